// Internal launchers shared by the per-stage entry points and m2_ssd_combined.
// Each validates its arguments, enqueues its kernel(s) on `stream` and returns
// an M2_* code (the message goes to m2_last_error).
#pragma once

#include "m2_common.h"

namespace m2 {
// The value m2_set_dispatch_override last set for a knob (M2_KNOB_*); 0 =
// the automatic choice.
int dispatch_override(int knob);
// compute units of the current device (queried once per device)
int cu_count();

int launch_chunk_cumsum(const m2_chunk_cumsum_args& a, hipStream_t stream);
// chunk_cumsum that also writes the chunk-state weights wts [b, H, nc, Q] and
// the carried-state decay scl [b, H, nc] (seq_idx rules applied) when non-NULL
int launch_chunk_cumsum_ex(const m2_chunk_cumsum_args& a, const int32_t* seq_idx, float* wts,
                           float* scl, hipStream_t stream);
int launch_chunk_state(const m2_chunk_state_args& a, hipStream_t stream);
bool chunk_state_cumsum_supported(const m2_chunk_cumsum_args& c1, const m2_chunk_state_args& a);
int launch_chunk_state_cumsum(const m2_chunk_cumsum_args& c1, const m2_chunk_state_args& a,
                              hipStream_t stream);
int launch_state_passing(const m2_state_passing_args& a, hipStream_t stream);
int launch_bmm_chunk(const m2_bmm_chunk_args& a, hipStream_t stream);
bool bmm_uses_tiles(const m2_bmm_chunk_args& a);
int check_bmm_chunk_args(const m2_bmm_chunk_args& a);
// state_passing (fp32 out) and bmm_chunk (fp32 in and out, tiled kernel) in one launch
bool state_passing_bmm_supported(const m2_state_passing_args& p, const m2_bmm_chunk_args& m);
int launch_state_passing_bmm(const m2_state_passing_args& p, const m2_bmm_chunk_args& m,
                             hipStream_t stream);
int launch_chunk_scan(const m2_chunk_scan_args& a, hipStream_t stream);
// chunk_scan for fp32 x / C / CB / states at chunk 128, head dim 64, dstate 64 /
// 128: one workgroup per (batch, chunk, group, slice of the group's heads)
// (csrc/scan_f32g.hip)
bool scan_f32g_supported(const m2_chunk_scan_args& a);
int launch_scan_f32g(const m2_chunk_scan_args& a, hipStream_t stream);
// the same kernel in the combined forward, building CB = C B^T itself (no
// bmm_chunk launch): fp32 inputs at the internal chunk 128, head dim 64,
// dstate 64 / 128
bool scan_f32g_layer_supported(const m2_ssd_combined_args& a);
int launch_scan_f32g_layer(const m2_ssd_combined_args& a, const float* dA, const float* dt_out,
                           const void* states_passed, hipStream_t stream);
int scan_f32g_heads_per_wg(int64_t batch, int64_t nc, int64_t G, int64_t hpg, int64_t N, bool cbb);
int launch_chunk_state_varlen(const m2_chunk_state_varlen_args& a, hipStream_t stream);
int launch_ssu(const m2_ssu_args& a, hipStream_t stream);
int launch_causal_conv1d(const m2_causal_conv1d_args& a, hipStream_t stream);
int launch_causal_conv1d_update(const m2_causal_conv1d_update_args& a, hipStream_t stream);
int launch_rms_norm_gated(const m2_rms_norm_gated_args& a, hipStream_t stream);
int launch_skinny_gemm(const m2_skinny_gemm_args& a, hipStream_t stream);
int launch_skinny_gemm_norm(const m2_skinny_gemm_norm_args& a, hipStream_t stream);

// chunk_state_varlen for bf16, head dim 64, dstate % 64 == 0, chunk_size % 32
// == 0 (<= 256): one workgroup per (sequence, head, 64-column dstate block)
bool varlen_states_fast_supported(const m2_chunk_state_varlen_args& a);
int launch_varlen_states(const m2_chunk_state_varlen_args& a, hipStream_t stream);
bool chunk_state_fast_supported(const m2_chunk_state_args& a);
int launch_chunk_state_fast(const m2_chunk_state_args& a, hipStream_t stream);

// Arguments of the fused bmm_chunk + chunk_scan kernels (one workgroup per
// (batch, chunk, group, slice of the group's heads)).
struct ScanFusedArgs {
    const bf16* x;
    const bf16* B;
    const bf16* C;
    const bf16* states;    // state entering each chunk, [b, nc, H, P, N]
    const float* dt;       // [b, H, nc, Q]
    const float* dA;       // [b, H, nc, Q]
    const float* D;
    const bf16* z;
    const int32_t* seq_idx;
    const void* cb;        // given CB [b, nc, G, Q, Q] (fp32 or bf16), or NULL: built here
    float* out;
    int D_has_hdim, cb_bf16;
    int L, H, G, nc, hpg, nwork;
    int hps, nslice;          // heads per workgroup (a slice of the group's), slices
    int ntl;                  // chunk-128 kernel: x / state rows loaded non-temporally
};
// the chunk-128 scan kernel (csrc/ssd_scan128.hip) for dstate 32 * ns (ns 2, 4,
// 8), with the z gate / with CB given / with non-temporal output stores (not
// with CB given); NULL for other sizes; its block size
typedef void (*ScanKernel)(ScanFusedArgs);
ScanKernel scan_q128_kernel(int ns, bool hasz, bool cbin, bool nt);
constexpr int SCAN_Q128_THREADS = 768;

// fused bmm_chunk + chunk_scan of the combined forward (bf16 inputs)
bool scan_fused_supported(int64_t headdim, int64_t dstate, int64_t chunk_size);
bool scan_fused_cb_supported(const m2_chunk_scan_args& a);
int launch_scan_fused_cb(const m2_chunk_scan_args& a, hipStream_t stream);
int launch_scan_fused(const m2_ssd_combined_args& a, const float* dA, const float* dt_out,
                      const void* states_passed, hipStream_t stream);

// m2_ssd_combined over the workspace `ws` of `ws_bytes` (the argument
// struct's own workspace fields are not read)
int ssd_combined_on(const m2_ssd_combined_args& a, void* ws, size_t ws_bytes, hipStream_t stream);

// chunk_state + state_passing of the combined forward in one chunk-sequential
// pass, from the weights / decay of launch_chunk_cumsum_ex; writes the states
// entering each chunk (in the input dtype) and the final states.  bf16 inputs
// (csrc/ssd_states.hip), and fp32 inputs where the pass fills the CUs
// (csrc/ssd_states_f32.hip; launch_states_fused dispatches on the dtype)
bool states_fused_supported(const m2_ssd_combined_args& a);
int launch_states_fused(const m2_ssd_combined_args& a, const float* wts, const float* scl,
                        void* states_passed, hipStream_t stream);
bool states_fused_f32_supported(const m2_ssd_combined_args& a);
int launch_states_fused_f32(const m2_ssd_combined_args& a, const float* wts, const float* scl,
                            void* states_passed, hipStream_t stream);
}  // namespace m2
