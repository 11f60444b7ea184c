// C-ABI plumbing: thread-local error messages, version, the per-stage entry
// points, and m2_ssd_combined (the whole forward over a caller workspace).
#include <stdarg.h>
#include <stdio.h>

#include <atomic>

#include "m2_internal.h"

namespace m2 {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return set_error(M2_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
    return M2_OK;
}

constexpr int NKNOBS = 4;
static std::atomic<int> g_knob[NKNOBS];

int dispatch_override(int knob) {
    return knob >= 0 && knob < NKNOBS ? g_knob[knob].load(std::memory_order_relaxed) : 0;
}

// compute units of the current device, queried once per device (256 on
// MI355X); 256 where the query fails
int cu_count() {
    constexpr int MAXDEV = 64;
    static std::atomic<int> cache[MAXDEV];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAXDEV) return 256;
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        n = 256;
    cache[dev].store(n, std::memory_order_relaxed);
    return n;
}

}  // namespace m2

extern "C" const char* m2_last_error(void) { return m2::g_err; }
extern "C" int m2_abi_version(void) { return M2SSD_ABI_VERSION; }

extern "C" int m2_set_dispatch_override(int knob, int value) {
    static const int maxval[m2::NKNOBS] = {3, 2, 1, 65};
    if (knob < 0 || knob >= m2::NKNOBS || value < 0 || value > maxval[knob])
        return m2::set_error(M2_ERR_INVALID, "m2_set_dispatch_override: knob %d value %d", knob,
                             value);
    return m2::g_knob[knob].exchange(value, std::memory_order_relaxed);
}

#define M2_ENTRY(name, T, launcher)                                  \
    extern "C" int name(const T* a, void* stream) {                  \
        if (!a) return m2::set_error(M2_ERR_INVALID, #name ": NULL args"); \
        return m2::launcher(*a, (hipStream_t)stream);                \
    }

M2_ENTRY(m2_chunk_cumsum, m2_chunk_cumsum_args, launch_chunk_cumsum)
M2_ENTRY(m2_chunk_state, m2_chunk_state_args, launch_chunk_state)
M2_ENTRY(m2_state_passing, m2_state_passing_args, launch_state_passing)
M2_ENTRY(m2_bmm_chunk, m2_bmm_chunk_args, launch_bmm_chunk)
M2_ENTRY(m2_chunk_scan, m2_chunk_scan_args, launch_chunk_scan)
M2_ENTRY(m2_chunk_state_varlen, m2_chunk_state_varlen_args, launch_chunk_state_varlen)
M2_ENTRY(m2_selective_state_update, m2_ssu_args, launch_ssu)
M2_ENTRY(m2_causal_conv1d, m2_causal_conv1d_args, launch_causal_conv1d)
M2_ENTRY(m2_causal_conv1d_update, m2_causal_conv1d_update_args, launch_causal_conv1d_update)
M2_ENTRY(m2_rms_norm_gated, m2_rms_norm_gated_args, launch_rms_norm_gated)
M2_ENTRY(m2_skinny_gemm, m2_skinny_gemm_args, launch_skinny_gemm)
M2_ENTRY(m2_skinny_gemm_norm, m2_skinny_gemm_norm_args, launch_skinny_gemm_norm)

// ---------------------------------------------------------------------------
// combined forward
// ---------------------------------------------------------------------------
namespace {

struct Layout {
    size_t dA, dt, wts, scl, states, passed, cb, total;
};

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// fp32 at chunk 128, head dim 64: the group scan builds CB itself, except
// where the staged path runs bmm_chunk in the state_passing launch (fewer
// than 128 (chunk, group) blocks), whose CB blocks fill CUs the walk leaves
// idle: mamba2-130m 37.2 us that way against 39.8 us with CB built in the
// scan (its 12 slices per group each load B).
bool layer_scan_builds_cb(const m2_ssd_combined_args& a) {
    if (!m2::scan_f32g_layer_supported(a)) return false;
    if (m2::states_fused_supported(a)) return true;
    m2_bmm_chunk_args m{};
    m.batch = a.batch; m.seqlen = a.seqlen; m.ngroups = a.ngroups; m.k = a.dstate;
    m.chunk_size = a.chunk_size; m.dtype = M2_F32; m.out_dtype = M2_F32;
    return !m2::bmm_uses_tiles(m);
}

Layout layout_of(const m2_ssd_combined_args& a) {
    // slots the fused kernels make unnecessary are left empty: the fp32 chunk
    // states (chunk_state + state_passing fused, which need the weights and
    // decay instead) and CB (bmm_chunk fused)
    Layout l{};
    const int64_t nc = (a.seqlen + a.chunk_size - 1) / a.chunk_size;
    const size_t es = m2_dtype_size(a.dtype);
    const size_t bhcq = (size_t)a.batch * a.nheads * nc * a.chunk_size;
    const size_t S = (size_t)a.batch * nc * a.nheads * a.headdim * a.dstate;
    const bool states_fused = m2::states_fused_supported(a);
    const bool scan_fused = (a.dtype == M2_BF16 &&
                             m2::scan_fused_supported(a.headdim, a.dstate, a.chunk_size)) ||
                            layer_scan_builds_cb(a);
    size_t off = 0;
    l.dA = off;     off += align256(bhcq * 4);
    l.dt = off;     off += align256(bhcq * 4);
    l.wts = off;    off += states_fused ? align256(bhcq * 4) : 0;
    l.scl = off;    off += states_fused ? align256((size_t)a.batch * a.nheads * nc * 4) : 0;
    l.states = off; off += states_fused ? 0 : align256(S * 4);
    l.passed = off; off += align256(S * es);
    l.cb = off;
    off += scan_fused ? 0 : align256((size_t)a.batch * nc * a.ngroups * a.chunk_size * a.chunk_size * es);
    l.total = off;
    return l;
}

int record(void** ev, int i, hipStream_t s) {
    if (!ev || !ev[i]) return M2_OK;
    if (hipEventRecord((hipEvent_t)ev[i], s) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "m2_ssd_combined: hipEventRecord failed");
    return M2_OK;
}

// The combined forward returns only y and the final (and varlen) states: the
// same function of the inputs for every chunk size (the chunked algorithm is
// exact; only the rounding points at chunk boundaries move).  bf16 chunk
// sizes the fused kernels do not take (256: the fused scan keeps at most 128
// positions of a chunk in LDS; 32; ...) run as chunks of 128 when that puts
// both halves of the layer on the fused kernels; fp32 chunks of 256 always
// run as chunks of 128; chunk sizes other than 64, 128 and 256 run as chunks
// of 128 (the tile sizes every kernel of the layer is built and tested for).
bool layer_fused(const m2_ssd_combined_args& a) {
    return m2::states_fused_supported(a) &&
           m2::scan_fused_supported(a.headdim, a.dstate, a.chunk_size);
}

m2_ssd_combined_args internal_args(const m2_ssd_combined_args& a0) {
    m2_ssd_combined_args a = a0;
    if (a0.dtype == M2_BF16 && a0.chunk_size != 128 && !layer_fused(a0)) {
        a.chunk_size = 128;
        if (!layer_fused(a)) a.chunk_size = a0.chunk_size;
    }
    // fp32 has no rounding points at chunk boundaries: chunks of 128 give the
    // same result up to fp32 summation order, with twice the workgroups and
    // half the intra-chunk work
    if (a0.dtype == M2_F32 && a0.chunk_size == 256) a.chunk_size = 128;
    if (a.chunk_size > 0 && a.chunk_size != 64 && a.chunk_size != 128 && a.chunk_size != 256)
        a.chunk_size = 128;
    return a;
}

}  // namespace

extern "C" size_t m2_ssd_combined_workspace_size(const m2_ssd_combined_args* a) {
    if (!a || a->chunk_size <= 0 || !m2_dtype_size(a->dtype)) return 0;
    return layout_of(internal_args(*a)).total;
}

extern "C" int m2_ssd_combined(const m2_ssd_combined_args* ap, void* stream_) {
    if (!ap) return m2::set_error(M2_ERR_INVALID, "m2_ssd_combined: NULL args");
    return m2::ssd_combined_on(*ap, ap->workspace, ap->workspace_bytes, (hipStream_t)stream_);
}

// The whole forward over the workspace ws (ws_bytes long): both entry points
// (m2_ssd_combined with the caller's workspace, m2_ssd_combined_noalloc with
// the library's static scratch) run this.
int m2::ssd_combined_on(const m2_ssd_combined_args& a0, void* workspace, size_t workspace_bytes,
                        hipStream_t s) {
    const m2_ssd_combined_args a = internal_args(a0);
    M2_REQUIRE(a.chunk_size > 0 && a.batch > 0 && a.seqlen > 0, M2_ERR_INVALID,
               "m2_ssd_combined: batch, seqlen and chunk_size must be positive");
    M2_REQUIRE(m2_dtype_size(a.dtype) != 0, M2_ERR_UNSUPPORTED, "m2_ssd_combined: dtype %d", a.dtype);
    M2_REQUIRE(a.x && a.dt && a.A && a.B && a.C && a.out, M2_ERR_INVALID,
               "m2_ssd_combined: x, dt, A, B, C and out are required");
    M2_REQUIRE(!a.varlen_states || (a.cu_seqlens && a.batch == 1 && a.nseq > 0), M2_ERR_INVALID,
               "m2_ssd_combined: varlen states need cu_seqlens, nseq > 0 and batch == 1");
    const Layout l = layout_of(a);
    M2_REQUIRE(workspace && workspace_bytes >= l.total, M2_ERR_WORKSPACE,
               "m2_ssd_combined: workspace of %zu bytes needed, %zu given", l.total,
               workspace_bytes);
    char* ws = (char*)workspace;
    float* dA = (float*)(ws + l.dA);
    float* dto = (float*)(ws + l.dt);
    float* states = (float*)(ws + l.states);
    void* passed = ws + l.passed;
    void* cb = ws + l.cb;
    const int64_t nc = (a.seqlen + a.chunk_size - 1) / a.chunk_size;
    int rc;
    bool cb_done = false;                   // CB already computed (with state_passing)
    const bool scan_cb = layer_scan_builds_cb(a);   // fp32: CB built in the group scan
    if ((rc = record(a.stage_events, 0, s))) return rc;

    if (m2::states_fused_supported(a)) {
        // cumsum (+ weights and decay), then chunk states and state passing in
        // one kernel: its time lands in the second event interval, the third is
        // empty
        m2_chunk_cumsum_args c1{};
        c1.dt = a.dt; c1.A = a.A; c1.dt_bias = a.dt_bias; c1.dA_cumsum = dA; c1.dt_out = dto;
        c1.batch = a.batch; c1.seqlen = a.seqlen; c1.nheads = a.nheads; c1.chunk_size = a.chunk_size;
        c1.dt_dtype = a.dt_dtype; c1.dt_softplus = a.dt_softplus; c1.dt_min = a.dt_min; c1.dt_max = a.dt_max;
        float* wts = (float*)(ws + l.wts);
        float* scl = (float*)(ws + l.scl);
        if ((rc = m2::launch_chunk_cumsum_ex(c1, a.seq_idx, wts, scl, s))) return rc;
        if ((rc = record(a.stage_events, 1, s))) return rc;
        if ((rc = m2::launch_states_fused(a, wts, scl, passed, s))) return rc;
        if ((rc = record(a.stage_events, 2, s))) return rc;
        if ((rc = record(a.stage_events, 3, s))) return rc;
    } else {
        m2_chunk_cumsum_args c1{};
        c1.dt = a.dt; c1.A = a.A; c1.dt_bias = a.dt_bias; c1.dA_cumsum = dA; c1.dt_out = dto;
        c1.batch = a.batch; c1.seqlen = a.seqlen; c1.nheads = a.nheads; c1.chunk_size = a.chunk_size;
        c1.dt_dtype = a.dt_dtype; c1.dt_softplus = a.dt_softplus; c1.dt_min = a.dt_min; c1.dt_max = a.dt_max;
        m2_chunk_state_args c2{};
        c2.x = a.x; c2.B = a.B; c2.dt = dto; c2.dA_cumsum = dA; c2.seq_idx = a.seq_idx; c2.states = states;
        c2.batch = a.batch; c2.seqlen = a.seqlen; c2.nheads = a.nheads; c2.headdim = a.headdim;
        c2.ngroups = a.ngroups; c2.dstate = a.dstate; c2.chunk_size = a.chunk_size; c2.dtype = a.dtype;
        // fp32: chunk_cumsum inside the chunk_state kernel where it covers the
        // shape (the cumsum event interval then stays empty)
        if (m2::chunk_state_cumsum_supported(c1, c2)) {
            if ((rc = record(a.stage_events, 1, s))) return rc;
            if ((rc = m2::launch_chunk_state_cumsum(c1, c2, s))) return rc;
        } else {
            if ((rc = m2::launch_chunk_cumsum(c1, s))) return rc;
            if ((rc = record(a.stage_events, 1, s))) return rc;
            if ((rc = m2::launch_chunk_state(c2, s))) return rc;
        }
        if ((rc = record(a.stage_events, 2, s))) return rc;

        m2_state_passing_args c3{};
        c3.states = states; c3.dA_chunk_cumsum = dA + (a.chunk_size - 1);
        c3.dA_stride_batch = a.nheads * nc * a.chunk_size; c3.dA_stride_head = nc * a.chunk_size;
        c3.dA_stride_chunk = a.chunk_size;
        c3.initial_states = a.initial_states; c3.seq_idx = a.seq_idx; c3.out = passed;
        c3.final_states = a.final_states;
        c3.batch = a.batch; c3.nchunks = nc; c3.nheads = a.nheads; c3.dim = a.headdim * a.dstate;
        c3.seqlen = a.seqlen; c3.chunk_size = a.chunk_size; c3.out_dtype = a.dtype;
        // fp32 with the tiled bmm_chunk kernel: bmm_chunk (independent of the
        // state chain) in the same launch as state_passing; its time lands in
        // the bmm_chunk event interval
        m2_bmm_chunk_args c4{};
        c4.a = a.C; c4.b = a.B; c4.seq_idx = a.seq_idx; c4.out = cb;
        c4.batch = a.batch; c4.seqlen = a.seqlen; c4.ngroups = a.ngroups; c4.k = a.dstate;
        c4.chunk_size = a.chunk_size; c4.dtype = a.dtype; c4.out_dtype = a.dtype; c4.causal = 0;
        if (!scan_cb && m2::state_passing_bmm_supported(c3, c4)) {
            if ((rc = record(a.stage_events, 3, s))) return rc;
            if ((rc = m2::launch_state_passing_bmm(c3, c4, s))) return rc;
            cb_done = true;
        } else {
            if ((rc = m2::launch_state_passing(c3, s))) return rc;
            if ((rc = record(a.stage_events, 3, s))) return rc;
        }
    }

    // the packed sequences' final states: they read the passed states and x of
    // the chunks where sequences end
    auto varlen = [&]() -> int {
        m2_chunk_state_varlen_args c6{};
        c6.B = a.B; c6.x = a.x; c6.dt = dto; c6.dA_cumsum = dA; c6.cu_seqlens = a.cu_seqlens;
        c6.chunk_states = passed; c6.out = a.varlen_states;
        c6.seqlen = a.seqlen; c6.nseq = a.nseq; c6.nheads = a.nheads; c6.headdim = a.headdim;
        c6.ngroups = a.ngroups; c6.dstate = a.dstate; c6.nchunks = nc; c6.chunk_size = a.chunk_size;
        c6.dtype = a.dtype; c6.states_dtype = a.dtype;
        int r;
        if ((r = m2::launch_chunk_state_varlen(c6, s))) return r;
        return record(a.stage_events, 6, s);
    };
    if (a.dtype == M2_BF16 && m2::scan_fused_supported(a.headdim, a.dstate, a.chunk_size)) {
        // The varlen states run before the scan here: where the passed states
        // exceed the cache the scan reads them and x non-temporally, after
        // which they would come from HBM again (c3 varlen states 57 against
        // 42 us; layer 0.531 against 0.525 ms, A/B on one box).  Their event
        // (6) is then recorded before events 4 and 5.
        if (a.varlen_states && (rc = varlen())) return rc;
        // CB is built inside the scan kernel: the bmm interval stays empty
        if ((rc = record(a.stage_events, 4, s))) return rc;
        if ((rc = m2::launch_scan_fused(a, dA, dto, passed, s))) return rc;
        if ((rc = record(a.stage_events, 5, s))) return rc;
        return M2_OK;
    } else if (scan_cb) {
        if ((rc = record(a.stage_events, 4, s))) return rc;
        if ((rc = m2::launch_scan_f32g_layer(a, dA, dto, passed, s))) return rc;
        if ((rc = record(a.stage_events, 5, s))) return rc;
    } else {
        if (!cb_done) {
            m2_bmm_chunk_args c4{};
            c4.a = a.C; c4.b = a.B; c4.seq_idx = a.seq_idx; c4.out = cb;
            c4.batch = a.batch; c4.seqlen = a.seqlen; c4.ngroups = a.ngroups; c4.k = a.dstate;
            c4.chunk_size = a.chunk_size; c4.dtype = a.dtype; c4.out_dtype = a.dtype; c4.causal = 0;
            if ((rc = m2::launch_bmm_chunk(c4, s))) return rc;
        }
        if ((rc = record(a.stage_events, 4, s))) return rc;

        m2_chunk_scan_args c5{};
        c5.cb = cb; c5.x = a.x; c5.dt = dto; c5.dA_cumsum = dA; c5.C = a.C; c5.states = passed;
        c5.D = a.D; c5.z = a.z; c5.seq_idx = a.seq_idx; c5.out = a.out; c5.out_x = nullptr;
        c5.batch = a.batch; c5.seqlen = a.seqlen; c5.nheads = a.nheads; c5.headdim = a.headdim;
        c5.ngroups = a.ngroups; c5.dstate = a.dstate; c5.chunk_size = a.chunk_size;
        c5.dtype = a.dtype; c5.cb_dtype = a.dtype; c5.states_dtype = a.dtype; c5.D_has_hdim = a.D_has_hdim;
        if ((rc = m2::launch_chunk_scan(c5, s))) return rc;
        if ((rc = record(a.stage_events, 5, s))) return rc;
    }

    if (a.varlen_states && (rc = varlen())) return rc;
    return M2_OK;
}
