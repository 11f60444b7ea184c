// state_passing: the sequential inter-chunk recurrence
//   out[c] = s_c,  s_{c+1} = exp(dA_last[c]) * s_c + states[c],  final = s_nc
// over b * H independent rows of D = P * N float32 values.
//
// HBM-bound streaming kernel.  Each thread owns VW consecutive elements of one
// (batch, head) row and walks the chunks in order, keeping its running state
// in registers; loads and stores are 16 bytes per lane (8 for bf16 output)
// and contiguous across the workgroup.  Two walks:
//  * rows of at most DEPTH chunks (latency-bound shapes): every chunk's load is
//    issued up front, the walk waits once, and its combines and stores then
//    run with no wait between them (on this target a wait for a load also
//    waits for every store issued before it, so a load consumed after a store
//    serialises the walk on store acknowledgements);
//  * longer rows: chunk c + ROLL is loaded while chunk c is combined; the many
//    workgroups of such shapes keep HBM busy across those waits.
// The first loads are issued before anything else; while they are in flight
// the per-chunk decays (seq_idx resets applied) are computed into LDS, so
// neither a global load nor an exp sits on the walk's serial path.  The
// block size (64-256 threads) is chosen per shape so that short rows and few
// heads still spread over every CU.
//
// Follows reference kernels/state_passing_fwd.py:108-151 (recurrence),
// :208-225 (seq_idx reset: end-of-chunk id differs from the previous chunk's,
// previous id of chunk 0 is 0) and ops/ssd_naive.py:135-182.
#include "m2_internal.h"
#include "bmm_tile.h"

namespace {

constexpr int THREADS = 256;                 // largest block
constexpr int DEPTH = 16;                    // chunks of the one-batch walk
constexpr int ROLL = 8;                      // loads in flight in the rolling walk

template <int VW> struct Vec;
template <> struct Vec<4> {
    float v[4];
    M2_DEV void load(const float* p) {
        float4 t = *reinterpret_cast<const float4*>(p);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
    M2_DEV void store(float* p) const {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    }
    M2_DEV void store_nt(float* p) const {
        __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(p));
    }
    M2_DEV void store(bf16* p) const {
        typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
        bf16x4 t = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
        *reinterpret_cast<bf16x4*>(p) = t;
    }
};
template <> struct Vec<1> {
    float v[1];
    M2_DEV void load(const float* p) { v[0] = *p; }
    M2_DEV void store(float* p) const { *p = v[0]; }
    M2_DEV void store(bf16* p) const { *p = (bf16)v[0]; }
};

struct PassArgs {
    const float* states;
    const float* dAc;
    int64_t sb, sh, sc;
    const float* init;
    const int32_t* seq_idx;
    void* out;
    float* fin;
    int nc, H;
    int64_t D;
    int L, Q, blocks_per_row;
};

// the walk of block `block` (blockDim.x threads, `scl` nc floats of LDS);
// NT (fp32, VW 4, one-batch walk): non-temporal state stores
template <typename TO, int VW, bool ONE_BATCH, bool NT = false>
M2_DEV void pass_walk(const PassArgs& p, int block, float* scl) {
    const float* __restrict__ states = p.states;
    const float* __restrict__ dAc = p.dAc;
    const int64_t sb = p.sb, sh = p.sh, sc = p.sc;
    const float* __restrict__ init = p.init;
    const int32_t* __restrict__ seq_idx = p.seq_idx;
    TO* __restrict__ out = static_cast<TO*>(p.out);
    float* __restrict__ fin = p.fin;
    const int nc = p.nc, H = p.H, L = p.L, Q = p.Q, blocks_per_row = p.blocks_per_row;
    const int64_t D = p.D;
    const int row = block / blocks_per_row;               // (batch, head)
    const int blk = block % blocks_per_row;
    const int bi = row / H, h = row % H;
    const int64_t d0 = ((int64_t)blk * blockDim.x + threadIdx.x) * VW;
    const bool active = d0 < D;
    const int64_t cstride = (int64_t)H * D;                // between chunks
    const int64_t base = ((int64_t)bi * nc * H + h) * D + (active ? d0 : 0);
    const float* src = states + base;
    TO* dst = out + base;

    // one-batch walk: loads take the chunk index clamped to the last chunk, so
    // none is conditional and the compiler's wait analysis sees one batch
    Vec<VW> buf[ONE_BATCH ? DEPTH : ROLL], run;
    if (active) {
        if constexpr (ONE_BATCH) {
#pragma unroll
            for (int i = 0; i < DEPTH; ++i) buf[i].load(src + (int64_t)min(i, nc - 1) * cstride);
        } else {
#pragma unroll
            for (int i = 0; i < ROLL; ++i)
                if (i < nc) buf[i].load(src + i * cstride);
        }
        if (init) run.load(init + ((int64_t)bi * H + h) * D + d0);
    }
    if (!init || !active) {
#pragma unroll
        for (int j = 0; j < VW; ++j) run.v[j] = 0.f;
    }
    {
        const float* dAr = dAc + (int64_t)bi * sb + (int64_t)h * sh;
        for (int c = threadIdx.x; c < nc; c += blockDim.x) {
            float v = expf(dAr[(int64_t)c * sc]);
            if (seq_idx) {
                // reset where the chunk-end id differs from the previous
                // chunk's (0 before chunk 0)
                const int cur = seq_idx[(int64_t)bi * L + min((c + 1) * Q, L) - 1];
                const int prev = c > 0 ? seq_idx[(int64_t)bi * L + c * Q - 1] : 0;
                if (cur != prev) v = 0.f;
            }
            scl[c] = v;
        }
    }
    __syncthreads();
    if (!active) return;
    if constexpr (ONE_BATCH) {
        // nc <= DEPTH: one explicit wait (vmcnt 0) for all loads, so the
        // guarded stores below need none
        __builtin_amdgcn_s_waitcnt(0x0F70);
#pragma unroll
        for (int c = 0; c < DEPTH; ++c) {
            if (c < nc) {
                if constexpr (NT) run.store_nt(dst + (int64_t)c * cstride);
                else run.store(dst + (int64_t)c * cstride);
                const float scale = scl[c];
#pragma unroll
                for (int j = 0; j < VW; ++j) run.v[j] = fmaf(scale, run.v[j], buf[c].v[j]);
            }
        }
    } else {
        for (int c0 = 0; c0 < nc; c0 += ROLL) {
#pragma unroll
            for (int i = 0; i < ROLL; ++i) {
                const int c = c0 + i;
                if (c < nc) {
                    run.store(dst + (int64_t)c * cstride);
                    const float scale = scl[c];
                    const Vec<VW> st = buf[i];
                    if (c + ROLL < nc) buf[i].load(src + (int64_t)(c + ROLL) * cstride);
#pragma unroll
                    for (int j = 0; j < VW; ++j) run.v[j] = fmaf(scale, run.v[j], st.v[j]);
                }
            }
        }
    }
    if (fin) run.store(fin + ((int64_t)bi * H + h) * D + d0);
}

template <typename TO, int VW, bool ONE_BATCH>
__global__ void __launch_bounds__(THREADS) k_state_passing(PassArgs p) {
    extern __shared__ float scl[];                        // [nc] chunk decays
    pass_walk<TO, VW, ONE_BATCH>(p, blockIdx.x, scl);
}

// state_passing and the independent bmm_chunk of the same forward in one
// launch of 256-thread blocks: blocks below npass walk states, the others
// compute CB tiles (one launch less on the path, and the CB tiles fill the
// CUs the walk leaves idle)
template <int VW, bool ONE_BATCH, int CT, bool NT>
__global__ void __launch_bounds__(THREADS) k_pass_bmm(PassArgs p, m2::BmmTileArgs m, int npass) {
    extern __shared__ float scl[];
    if ((int)blockIdx.x < npass) pass_walk<float, VW, ONE_BATCH, NT>(p, blockIdx.x, scl);
    else m2::bmm_tile<float, float, CT>(m, xcd_remap(blockIdx.x - npass, m.nblocks));
}

PassArgs pass_args(const m2_state_passing_args& a, int bpr) {
    PassArgs p{};
    p.states = a.states; p.dAc = a.dA_chunk_cumsum;
    p.sb = a.dA_stride_batch; p.sh = a.dA_stride_head; p.sc = a.dA_stride_chunk;
    p.init = a.initial_states; p.seq_idx = a.seq_idx; p.out = a.out; p.fin = a.final_states;
    p.nc = (int)a.nchunks; p.H = (int)a.nheads; p.D = a.dim; p.L = (int)a.seqlen;
    p.Q = (int)a.chunk_size; p.blocks_per_row = bpr;
    return p;
}

template <typename TO>
int launch_typed(const m2_state_passing_args& a, hipStream_t s) {
    const int vw = (a.dim % 4 == 0) ? 4 : 1;
    // the largest block (of 64 / 128 / 256 threads) that still gives ~4
    // workgroups per CU
    int bs = THREADS;
    while (bs > 64 && a.batch * a.nheads * ((a.dim + (int64_t)bs * vw - 1) / ((int64_t)bs * vw)) < 1024)
        bs /= 2;
    const int64_t per_block = (int64_t)bs * vw;
    const int bpr = (int)((a.dim + per_block - 1) / per_block);
    const int64_t nblocks = a.batch * a.nheads * bpr;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "state_passing: too many blocks");
    M2_REQUIRE(a.nchunks <= 16384, M2_ERR_UNSUPPORTED, "state_passing: more than 16384 chunks");
    const size_t shm = (size_t)a.nchunks * sizeof(float);
    const bool one = a.nchunks <= DEPTH;
    auto kern = vw == 4 ? (one ? k_state_passing<TO, 4, true> : k_state_passing<TO, 4, false>)
                        : (one ? k_state_passing<TO, 1, true> : k_state_passing<TO, 1, false>);
    kern<<<(unsigned)nblocks, bs, shm, s>>>(pass_args(a, bpr));
    return m2::check_launch("state_passing");
}

}  // namespace

namespace m2 {

int check_state_passing_args(const m2_state_passing_args& a) {
    M2_REQUIRE(a.states && a.dA_chunk_cumsum && a.out, M2_ERR_INVALID,
               "state_passing: states, dA_chunk_cumsum and out are required");
    M2_REQUIRE(a.batch > 0 && a.nchunks > 0 && a.nheads > 0 && a.dim > 0, M2_ERR_INVALID,
               "state_passing: sizes must be positive");
    M2_REQUIRE(!a.seq_idx || (a.chunk_size > 0 && a.seqlen > 0 &&
                              a.seqlen > (a.nchunks - 1) * a.chunk_size &&
                              a.seqlen <= a.nchunks * a.chunk_size),
               M2_ERR_INVALID, "state_passing: seq_idx needs chunk_size and a seqlen that "
               "spans nchunks chunks");
    M2_REQUIRE(a.nchunks <= 16384, M2_ERR_UNSUPPORTED, "state_passing: more than 16384 chunks");
    return M2_OK;
}

bool state_passing_bmm_supported(const m2_state_passing_args& p, const m2_bmm_chunk_args& m) {
    return p.out_dtype == M2_F32 && m.dtype == M2_F32 && m.out_dtype == M2_F32 &&
           bmm_uses_tiles(m);
}

int launch_state_passing_bmm(const m2_state_passing_args& a, const m2_bmm_chunk_args& m,
                             hipStream_t s) {
    M2_REQUIRE(state_passing_bmm_supported(a, m), M2_ERR_UNSUPPORTED,
               "state_passing + bmm_chunk: fp32 with the tiled bmm_chunk kernel only");
    int rc;
    if ((rc = check_state_passing_args(a)) || (rc = check_bmm_chunk_args(m))) return rc;
    BmmTileArgs mt;
    const int ct = bmm_tile_plan(m, mt);
    const int vw = (a.dim % 4 == 0) ? 4 : 1;
    const int64_t per_block = (int64_t)THREADS * vw;
    const int bpr = (int)((a.dim + per_block - 1) / per_block);
    const int64_t npass = a.batch * a.nheads * bpr;
    M2_REQUIRE(mt.nblocks > 0 && npass + mt.nblocks < (1ll << 31), M2_ERR_UNSUPPORTED,
               "state_passing + bmm_chunk: too many blocks");
    const bool one = a.nchunks <= DEPTH;
    // Small passed states (at most 16 MiB, the fp32 mamba2-130m layer: 12 MiB)
    // leave non-temporally: there state_passing + bmm_chunk took 9.5 against
    // 11.3 us and the layer 34.6 against 35.5 us (A/B on one box), no dirty
    // state lines remaining in L2 for the end of the kernel.  At batch 2 / 4
    // (24 / 48 MiB) the scan, which reads them next, then lost more than the
    // walk gained (layer 54.4 against 50.9 us, 89.4 against 84.7).
    const bool nt = vw == 4 && one &&
                    (double)a.batch * a.nchunks * a.nheads * a.dim * 4 <= 16.0 * (1 << 20);
    void (*kern)(PassArgs, BmmTileArgs, int) = nullptr;
#define M2_PB_CASE(VWV, ONEV, CTV) \
    if (vw == VWV && one == ONEV && ct == CTV) kern = k_pass_bmm<VWV, ONEV, CTV, false>;
#define M2_PB_NT(CTV) \
    if (nt && ct == CTV) kern = k_pass_bmm<4, true, CTV, true>;
#define M2_PB_CT(VWV, ONEV) M2_PB_CASE(VWV, ONEV, 1) M2_PB_CASE(VWV, ONEV, 2) \
                            M2_PB_CASE(VWV, ONEV, 3) M2_PB_CASE(VWV, ONEV, 4)
    M2_PB_CT(4, true) M2_PB_CT(4, false) M2_PB_CT(1, true) M2_PB_CT(1, false)
    M2_PB_NT(1) M2_PB_NT(2) M2_PB_NT(3) M2_PB_NT(4)
#undef M2_PB_CT
#undef M2_PB_NT
#undef M2_PB_CASE
    M2_REQUIRE(kern, M2_ERR_UNSUPPORTED, "state_passing + bmm_chunk: chunk_size %lld",
               (long long)m.chunk_size);
    const size_t shm = (size_t)a.nchunks * sizeof(float);
    kern<<<(unsigned)(npass + mt.nblocks), THREADS, shm, s>>>(pass_args(a, bpr), mt, (int)npass);
    return check_launch("state_passing + bmm_chunk");
}

int launch_state_passing(const m2_state_passing_args& a, hipStream_t s) {
    int rc;
    if ((rc = check_state_passing_args(a))) return rc;
    if (a.out_dtype == M2_F32) return launch_typed<float>(a, s);
    if (a.out_dtype == M2_BF16) return launch_typed<bf16>(a, s);
    return set_error(M2_ERR_UNSUPPORTED, "state_passing: out dtype %d", a.out_dtype);
}

}  // namespace m2
