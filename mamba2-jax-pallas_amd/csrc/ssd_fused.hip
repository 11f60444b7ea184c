// Fused kernels of the combined forward for bf16 inputs.
//
// k_scan_fused = bmm_chunk + chunk_scan.  One workgroup per (batch, chunk,
// group, block of HB heads of that group), 4 wavefronts.  Everything that is
// shared by the heads of a group is built once per workgroup and kept in
// registers:
//   * C-row fragments of the wavefront's output rows (MFMA A operand of the
//     carried-state product),
//   * CB = C B^T of the chunk, computed as CB^T tiles with 16x16x32 MFMAs
//     (A = B rows, B = the C fragments).  The accumulator layout of a CB^T
//     tile (lane = column m, 4 consecutive rows k) is exactly the A-operand
//     layout of a 16x16x16 MFMA (lane = row m, 4 consecutive k), so the tiles
//     feed the intra-chunk product without any data movement.  CB is rounded
//     to bf16 and seq_idx-masked as the reference's bmm_chunk output is.
// The output rows of a chunk are split into pairs of 16-row tiles (t, Q/16-1-t)
// so that every wavefront does the same amount of causal (triangular) work; a
// pair's CB tiles occupy exactly Q/16+1 register slots.
// The group's B tile is staged in LDS once (all loads in flight); per head,
// x rows [Q x P] and the carried state [P x N] (bf16) are committed to LDS from
// registers that were prefetched during the previous head's compute; each
// wavefront then, for each of its row tiles,
//   1. multiplies its C rows by the state (16x16x32 MFMAs), rounds that
//      product to bf16 and scales it by exp(dA[m]) (reference ops/ssd_naive.py
//      :294-297),
//   2. adds sum_k CB[m,k] exp(dA[m]-dA[k]) dt[k] x[k,:] over k <= m, the
//      weighted operand split into bf16 hi + lo parts (near-fp32 accuracy),
//   3. applies D x and the silu(z) gate and stores fp32 y.
//
// Follows reference ops/ssd_naive.py:189-318 and kernels/chunk_scan_fwd.py
// :294-322 / kernels/bmm_chunk_fwd.py:353-372 (seq_idx masks).
#include "m2_internal.h"

namespace {

constexpr int THREADS = 256;
constexpr int HB = 4;  // heads per workgroup

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;

M2_DEV f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
M2_DEV f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
M2_DEV bf16x8 zero8() {
    bf16x8 z;
#pragma unroll
    for (int j = 0; j < 8; ++j) z[j] = (bf16)0.f;
    return z;
}
M2_DEV float rbf(float v) { return (float)(bf16)v; }

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
    float* out;
    int D_has_hdim;
    int L, H, G, nc, nhb, nblocks;
};

// LDS row strides (elements); state rows are padded by 16 bytes so that each
// quarter-wave's 16-byte reads hit 64 distinct banks.
template <int NS, int QT>
struct ScanShape {
    static constexpr int PT = 4, P = 64, N = 32 * NS, Q = 16 * QT;
    // x is kept transposed, [P][SQ]: a 16x16x16 B fragment (4 consecutive
    // positions of one column p) is one 8-byte read; SQ/2 = 4 * odd spreads
    // the 16 rows of a quarter-wave over distinct bank quads.
    static constexpr int SQ = Q + 8, SS = N + 8;
    static constexpr int NPAIRS = QT / 2, NSLOT = QT + 1;
};

// Register budget: LDS allows 2 workgroups per CU, i.e. 2 waves per SIMD.
template <int NS, int QT>
__global__ void __launch_bounds__(THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_scan_fused(ScanFusedArgs a) {
    typedef ScanShape<NS, QT> X;
    constexpr int PT = X::PT, P = X::P, N = X::N, Q = X::Q, SQ = X::SQ, SS = X::SS;
    constexpr int NPAIRS = X::NPAIRS, NSLOT = X::NSLOT;
    constexpr int XV = Q * P / 8 / THREADS;    // 16-byte vectors per thread: x tile
    constexpr int SV = P * N / 8 / THREADS;    //                              state
    constexpr int BV = Q * N / 8 / THREADS;    //                              B tile
    constexpr int SB = N + 8;                  // LDS row stride of the B tile
    static_assert(NPAIRS <= 4, "one row-tile pair per wavefront");
    static_assert(XV >= 1 && SV >= 1 && BV >= 1, "tiles too small for the workgroup");
    constexpr int XSB = (P * SQ + P * SS) > Q * SB ? (P * SQ + P * SS) : Q * SB;
    // xs (x transposed) / ss hold one head's x and state; before the head loop
    // the same bytes hold the group's B tile [Q][SB].
    __shared__ __align__(16) bf16 xsb[XSB];
    bf16* const xs = xsb;
    bf16* const ss = xsb + P * SQ;
    bf16* const bs = xsb;
    __shared__ __align__(16) bf16x4 cbl[4][NSLOT][64];   // per-wavefront CB^T tiles
    __shared__ __align__(16) float dAs[Q];                 // dA_cumsum * log2(e)
    __shared__ __align__(16) float dts[Q];
    __shared__ int seqs[Q];

    const int L = a.L, H = a.H, G = a.G, nc = a.nc;
    const int hpg = H / G;
    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int hb = work % a.nhb;
    int rest = work / a.nhb;
    const int g = rest % G;
    rest /= G;
    const int ci = rest % nc;
    const int bi = rest / nc;
    const int h0 = g * hpg + hb * HB;
    const int nh = min(HB, hpg - hb * HB);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int ln = lane & 15, kg = lane >> 4;
    const int64_t tok0 = (int64_t)bi * L + (int64_t)ci * Q;
    const int valid = min(Q, L - ci * Q);
    const int64_t rs = (int64_t)G * N;                       // row stride of B / C
    constexpr float LOG2E = 1.4426950408889634f;
    const bf16* Cg = a.C + (tok0 * G + g) * N + kg * 8;
    const int seq_prev = (a.seq_idx && ci > 0) ? a.seq_idx[tok0 - 1] : 0;

    // ---- register prefetch of one head's x rows, state, dA and dt ----------
    uint4 px[XV], ps[SV];
    float pdA = 0.f, pdt = 0.f;
#define M2_PREFETCH(HEAD)                                                                    \
    {                                                                                        \
        _Pragma("unroll") for (int u = 0; u < XV; ++u) {                                     \
            const int idx = threadIdx.x + u * THREADS;  /* 8 lanes per 128-byte row */       \
            const int rr = min(idx / (P / 8), valid - 1);   /* clamped, zeroed on commit */  \
            px[u] = *reinterpret_cast<const uint4*>(a.x + ((tok0 + rr) * H + (HEAD)) * P +  \
                                                    (idx % (P / 8)) * 8);                    \
        }                                                                                    \
        const bf16* sp_ = a.states + ((((int64_t)bi * nc + ci) * H + (HEAD)) * P) * N;       \
        _Pragma("unroll") for (int u = 0; u < SV; ++u)                                       \
            ps[u] = *reinterpret_cast<const uint4*>(sp_ + (int64_t)(threadIdx.x + u * THREADS) * 8); \
        if (threadIdx.x < Q) {                                                               \
            const int64_t cq = (((int64_t)bi * H + (HEAD)) * nc + ci) * Q + threadIdx.x;     \
            pdA = a.dA[cq] * LOG2E;                                                          \
            pdt = a.dt[cq];                                                                  \
        }                                                                                    \
    }

    // ---- stage the group's B tile (all loads in flight), seq ids ------------
    {
        const bf16* Bsrc = a.B + (tok0 * G + g) * N;
        uint4 pb[BV];
#pragma unroll
        for (int u = 0; u < BV; ++u) {
            const int idx = threadIdx.x + u * THREADS;
            const int r = min(idx / (N / 8), valid - 1), cv = idx % (N / 8);
            pb[u] = *reinterpret_cast<const uint4*>(Bsrc + r * rs + cv * 8);
        }
        for (int q = threadIdx.x; q < Q; q += THREADS)
            seqs[q] = (a.seq_idx && q < valid) ? a.seq_idx[tok0 + q] : -1;
#pragma unroll
        for (int u = 0; u < BV; ++u) {
            const int idx = threadIdx.x + u * THREADS;
            const int r = idx / (N / 8), cv = idx % (N / 8);
            *reinterpret_cast<uint4*>(bs + r * SB + cv * 8) = pb[u];   // rows >= valid: masked later
        }
    }
    // C fragments of this wavefront's row-tile pair (w, QT-1-w)
    const bool active = w < NPAIRS;
    const int t1 = w, t2 = QT - 1 - w;
    bf16x8 cfr[2][NS];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int row = min(16 * (tt ? t2 : t1) + ln, valid - 1);   // clamped; masked below
#pragma unroll
        for (int ns = 0; ns < NS; ++ns)
            cfr[tt][ns] = *reinterpret_cast<const bf16x8*>(Cg + row * rs + ns * 32);
    }
    lds_barrier();   // B tile and seq ids visible

    // ---- CB^T tiles (k-tile kt, row tile t), kt <= t, into LDS slots -------
    if (active) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = tt ? t2 : t1;
            const int slot0 = tt ? t1 + 1 : 0;
            const int m = 16 * t + ln;
            for (int kt = 0; kt <= t; ++kt) {
                f32x4 acc = zero4();
#pragma unroll
                for (int ns = 0; ns < NS; ++ns)
                    acc = mma32(*reinterpret_cast<const bf16x8*>(
                                    bs + (16 * kt + ln) * SB + ns * 32 + kg * 8),
                                cfr[tt][ns], acc);
                bf16x4 v4;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int k = 16 * kt + 4 * kg + i;
                    float v = acc[i];
                    if (k > m || m >= valid) v = 0.f;          // causal, k <= m < valid
                    if (a.seq_idx && seqs[m] != seqs[k]) v = 0.f;
                    v4[i] = (bf16)v;                            // CB is bf16 (reference)
                }
                cbl[w][slot0 + kt][lane] = v4;
            }
        }
    }
    // D values of this workgroup's heads, loaded before any prefetch so that
    // no later vector load forces a wait on the (in-order) prefetch queue
    float dvl[HB][PT];
#pragma unroll
    for (int hi = 0; hi < HB; ++hi)
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
            const int hh = h0 + min(hi, nh - 1);
            dvl[hi][pt] = a.D ? (a.D_has_hdim ? a.D[hh * P + pt * 16 + ln] : a.D[hh]) : 0.f;
        }
    M2_PREFETCH(h0)

#pragma unroll
    for (int hi = 0; hi < HB; ++hi) {          // unrolled: exact waitcnt accounting
        if (hi >= nh) break;
        const int h = h0 + hi;
        lds_barrier();               // B tile / previous head no longer read
#pragma unroll
        for (int u = 0; u < XV; ++u) {
            const int idx = threadIdx.x + u * THREADS;
            const int r = idx / (P / 8), cv = idx % (P / 8);
            const uint4 v = r < valid ? px[u] : make_uint4(0, 0, 0, 0);
            const uint32_t wds[4] = {v.x, v.y, v.z, v.w};
            unsigned short* d = reinterpret_cast<unsigned short*>(xs) + (cv * 8) * SQ + r;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                d[(2 * j) * SQ] = (unsigned short)(wds[j] & 0xffff);
                d[(2 * j + 1) * SQ] = (unsigned short)(wds[j] >> 16);
            }
        }
#pragma unroll
        for (int u = 0; u < SV; ++u) {
            const int idx = threadIdx.x + u * THREADS;
            const uint4 v = ps[u];
            uint2* d = reinterpret_cast<uint2*>(ss + (idx / (N / 8)) * SS + (idx % (N / 8)) * 8);
            d[0] = make_uint2(v.x, v.y);
            d[1] = make_uint2(v.z, v.w);
        }
        if (threadIdx.x < Q) {
            dAs[threadIdx.x] = pdA;
            dts[threadIdx.x] = pdt;
        }
        lds_barrier();
        if (hi + 1 < nh) M2_PREFETCH(h + 1)   // in flight during this head's compute
        if (!active) continue;
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int t = tt ? t2 : t1;
            f32x4 acc[PT];
#pragma unroll
            for (int pt = 0; pt < PT; ++pt) acc[pt] = zero4();
            // 1. carried state: C rows @ state^T, rounded to bf16, times exp(dA[m])
#pragma unroll
            for (int ns = 0; ns < NS; ++ns) {
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) {
                    const bf16x8 bfr = *reinterpret_cast<const bf16x8*>(
                        ss + (pt * 16 + ln) * SS + ns * 32 + kg * 8);
                    acc[pt] = mma32(cfr[tt][ns], bfr, acc[pt]);
                }
                __builtin_amdgcn_sched_barrier(0);   // bound the live fragments
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mr = 16 * t + 4 * kg + i;
                float f = __builtin_amdgcn_exp2f(dAs[mr]);
                if (a.seq_idx && seqs[mr] != seq_prev) f = 0.f;
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) acc[pt][i] = rbf(acc[pt][i]) * f;
            }
            // 2. intra-chunk: CB[m,k] exp(dA[m]-dA[k]) dt[k] (bf16 hi + lo) @ x[k,:]
            const int m = 16 * t + ln;
            const float dAm = dAs[m];
            const int slot0 = tt ? t1 + 1 : 0;
            for (int kt = 0; kt <= t; ++kt) {
                const bf16x4 cb4 = cbl[w][slot0 + kt][lane];
                const int k0 = 16 * kt + 4 * kg;
                const float4 dk = *reinterpret_cast<const float4*>(dAs + k0);
                const float4 tk = *reinterpret_cast<const float4*>(dts + k0);
                const float dkv[4] = {dk.x, dk.y, dk.z, dk.w};
                const float tkv[4] = {tk.x, tk.y, tk.z, tk.w};
                bf16x4 ahi, alo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // decay exp(dA[m]-dA[k]) in the log2 domain; k > m is masked
                    const float e = __builtin_amdgcn_exp2f(fminf(dAm - dkv[i], 0.f));
                    const float v = (k0 + i <= m) ? (float)cb4[i] * e * tkv[i] : 0.f;
                    const bf16 hv = (bf16)v;
                    ahi[i] = hv;
                    alo[i] = (bf16)(v - (float)hv);
                }
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) {
                    const bf16x4 bfr =
                        *reinterpret_cast<const bf16x4*>(xs + (pt * 16 + ln) * SQ + k0);
                    acc[pt] = mma16(ahi, bfr, acc[pt]);
                    acc[pt] = mma16(alo, bfr, acc[pt]);
                }
            }
            // 3. epilogue: + D x, silu(z) gate in z's dtype, fp32 store
#pragma unroll
            for (int pt = 0; pt < PT; ++pt) {
                const int pcol = pt * 16 + ln;
                const float dv = dvl[hi][pt];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int mr = 16 * t + 4 * kg + i;
                    if (mr >= valid) continue;
                    float v = acc[pt][i];
                    if (a.D) v += dv * (float)xs[pcol * SQ + mr];
                    const int64_t o = ((tok0 + mr) * H + h) * (int64_t)P + pcol;
                    if (a.z) v *= rbf(silu_f((float)a.z[o]));
                    a.out[o] = v;
                }
            }
        }
    }
}
#undef M2_PREFETCH

}  // namespace

namespace m2 {

// True when the fused path covers these sizes (bf16, headdim 64).
bool scan_fused_supported(int64_t headdim, int64_t dstate, int64_t chunk_size) {
    return headdim == 64 && (dstate == 64 || dstate == 128 || dstate == 256) &&
           (chunk_size == 64 || chunk_size == 128);
}

int launch_scan_fused(const m2_ssd_combined_args& a, const float* dA, const float* dto,
                      const void* passed, hipStream_t s) {
    const int64_t nc = (a.seqlen + a.chunk_size - 1) / a.chunk_size;
    const int64_t hpg = a.nheads / a.ngroups;
    const int64_t nhb = (hpg + HB - 1) / HB;
    const int64_t nblocks = a.batch * nc * a.ngroups * nhb;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "scan_fused: too many blocks");
    ScanFusedArgs f{};
    f.x = (const bf16*)a.x; f.B = (const bf16*)a.B; f.C = (const bf16*)a.C;
    f.states = (const bf16*)passed; f.dt = dto; f.dA = dA; f.D = a.D; f.z = (const bf16*)a.z;
    f.seq_idx = a.seq_idx; f.out = a.out; f.D_has_hdim = a.D_has_hdim;
    f.L = (int)a.seqlen; f.H = (int)a.nheads; f.G = (int)a.ngroups; f.nc = (int)nc;
    f.nhb = (int)nhb; f.nblocks = (int)nblocks;
    void (*kern)(ScanFusedArgs) = nullptr;
#define M2_SF_CASE(NSV, QTV) \
    if (a.dstate == 32 * NSV && a.chunk_size == 16 * QTV) kern = k_scan_fused<NSV, QTV>;
    M2_SF_CASE(2, 4) M2_SF_CASE(2, 8)
    M2_SF_CASE(4, 4) M2_SF_CASE(4, 8)
    M2_SF_CASE(8, 4) M2_SF_CASE(8, 8)
#undef M2_SF_CASE
    M2_REQUIRE(kern && a.headdim == 64, M2_ERR_UNSUPPORTED, "scan_fused: unsupported sizes");
    kern<<<(unsigned)nblocks, THREADS, 0, s>>>(f);
    return check_launch("scan_fused");
}

}  // namespace m2
