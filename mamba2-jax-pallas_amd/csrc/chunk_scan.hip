// chunk_scan: the SSD output of one chunk and head
//   y[m,:] = sum_{k<=m} cb[m,k] exp(dA[m]-dA[k]) dt[k] x[k,:]      (intra-chunk)
//          + exp(dA[m]) * C[m,:] @ states^T                        (carried state)
//          + D x[m,:],   then y *= silu(z[m,:])
//
// One workgroup per (b, c, h), 8 wavefronts; the chunk's x rows [Q x P] and
// the carried state [P x N] are staged in LDS (16-byte coalesced loads; the
// state is rounded to x's dtype on the way in).  Each wavefront takes 16-row
// tiles of the output in a snake order so that the causal (triangular) work
// is balanced, and for each tile accumulates
//   1. C-rows (16-byte loads straight into VGPRs) x state  -> scaled by exp(dA[m])
//   2. decay-weighted CB-rows x x-tile, for k-tiles up to the diagonal only.
// The decay exp(dA[m]-dA[k]) is evaluated per element in registers while the
// CB fragment is built -- never factored into exp(dA[m]) * exp(-dA[k]), which
// overflows once |dA| inside a chunk exceeds ~88.  The D skip and z gate are
// fused into the store.
//
// Follows reference ops/ssd_naive.py:223-318 (math), kernels/chunk_scan_fwd.py
// :294-322 (seq_idx rule for the carried-state term) and :545-570 (epilogue).
#include "m2_internal.h"

namespace {

constexpr int THREADS = 512;
constexpr int NW = THREADS / 64;      // wavefronts: two per SIMD (one workgroup per CU
                                      // when the fp32 x tile fills the LDS)

template <typename T> struct ScanPad;
template <> struct ScanPad<bf16> { static constexpr int x = 2; static constexpr int s = 8; };
template <> struct ScanPad<float> { static constexpr int x = 16; static constexpr int s = 4; };

struct ScanArgs {
    const void* cb;
    const void* x;
    const float* dt;
    const float* dA;
    const void* C;
    const void* states;
    const float* D;
    const void* z;
    const int32_t* seq_idx;
    float* out;
    float* out_x;
    int states_same;      // states dtype == x dtype
    int states_bf16;      // states dtype is bf16
    int D_has_hdim;
    int L, H, G, P, N, Q, nc, nblocks;
};

// KPL consecutive cb values of one row, as float
template <int KPL> M2_DEV void load_cb(const float* p, float* v) {
    if constexpr (KPL == 8) {
        const float4 a = reinterpret_cast<const float4*>(p)[0];
        const float4 b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < KPL; ++j) v[j] = p[j];
    }
}
template <int KPL> M2_DEV void load_cb(const bf16* p, float* v) {
    if constexpr (KPL == 8) {
        const bf16x8 a = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = (float)a[j];
    } else {
#pragma unroll
        for (int j = 0; j < KPL; ++j) v[j] = (float)p[j];
    }
}

// SG: the carried state is read from global memory (an L2-resident 32 KB per
// head and chunk at head dim 128) instead of staged in LDS, for the shapes
// whose x tile and state together exceed the LDS (fp32, head dim 128, chunk
// 256); needs the state in x's dtype.
template <typename T, typename TCB, int PT, bool SG>
__global__ void __launch_bounds__(THREADS) k_chunk_scan(ScanArgs a) {
    typedef MF<T> M;
    constexpr int KPL = M::KPL;
    extern __shared__ __align__(16) char smem[];
    const int P = PT * 16;
    const int Q = a.Q, L = a.L, H = a.H, N = a.N, nc = a.nc;
    const int SX = P + ScanPad<T>::x, SS = N + ScanPad<T>::s;
    T* xs = reinterpret_cast<T*>(smem);                  // [Q][SX]
    T* ss = xs + Q * SX;                                  // [P][SS]
    float* dAs = reinterpret_cast<float*>(ss + (SG ? 0 : P * SS));   // [Q]
    float* dts = dAs + Q;                                 // [Q]
    int* seqs = reinterpret_cast<int*>(dts + Q);          // [Q] (seq_idx only)

    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int h = work % H;
    const int rest = work / H;
    const int c = rest % nc;
    const int bi = rest / nc;
    const int g = h / (H / a.G);
    const int valid = min(Q, L - c * Q);
    const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;

    // --- stage dA, dt, seq_idx, x rows and the carried state ----------------
    const int64_t cq = (((int64_t)bi * H + h) * nc + c) * Q;
    int seq_prev = 0;
    if (a.seq_idx && c > 0) seq_prev = a.seq_idx[tok0 - 1];
    for (int q = threadIdx.x; q < Q; q += THREADS) {
        dAs[q] = a.dA[cq + q];
        dts[q] = a.dt[cq + q];
        if (a.seq_idx) seqs[q] = q < valid ? a.seq_idx[tok0 + q] : -1;
    }
    {
        constexpr int VE = 16 / sizeof(T);
        const T* xsrc = reinterpret_cast<const T*>(a.x) + (tok0 * H + h) * P;
        const int vpr = P / VE, total = Q * vpr;
        for (int idx = threadIdx.x; idx < total; idx += THREADS) {
            const int r = idx / vpr, cv = idx % vpr;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (r < valid) v = *reinterpret_cast<const uint4*>(xsrc + (int64_t)r * H * P + cv * VE);
            uint32_t* d = reinterpret_cast<uint32_t*>(xs + r * SX + cv * VE);
            d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
        }
    }
    const int64_t soff = (((int64_t)bi * nc + c) * H + h) * (int64_t)P * N;
    if (!SG) {
        if (a.states_same) {
            constexpr int VE = 16 / sizeof(T);
            const T* src = reinterpret_cast<const T*>(a.states) + soff;
            const int vpr = N / VE, total = P * vpr;
            for (int idx = threadIdx.x; idx < total; idx += THREADS) {
                const int r = idx / vpr, cv = idx % vpr;
                *reinterpret_cast<uint4*>(ss + r * SS + cv * VE) =
                    *reinterpret_cast<const uint4*>(src + (int64_t)r * N + cv * VE);
            }
        } else {
            for (int idx = threadIdx.x; idx < P * N; idx += THREADS) {
                const int r = idx / N, cl = idx % N;
                const float v = a.states_bf16
                                    ? (float)reinterpret_cast<const bf16*>(a.states)[soff + idx]
                                    : reinterpret_cast<const float*>(a.states)[soff + idx];
                ss[r * SS + cl] = from_f32<T>(v);
            }
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    const T* Cbase = reinterpret_cast<const T*>(a.C) + (tok0 * a.G + g) * N;
    const TCB* cbbase = reinterpret_cast<const TCB*>(a.cb) +
                        (((int64_t)bi * nc + c) * a.G + g) * (int64_t)Q * Q;
    typename M::frag zf;
#pragma unroll
    for (int j = 0; j < KPL; ++j) M::set(zf, j, 0.f);

    const int ntiles = Q / 16;
    for (int r = 0;; ++r) {
        const int t = r * NW + ((r & 1) ? (NW - 1 - w) : w);
        if (t >= ntiles) break;
        const int m0 = t * 16;
        f32x4 acc[PT];
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) acc[pt] = zero4();

        // 1. carried state: C[m, :] @ state^T.  The C fragments of BATCH K
        // steps are loaded (unconditionally: rows past the end are clamped and
        // zeroed afterwards) before any is used, so they are in flight together.
        {
            const int m = m0 + ln;
            const bool mok = m < valid;
            const T* crow = Cbase + (int64_t)min(m, valid - 1) * a.G * N + kg * KPL;
            constexpr int BATCH = KPL == 1 ? 8 : 2;
            for (int k0 = 0; k0 < N; k0 += BATCH * M::K) {
                typename M::frag cf[BATCH];
#pragma unroll
                for (int u = 0; u < BATCH; ++u) cf[u] = load_frag(crow + min(k0 + u * M::K, N - M::K));
#pragma unroll
                for (int u = 0; u < BATCH; ++u) {
                    // steps past N (N not a multiple of the batch) add zero
                    const int k = min(k0 + u * M::K, N - M::K);
                    const typename M::frag af = (mok && k0 + u * M::K < N) ? cf[u] : zf;
#pragma unroll
                    for (int pt = 0; pt < PT; ++pt) {
                        const typename M::frag bfr =
                            SG ? load_frag(reinterpret_cast<const T*>(a.states) + soff +
                                           (int64_t)(pt * 16 + ln) * N + k + kg * KPL)
                               : load_frag(ss + (pt * 16 + ln) * SS + k + kg * KPL);
                        acc[pt] = M::mma(af, bfr, acc[pt]);
                    }
                }
            }
            // C @ states has x's dtype as result type in the reference
            // (ops/ssd_naive.py:294-297): round it before the fp32 decay
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mr = m0 + kg * 4 + i;
                float f = expf(dAs[mr]);
                if (a.seq_idx && seqs[mr] != seq_prev) f = 0.f;
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) acc[pt][i] = to_f32(from_f32<T>(acc[pt][i])) * f;
            }
        }

        // 2. intra-chunk: (cb o decay o dt)[m, k<=m] @ x[k, :]; the cb values of
        // BATCH K steps are loaded before any is used
        {
            const int m = m0 + ln;
            const float dAm = dAs[m];
            const TCB* cbrow = cbbase + (int64_t)m * Q;
            const int kend = m0 + 16;
            constexpr int BATCH = KPL == 1 ? 8 : 2;
            for (int kB = 0; kB < kend; kB += BATCH * M::K) {
            float cbb[BATCH][KPL];
#pragma unroll
            for (int u = 0; u < BATCH; ++u)
                load_cb<KPL>(cbrow + min(kB + u * M::K + kg * KPL, Q - KPL), cbb[u]);
#pragma unroll
            for (int u = 0; u < BATCH; ++u) {
                const int k0 = kB + u * M::K;
                if (k0 >= kend) break;
                const int kb = k0 + kg * KPL;
                const float* cbv = cbb[u];
                // the weighted operand is split into bf16 hi + lo parts (x is
                // exact in bf16): the intra-chunk sum keeps near-fp32 accuracy
                typename M::frag af, al;
#pragma unroll
                for (int j = 0; j < KPL; ++j) {
                    const int k = kb + j;
                    float v = 0.f;
                    if (k <= m && k < Q) v = cbv[j] * expf(dAm - dAs[k]) * dts[k];
                    M::set_split(af, al, j, v);
                }
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) {
                    typename M::frag bfr;
#pragma unroll
                    for (int j = 0; j < KPL; ++j) {
                        const int k = kb + j;
                        M::set_raw(bfr, j, k < Q ? xs[k * SX + pt * 16 + ln] : T(0.f));
                    }
                    acc[pt] = M::mma(af, bfr, acc[pt]);
                    if constexpr (M::kSplit) acc[pt] = M::mma(al, bfr, acc[pt]);
                }
            }
            }
        }

        // 3. epilogue: + D x, out_x, z gate, store
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
            const int p = pt * 16 + ln;
            const float dv = a.D ? (a.D_has_hdim ? a.D[h * P + p] : a.D[h]) : 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mr = m0 + kg * 4 + i;
                if (mr >= valid) continue;
                float v = acc[pt][i];
                if (a.D) v += dv * to_f32(xs[mr * SX + p]);
                const int64_t o = ((tok0 + mr) * H + h) * (int64_t)P + p;
                if (a.out_x) a.out_x[o] = v;
                // silu(z) is evaluated in z's dtype by the reference (ops/ssd_naive.py:316)
                if (a.z) v *= to_f32(from_f32<T>(silu_f(to_f32(reinterpret_cast<const T*>(a.z)[o]))));
                a.out[o] = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// k_chunk_scan_f32: the same computation for fp32 x / C / states (head dim
// 64), with every fp32 operand split into bf16 hi + lo parts once, when it is
// staged, rather than at each use: x goes to LDS as two row-major bf16
// planes [Q][64] with XOR-swizzled 16-byte chunks, whose columns (8 positions
// of one head-dim column: the B operand of the intra-chunk product) come
// through the gfx950 LDS transpose read, and the carried state as two planes
// [P][N]; a product of two split operands is three 16x16x32 bf16 MFMAs
// (hi.hi + hi.lo + lo.hi, ~2^-16 relative).  The decay weights use the
// hardware exp2.  One workgroup per (b, c, h), 8 wavefronts, snake tile order
// (two heads per workgroup, sharing the C / CB fragments, measured slower:
// half the workgroups, one per CU).
// ---------------------------------------------------------------------------
constexpr float LOG2E = 1.4426950408889634f;

// padded row lengths (bf16 elements) of the planes: rows 16 bytes apart in
// the bank map, so 16 lanes reading one 16-byte column of 16 rows hit
// distinct banks
__host__ __device__ inline int f32_srow(int N) { return N + 8; }
__host__ __device__ inline size_t f32_scan_lds(int Q, int P, int N) {
    return (size_t)2 * Q * P * 2 + (size_t)2 * P * f32_srow(N) * 2 + (size_t)Q * 3 * 4;
}
// 16-byte chunk swizzle of an x plane row R (128-byte rows, head dim 64): the
// 8 rows of a transpose read at one chunk pair land on distinct banks
M2_DEV int xpswz(int R) { return ((R >> 1) & 3) << 1; }

M2_DEV f32x4 mma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
}
// 8 floats as bf16 hi / lo parts
M2_DEV void split8(const float* v, bf16x8& hi, bf16x8& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) split2(v[2 * i], v[2 * i + 1], h[i], l[i]);
    hi = as_bf16x8(h[0], h[1], h[2], h[3]);
    lo = as_bf16x8(l[0], l[1], l[2], l[3]);
}

template <int PT, int NS, int QT, typename TCB>
__global__ void __launch_bounds__(THREADS, 4) k_chunk_scan_f32(ScanArgs a) {
    // NS: dstate / 32, QT: chunk / 32 (compile-time, so every load of a stage
    // is issued before the first of them is used)
    extern __shared__ __align__(16) char smem[];
    constexpr int P = PT * 16;
    constexpr int Q = 32 * QT, N = 32 * NS;
    static_assert(P == 64, "x planes: 128-byte rows");
    const int L = a.L, H = a.H, nc = a.nc;
    constexpr int XROW = P * 2, SR = N + 8;
    char* xh = smem;                                     // [Q] rows of XROW: x hi
    char* xl = xh + Q * XROW;                            // x lo
    bf16* sh = reinterpret_cast<bf16*>(xl + Q * XROW);   // [P][SR]: state hi
    bf16* sl = sh + P * SR;                              // [P][SR]: state lo
    float* dAs = reinterpret_cast<float*>(sl + P * SR);  // [Q]
    float* dts = dAs + Q;                                // [Q]
    int* seqs = reinterpret_cast<int*>(dts + Q);         // [Q] (seq_idx only)

    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int h = work % H;
    const int rest = work / H;
    const int c = rest % nc;
    const int bi = rest / nc;
    const int g = h / (H / a.G);
    const int valid = min(Q, L - c * Q);
    const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;

    // --- stage dA, dt, seq_idx; x and the carried state as hi / lo planes ---
    const int64_t cq = (((int64_t)bi * H + h) * nc + c) * Q;
    int seq_prev = 0;
    if (a.seq_idx && c > 0) seq_prev = a.seq_idx[tok0 - 1];
    for (int q = threadIdx.x; q < Q; q += THREADS) {
        dAs[q] = a.dA[cq + q];
        dts[q] = a.dt[cq + q];
        if (a.seq_idx) seqs[q] = q < valid ? a.seq_idx[tok0 + q] : -1;
    }
    {
        // x[r][4 v .. 4 v + 3] -> an 8-byte half of a swizzled chunk of row r
        const float* xsrc = reinterpret_cast<const float*>(a.x) + (tok0 * H + h) * P;
        constexpr int VPR = P / 4, XI = Q * VPR / THREADS;
        static_assert(Q * VPR % THREADS == 0 && P * (N / 4) % THREADS == 0, "even staging split");
        float4 xf[XI];
#pragma unroll
        for (int it = 0; it < XI; ++it) {
            const int idx = threadIdx.x + it * THREADS, r = idx / VPR, v = idx % VPR;
            xf[it] = *reinterpret_cast<const float4*>(xsrc + (int64_t)min(r, valid - 1) * H * P + 4 * v);
        }
        constexpr int VS = N / 4, SI = P * VS / THREADS;
        const int64_t soff = (((int64_t)bi * nc + c) * H + h) * (int64_t)P * N;
        float sv[SI][4];
#pragma unroll
        for (int it = 0; it < SI; ++it) {
            const int idx = threadIdx.x + it * THREADS, r = idx / VS, v = idx % VS;
            if (a.states_bf16) {
                const bf16x4 b4 = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16*>(a.states) + soff + (int64_t)r * N + 4 * v);
#pragma unroll
                for (int i = 0; i < 4; ++i) sv[it][i] = (float)b4[i];
            } else {
                const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.states) + soff + (int64_t)r * N + 4 * v);
                sv[it][0] = f.x; sv[it][1] = f.y; sv[it][2] = f.z; sv[it][3] = f.w;
            }
        }
#pragma unroll
        for (int it = 0; it < XI; ++it) {
            const int idx = threadIdx.x + it * THREADS, r = idx / VPR, v = idx % VPR;
            const float4 f = r < valid ? xf[it] : make_float4(0.f, 0.f, 0.f, 0.f);
            uint32_t h01, l01, h23, l23;
            split2(f.x, f.y, h01, l01);
            split2(f.z, f.w, h23, l23);
            typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
            const int off = r * XROW + (((v >> 1) ^ xpswz(r)) * 16) + 8 * (v & 1);
            *reinterpret_cast<u2*>(xh + off) = u2{h01, h23};
            *reinterpret_cast<u2*>(xl + off) = u2{l01, l23};
        }
#pragma unroll
        for (int it = 0; it < SI; ++it) {
            const int idx = threadIdx.x + it * THREADS, r = idx / VS, v = idx % VS;
            uint32_t h01, l01, h23, l23;
            split2(sv[it][0], sv[it][1], h01, l01);
            split2(sv[it][2], sv[it][3], h23, l23);
            typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
            *reinterpret_cast<u2*>(sh + r * SR + 4 * v) = u2{h01, h23};
            *reinterpret_cast<u2*>(sl + r * SR + 4 * v) = u2{l01, l23};
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    const float* Cbase = reinterpret_cast<const float*>(a.C) + (tok0 * a.G + g) * N;
    const TCB* cbbase = reinterpret_cast<const TCB*>(a.cb) + (((int64_t)bi * nc + c) * a.G + g) * (int64_t)Q * Q;
    const bf16x8 zero8 = as_bf16x8(0u, 0u, 0u, 0u);
    const int ntiles = Q / 16;
    for (int r = 0;; ++r) {
        const int t = r * NW + ((r & 1) ? (NW - 1 - w) : w);
        if (t >= ntiles) break;
        const int m0 = t * 16;
        const int m = m0 + ln;
        f32x4 acc[PT];
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) acc[pt] = zero4();

        // 1. carried state: C[m, :] @ state^T (C split as its rows arrive)
        {
            const bool mok = m < valid;
            const float* crow = Cbase + (int64_t)min(m, valid - 1) * a.G * N + kg * 8;
            constexpr int NS4 = NS < 4 ? NS : 4;             // C loads in flight together
#pragma unroll
            for (int ks0 = 0; ks0 < NS; ks0 += NS4) {
            float4 cf[NS4][2];
#pragma unroll
            for (int u = 0; u < NS4; ++u) {
                cf[u][0] = *reinterpret_cast<const float4*>(crow + 32 * (ks0 + u));
                cf[u][1] = *reinterpret_cast<const float4*>(crow + 32 * (ks0 + u) + 4);
            }
#pragma unroll
            for (int u = 0; u < NS4; ++u) {
                const int ks = ks0 + u;
                __builtin_amdgcn_sched_barrier(0);           // one k-step's operands live at a time
                const float cv[8] = {cf[u][0].x, cf[u][0].y, cf[u][0].z, cf[u][0].w,
                                     cf[u][1].x, cf[u][1].y, cf[u][1].z, cf[u][1].w};
                bf16x8 ch, cl;
                split8(cv, ch, cl);
                if (!mok) { ch = zero8; cl = zero8; }
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) {
                    const int pr = pt * 16 + ln;
                    const bf16x8 bh = *reinterpret_cast<const bf16x8*>(sh + pr * SR + 32 * ks + kg * 8);
                    const bf16x8 bl = *reinterpret_cast<const bf16x8*>(sl + pr * SR + 32 * ks + kg * 8);
                    acc[pt] = mma3(ch, cl, bh, bl, acc[pt]);
                }
            }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mr = m0 + kg * 4 + i;
                float f = __builtin_amdgcn_exp2f(dAs[mr] * LOG2E);
                if (a.seq_idx && seqs[mr] != seq_prev) f = 0.f;
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) acc[pt][i] *= f;
            }
        }

        // 2. intra-chunk: (cb o decay o dt)[m, k <= m] @ x[k, :], the weights
        // split into hi / lo.  In K step ks, MFMA k index j < 4 is position
        // 32 ks + 4 kg + j and j >= 4 is 16 more: the rows the transpose read
        // of the x planes gives this lane group
        {
            const float dAm = dAs[m];
            const TCB* cbrow = cbbase + (int64_t)m * Q;
            const int nks = (m0 + 16 + 31) / 32;             // k-steps up to the diagonal
            const int rA = 4 * kg + (ln >> 2), c1 = ln & 3;
            int xo[PT];
#pragma unroll
            for (int pt = 0; pt < PT; ++pt)
                xo[pt] = rA * XROW + (((2 * pt + (c1 >> 1)) ^ xpswz(rA)) * 16) + 8 * (c1 & 1);
            constexpr int KB4 = QT < 4 ? QT : 4;             // CB loads in flight together
            for (int ks0 = 0; ks0 < nks; ks0 += KB4) {
            float cbv[KB4][8];
#pragma unroll
            for (int u = 0; u < KB4; ++u)
                if (ks0 + u < nks) {
                    load_cb<4>(cbrow + 32 * (ks0 + u) + 4 * kg, cbv[u]);
                    load_cb<4>(cbrow + 32 * (ks0 + u) + 16 + 4 * kg, cbv[u] + 4);
                }
#pragma unroll
            for (int u = 0; u < KB4; ++u) {
                const int ks = ks0 + u;
                if (ks >= nks) break;
                __builtin_amdgcn_sched_barrier(0);           // one k-step's operands live at a time
                float v[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int k = 32 * ks + 4 * kg + (j & 3) + (j >> 2) * 16;
                    v[j] = k <= m ? cbv[u][j] * __builtin_amdgcn_exp2f((dAm - dAs[k]) * LOG2E) * dts[k] : 0.f;
                }
                bf16x8 wh, wl;
                split8(v, wh, wl);
                const int xs = ks * 32 * XROW;
#pragma unroll
                for (int pt = 0; pt < PT; ++pt) {
                    const char* ph = xh + xs + xo[pt];
                    const char* pl = xl + xs + xo[pt];
                    const bf16x8 bh = __builtin_shufflevector(ds_read_tr(ph), ds_read_tr(ph + 16 * XROW), 0, 1, 2, 3, 4, 5, 6, 7);
                    const bf16x8 bl = __builtin_shufflevector(ds_read_tr(pl), ds_read_tr(pl + 16 * XROW), 0, 1, 2, 3, 4, 5, 6, 7);
                    acc[pt] = mma3(wh, wl, bh, bl, acc[pt]);
                }
            }
            }
        }

        // 3. epilogue: + D x, out_x, z gate, store
#pragma unroll
        for (int pt = 0; pt < PT; ++pt) {
            const int p = pt * 16 + ln;
            const float dv = a.D ? (a.D_has_hdim ? a.D[h * P + p] : a.D[h]) : 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int mr = m0 + kg * 4 + i;
                if (mr >= valid) continue;
                float v = acc[pt][i];
                if (a.D) {
                    const int xoff = mr * XROW + (((p >> 3) ^ xpswz(mr)) * 16) + 2 * (p & 7);
                    v += dv * ((float)*reinterpret_cast<const bf16*>(xh + xoff) +
                               (float)*reinterpret_cast<const bf16*>(xl + xoff));
                }
                const int64_t o = ((tok0 + mr) * H + h) * (int64_t)P + p;
                if (a.out_x) a.out_x[o] = v;
                if (a.z) v *= silu_f(reinterpret_cast<const float*>(a.z)[o]);
                a.out[o] = v;
            }
        }
    }
}

// head dim 64, compile-time chunk 64 / 128 / 256 and dstate 64 / 128 / 256
// (others: the generic kernel)
template <typename TCB>
int launch_f32(const ScanArgs& sa, hipStream_t s) {
    const size_t shm = f32_scan_lds(sa.Q, sa.P, sa.N);
    void (*kern)(ScanArgs) = nullptr;
#define M2_F32_SCAN(PTV, NSV, QTV) \
    if (sa.P == 16 * PTV && sa.N == 32 * NSV && sa.Q == 32 * QTV) kern = k_chunk_scan_f32<PTV, NSV, QTV, TCB>;
    M2_F32_SCAN(4, 2, 2) M2_F32_SCAN(4, 4, 2) M2_F32_SCAN(4, 8, 2)
    M2_F32_SCAN(4, 2, 4) M2_F32_SCAN(4, 4, 4) M2_F32_SCAN(4, 8, 4)
    M2_F32_SCAN(4, 2, 8) M2_F32_SCAN(4, 4, 8) M2_F32_SCAN(4, 8, 8)
#undef M2_F32_SCAN
    if (!kern) return M2_ERR_UNSUPPORTED;
    if (shm > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "chunk_scan: cannot reserve %zu B of LDS", shm);
    kern<<<(unsigned)sa.nblocks, THREADS, shm, s>>>(sa);
    return m2::check_launch("chunk_scan");
}

template <typename T, typename TCB>
int launch_typed(const ScanArgs& sa, hipStream_t s) {
    const size_t xb = (size_t)sa.Q * (sa.P + ScanPad<T>::x) * sizeof(T) + (size_t)sa.Q * 3 * sizeof(float);
    const size_t sb = (size_t)sa.P * (sa.N + ScanPad<T>::s) * sizeof(T);
    // the state from global memory when x tile + state exceed the LDS
    const bool sg = xb + sb > 160 * 1024 && sa.states_same;
    const size_t shm = sg ? xb : xb + sb;
    void (*kern)(ScanArgs) = nullptr;
    switch (sa.P) {
        case 32: kern = sg ? k_chunk_scan<T, TCB, 2, true> : k_chunk_scan<T, TCB, 2, false>; break;
        case 64: kern = sg ? k_chunk_scan<T, TCB, 4, true> : k_chunk_scan<T, TCB, 4, false>; break;
        case 128: kern = sg ? k_chunk_scan<T, TCB, 8, true> : k_chunk_scan<T, TCB, 8, false>; break;
        default:
            return m2::set_error(M2_ERR_UNSUPPORTED,
                                 "chunk_scan: headdim %d not supported (32, 64, 128)", sa.P);
    }
    if (shm > 160 * 1024)
        return m2::set_error(M2_ERR_UNSUPPORTED, "chunk_scan: %zu B of LDS needed", shm);
    if (shm > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "chunk_scan: cannot reserve %zu B of LDS", shm);
    kern<<<(unsigned)sa.nblocks, THREADS, shm, s>>>(sa);
    return m2::check_launch("chunk_scan");
}

}  // namespace

namespace m2 {

int launch_chunk_scan(const m2_chunk_scan_args& a, hipStream_t s) {
    M2_REQUIRE(a.cb && a.x && a.dt && a.dA_cumsum && a.C && a.states && a.out, M2_ERR_INVALID,
               "chunk_scan: cb, x, dt, dA_cumsum, C, states and out are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.nheads > 0 && a.ngroups > 0 &&
                   a.nheads % a.ngroups == 0 && a.chunk_size > 0,
               M2_ERR_INVALID, "chunk_scan: bad sizes (nheads must be a multiple of ngroups)");
    M2_REQUIRE(a.chunk_size % 16 == 0 && a.chunk_size <= 256, M2_ERR_UNSUPPORTED,
               "chunk_scan: chunk_size must be a multiple of 16 and <= 256");
    M2_REQUIRE(a.states_dtype == M2_F32 || a.states_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "chunk_scan: states dtype %d", a.states_dtype);
    // bf16, headdim 64, no z: the fused scan kernel with CB read in
    if (scan_fused_cb_supported(a)) return launch_scan_fused_cb(a, s);
    ScanArgs sa{};
    sa.cb = a.cb; sa.x = a.x; sa.dt = a.dt; sa.dA = a.dA_cumsum; sa.C = a.C; sa.states = a.states;
    sa.D = a.D; sa.z = a.z; sa.seq_idx = a.seq_idx; sa.out = a.out; sa.out_x = a.out_x;
    sa.states_same = a.states_dtype == a.dtype; sa.states_bf16 = a.states_dtype == M2_BF16;
    sa.D_has_hdim = a.D_has_hdim;
    sa.L = (int)a.seqlen; sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.P = (int)a.headdim;
    sa.N = (int)a.dstate; sa.Q = (int)a.chunk_size;
    sa.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    const int64_t nblocks = a.batch * sa.nc * a.nheads;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_scan: too many blocks");
    sa.nblocks = (int)nblocks;
    if (a.dtype == M2_BF16) {
        M2_REQUIRE(a.dstate % 32 == 0, M2_ERR_UNSUPPORTED, "chunk_scan: bf16 needs dstate %% 32 == 0");
        if (a.cb_dtype == M2_F32) return launch_typed<bf16, float>(sa, s);
        if (a.cb_dtype == M2_BF16) return launch_typed<bf16, bf16>(sa, s);
    } else if (a.dtype == M2_F32) {
        M2_REQUIRE(a.dstate % 32 == 0, M2_ERR_UNSUPPORTED, "chunk_scan: f32 needs dstate %% 32 == 0");
        // chunk 128, head dim 64, fp32 CB and states: the group kernel
        if (scan_f32g_supported(a)) return launch_scan_f32g(a, s);
        // split planes when they fit (head dim 32 / 64): x, C and states fp32
        if (sa.P == 64 && sa.states_same && f32_scan_lds(sa.Q, sa.P, sa.N) <= 160 * 1024) {
            const int rc = a.cb_dtype == M2_F32 ? launch_f32<float>(sa, s)
                         : a.cb_dtype == M2_BF16 ? launch_f32<bf16>(sa, s) : M2_ERR_UNSUPPORTED;
            if (rc != M2_ERR_UNSUPPORTED) return rc;
        }
        if (a.cb_dtype == M2_F32) return launch_typed<float, float>(sa, s);
        if (a.cb_dtype == M2_BF16) return launch_typed<float, bf16>(sa, s);
    }
    return set_error(M2_ERR_UNSUPPORTED, "chunk_scan: dtype %d / cb dtype %d", a.dtype, a.cb_dtype);
}

}  // namespace m2
