// k_scan_q128: bmm_chunk + chunk_scan of the combined forward for bf16 inputs
// at chunk 128 (head dim 64, dstate 64 / 128 / 256).
//
//   y[m, :] = exp(dA[m]) * bf16(C[m, :] h_c^T)                     (carried state)
//           + sum_{k <= m} CB[m, k] exp(dA[m] - dA[k]) dt[k] x[k, :] (intra chunk)
//           + D x[m, :],   then y *= silu(z[m, :]) when z is given
// with CB = bf16(C B^T) (seq_idx-masked), h_c the bf16 state entering chunk c.
//
// One workgroup per (batch, chunk, group[, slice of the group's heads]), as in
// k_scan_fused: 8 compute wavefronts + 4 that only move data.  The 8 row tiles
// of the chunk form 4 pairs (t, 7 - t) of equal causal work; pair pi is split
// between two wavefronts (half 0 and half 1) into fixed lists of (row tile,
// k-tile) units:
//   half 0: tile 7 - pi over k-tiles 0..3, and its diagonal tile;
//   half 1: tile 7 - pi over k-tiles 4..6 - pi (a partial of that tile,
//           handed to half 0 through LDS), tile pi over k-tiles 0..pi - 1,
//           and its diagonal tile.
// Both lists are compile-time (one instantiation of the compute path per
// (pair, half)), so every LDS offset is an immediate and no loop bound is
// computed per head.  Each wavefront builds the CB^T tiles of its own units
// once, with 16x16x32 MFMAs (A = B rows, B = C rows), keeps them in
// registers as floats (bf16-rounded and masked), and reuses them for every
// head: their accumulator layout (lane = output row m, 4 consecutive k) is
// the B-operand layout of the intra-chunk product y^T += x^T W^T, and a pair
// of units of one tile fills the 8 k of a 16x16x32 MFMA (a lone unit uses two
// 16x16x16 MFMAs, one per split half).  W is split into bf16 hi + lo parts.
//
// Off-diagonal units factor the decay through the row tile's first row r:
//   exp(dA[m] - dA[k]) = exp(dA[m] - dA[r]) exp(dA[r] - dA[k]),
// both <= 1 when dA does not increase over the chunk (dt' >= 0, A <= 0);
// the second factor (times dt[k]) is one exp per lane from a per-wavefront
// table, the first scales the tile once.  Otherwise (checked per head) the
// decay is evaluated per element.  A per-head D is folded into the diagonal of
// W (D x[m] is the k = m term), so it costs no pass of its own.
//
// Per head, x [128 x 64], the carried state [64 x N], dA / dt and D arrive in
// a ring of R LDS slots through direct global -> LDS loads issued by the four
// data wavefronts, R - 1 heads ahead; they also store the output tiles the
// compute wavefronts stage in LDS (when LDS allows), so no compute wavefront
// ever waits on vmcnt for a store.
//
// Follows reference ops/ssd_naive.py:189-318 and kernels/chunk_scan_fwd.py
// :294-322 / kernels/bmm_chunk_fwd.py:353-372 (seq_idx masks).
#include <type_traits>

#include "m2_internal.h"

namespace {

using m2::ScanFusedArgs;

constexpr int NWAVES = 8;                 // compute wavefronts
constexpr int NLOAD = 4;                  // data wavefronts
constexpr int THREADS = (NWAVES + NLOAD) * 64;
static_assert(THREADS == m2::SCAN_Q128_THREADS, "block size");
constexpr int P = 64;
constexpr int Q = 128, QT = 8;
constexpr float LOG2E = 1.4426950408889634f;
constexpr int LDS_BYTES = 160 * 1024;

// a 16-byte output store, non-temporal for NT (a compile-time choice: the
// compiler merges the two stores of a runtime branch and drops the hint)
template <bool NT> M2_DEV void store_out(const f32x4& v, float* p) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
    else *reinterpret_cast<f32x4*>(p) = v;
}

template <int V> using IC = std::integral_constant<int, V>;

M2_DEV f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
M2_DEV f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
M2_DEV float rbf(float v) { return (float)(bf16)v; }
M2_DEV float ex2(float v) { return __builtin_amdgcn_exp2f(v); }

// 16-byte chunk swizzles: x rows are 128 bytes, read as chunk pairs / 8-byte
// halves (an even mask keeps pairs together); state / B rows (CPR chunks) are
// read 16 bytes per lane by 16 consecutive rows at one chunk.
M2_DEV int xswz(int r) { return ((r >> 1) & 3) << 1; }
template <int CPR> M2_DEV int sswz(int r) { return CPR == 8 ? ((r >> 1) & 7) : (r & 15); }

template <int NS>
struct Cfg {
    static constexpr int N = 32 * NS;
    static constexpr int SCPR = N / 8;                       // 16-byte chunks per state row
    static constexpr int XB = Q * P * 2, SB = P * N * 2;
    static constexpr int AUXB = 2 * Q * 4 + 64 * 4;          // dA, dt, D
    static constexpr int SLOT = XB + SB + AUXB;
    static constexpr int BT = Q * N * 2;                     // the group's B rows (CB build)
    static constexpr int XCHG = 4 * 4 * 64 * 16;             // half 1's partial tiles
    static constexpr int FTAB = NWAVES * 64 * 4;             // decay factor tables
    static constexpr int FIXED = XCHG + FTAB + Q * 4 + 256;
    static constexpr int ring_bytes(int r) { return r * SLOT > SLOT + BT ? r * SLOT : SLOT + BT; }
    static constexpr int STW = 16 * 64 * 4, STG = NWAVES * STW;   // staged output tiles
    static constexpr bool STAGE = ring_bytes(2) + FIXED + STG <= LDS_BYTES;
    // without room for whole tiles (N 256) each compute wavefront stages its
    // own tile, 32 columns (128-byte row pieces) at a time, and stores it
    // itself: whole 128-byte lines per store instead of 64-byte pieces (the
    // scan at c3: 323 against 332 us)
    static constexpr int WSTW = 16 * 32 * 4, WSTG = NWAVES * WSTW;
    static constexpr bool WST = !STAGE && ring_bytes(2) + FIXED + WSTG <= LDS_BYTES;
    static constexpr int EXTRA = FIXED + (STAGE ? STG : WST ? WSTG : 0);
    static constexpr int R = ring_bytes(4) + EXTRA <= LDS_BYTES ? 4
                           : ring_bytes(3) + EXTRA <= LDS_BYTES ? 3 : 2;
    static constexpr int RING = ring_bytes(R);
    // 1 KB direct loads per head (x, state) and for the B rows; per data wavefront
    static constexpr int XI = XB / 1024, SI = SB / 1024, BI = BT / 1024;
    static constexpr int XL = XI / NLOAD, SL = SI / NLOAD, BL = BI / NLOAD;
    static constexpr int WAIT01 = (R - 2) * (XL + SL + 1), WAIT23 = (R - 2) * (XL + SL);
    static_assert(XI % NLOAD == 0 && SI % NLOAD == 0 && BI % NLOAD == 0, "even load split");
    static_assert(RING + EXTRA <= LDS_BYTES, "LDS budget");
    static_assert(WAIT01 <= 63, "vmcnt range");
};

// The units of pair PI, half KH.  Off-diagonal units first (those of the
// long tile, then those of the short one), the diagonal unit last.
template <int PI, int KH>
struct Units {
    static constexpr int T1 = PI, T2 = QT - 1 - PI;
    static constexpr int TM = KH ? T1 : T2;                  // the tile this half stores
    static constexpr int NL = KH ? 3 - PI : 4;               // off-diagonal units of T2
    static constexpr int NSH = KH ? PI : 0;                  // off-diagonal units of T1
    static constexpr int NOFF = NL + NSH;
    static constexpr int NU = NOFF + 1;
    static constexpr int tile(int u) { return u < NL ? T2 : u < NOFF ? T1 : TM; }
    static constexpr int kt(int u) { return u < NL ? (KH ? 4 + u : u) : u < NOFF ? u - NL : TM; }
};

template <int NS, bool HASZ, bool CBIN, bool NT, int PI, int KH>
M2_DEV void compute_path(const ScanFusedArgs& a, char* ring, f32x4 (*xchg)[4][64], float* ftab,
                         char* stg, const int* seqs, int bi, int ci, int g, int h0, int nh,
                         int valid, int seq_prev) {
    typedef Cfg<NS> S;
    typedef Units<PI, KH> U;
    constexpr int N = S::N, SCPR = S::SCPR, R = S::R, XB = S::XB, SLOT = S::SLOT;
    constexpr int NU = U::NU, NOFF = U::NOFF, TM = U::TM;
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    const int G = a.G, H = a.H, L = a.L, nc = a.nc;
    const int64_t tok0 = (int64_t)bi * L + (int64_t)ci * Q;

    // ---- C fragments: rows of the stored tile (kept), of the long tile for
    // half 1's long-tile units (CB build only)
    bf16x8 cst[NS], cot[NS];
    {
        const int row = min(16 * TM + ln, valid - 1);          // clamped; masked below
        const bf16* cp = a.C + ((tok0 + row) * G + g) * N + kg * 8;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) cst[ns] = *reinterpret_cast<const bf16x8*>(cp + ns * 32);
        if (KH && U::NL > 0) {
            const int row2 = min(16 * U::T2 + ln, valid - 1);
            const bf16* cp2 = a.C + ((tok0 + row2) * G + g) * N + kg * 8;
#pragma unroll
            for (int ns = 0; ns < NS; ++ns) cot[ns] = *reinterpret_cast<const bf16x8*>(cp2 + ns * 32);
        }
    }
    __syncthreads();                                          // B rows and head 0 in LDS

    // ---- CB^T of this wavefront's units, bf16-rounded, masked, as floats:
    // cbv[u][i] = CB[m, k], m = 16 tile(u) + ln, k = 16 kt(u) + 4 kg + i
    float cbv[NU][4];
    {
        const char* bt = ring + SLOT;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int t = U::tile(u), kt = U::kt(u);
            const int m = 16 * t + ln;
            f32x4 acc = zero4();
            if (CBIN) {
                // row m, columns 16 kt + 4 kg .. + 3 of the given CB
                const int64_t o = ((((int64_t)bi * nc + ci) * G + g) * Q + m) * Q + 16 * kt + 4 * kg;
                if (a.cb_bf16) {
                    const bf16x4 c4 = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16*>(a.cb) + o);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = (float)c4[i];
                } else {
                    const float4 c4 = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.cb) + o);
                    acc[0] = c4.x; acc[1] = c4.y; acc[2] = c4.z; acc[3] = c4.w;
                }
            } else {
                const int r = 16 * kt + ln;
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    const bf16x8 bfr = *reinterpret_cast<const bf16x8*>(
                        bt + r * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(r)) * 16));
                    acc = mma32(bfr, (t == TM) ? cst[ns] : cot[ns], acc);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = 16 * kt + 4 * kg + i;
                float v = acc[i];
                if (k > m || m >= valid) v = 0.f;                // causal, k <= m < valid
                if (!CBIN && a.seq_idx && seqs[m] != seqs[k]) v = 0.f;
                cbv[u][i] = rbf(v);                              // CB is bf16 (reference)
            }
        }
    }
    __syncthreads();                                          // B rows no longer read

    const int mrow = 16 * TM + ln;                            // this lane's stored output row
    const float fmask = (a.seq_idx && seqs[mrow] != seq_prev) ? 0.f : 1.f;
    const bool fold_d = a.D && !a.D_has_hdim;
    // x^T fragment reads: lane (ln, kg) of a 16-lane group reads row
    // 16 kt + r0 of the group's 4 x 16 block at column chunk ch; the row
    // swizzle repeats every 8 rows, so a k-tile moves the offset by 2048 bytes
    int xo[4];
    {
        const int r0 = 4 * kg + (ln >> 2);
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
            const int ch = 2 * pt + ((ln & 3) >> 1);
            xo[pt] = r0 * 128 + ((ch ^ xswz(r0)) * 16) + 8 * (ln & 1);
        }
    }
    float* ft = ftab + w * 64;

    for (int j = 0; j < nh; ++j) {
        const int k = j % R;
        lds_barrier();                                        // slot k complete
        const char* slot = ring + k * SLOT;
        const float* dAs = reinterpret_cast<const float*>(slot + XB + S::SB);
        const float* dts = dAs + Q;
        const float* Ds = dAs + 2 * Q;
        const int h = h0 + j;
        bf16x4 zr[4];
        if (HASZ) {
            // gate rows from HBM, in flight during the compute below
            const bf16* zp = a.z + ((tok0 + min(mrow, valid - 1)) * H + h) * P;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) zr[pt] = *reinterpret_cast<const bf16x4*>(zp + 16 * pt + 4 * kg);
        }
        const float dval = fold_d ? Ds[0] : 0.f;

        // acc[0]: the stored tile; acc[1]: half 1's partial of the long tile
        f32x4 acc[2][4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) { acc[0][pt] = zero4(); acc[1][pt] = zero4(); }

        // hi / lo split of 4 weights of one unit
        auto split4 = [&](const float (&v)[4], bf16x4& hi, bf16x4& lo) {
            uint32_t h01, l01, h23, l23;
            split2(v[0], v[1], h01, l01);
            split2(v[2], v[3], h23, l23);
            typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
            const u2 hv = {h01, h23}, lv = {l01, l23};
            hi = __builtin_bit_cast(bf16x4, hv);
            lo = __builtin_bit_cast(bf16x4, lv);
        };
        // acc[SEL] += x^T W^T over one unit (two 16x16x16 MFMAs per head-dim tile)
        auto mac1 = [&](auto selc, int kt, const float (&v)[4]) {
            constexpr int SEL = decltype(selc)::value;
            bf16x4 wh, wl;
            split4(v, wh, wl);
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const bf16x4 xf = ds_read_tr(slot + kt * 2048 + xo[pt]);
                acc[SEL][pt] = mma16(xf, wh, acc[SEL][pt]);
                acc[SEL][pt] = mma16(xf, wl, acc[SEL][pt]);
            }
        };
        // acc += x^T W^T over two units of one tile (k index j < 4: unit a,
        // j >= 4: unit b; the hi parts in one 16x16x32 MFMA, the lo parts in another)
        auto mac2 = [&](auto selc, int ka, const float (&va)[4], int kb, const float (&vb)[4]) {
            constexpr int SEL = decltype(selc)::value;
            bf16x4 ha, la, hb, lb;
            split4(va, ha, la);
            split4(vb, hb, lb);
            const bf16x8 wh = __builtin_shufflevector(ha, hb, 0, 1, 2, 3, 4, 5, 6, 7);
            const bf16x8 wl = __builtin_shufflevector(la, lb, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const bf16x4 xa = ds_read_tr(slot + ka * 2048 + xo[pt]);
                const bf16x4 xb = ds_read_tr(slot + kb * 2048 + xo[pt]);
                const bf16x8 x8 = __builtin_shufflevector(xa, xb, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[SEL][pt] = mma32(x8, wh, acc[SEL][pt]);
                acc[SEL][pt] = mma32(x8, wl, acc[SEL][pt]);
            }
        };

        // 1. intra chunk, off-diagonal units.  When dA does not increase over
        // the chunk the decay factors through each tile's first row r:
        // ft[16 u + kk] = exp(dA[r] - dA[k]) dt[k] (k = 16 kt(u) + kk), and
        // exp(dA[m] - dA[r]) scales the tile's sum afterwards.
        bool mono = true;
        for (int q = lane; q < Q - 1; q += 64) mono = mono && dAs[q + 1] <= dAs[q];
        mono = __all(mono);
        float w_off[NOFF > 0 ? NOFF : 1][4];
        if (NOFF > 0) {
            if (mono) {
                const int s = lane >> 4, kk = lane & 15;
                if (s < NOFF) {
                    const int t = s < U::NL ? U::T2 : U::T1;
                    const int kt = s < U::NL ? (KH ? 4 + s : s) : s - U::NL;
                    const int kq = 16 * kt + kk;
                    ft[16 * s + kk] = ex2((dAs[16 * t] - dAs[kq]) * LOG2E) * dts[kq];
                }
#pragma unroll
                for (int u = 0; u < NOFF; ++u) {
                    const float4 f = *reinterpret_cast<const float4*>(ft + 16 * u + 4 * kg);
                    w_off[u][0] = cbv[u][0] * f.x; w_off[u][1] = cbv[u][1] * f.y;
                    w_off[u][2] = cbv[u][2] * f.z; w_off[u][3] = cbv[u][3] * f.w;
                }
            } else {
#pragma unroll
                for (int u = 0; u < NOFF; ++u) {
                    const int m = 16 * U::tile(u) + ln, k0 = 16 * U::kt(u) + 4 * kg;
                    const float dAm = dAs[m];
                    const float4 dk = *reinterpret_cast<const float4*>(dAs + k0);
                    const float4 tk = *reinterpret_cast<const float4*>(dts + k0);
                    w_off[u][0] = cbv[u][0] * ex2((dAm - dk.x) * LOG2E) * tk.x;
                    w_off[u][1] = cbv[u][1] * ex2((dAm - dk.y) * LOG2E) * tk.y;
                    w_off[u][2] = cbv[u][2] * ex2((dAm - dk.z) * LOG2E) * tk.z;
                    w_off[u][3] = cbv[u][3] * ex2((dAm - dk.w) * LOG2E) * tk.w;
                }
            }
            // units of one tile in pairs, a lone one last
            auto run_tile = [&](auto u0c, auto cntc) {
                constexpr int u0 = decltype(u0c)::value, cnt = decltype(cntc)::value;
                constexpr int SEL = (KH && U::tile(u0) == U::T2) ? 1 : 0;
#pragma unroll
                for (int p2 = 0; p2 + 1 < cnt; p2 += 2)
                    mac2(IC<SEL>{}, U::kt(u0 + p2), w_off[u0 + p2], U::kt(u0 + p2 + 1), w_off[u0 + p2 + 1]);
                if constexpr (cnt % 2 == 1) mac1(IC<SEL>{}, U::kt(u0 + cnt - 1), w_off[u0 + cnt - 1]);
            };
            run_tile(IC<0>{}, IC<U::NL>{});
            run_tile(IC<U::NL>{}, IC<U::NSH>{});
            if (mono) {
                // exp(dA[m] - dA[r]) of each tile with off-diagonal work
                if (U::NL > 0) {
                    constexpr int SEL = KH ? 1 : 0;
                    const float e = ex2((dAs[16 * U::T2 + ln] - dAs[16 * U::T2]) * LOG2E);
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[SEL][pt][i] *= e;
                }
                if (U::NSH > 0) {
                    const float e = ex2((dAs[16 * U::T1 + ln] - dAs[16 * U::T1]) * LOG2E);
#pragma unroll
                    for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) acc[0][pt][i] *= e;
                }
            }
        }
        // 2. the diagonal unit (the stored tile): direct weights for k <= m, 0
        // above (where the exponent may overflow), + D on the diagonal
        {
            constexpr int ud = NU - 1;
            const int k0 = 16 * TM + 4 * kg;
            const float dAm = dAs[mrow];
            const float4 dk = *reinterpret_cast<const float4*>(dAs + k0);
            const float4 tk = *reinterpret_cast<const float4*>(dts + k0);
            const float dkv[4] = {dk.x, dk.y, dk.z, dk.w}, tkv[4] = {tk.x, tk.y, tk.z, tk.w};
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = ex2((dAm - dkv[i]) * LOG2E);
                v[i] = k0 + i > mrow ? 0.f : cbv[ud][i] * e * tkv[i];
                if (k0 + i == mrow) v[i] += dval;
            }
            mac1(IC<0>{}, TM, v);
        }
        // 3. carried state of the stored tile: y^T += bf16(h_c C^T) exp(dA[m])
        {
            f32x4 cs[4];
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) cs[pt] = zero4();
            constexpr int NF = 4 * NS, BR = NS >= 8 ? 4 : 8;
#pragma unroll
            for (int f0 = 0; f0 < NF; f0 += BR) {
                bf16x8 sfr[BR];
#pragma unroll
                for (int q = 0; q < BR; ++q) {
                    const int pt = (f0 + q) / NS, ns = (f0 + q) % NS;
                    const int p = 16 * pt + ln;
                    sfr[q] = *reinterpret_cast<const bf16x8*>(
                        slot + XB + p * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(p)) * 16));
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < BR; ++q) {
                    const int pt = (f0 + q) / NS, ns = (f0 + q) % NS;
                    cs[pt] = mma32(sfr[q], cst[ns], cs[pt]);
                }
            }
            const float f = ex2(dAs[mrow] * LOG2E) * fmask;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[0][pt][i] += rbf(cs[pt][i]) * f;
        }
        // 4. + D x for a per-head-dim D
        if (a.D && a.D_has_hdim) {
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const int p0 = 16 * pt + 4 * kg;
                const int xoff = mrow * 128 + (((p0 >> 3) ^ xswz(mrow)) * 16) + 2 * (p0 & 7);
                const bf16x4 xv = *reinterpret_cast<const bf16x4*>(slot + xoff);
                const float4 d4 = *reinterpret_cast<const float4*>(Ds + p0);
                const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[0][pt][i] += dv[i] * (float)xv[i];
            }
        }
        // half 1's part of the long tile joins half 0's
        if (KH && U::NL > 0) {
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) xchg[PI][pt][lane] = acc[1][pt];
        }
        lds_barrier();
        if (!KH && Units<PI, 1>::NL > 0) {
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const f32x4 o = xchg[PI][pt][lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[0][pt][i] += o[i];
            }
        }
        // 5. epilogue: silu(z) gate in z's dtype; the tile goes to the staging
        // area (stored by the data wavefronts), through the wavefront's own
        // staging rows to HBM, or straight to HBM
        f32x4 vo[4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) {
            float v[4] = {acc[0][pt][0], acc[0][pt][1], acc[0][pt][2], acc[0][pt][3]};
            if (HASZ) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] *= rbf(silu_f((float)zr[pt][i]));
            }
            vo[pt] = f32x4{v[0], v[1], v[2], v[3]};
            if (S::STAGE) {
                // row ln, 16-byte chunk 4 pt + kg, XOR-swizzled by the row
                const int c = (4 * pt + kg) ^ ln;
                *reinterpret_cast<float4*>(stg + w * S::STW + ln * 256 + 16 * c) =
                    make_float4(v[0], v[1], v[2], v[3]);
            } else if (!S::WST && mrow < valid) {
                store_out<NT>(vo[pt], a.out + ((tok0 + mrow) * H + h) * P + 16 * pt + 4 * kg);
            }
        }
        if constexpr (S::WST) {
            // half hf (columns 32 hf ..): row ln, 16-byte chunk 4 pl + kg of the
            // 128-byte row, XOR-swizzled by the row; read back as whole rows
            char* sw = stg + w * S::WSTW;
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
                for (int pl = 0; pl < 2; ++pl)
                    *reinterpret_cast<f32x4*>(sw + ln * 128 + 16 * ((4 * pl + kg) ^ (ln & 7))) = vo[2 * hf + pl];
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                f32x4 o[2];
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int r = 8 * q + (lane >> 3);
                    o[q] = *reinterpret_cast<const f32x4*>(sw + r * 128 + 16 * ((lane & 7) ^ (r & 7)));
                }
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const int m = 16 * TM + 8 * q + (lane >> 3);
                    if (m < valid)
                        store_out<NT>(o[q], a.out + ((tok0 + m) * H + h) * P + 32 * hf + 4 * (lane & 7));
                }
            }
        }
    }
    if (S::STAGE) lds_barrier();                              // the last head's outputs staged
}

template <int NS, bool HASZ, bool CBIN, bool NT>
__global__ void __launch_bounds__(THREADS) k_scan_q128(ScanFusedArgs a) {
    typedef Cfg<NS> S;
    constexpr int N = S::N, SCPR = S::SCPR, R = S::R, XB = S::XB, SB = S::SB, SLOT = S::SLOT;
    __shared__ __align__(16) char ring[S::RING];
    __shared__ __align__(16) f32x4 xchg[4][4][64];
    __shared__ __align__(16) float ftab[NWAVES * 64];
    __shared__ __align__(16) char stg[S::STAGE ? S::STG : S::WST ? S::WSTG : 16];
    __shared__ int seqs[Q];

    const int L = a.L, H = a.H, G = a.G, nc = a.nc, hpg = a.hpg;
    // work = ((b nc + chunk) G + group) nslice + slice: the slices of a (chunk,
    // group), which read the same B / C rows, share an XCD
    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int sl = work % a.nslice;
    const int g = (work / a.nslice) % G;
    const int rest = work / (a.nslice * G);
    const int ci = rest % nc, bi = rest / nc;
    const int h0 = g * hpg + sl * a.hps;                  // this workgroup's heads h0 + j, j < nh
    const int nh = min(a.hps, hpg - sl * a.hps);
    const int lane = threadIdx.x & 63, w = wave_id();
    const int64_t tok0 = (int64_t)bi * L + (int64_t)ci * Q;
    const int valid = min(Q, L - ci * Q);
    const int64_t rs = (int64_t)G * N;                    // row stride of B / C
    const int seq_prev = (a.seq_idx && ci > 0) ? a.seq_idx[tok0 - 1] : 0;
    const uint32_t ring_lds = lds_addr(ring);
    for (int q = threadIdx.x; q < Q; q += THREADS)
        seqs[q] = (a.seq_idx && q < valid) ? a.seq_idx[tok0 + q] : -1;

    if (w < NWAVES) {
        // one instantiation of the compute path per (pair, half)
#define M2_Q128_CASE(W) \
        case W: compute_path<NS, HASZ, CBIN, NT, ((W) & 3), ((W) >> 2)>(a, ring, xchg, ftab, stg, seqs, bi, ci, g, h0, nh, valid, seq_prev); break;
        switch (w) {
            M2_Q128_CASE(0) M2_Q128_CASE(1) M2_Q128_CASE(2) M2_Q128_CASE(3)
            M2_Q128_CASE(4) M2_Q128_CASE(5) M2_Q128_CASE(6) M2_Q128_CASE(7)
        }
#undef M2_Q128_CASE
        return;
    }

    // ---- the data wavefronts: head j -> slot k.  Lane l of load u brings
    // 16-byte chunk 64 u + l of a tile (row, swizzled column); data wavefront
    // li takes its share of every tile's loads.
    const int li = w - NWAVES;
    const int64_t cq0 = ((int64_t)bi * H * nc + ci) * Q;  // dA / dt row of head 0 (+ h nc Q)
    const int64_t st0 = ((int64_t)bi * nc + ci) * H * P * N;
    // x and state rows non-temporally where the states exceed the cache
    const bool ntl = a.ntl;
    auto issue = [&](int j, int k) {
        const int h = h0 + j;
        const uint32_t sb = ring_lds + k * SLOT;
#pragma unroll
        for (int uu = 0; uu < S::XL; ++uu) {
            const int u = li * S::XL + uu;
            const int gi = 64 * u + lane, r = gi / 8;
            const int64_t off = (tok0 + min(r, valid - 1)) * H * P + h * P + 8 * ((gi % 8) ^ xswz(r));
            if (ntl) dma16nt(a.x + off, sb + 1024 * u);
            else dma16(a.x + off, sb + 1024 * u);
        }
        const bf16* sp = a.states + st0 + (int64_t)h * P * N;
#pragma unroll
        for (int uu = 0; uu < S::SL; ++uu) {
            const int u = li * S::SL + uu;
            const int gi = 64 * u + lane, p = gi / SCPR;
            const bf16* src = sp + p * N + 8 * ((gi % SCPR) ^ sswz<SCPR>(p));
            if (ntl) dma16nt(src, sb + XB + 1024 * u);
            else dma16(src, sb + XB + 1024 * u);
        }
        const int64_t row = cq0 + (int64_t)h * nc * Q;
        if (li == 0 && lane < Q / 2) {
            const float* src = lane < Q / 4 ? a.dA + row + 4 * lane : a.dt + row + 4 * (lane - Q / 4);
            dma16(src, sb + XB + SB);
        }
        if (li == 1) {
            const float* dsrc = a.D ? (a.D_has_hdim ? a.D + h * P + lane : a.D + h) : a.dA + cq0;
            dma4(dsrc, sb + XB + SB + 2 * Q * 4);
        }
    };
    // the group's B rows (aliasing ring slots 1..) and head 0
    const bf16* Bg = a.B + (tok0 * G + g) * N;
#pragma unroll
    for (int uu = 0; uu < (CBIN ? 0 : S::BL); ++uu) {
        const int u = li * S::BL + uu;
        const int gi = 64 * u + lane, r = gi / SCPR;
        dma16(Bg + min(r, valid - 1) * rs + 8 * ((gi % SCPR) ^ sswz<SCPR>(r)), ring_lds + SLOT + 1024 * u);
    }
    issue(0, 0);
    wait_vmem<0>();
    __syncthreads();                                      // B rows and head 0 in LDS
    __syncthreads();                                      // the CB build is done with the B rows

    // the output tiles of head j (staged by the compute wavefronts) to HBM:
    // data wavefront li stores those of compute wavefronts li and li + 4, one
    // 16-byte chunk per lane, 16 per store
    auto store_staged = [&](int j) {
        const int h = h0 + j;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int cw = li + 4 * half;                   // compute wavefront
            const int ct = half ? (cw & 3) : QT - 1 - (cw & 3);   // its stored row tile
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int o = 1024 * it + 16 * lane;
                const int row = o / 256, c = ((o % 256) / 16) ^ row;
                const f32x4 v = *reinterpret_cast<const f32x4*>(stg + cw * S::STW + o);
                const int m = 16 * ct + row;
                if (m < valid)
                    store_out<NT>(v, a.out + ((tok0 + m) * H + h) * P + 4 * c);
            }
        }
    };
#pragma unroll
    for (int i = 1; i < R - 1; ++i) issue(min(i, nh - 1), i);
    for (int j = 0; j < nh; ++j) {
        // head j's loads done (R - 2 later heads may still be in flight; the
        // output stores issued in between only make the wait longer)
        if (li < 2) wait_vmem<S::WAIT01>();
        else wait_vmem<S::WAIT23>();
        lds_barrier();                                      // slot j % R complete, slot (j-1) % R free,
                                                            // head j-1's outputs staged
        if (S::STAGE && j > 0) store_staged(j - 1);
        issue(min(j + R - 1, nh - 1), (j + R - 1) % R);
        lds_barrier();                                      // the compute wavefronts' exchange
    }
    if (S::STAGE) {
        lds_barrier();                                      // the last head's outputs staged
        store_staged(nh - 1);
    }
    wait_vmem<0>();     // the tail heads re-loaded into unused slots
}

}  // namespace

namespace m2 {

ScanKernel scan_q128_kernel(int ns, bool hasz, bool cbin, bool nt) {
#define M2_Q128_PICK(NSV)                                                                  \
    if (ns == NSV) return cbin ? k_scan_q128<NSV, false, true, false>                      \
                         : hasz ? (nt ? k_scan_q128<NSV, true, false, true> : k_scan_q128<NSV, true, false, false>) \
                                : (nt ? k_scan_q128<NSV, false, false, true> : k_scan_q128<NSV, false, false, false>);
    M2_Q128_PICK(2) M2_Q128_PICK(4) M2_Q128_PICK(8)
#undef M2_Q128_PICK
    return nullptr;
}

}  // namespace m2
