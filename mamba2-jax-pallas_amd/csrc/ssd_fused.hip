// k_scan_fused: bmm_chunk + chunk_scan of the combined forward for bf16 inputs.
//
//   y[m, :] = exp(dA[m]) * bf16(C[m, :] h_c^T)                     (carried state)
//           + sum_{k <= m} CB[m, k] exp(dA[m] - dA[k]) dt[k] x[k, :] (intra chunk)
//           + D x[m, :],   then y *= silu(z[m, :]) when z is given
// with CB = bf16(C B^T) (seq_idx-masked), h_c the bf16 state entering chunk c.
//
// One workgroup per (batch, chunk, group) covers every head of the group, so
// CB is built once and used by all of them (or a slice of them, when fewer
// than 256 (batch, chunk, group) items would leave CUs idle).  8 compute wavefronts (+ four that
// only load, below); the chunk's 16-row
// output tiles are paired (t, Q/16-1-t) so that every pair carries the same
// causal (triangular) work; the wavefronts of a pair split that work in two
// halves of (row tile, k-tile) units, the first accumulating the long tile's
// first KA k-tiles and its diagonal tile, the second the rest of it (a
// partial, summed through LDS) and the short tile (each half one of the two
// diagonal tiles, the dearer units), and (for Q = 64) the head dim in PPARTS
// parts.
//
// Per head, the x rows [Q x 64], the carried state [64 x N], dA / dt of the
// chunk and D are brought into a ring of R LDS slots by direct
// global -> LDS loads (global_load_lds_dwordx4), R - 1 heads ahead of use;
// the group's B rows use the same path once, for the CB build.  Four
// wavefronts besides the compute ones issue these loads (one alone cannot keep
// enough in flight) and wait for them (vmcnt) before the barrier that hands a
// slot over: vmcnt is one in-order counter per wavefront for loads and stores
// alike, so a wavefront that also stored the outputs would wait for its
// stores as well.  Rows are dense in LDS with their
// 16-byte chunks XOR-swizzled so that the reads below hit distinct banks.
//
// The products are computed transposed, y^T = h_c C^T + x^T W^T with
// W[m, k] = CB[m, k] exp(dA[m] - dA[k]) dt[k], so that each lane ends with 4
// consecutive head-dim values of one output row (16-byte stores, 8-byte D / z
// reads; the z rows come straight from HBM, issued before the compute):
//   * carried state: A = state rows (16-byte reads), B = C rows (registers),
//     16x16x32 MFMAs; the product is rounded to bf16 and scaled by exp(dA[m])
//     as in the reference (ops/ssd_naive.py:294-297);
//   * intra chunk: A = x^T via the gfx950 LDS transpose read, B = W^T, whose
//     layout (lane = output row m, 4 consecutive k) is exactly the
//     accumulator layout of the CB^T tiles built with 16x16x32 MFMAs
//     (A = B rows, B = C rows), so they feed 16x16x16 MFMAs without data
//     movement; W is split into bf16 hi + lo parts (two MFMAs, near-fp32).
//
// The same kernel serves the stage operator chunk_scan (bf16, no z) when CB
// comes in from bmm_chunk: the CB^T tiles are then read from HBM (fp32 or
// bf16, rounded to bf16 as the reference's chunk_scan kernel does,
// kernels/chunk_scan_fwd.py:386-394) with only the causal mask applied, since
// the seq_idx mask of CB belongs to bmm_chunk (kernels/chunk_scan_fwd.py
// :295-322 masks C only).
//
// Follows reference ops/ssd_naive.py:189-318 and kernels/chunk_scan_fwd.py
// :294-322 / kernels/bmm_chunk_fwd.py:353-372 (seq_idx masks).
#include <algorithm>
#include <type_traits>

#include "m2_internal.h"

namespace {

constexpr int NWAVES = 8;                 // compute wavefronts
constexpr int NLOAD = 4;                  // load wavefronts (one alone cannot keep
                                          // enough direct loads in flight)
constexpr int THREADS = (NWAVES + NLOAD) * 64;
constexpr int P = 64;
constexpr float LOG2E = 1.4426950408889634f;
constexpr int LDS_BYTES = 160 * 1024;

M2_DEV f32x4 mma16(bf16x4 a, bf16x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}
M2_DEV f32x4 mma32(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
M2_DEV float rbf(float v) { return (float)(bf16)v; }

// 16-byte chunk swizzles.  x rows are 128 bytes and read as chunk pairs by
// 16-lane groups (4 rows each) or as single 8-byte halves: an even mask keeps
// pairs together.  State / B rows (CPR chunks) are read 16 bytes per lane by
// 16 consecutive rows at one chunk.
M2_DEV int xswz(int r) { return ((r >> 1) & 3) << 1; }
template <int CPR> M2_DEV int sswz(int r) { return CPR == 8 ? ((r >> 1) & 7) : (r & 15); }

using m2::ScanFusedArgs;

template <int NS, int QT, bool HASZ>
struct Shape {
    static constexpr int N = 32 * NS, Q = 16 * QT;
    // wavefronts per row-tile pair: two halves of the pair's causal work (the
    // long row tile's first KA k-tiles and diagonal, and the rest) times
    // PPARTS parts of the head dim with PTW 16-column tiles each
    static constexpr int NPAIRS = QT / 2, WPP = NWAVES / NPAIRS, PPARTS = WPP / 2, PTW = 4 / PPARTS;
    static constexpr int KA = QT / 2;                       // <= the long tile t2
    static constexpr int SCPR = N / 8;                      // 16-byte chunks per state row
    static constexpr int XB = Q * P * 2, SB = P * N * 2, ZB = 0;
    static constexpr int AUXB = 2 * Q * 4 + 64 * 4;         // dA, dt, D
    static constexpr int SLOT = XB + SB + ZB + AUXB;
    static constexpr int BT = Q * N * 2;                    // the group's B rows
    static constexpr int CBL = NPAIRS * (QT + 1) * 64 * 8;  // CB^T tiles
    static constexpr int XCHG = NPAIRS * 4 * 64 * 16;       // second-half partials
    static constexpr int FTAB = NWAVES * 8 * 16 * 4;            // decay factor tables
    static constexpr int FIXED = CBL + XCHG + FTAB + Q * 4 + 256;
    static constexpr int ring_bytes(int r) { return r * SLOT > SLOT + BT ? r * SLOT : SLOT + BT; }
    // output staging: each compute wavefront's finished 16 x 16 PTW fp32 tile,
    // stored to HBM by the load wavefronts (when it fits beside the ring)
    static constexpr int STW = 16 * 16 * PTW * 4, STG = NWAVES * STW;
    static constexpr bool STAGE = ring_bytes(2) + FIXED + STG <= LDS_BYTES;
    static constexpr int R = ring_bytes(3) + FIXED + (STAGE ? STG : 0) <= LDS_BYTES ? 3 : 2;
    static constexpr int RING = ring_bytes(R);
    // 1 KB direct loads of the load wavefront per head / for the B rows
    static constexpr int XI = XB / 1024, SI = SB / 1024, ZI = ZB / 1024, BI = BT / 1024;
    // per load wavefront: XL + SL tile loads (+ dA / dt or D for wavefronts 0, 1)
    static constexpr int XL = XI / NLOAD, SL = SI / NLOAD, BL = BI / NLOAD;
    static constexpr int WAIT01 = (R - 2) * (XL + SL + 1), WAIT23 = (R - 2) * (XL + SL);
    static_assert(XI % NLOAD == 0 && SI % NLOAD == 0 && BI % NLOAD == 0, "even load split");
    static_assert(NPAIRS * WPP == NWAVES && PPARTS * PTW == 4 && PPARTS >= 1, "wavefront split");
    static_assert(ring_bytes(R) + FIXED + (STAGE ? STG : 0) <= LDS_BYTES, "LDS budget");
    static_assert(WAIT01 <= 63, "vmcnt range");
};

// CBIN: CB given in a.cb (the chunk_scan stage operator) instead of built here
template <int NS, int QT, bool HASZ, bool CBIN>
__global__ void __launch_bounds__(THREADS) k_scan_fused(ScanFusedArgs a) {
    typedef Shape<NS, QT, HASZ> S;
    constexpr int N = S::N, Q = S::Q, NPAIRS = S::NPAIRS, PTW = S::PTW, R = S::R;
    constexpr int XB = S::XB, SB = S::SB, ZB = S::ZB, SLOT = S::SLOT, SCPR = S::SCPR;
    __shared__ __align__(16) char ring[S::RING];
    __shared__ __align__(16) bf16x4 cbl[NPAIRS][QT + 1][64];
    __shared__ __align__(16) f32x4 xchg[NPAIRS][4][64];
    __shared__ __align__(16) float ftab[NWAVES][8 * 16];   // decay factors of each wavefront's units
    __shared__ __align__(16) char stg[S::STAGE ? S::STG : 16];  // output tiles on their way to HBM
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
    const int ln = lane & 15, kg = lane >> 4;
    const int pi = w % NPAIRS, ph = w / NPAIRS;
    const int kh = ph & 1, pp = ph >> 1;                  // work half, head-dim part
    const int t1 = pi, t2 = QT - 1 - pi;
    const int64_t tok0 = (int64_t)bi * L + (int64_t)ci * Q;
    const int valid = min(Q, L - ci * Q);
    const int64_t rs = (int64_t)G * N;                    // row stride of B / C
    const int seq_prev = (a.seq_idx && ci > 0) ? a.seq_idx[tok0 - 1] : 0;
    const uint32_t ring_lds = lds_addr(ring);

    const bool loader = w >= NWAVES;
    const int li = w - NWAVES;                            // load wavefront index

    // ---- plain loads: C fragments of the pair's two row tiles, seq ids -----
    bf16x8 cfr[2][NS];
    if (!loader) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int row = min(16 * (tt ? t2 : t1) + ln, valid - 1);   // clamped; masked below
            const bf16* cp = a.C + ((tok0 + row) * G + g) * N + kg * 8;
#pragma unroll
            for (int ns = 0; ns < NS; ++ns) cfr[tt][ns] = *reinterpret_cast<const bf16x8*>(cp + ns * 32);
        }
    }
    for (int q = threadIdx.x; q < Q; q += THREADS)
        seqs[q] = (a.seq_idx && q < valid) ? a.seq_idx[tok0 + q] : -1;

    // ---- the load wavefronts: head j -> slot k.  Lane l of load u brings
    // 16-byte chunk 64 u + l of a tile (row, swizzled column); load wavefront
    // li takes its share of every tile's loads.
    const int64_t cq0 = ((int64_t)bi * H * nc + ci) * Q;  // dA / dt row of head 0 (+ h nc Q)
    const int64_t st0 = ((int64_t)bi * nc + ci) * H * P * N;
    auto issue = [&](int j, int k) {
        const int h = h0 + j;
        const uint32_t sb = ring_lds + k * SLOT;
#pragma unroll
        for (int uu = 0; uu < S::XL; ++uu) {
            const int u = li * S::XL + uu;
            const int gi = 64 * u + lane, r = gi / 8;
            const int64_t off = (tok0 + min(r, valid - 1)) * H * P + h * P + 8 * ((gi % 8) ^ xswz(r));
            dma16(a.x + off, sb + 1024 * u);
        }
        const bf16* sp = a.states + st0 + (int64_t)h * P * N;
#pragma unroll
        for (int uu = 0; uu < S::SL; ++uu) {
            const int u = li * S::SL + uu;
            const int gi = 64 * u + lane, p = gi / SCPR;
            dma16(sp + p * N + 8 * ((gi % SCPR) ^ sswz<SCPR>(p)), sb + XB + 1024 * u);
        }
        const int64_t row = cq0 + (int64_t)h * nc * Q;
        if (li == 0 && lane < Q / 2) {
            const float* src = lane < Q / 4 ? a.dA + row + 4 * lane : a.dt + row + 4 * (lane - Q / 4);
            dma16(src, sb + XB + SB + ZB);
        }
        if (li == 1) {
            const float* dsrc = a.D ? (a.D_has_hdim ? a.D + h * P + lane : a.D + h) : a.dA + cq0;
            dma4(dsrc, sb + XB + SB + ZB + 2 * Q * 4);
        }
    };

    // ---- the group's B rows (aliasing ring slots 1..) and head 0 -----------
    if (loader) {
        const bf16* Bg = a.B + (tok0 * G + g) * N;
#pragma unroll
        for (int uu = 0; uu < (CBIN ? 0 : S::BL); ++uu) {
            const int u = li * S::BL + uu;
            const int gi = 64 * u + lane, r = gi / SCPR;
            dma16(Bg + min(r, valid - 1) * rs + 8 * ((gi % SCPR) ^ sswz<SCPR>(r)),
                  ring_lds + SLOT + 1024 * u);
        }
        issue(0, 0);
        wait_vmem<0>();
    }
    __syncthreads();

    // ---- CB^T tiles of each pair: (t1, kt <= t1) in slots 0..t1, (t2, kt <= t2)
    // in slots t1+1..; the pair's wavefronts share them out
    if (!loader) {
        const char* bt = ring + SLOT;
        for (int j = ph; j < QT + 1; j += S::WPP) {
            const bool second = j > t1;
            const int t = second ? t2 : t1;
            const int kt = second ? j - t1 - 1 : j;
            const int m = 16 * t + ln;
            f32x4 acc = zero4();
            if (CBIN) {
                // row m, columns 16 kt + 4 kg .. + 3 of the given CB
                const int64_t o = ((((int64_t)bi * nc + ci) * G + g) * Q + m) * Q + 16 * kt + 4 * kg;
                if (a.cb_bf16) {
                    const bf16x4 c4 = *reinterpret_cast<const bf16x4*>(
                        reinterpret_cast<const bf16*>(a.cb) + o);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[i] = (float)c4[i];
                } else {
                    const float4 c4 = *reinterpret_cast<const float4*>(
                        reinterpret_cast<const float*>(a.cb) + o);
                    acc[0] = c4.x; acc[1] = c4.y; acc[2] = c4.z; acc[3] = c4.w;
                }
            } else {
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    const int r = 16 * kt + ln;
                    const bf16x8 bfr = *reinterpret_cast<const bf16x8*>(
                        bt + r * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(r)) * 16));
                    acc = mma32(bfr, second ? cfr[1][ns] : cfr[0][ns], acc);
                }
            }
            bf16x4 v4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = 16 * kt + 4 * kg + i;
                float v = acc[i];
                if (k > m || m >= valid) v = 0.f;          // causal, k <= m < valid
                if (!CBIN && a.seq_idx && seqs[m] != seqs[k]) v = 0.f;
                v4[i] = (bf16)v;                            // CB is bf16 (reference)
            }
            cbl[pi][j][lane] = v4;
        }
    }
    __syncthreads();                                        // B rows no longer read

    // seq masks of the carried-state term (per output row m = 16 t + ln)
    float fmask[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int m = 16 * (tt ? t2 : t1) + ln;
        fmask[tt] = (a.seq_idx && seqs[m] != seq_prev) ? 0.f : 1.f;
    }

    // the output tiles of head j (staged by the compute wavefronts) to HBM:
    // load wavefront li stores those of compute wavefronts li and li + 4, one
    // 16-byte chunk per lane, 16 PTW (4 PTW with PTW 16 KB rows) per store
    auto store_staged = [&](int j) {
        const int h = h0 + j;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const int cw = li + 4 * half;                   // compute wavefront
            const int cph = cw / NPAIRS, ckh = cph & 1, cpp = cph >> 1, cpi = cw % NPAIRS;
            const int ct = ckh ? cpi : QT - 1 - cpi;        // its row tile
#pragma unroll
            for (int it = 0; it < PTW; ++it) {
                const int o = 1024 * it + 16 * lane;
                const int row = o / (64 * PTW), c = ((o % (64 * PTW)) / 16) ^ (row & (4 * PTW - 1));
                const float4 v = *reinterpret_cast<const float4*>(stg + cw * S::STW + o);
                const int m = 16 * ct + row;
                if (m < valid)
                    *reinterpret_cast<float4*>(a.out + ((tok0 + m) * H + h) * P + 16 * PTW * cpp + 4 * c) = v;
            }
        }
    };
    if (loader) {
#pragma unroll
        for (int i = 1; i < R - 1; ++i) issue(min(i, nh - 1), i);
        for (int j = 0; j < nh; ++j) {
            // head j's loads done (R - 2 later heads may still be in flight;
            // the output stores issued in between only make the wait longer)
            if (li < 2) wait_vmem<S::WAIT01>();
            else wait_vmem<S::WAIT23>();
            lds_barrier();                                  // slot j % R complete, slot (j-1) % R free,
                                                            // head j-1's outputs staged
            if (S::STAGE && j > 0) store_staged(j - 1);
            issue(min(j + R - 1, nh - 1), (j + R - 1) % R);
            lds_barrier();                                  // the compute wavefronts' exchange
        }
        if (S::STAGE) {
            lds_barrier();                                  // the last head's outputs staged
            store_staged(nh - 1);
        }
        wait_vmem<0>();     // the tail heads re-loaded into unused slots
        return;
    }
    // this wavefront's row tiles: the first half (kh == 0) accumulates the
    // long tile t2 over k-tiles [0, KA) and t2; the second half t2 over
    // [KA, t2) (a partial, added in through LDS) and the short tile t1 over
    // [0, t1]
    constexpr int KA = S::KA;
    const int tmine = kh ? t1 : t2;                    // the tile this wavefront stores
    // x^T fragment reads: lane (ln, kg) of a 16-lane group reads row
    // 16 kt + r0 of the group's 4 x 16 block at column chunk ch; the row
    // swizzle repeats every 8 rows, so only 16 kt rows (2048 bytes) change
    int xo[PTW];
    {
        const int r0 = 4 * kg + (ln >> 2);
#pragma unroll
        for (int pt = 0; pt < PTW; ++pt) {
            const int ch = 2 * (PTW * pp + pt) + ((ln & 3) >> 1);
            xo[pt] = r0 * 128 + ((ch ^ xswz(r0)) * 16) + 8 * (ln & 1);
        }
    }
    for (int j = 0; j < nh; ++j) {
        const int k = j % R;
        lds_barrier();
        const char* slot = ring + k * SLOT;
        const float* dAs = reinterpret_cast<const float*>(slot + XB + SB + ZB);
        const float* dts = dAs + Q;
        const float* Ds = dAs + 2 * Q;
        const int h = h0 + j;
        const int mrow = 16 * tmine + ln;              // output row of this lane
        bf16x4 zr[PTW];
        if (HASZ) {
            // gate rows from HBM, in flight during the compute below
            const bf16* zp = a.z + ((tok0 + min(mrow, valid - 1)) * H + h) * P;
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt)
                zr[pt] = *reinterpret_cast<const bf16x4*>(zp + 16 * (PTW * pp + pt) + 4 * kg);
        }

        f32x4 acc[2][PTW];                             // [0]: tile t1, [1]: tile t2
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) acc[tt][pt] = zero4();

        // acc[TT] += x^T W^T over k-tile kt, from this lane's 4 values of W^T
        // (output row m = 16 t + ln, k = 16 kt + 4 kg + i), split into bf16
        // hi + lo parts: one K = 32 MFMA, k index i < 4 pairs x with the hi
        // part, 4 + i the same x with the lo part
        auto mac1 = [&](auto ttc, int kt, const float (&v)[4]) {
            constexpr int TT = decltype(ttc)::value;
            uint32_t h01, l01, h23, l23;
            split2(v[0], v[1], h01, l01);
            split2(v[2], v[3], h23, l23);
            const bf16x8 w8 = as_bf16x8(h01, h23, l01, l23);
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const bf16x4 xf = ds_read_tr(slot + kt * 2048 + xo[pt]);
                const bf16x8 x8 = __builtin_shufflevector(xf, xf, 0, 1, 2, 3, 0, 1, 2, 3);
                acc[TT][pt] = mma32(x8, w8, acc[TT][pt]);
            }
        };
        // two k-tiles: k index i < 4 is k-tile ka, 4 + i k-tile kb; the hi
        // parts in one K = 32 MFMA, the lo parts in another
        auto mac2 = [&](auto ttc, int ka, const float (&va)[4], int kb, const float (&vb)[4]) {
            constexpr int TT = decltype(ttc)::value;
            uint32_t ha01, la01, ha23, la23, hb01, lb01, hb23, lb23;
            split2(va[0], va[1], ha01, la01);
            split2(va[2], va[3], ha23, la23);
            split2(vb[0], vb[1], hb01, lb01);
            split2(vb[2], vb[3], hb23, lb23);
            const bf16x8 wh = as_bf16x8(ha01, ha23, hb01, hb23);
            const bf16x8 wl = as_bf16x8(la01, la23, lb01, lb23);
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const bf16x4 xa = ds_read_tr(slot + ka * 2048 + xo[pt]);
                const bf16x4 xb = ds_read_tr(slot + kb * 2048 + xo[pt]);
                const bf16x8 x8 = __builtin_shufflevector(xa, xb, 0, 1, 2, 3, 4, 5, 6, 7);
                acc[TT][pt] = mma32(x8, wh, acc[TT][pt]);
                acc[TT][pt] = mma32(x8, wl, acc[TT][pt]);
            }
        };
        // direct weights W[m, k] = CB[m, k] exp(dA[m] - dA[k]) dt[k] for k <= m,
        // 0 above the diagonal (where the exponent may overflow); the decay in
        // the log2 domain
        auto direct = [&](auto ttc, int kt) {
            constexpr int TT = decltype(ttc)::value;
            const int t = TT ? t2 : t1;
            const int k0 = 16 * kt + 4 * kg, m = 16 * t + ln;
            const float dAm = dAs[m];
            const float4 dk = *reinterpret_cast<const float4*>(dAs + k0);
            const float4 tk = *reinterpret_cast<const float4*>(dts + k0);
            const float dkv[4] = {dk.x, dk.y, dk.z, dk.w}, tkv[4] = {tk.x, tk.y, tk.z, tk.w};
            const bf16x4 cb4 = cbl[pi][TT ? t1 + 1 + kt : kt][lane];
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float e = __builtin_amdgcn_exp2f((dAm - dkv[i]) * LOG2E);
                v[i] = k0 + i > m ? 0.f : (float)cb4[i] * e * tkv[i];
            }
            mac1(ttc, kt, v);
        };
        const std::integral_constant<int, 0> T1c{};
        const std::integral_constant<int, 1> T2c{};

        // 1. intra chunk: y^T += x^T W^T over this wavefront's (tile, k-tile)
        // units: the first half (kh == 0) the long tile t2 over k-tiles
        // [0, KA) and its diagonal k-tile t2, the second half t2 over
        // [KA, t2) (a partial, added in through LDS) and the short tile t1
        // over [0, t1].
        // When dA does not increase over the chunk (dt >= 0, A <= 0: every
        // Mamba2 layer) the off-diagonal k-tiles (kt < t) of row tile t factor
        // through its first row r = 16 t:
        //   exp(dA[m] - dA[k]) = exp(dA[m] - dA[r]) exp(dA[r] - dA[k]),
        // both factors <= 1 (no overflow; a factor that underflows bounds the
        // product).  F[k] = exp(dA[r] - dA[k]) dt[k] is computed once per unit
        // (16 values, a wavefront-private table) and exp(dA[m] - dA[r]) scales
        // the off-diagonal sum; the diagonal tiles keep the direct weights.
        bool mono = true;
        for (int q = lane; q < Q - 1; q += 64) mono = mono && dAs[q + 1] <= dAs[q];
        if (__all(mono)) {
            // units: tile t2 over k-tiles [lo2, hi2) -> table slots kt - lo2,
            // tile t1 over [0, hi1) -> slots 4 + kt
            const int lo2 = kh ? KA : 0, hi2 = kh ? t2 : KA, hi1 = kh ? t1 : 0;
            float* ft = ftab[w];
#pragma unroll
            for (int pass = 0; pass < 2; ++pass) {
                const int sl = 4 * pass + kg;
                const bool is2 = !kh || sl < 4;
                const int kt = is2 ? lo2 + sl : sl - 4;
                if (kt < (is2 ? hi2 : hi1)) {
                    const int kk = 16 * kt + ln, r0 = 16 * (is2 ? t2 : t1);
                    ft[16 * sl + ln] = __builtin_amdgcn_exp2f((dAs[r0] - dAs[kk]) * LOG2E) * dts[kk];
                }
            }
            auto fw = [&](int sl, int ci, float (&v)[4]) {   // CB (slot ci of the pair) x F
                const float4 f = *reinterpret_cast<const float4*>(ft + 16 * sl + 4 * kg);
                const bf16x4 cb4 = cbl[pi][ci][lane];
                v[0] = (float)cb4[0] * f.x; v[1] = (float)cb4[1] * f.y;
                v[2] = (float)cb4[2] * f.z; v[3] = (float)cb4[3] * f.w;
            };
            int kt = lo2;
            for (; kt + 1 < hi2; kt += 2) {
                float va[4], vb[4];
                fw(kt - lo2, t1 + 1 + kt, va);
                fw(kt + 1 - lo2, t1 + 2 + kt, vb);
                mac2(T2c, kt, va, kt + 1, vb);
            }
            if (kt < hi2) {
                float va[4];
                fw(kt - lo2, t1 + 1 + kt, va);
                mac1(T2c, kt, va);
            }
            for (kt = 0; kt + 1 < hi1; kt += 2) {
                float va[4], vb[4];
                fw(4 + kt, kt, va);
                fw(5 + kt, kt + 1, vb);
                mac2(T1c, kt, va, kt + 1, vb);
            }
            if (kt < hi1) {
                float va[4];
                fw(4 + kt, kt, va);
                mac1(T1c, kt, va);
            }
            const float e1 = __builtin_amdgcn_exp2f((dAs[16 * t1 + ln] - dAs[16 * t1]) * LOG2E);
            const float e2 = __builtin_amdgcn_exp2f((dAs[16 * t2 + ln] - dAs[16 * t2]) * LOG2E);
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc[0][pt][i] *= e1;
                    acc[1][pt][i] *= e2;
                }
            if (kh) direct(T1c, t1);
            else direct(T2c, t2);
        } else {
            for (int kt = 0; kt <= t2; ++kt) {
                if (kh && kt <= t1) direct(T1c, kt);
                if (kh ? kt >= KA && kt < t2 : kt < KA || kt == t2) direct(T2c, kt);
            }
        }

        // 2. carried state of the stored tile: y^T += bf16(h_c C^T) exp(dA[m])
        {
            f32x4 ci_[PTW];
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) ci_[pt] = zero4();
            // state fragments in blocks of BR reads, each block read before
            // its MFMAs are issued (fragment f: head-dim tile f / NS, k step f % NS)
            constexpr int NF = PTW * NS, BR = (NS >= 8 ? 4 : 8) < NF ? (NS >= 8 ? 4 : 8) : NF;
#pragma unroll
            for (int f0 = 0; f0 < NF; f0 += BR) {
                bf16x8 sfr[BR];
#pragma unroll
                for (int q = 0; q < BR; ++q) {
                    const int pt = (f0 + q) / NS, ns = (f0 + q) % NS;
                    const int p = 16 * (PTW * pp + pt) + ln;
                    sfr[q] = *reinterpret_cast<const bf16x8*>(
                        slot + XB + p * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(p)) * 16));
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < BR; ++q) {
                    const int pt = (f0 + q) / NS, ns = (f0 + q) % NS;
                    ci_[pt] = mma32(sfr[q], kh ? cfr[0][ns] : cfr[1][ns], ci_[pt]);
                }
            }
            const float f = __builtin_amdgcn_exp2f(dAs[mrow] * LOG2E) * (kh ? fmask[0] : fmask[1]);
            if (kh) {
#pragma unroll
                for (int pt = 0; pt < PTW; ++pt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[0][pt][i] += rbf(ci_[pt][i]) * f;
            } else {
#pragma unroll
                for (int pt = 0; pt < PTW; ++pt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[1][pt][i] += rbf(ci_[pt][i]) * f;
            }
        }
        // 3. + D x for the stored tile
        if (a.D) {
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const int p0 = 16 * (PTW * pp + pt) + 4 * kg;
                const int xoff = mrow * 128 + (((p0 >> 3) ^ xswz(mrow)) * 16) + 2 * (p0 & 7);
                const bf16x4 xv = *reinterpret_cast<const bf16x4*>(slot + xoff);
                float dv[4];
                if (a.D_has_hdim) {
                    const float4 d4 = *reinterpret_cast<const float4*>(Ds + p0);
                    dv[0] = d4.x; dv[1] = d4.y; dv[2] = d4.z; dv[3] = d4.w;
                } else {
                    dv[0] = dv[1] = dv[2] = dv[3] = Ds[0];
                }
                if (kh) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[0][pt][i] += dv[i] * (float)xv[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[1][pt][i] += dv[i] * (float)xv[i];
                }
            }
        }
        // the second half's part of tile t2 joins the first half's
        if (kh) {
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) xchg[pi][PTW * pp + pt][lane] = acc[1][pt];
        }
        lds_barrier();
        if (!kh) {
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const f32x4 o = xchg[pi][PTW * pp + pt][lane];
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[1][pt][i] += o[i];
            }
        }
        // 4. epilogue: silu(z) gate in z's dtype; the tile goes to the staging
        // area (stored by the load wavefronts) or straight to HBM
#pragma unroll
        for (int pt = 0; pt < PTW; ++pt) {
            const f32x4 r = kh ? acc[0][pt] : acc[1][pt];
            float v[4] = {r[0], r[1], r[2], r[3]};
            if (HASZ) {
#pragma unroll
                for (int i = 0; i < 4; ++i) v[i] *= rbf(silu_f((float)zr[pt][i]));
            }
            if (S::STAGE) {
                // row ln, 16-byte chunk 4 pt + kg, XOR-swizzled by the row
                const int c = (4 * pt + kg) ^ (ln & (4 * PTW - 1));
                *reinterpret_cast<float4*>(stg + w * S::STW + ln * (64 * PTW) + 16 * c) =
                    make_float4(v[0], v[1], v[2], v[3]);
            } else if (mrow < valid) {
                const int p0 = 16 * (PTW * pp + pt) + 4 * kg;
                *reinterpret_cast<float4*>(a.out + ((tok0 + mrow) * H + h) * P + p0) =
                    make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
    if (S::STAGE) lds_barrier();                       // the last head's outputs staged
}

}  // namespace

namespace m2 {

// True when the fused path covers these sizes (bf16, headdim 64).
bool scan_fused_supported(int64_t headdim, int64_t dstate, int64_t chunk_size) {
    return headdim == 64 && (dstate == 64 || dstate == 128 || dstate == 256) &&
           (chunk_size == 64 || chunk_size == 128);
}

namespace {

// f: pointers filled in; a: the sizes (batch, seqlen, nheads, ngroups,
// headdim, dstate, chunk_size); hz: with the z gate; cbin: CB given in f.cb
template <typename Sizes>
int launch_scan_fused_common(ScanFusedArgs& f, const Sizes& a, bool hz, bool cbin, hipStream_t s) {
    M2_REQUIRE(a.ngroups > 0 && a.nheads % a.ngroups == 0, M2_ERR_INVALID,
               "scan_fused: nheads %% ngroups != 0");
    const int64_t nc = (a.seqlen + a.chunk_size - 1) / a.chunk_size;
    const int hpg = (int)(a.nheads / a.ngroups);
    // a group's heads split over enough workgroups to fill the 256 CUs (each
    // slice builds CB again: cheap next to its heads' work)
    const int64_t items = a.batch * nc * a.ngroups;
    int nslice = (int)std::min<int64_t>(hpg, std::max<int64_t>(1, (256 + items - 1) / items));
    const int hps = (hpg + nslice - 1) / nslice;
    nslice = (hpg + hps - 1) / hps;
    const int64_t nwork = items * nslice;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "scan_fused: too many blocks");
    f.L = (int)a.seqlen; f.H = (int)a.nheads; f.G = (int)a.ngroups; f.nc = (int)nc;
    f.hpg = hpg; f.nwork = (int)nwork; f.hps = hps; f.nslice = nslice;
    // The fp32 output is written once and not read again by the layer.  For the
    // chunk-128 kernel (csrc/ssd_scan128.hip; the chunk-64 one ignores it): while
    // it is at most the 256 MB Infinity Cache, non-temporal stores keep it from
    // evicting the states entering each chunk that the scan is still reading
    // (and the inputs): measured (A/B on one box) c2 0.0967 -> 0.0946 ms per
    // layer, c1 0.135 -> 0.120 ms.  Larger outputs (c3: 537 MB) stream better
    // as ordinary stores (0.637 against 0.645 ms).
    const bool nt = (double)a.batch * a.seqlen * a.nheads * a.headdim * 4 <= 256.0 * (1 << 20);
    // States entering the chunks beyond the cache (c3: 537 MB of bf16) are
    // read once here: the chunk-128 kernel loads them and x non-temporally, so
    // they do not displace what the cache still holds (A/B on one box at c3:
    // scan 302 -> 262 us; with the varlen states moved before the scan, layer
    // 0.553 -> 0.525 ms).  At c1 / c2 (states in the cache) the same loads
    // cost the next call's state pass more than the scan gains (c2 0.092 ->
    // 0.105 ms).
    f.ntl = (double)a.batch * nc * a.nheads * a.headdim * a.dstate * 2 > 256.0 * (1 << 20);
    void (*kern)(ScanFusedArgs) = nullptr;
    // chunk 128: the kernel with per-wavefront compile-time unit lists
    // (csrc/ssd_scan128.hip); chunk 64: k_scan_fused
    if (a.chunk_size == 128 && a.dstate % 32 == 0) kern = m2::scan_q128_kernel((int)(a.dstate / 32), hz, cbin, nt);
#define M2_SF_CASE(NSV, QTV)                                                        \
    if (a.dstate == 32 * NSV && a.chunk_size == 16 * QTV)                           \
        kern = cbin ? k_scan_fused<NSV, QTV, false, true>                          \
                    : hz ? k_scan_fused<NSV, QTV, true, false> : k_scan_fused<NSV, QTV, false, false>;
    M2_SF_CASE(2, 4) M2_SF_CASE(4, 4) M2_SF_CASE(8, 4)
#undef M2_SF_CASE
    static_assert(THREADS == m2::SCAN_Q128_THREADS, "both scan kernels take the same block");
    M2_REQUIRE(kern && a.headdim == P, M2_ERR_UNSUPPORTED, "scan_fused: unsupported sizes");
    kern<<<(unsigned)nwork, THREADS, 0, s>>>(f);
    return m2::check_launch("scan_fused");
}

}  // namespace

int launch_scan_fused(const m2_ssd_combined_args& a, const float* dA, const float* dto,
                      const void* passed, hipStream_t s) {
    ScanFusedArgs f{};
    f.x = (const bf16*)a.x; f.B = (const bf16*)a.B; f.C = (const bf16*)a.C;
    f.states = (const bf16*)passed; f.dt = dto; f.dA = dA; f.D = a.D; f.z = (const bf16*)a.z;
    f.seq_idx = a.seq_idx; f.out = a.out; f.D_has_hdim = a.D_has_hdim;
    return launch_scan_fused_common(f, a, a.z != nullptr, false, s);
}

bool scan_fused_cb_supported(const m2_chunk_scan_args& a) {
    return a.dtype == M2_BF16 && a.states_dtype == M2_BF16 && !a.z && !a.out_x &&
           (a.cb_dtype == M2_F32 || a.cb_dtype == M2_BF16) &&
           scan_fused_supported(a.headdim, a.dstate, a.chunk_size);
}

int launch_scan_fused_cb(const m2_chunk_scan_args& a, hipStream_t s) {
    M2_REQUIRE(scan_fused_cb_supported(a), M2_ERR_UNSUPPORTED,
               "chunk_scan: unsupported shape / dtype for the fused kernel");
    ScanFusedArgs f{};
    f.x = (const bf16*)a.x; f.C = (const bf16*)a.C; f.states = (const bf16*)a.states;
    f.dt = a.dt; f.dA = a.dA_cumsum; f.D = a.D; f.seq_idx = a.seq_idx; f.out = a.out;
    f.D_has_hdim = a.D_has_hdim; f.cb = a.cb; f.cb_bf16 = a.cb_dtype == M2_BF16;
    return launch_scan_fused_common(f, a, false, true, s);
}

}  // namespace m2
