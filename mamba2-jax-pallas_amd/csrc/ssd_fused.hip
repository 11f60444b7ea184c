// k_scan_fused: bmm_chunk + chunk_scan of the combined forward for bf16 inputs.
//
//   y[m, :] = exp(dA[m]) * bf16(C[m, :] h_c^T)                     (carried state)
//           + sum_{k <= m} CB[m, k] exp(dA[m] - dA[k]) dt[k] x[k, :] (intra chunk)
//           + D x[m, :],   then y *= silu(z[m, :]) when z is given
// with CB = bf16(C B^T) (seq_idx-masked), h_c the bf16 state entering chunk c.
//
// One workgroup per (batch, chunk, group) covers every head of the group, so
// CB is built once and used by all of them.  8 compute wavefronts (+ four that
// only load, below); the chunk's 16-row
// output tiles are paired (t, Q/16-1-t) so that every pair carries the same
// causal (triangular) work; the wavefronts of a pair split that work in two
// halves of (row tile, k-tile) units, the first accumulating the long tile's
// first KA k-tiles, the second the rest of it (a partial, summed through LDS)
// and the short tile, and (for Q = 64) the head dim in PPARTS parts.
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
// Follows reference ops/ssd_naive.py:189-318 and kernels/chunk_scan_fwd.py
// :294-322 / kernels/bmm_chunk_fwd.py:353-372 (seq_idx masks).
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
    int L, H, G, nc, hpg, nwork;
};

template <int NS, int QT, bool HASZ>
struct Shape {
    static constexpr int N = 32 * NS, Q = 16 * QT;
    // wavefronts per row-tile pair: two halves of the pair's causal work (the
    // k-tiles of the long row tile up to KA, and the rest) times PPARTS parts
    // of the head dim with PTW 16-column tiles each
    static constexpr int NPAIRS = QT / 2, WPP = NWAVES / NPAIRS, PPARTS = WPP / 2, PTW = 4 / PPARTS;
    static constexpr int KA = QT / 2 + 1;
    static constexpr int SCPR = N / 8;                      // 16-byte chunks per state row
    static constexpr int XB = Q * P * 2, SB = P * N * 2, ZB = 0;
    static constexpr int AUXB = 2 * Q * 4 + 64 * 4;         // dA, dt, D
    static constexpr int SLOT = XB + SB + ZB + AUXB;
    static constexpr int BT = Q * N * 2;                    // the group's B rows
    static constexpr int CBL = NPAIRS * (QT + 1) * 64 * 8;  // CB^T tiles
    static constexpr int XCHG = NPAIRS * 4 * 64 * 16;       // second-half partials
    static constexpr int FIXED = CBL + XCHG + Q * 4 + 256;
    static constexpr int ring_bytes(int r) { return r * SLOT > SLOT + BT ? r * SLOT : SLOT + BT; }
    static constexpr int R = ring_bytes(3) + FIXED <= LDS_BYTES ? 3 : 2;
    static constexpr int RING = ring_bytes(R);
    // 1 KB direct loads of the load wavefront per head / for the B rows
    static constexpr int XI = XB / 1024, SI = SB / 1024, ZI = ZB / 1024, BI = BT / 1024;
    // per load wavefront: XL + SL tile loads (+ dA / dt or D for wavefronts 0, 1)
    static constexpr int XL = XI / NLOAD, SL = SI / NLOAD, BL = BI / NLOAD;
    static constexpr int WAIT01 = (R - 2) * (XL + SL + 1), WAIT23 = (R - 2) * (XL + SL);
    static_assert(XI % NLOAD == 0 && SI % NLOAD == 0 && BI % NLOAD == 0, "even load split");
    static_assert(NPAIRS * WPP == NWAVES && PPARTS * PTW == 4 && PPARTS >= 1, "wavefront split");
    static_assert(ring_bytes(R) + FIXED <= LDS_BYTES, "LDS budget");
    static_assert(WAIT01 <= 63, "vmcnt range");
};

template <int NS, int QT, bool HASZ>
__global__ void __launch_bounds__(THREADS) k_scan_fused(ScanFusedArgs a) {
    typedef Shape<NS, QT, HASZ> S;
    constexpr int N = S::N, Q = S::Q, NPAIRS = S::NPAIRS, PTW = S::PTW, R = S::R;
    constexpr int XB = S::XB, SB = S::SB, ZB = S::ZB, SLOT = S::SLOT, SCPR = S::SCPR;
    __shared__ __align__(16) char ring[S::RING];
    __shared__ __align__(16) bf16x4 cbl[NPAIRS][QT + 1][64];
    __shared__ __align__(16) f32x4 xchg[NPAIRS][4][64];
    __shared__ int seqs[Q];

    const int L = a.L, H = a.H, G = a.G, nc = a.nc, hpg = a.hpg;
    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int g = work % G;
    const int rest = work / G;
    const int ci = rest % nc, bi = rest / nc;
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
        const int h = g * hpg + j;
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
        for (int uu = 0; uu < S::BL; ++uu) {
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
#pragma unroll
            for (int ns = 0; ns < NS; ++ns) {
                const int r = 16 * kt + ln;
                const bf16x8 bfr = *reinterpret_cast<const bf16x8*>(
                    bt + r * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(r)) * 16));
                acc = mma32(bfr, second ? cfr[1][ns] : cfr[0][ns], acc);
            }
            bf16x4 v4;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int k = 16 * kt + 4 * kg + i;
                float v = acc[i];
                if (k > m || m >= valid) v = 0.f;          // causal, k <= m < valid
                if (a.seq_idx && seqs[m] != seqs[k]) v = 0.f;
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

    if (loader) {
#pragma unroll
        for (int i = 1; i < R - 1; ++i) issue(min(i, hpg - 1), i);
        for (int j = 0; j < hpg; ++j) {
            // head j's loads done (R - 2 later heads may still be in flight)
            if (li < 2) wait_vmem<S::WAIT01>();
            else wait_vmem<S::WAIT23>();
            lds_barrier();                                  // slot j % R complete, slot (j-1) % R free
            issue(min(j + R - 1, hpg - 1), (j + R - 1) % R);
            lds_barrier();                                  // the compute wavefronts' exchange
        }
        wait_vmem<0>();     // the tail heads re-loaded into unused slots
        return;
    }
    // this wavefront's row tiles: the first half (kh == 0) accumulates the
    // long tile t2 over k-tiles [0, KA); the second half t2 over [KA, t2] (a
    // partial, added in through LDS) and the short tile t1 over [0, t1]
    constexpr int KA = S::KA;
    const int tmine = kh ? t1 : t2;                    // the tile this wavefront stores
    for (int j = 0; j < hpg; ++j) {
        const int k = j % R;
        lds_barrier();
        const char* slot = ring + k * SLOT;
        const float* dAs = reinterpret_cast<const float*>(slot + XB + SB + ZB);
        const float* dts = dAs + Q;
        const float* Ds = dAs + 2 * Q;
        const int h = g * hpg + j;
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
        // 1. carried state of the stored tile: y^T = h_c C^T, rounded to bf16,
        // times exp(dA[m])
        {
            f32x4 ci_[PTW];
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) ci_[pt] = zero4();
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const int p = 16 * (PTW * pp + pt) + ln;
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    const bf16x8 sfr = *reinterpret_cast<const bf16x8*>(
                        slot + XB + p * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(p)) * 16));
                    ci_[pt] = mma32(sfr, kh ? cfr[0][ns] : cfr[1][ns], ci_[pt]);
                }
            }
            const float f = __builtin_amdgcn_exp2f(dAs[mrow] * LOG2E) * (kh ? fmask[0] : fmask[1]);
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) ci_[pt][i] = rbf(ci_[pt][i]) * f;
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                if (kh) acc[0][pt] = ci_[pt];
                else acc[1][pt] = ci_[pt];
            }
        }
        // 2. intra chunk: y^T += x^T W^T over this wavefront's (tile, k-tile) units
        const float dAm1 = dAs[16 * t1 + ln] * LOG2E, dAm2 = dAs[16 * t2 + ln] * LOG2E;
        for (int kt = 0; kt <= t2; ++kt) {
            const bool do2 = kh ? kt >= KA : kt < KA;    // tile t2
            const bool do1 = kh && kt <= t1;             // tile t1
            if (!do1 && !do2) continue;
            const int k0 = 16 * kt + 4 * kg;
            bf16x4 xfr[PTW];
            {
                const int r = k0 + (ln >> 2);            // rows k0 .. k0+3 of the group
#pragma unroll
                for (int pt = 0; pt < PTW; ++pt) {
                    const int ch = 2 * (PTW * pp + pt) + ((ln & 3) >> 1);
                    xfr[pt] = ds_read_tr(slot + r * 128 + ((ch ^ xswz(r)) * 16) + 8 * (ln & 1));
                }
            }
            const float4 dk = *reinterpret_cast<const float4*>(dAs + k0);
            const float4 tk = *reinterpret_cast<const float4*>(dts + k0);
            const float dkv[4] = {dk.x * LOG2E, dk.y * LOG2E, dk.z * LOG2E, dk.w * LOG2E};
            const float tkv[4] = {tk.x, tk.y, tk.z, tk.w};
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                if (tt ? !do2 : !do1) continue;
                const bf16x4 cb4 = cbl[pi][tt ? t1 + 1 + kt : kt][lane];
                const float dAm = tt ? dAm2 : dAm1;
                bf16x4 whi, wlo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // decay exp(dA[m]-dA[k]) in the log2 domain; CB is 0 for k > m
                    const float e = __builtin_amdgcn_exp2f(fminf(dAm - dkv[i], 0.f));
                    const float v = (float)cb4[i] * e * tkv[i];
                    const bf16 hv = (bf16)v;
                    whi[i] = hv;
                    wlo[i] = (bf16)(v - (float)hv);
                }
                // one K = 32 MFMA: k index i < 4 pairs x with the hi part,
                // 4 + i the same x with the lo part
                const bf16x8 w8 = __builtin_shufflevector(whi, wlo, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
                for (int pt = 0; pt < PTW; ++pt) {
                    const bf16x8 x8 = __builtin_shufflevector(xfr[pt], xfr[pt], 0, 1, 2, 3, 0, 1, 2, 3);
                    acc[tt][pt] = mma32(x8, w8, acc[tt][pt]);
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
        // 3. epilogue: + D x, silu(z) gate in z's dtype, 16-byte fp32 stores
        if (mrow < valid) {
            float* op = a.out + ((tok0 + mrow) * H + h) * P;
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const int p0 = 16 * (PTW * pp + pt) + 4 * kg;
                const f32x4 r = kh ? acc[0][pt] : acc[1][pt];
                float v[4] = {r[0], r[1], r[2], r[3]};
                if (a.D) {
                    const int xoff = mrow * 128 + (((p0 >> 3) ^ xswz(mrow)) * 16) + 2 * (p0 & 7);
                    const bf16x4 xv = *reinterpret_cast<const bf16x4*>(slot + xoff);
                    float dv[4];
                    if (a.D_has_hdim) {
                        const float4 d4 = *reinterpret_cast<const float4*>(Ds + p0);
                        dv[0] = d4.x; dv[1] = d4.y; dv[2] = d4.z; dv[3] = d4.w;
                    } else {
                        dv[0] = dv[1] = dv[2] = dv[3] = Ds[0];
                    }
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] += dv[i] * (float)xv[i];
                }
                if (HASZ) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] *= rbf(silu_f((float)zr[pt][i]));
                }
                *reinterpret_cast<float4*>(op + p0) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

}  // namespace

namespace m2 {

// True when the fused path covers these sizes (bf16, headdim 64).
bool scan_fused_supported(int64_t headdim, int64_t dstate, int64_t chunk_size) {
    return headdim == 64 && (dstate == 64 || dstate == 128 || dstate == 256) &&
           (chunk_size == 64 || chunk_size == 128);
}

int launch_scan_fused(const m2_ssd_combined_args& a, const float* dA, const float* dto,
                      const void* passed, hipStream_t s) {
    M2_REQUIRE(a.ngroups > 0 && a.nheads % a.ngroups == 0, M2_ERR_INVALID,
               "scan_fused: nheads %% ngroups != 0");
    const int64_t nc = (a.seqlen + a.chunk_size - 1) / a.chunk_size;
    const int64_t nwork = a.batch * nc * a.ngroups;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "scan_fused: too many blocks");
    ScanFusedArgs f{};
    f.x = (const bf16*)a.x; f.B = (const bf16*)a.B; f.C = (const bf16*)a.C;
    f.states = (const bf16*)passed; f.dt = dto; f.dA = dA; f.D = a.D; f.z = (const bf16*)a.z;
    f.seq_idx = a.seq_idx; f.out = a.out; f.D_has_hdim = a.D_has_hdim;
    f.L = (int)a.seqlen; f.H = (int)a.nheads; f.G = (int)a.ngroups; f.nc = (int)nc;
    f.hpg = (int)(a.nheads / a.ngroups); f.nwork = (int)nwork;
    void (*kern)(ScanFusedArgs) = nullptr;
    const bool hz = a.z != nullptr;
#define M2_SF_CASE(NSV, QTV)                                                        \
    if (a.dstate == 32 * NSV && a.chunk_size == 16 * QTV)                           \
        kern = hz ? k_scan_fused<NSV, QTV, true> : k_scan_fused<NSV, QTV, false>;
    M2_SF_CASE(2, 4) M2_SF_CASE(2, 8)
    M2_SF_CASE(4, 4) M2_SF_CASE(4, 8)
    M2_SF_CASE(8, 4) M2_SF_CASE(8, 8)
#undef M2_SF_CASE
    M2_REQUIRE(kern && a.headdim == P, M2_ERR_UNSUPPORTED, "scan_fused: unsupported sizes");
    kern<<<(unsigned)nwork, THREADS, 0, s>>>(f);
    return check_launch("scan_fused");
}

}  // namespace m2
