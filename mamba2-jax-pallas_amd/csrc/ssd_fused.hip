// k_scan_fused: bmm_chunk + chunk_scan of the combined forward for bf16 inputs.
//
//   y[m, :] = exp(dA[m]) * bf16(C[m, :] h_c^T)                     (carried state)
//           + sum_{k <= m} CB[m, k] exp(dA[m] - dA[k]) dt[k] x[k, :] (intra chunk)
//           + D x[m, :],   then y *= silu(z[m, :]) when z is given
// with CB = bf16(C B^T) (seq_idx-masked), h_c the bf16 state entering chunk c.
//
// One workgroup per (batch, chunk, group) covers every head of the group, so
// CB is built once and used by all of them.  8 wavefronts; the chunk's 16-row
// output tiles are paired (t, Q/16-1-t) so that every pair carries the same
// causal (triangular) work, and the head dim is split among the wavefronts of
// a pair: wavefront w owns pair w % NPAIRS and PTW 16-column head-dim tiles.
//
// Per head, the x rows [Q x 64], the carried state [64 x N], dA / dt of the
// chunk, D (and the z rows) are brought into a ring of R LDS slots by direct
// global -> LDS loads (global_load_lds_dwordx4), R - 1 heads ahead of use,
// with explicit vmcnt waits; the group's B rows use the same path once, for
// the CB build.  Rows are dense in LDS with their 16-byte chunks
// XOR-swizzled so that the reads below hit distinct banks.
//
// The products are computed transposed, y^T = h_c C^T + x^T W^T with
// W[m, k] = CB[m, k] exp(dA[m] - dA[k]) dt[k], so that each lane ends with 4
// consecutive head-dim values of one output row (16-byte stores, 8-byte D / z
// reads):
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

constexpr int THREADS = 512;
constexpr int NWAVES = THREADS / 64;
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
    static constexpr int NPAIRS = QT / 2, PSPLIT = NWAVES / NPAIRS, PTW = 4 / PSPLIT;
    static constexpr int SCPR = N / 8;                      // 16-byte chunks per state row
    static constexpr int XB = Q * P * 2, SB = P * N * 2, ZB = HASZ ? Q * P * 2 : 0;
    static constexpr int AUXB = 2 * Q * 4 + 64 * 4;         // dA, dt, D
    static constexpr int SLOT = XB + SB + ZB + AUXB;
    static constexpr int BT = Q * N * 2;                    // the group's B rows
    static constexpr int CBL = NPAIRS * (QT + 1) * 64 * 8;  // CB^T tiles
    static constexpr int FIXED = CBL + Q * 4 + 256;
    static constexpr int ring_bytes(int r) { return r * SLOT > SLOT + BT ? r * SLOT : SLOT + BT; }
    static constexpr int R = ring_bytes(3) + FIXED <= LDS_BYTES ? 3 : 2;
    static constexpr int RING = ring_bytes(R);
    static constexpr int XV = XB / 16 / THREADS, SV = SB / 16 / THREADS;
    static constexpr int ZV = ZB / 16 / THREADS, BV = BT / 16 / THREADS;
    static_assert(NPAIRS * PSPLIT == NWAVES && PTW * PSPLIT == 4, "wavefront split");
    static_assert(XV >= 1 && SV >= 1 && BV >= 1, "tiles too small for the workgroup");
    static_assert(ring_bytes(R) + FIXED <= LDS_BYTES, "LDS budget");
};

template <int NS, int QT, bool HASZ>
__global__ void __launch_bounds__(THREADS) k_scan_fused(ScanFusedArgs a) {
    typedef Shape<NS, QT, HASZ> S;
    constexpr int N = S::N, Q = S::Q, NPAIRS = S::NPAIRS, PTW = S::PTW, R = S::R;
    constexpr int XB = S::XB, SB = S::SB, ZB = S::ZB, SLOT = S::SLOT, SCPR = S::SCPR;
    __shared__ __align__(16) char ring[S::RING];
    __shared__ __align__(16) bf16x4 cbl[NPAIRS][QT + 1][64];
    __shared__ int seqs[Q];

    const int L = a.L, H = a.H, G = a.G, nc = a.nc, hpg = a.hpg;
    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int g = work % G;
    const int rest = work / G;
    const int ci = rest % nc, bi = rest / nc;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int ln = lane & 15, kg = lane >> 4;
    const int pi = w % NPAIRS, ph = w / NPAIRS;
    const int t1 = pi, t2 = QT - 1 - pi;
    const int64_t tok0 = (int64_t)bi * L + (int64_t)ci * Q;
    const int valid = min(Q, L - ci * Q);
    const int64_t rs = (int64_t)G * N;                    // row stride of B / C
    const int seq_prev = (a.seq_idx && ci > 0) ? a.seq_idx[tok0 - 1] : 0;
    const uint32_t ring_lds = lds_addr(ring);

    // ---- plain loads: C fragments of the pair's two row tiles, seq ids -----
    bf16x8 cfr[2][NS];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int row = min(16 * (tt ? t2 : t1) + ln, valid - 1);   // clamped; masked below
        const bf16* cp = a.C + ((tok0 + row) * G + g) * N + kg * 8;
#pragma unroll
        for (int ns = 0; ns < NS; ++ns) cfr[tt][ns] = *reinterpret_cast<const bf16x8*>(cp + ns * 32);
    }
    for (int q = threadIdx.x; q < Q; q += THREADS)
        seqs[q] = (a.seq_idx && q < valid) ? a.seq_idx[tok0 + q] : -1;

    // ---- per-thread direct-load sources (row, swizzled column) -------------
    int64_t xo[S::XV];
#pragma unroll
    for (int u = 0; u < S::XV; ++u) {
        const int gi = u * THREADS + threadIdx.x, r = gi / 8;
        xo[u] = (tok0 + min(r, valid - 1)) * H * P + 8 * ((gi % 8) ^ xswz(r));
    }
    int so[S::SV];
#pragma unroll
    for (int u = 0; u < S::SV; ++u) {
        const int gi = u * THREADS + threadIdx.x, p = gi / SCPR;
        so[u] = p * N + 8 * ((gi % SCPR) ^ sswz<SCPR>(p));
    }
    const int64_t cq0 = ((int64_t)bi * H * nc + ci) * Q;  // dA / dt row of head 0 (+ h nc Q)
    const int64_t st0 = ((int64_t)bi * nc + ci) * H * P * N;
    // head j -> slot k: XV + SV (+ ZV) loads per thread; wavefront 0 adds dA / dt
    // (lanes < Q/2, 16 bytes each), wavefront 1 adds D (64 words)
    auto issue = [&](int j, int k) {
        const int h = g * hpg + j;
        const uint32_t sb = ring_lds + k * SLOT;
#pragma unroll
        for (int u = 0; u < S::XV; ++u)
            dma16(a.x + xo[u] + h * P, sb + (u * THREADS + 64 * w) * 16);
        const bf16* sp = a.states + st0 + (int64_t)h * P * N;
#pragma unroll
        for (int u = 0; u < S::SV; ++u)
            dma16(sp + so[u], sb + XB + (u * THREADS + 64 * w) * 16);
        if (HASZ) {
#pragma unroll
            for (int u = 0; u < S::ZV; ++u)
                dma16(a.z + xo[u] + h * P, sb + XB + SB + (u * THREADS + 64 * w) * 16);
        }
        if (w == 0) {
            const int64_t row = cq0 + (int64_t)h * nc * Q;
            if (lane < Q / 2) {
                const float* src = lane < Q / 4 ? a.dA + row + 4 * lane : a.dt + row + 4 * (lane - Q / 4);
                dma16(src, sb + XB + SB + ZB);
            }
        } else if (w == 1) {
            const float* src = a.D ? (a.D_has_hdim ? a.D + h * P + lane : a.D + h) : a.dA + cq0;
            dma4(src, sb + XB + SB + ZB + 2 * Q * 4);
        }
    };
    constexpr int CNT = S::XV + S::SV + S::ZV;   // loads per head, wavefronts >= 2

    // ---- the group's B rows (aliasing ring slots 1..) and head 0 -----------
    {
        const bf16* Bg = a.B + (tok0 * G + g) * N;
#pragma unroll
        for (int u = 0; u < S::BV; ++u) {
            const int gi = u * THREADS + threadIdx.x, r = gi / SCPR;
            dma16(Bg + min(r, valid - 1) * rs + 8 * ((gi % SCPR) ^ sswz<SCPR>(r)),
                  ring_lds + SLOT + (u * THREADS + 64 * w) * 16);
        }
    }
    issue(0, 0);
    wait_vmem<0>();
    __syncthreads();

    // ---- CB^T tiles of each pair: (t1, kt <= t1) in slots 0..t1, (t2, kt <= t2)
    // in slots t1+1..; the pair's wavefronts share them out
    {
        const char* bt = ring + SLOT;
        for (int j = ph; j < QT + 1; j += NWAVES / NPAIRS) {
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
#pragma unroll
    for (int i = 1; i < R; ++i) issue(min(i, hpg - 1), i);

    // seq masks of the carried-state term (per output row m = 16 t + ln)
    float fmask[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int m = 16 * (tt ? t2 : t1) + ln;
        fmask[tt] = (a.seq_idx && seqs[m] != seq_prev) ? 0.f : 1.f;
    }

    for (int j = 0; j < hpg; ++j) {
        const int k = j % R;
        // own loads of head j done (R - 2 later heads may still be in flight)
        if (w == 0 || w == 1) wait_vmem<(R - 2) * (CNT + 1)>();
        else wait_vmem<(R - 2) * CNT>();
        lds_barrier();                                      // slot k complete, slot k-1 free
        issue(min(j + R - 1, hpg - 1), (j + R - 1) % R);
        const char* slot = ring + k * SLOT;
        const float* dAs = reinterpret_cast<const float*>(slot + XB + SB + ZB);
        const float* dts = dAs + Q;
        const float* Ds = dAs + 2 * Q;
        const int h = g * hpg + j;

        f32x4 acc[2][PTW];
        // 1. carried state: y^T = h_c C^T, rounded to bf16, times exp(dA[m])
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) acc[tt][pt] = zero4();
#pragma unroll
        for (int pt = 0; pt < PTW; ++pt) {
            const int p = 16 * (PTW * ph + pt) + ln;
#pragma unroll
            for (int ns = 0; ns < NS; ++ns) {
                const bf16x8 sfr = *reinterpret_cast<const bf16x8*>(
                    slot + XB + p * (2 * N) + (((4 * ns + kg) ^ sswz<SCPR>(p)) * 16));
                acc[0][pt] = mma32(sfr, cfr[0][ns], acc[0][pt]);
                acc[1][pt] = mma32(sfr, cfr[1][ns], acc[1][pt]);
            }
        }
        float dAm[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int m = 16 * (tt ? t2 : t1) + ln;
            dAm[tt] = dAs[m] * LOG2E;
            const float f = __builtin_amdgcn_exp2f(dAm[tt]) * fmask[tt];
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[tt][pt][i] = rbf(acc[tt][pt][i]) * f;
        }
        // 2. intra chunk: y^T += x^T W^T over k-tiles kt <= t
        for (int kt = 0; kt <= t2; ++kt) {
            const int k0 = 16 * kt + 4 * kg;
            bf16x4 xfr[PTW];
            {
                const int r = k0 + (ln >> 2);                   // rows k0 .. k0+3 of the group
#pragma unroll
                for (int pt = 0; pt < PTW; ++pt) {
                    const int ch = 2 * (PTW * ph + pt) + ((ln & 3) >> 1);
                    xfr[pt] = ds_read_tr(slot + r * 128 + ((ch ^ xswz(r)) * 16) + 8 * (ln & 1));
                }
            }
            const float4 dk = *reinterpret_cast<const float4*>(dAs + k0);
            const float4 tk = *reinterpret_cast<const float4*>(dts + k0);
            const float dkv[4] = {dk.x * LOG2E, dk.y * LOG2E, dk.z * LOG2E, dk.w * LOG2E};
            const float tkv[4] = {tk.x, tk.y, tk.z, tk.w};
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int t = tt ? t2 : t1;
                if (kt > t) continue;
                const int m = 16 * t + ln;
                const bf16x4 cb4 = cbl[pi][tt ? t1 + 1 + kt : kt][lane];
                bf16x4 whi, wlo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    // decay exp(dA[m]-dA[k]) in the log2 domain; k > m is masked
                    const float e = __builtin_amdgcn_exp2f(fminf(dAm[tt] - dkv[i], 0.f));
                    const float v = (k0 + i <= m) ? (float)cb4[i] * e * tkv[i] : 0.f;
                    const bf16 hv = (bf16)v;
                    whi[i] = hv;
                    wlo[i] = (bf16)(v - (float)hv);
                }
#pragma unroll
                for (int pt = 0; pt < PTW; ++pt) {
                    acc[tt][pt] = mma16(xfr[pt], whi, acc[tt][pt]);
                    acc[tt][pt] = mma16(xfr[pt], wlo, acc[tt][pt]);
                }
            }
        }
        // 3. epilogue: + D x, silu(z) gate in z's dtype, 16-byte fp32 stores
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int m = 16 * (tt ? t2 : t1) + ln;
            if (m >= valid) continue;
            float* op = a.out + ((tok0 + m) * H + h) * P;
#pragma unroll
            for (int pt = 0; pt < PTW; ++pt) {
                const int p0 = 16 * (PTW * ph + pt) + 4 * kg;
                const int xoff = m * 128 + (((p0 >> 3) ^ xswz(m)) * 16) + 2 * (p0 & 7);
                float v[4] = {acc[tt][pt][0], acc[tt][pt][1], acc[tt][pt][2], acc[tt][pt][3]};
                if (a.D) {
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
                    const bf16x4 zv = *reinterpret_cast<const bf16x4*>(slot + XB + SB + xoff);
#pragma unroll
                    for (int i = 0; i < 4; ++i) v[i] *= rbf(silu_f((float)zv[i]));
                }
                *reinterpret_cast<float4*>(op + p0) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
    wait_vmem<0>();     // the tail heads re-loaded into unused slots
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
