// k_scan_f32g: chunk_scan for fp32 inputs at chunk 128, head dim 64 and
// dstate 64 / 128, one workgroup per (batch, chunk, group, slice of the
// group's heads).
//
//   y[m, :] = exp(dA[m]) * C[m, :] h_c^T                            (carried state)
//           + sum_{k <= m} CB[m, k] exp(dA[m] - dA[k]) dt[k] x[k, :] (intra chunk)
//           + D x[m, :],   then y *= silu(z[m, :]) when z is given
// with CB = C B^T (seq_idx-masked; the fp32 bmm_chunk output, or built here
// in the combined forward: CBB below) and h_c the fp32 state entering chunk c.
//
// The per-(chunk, head) fp32 kernel (chunk_scan.hip) brings the group's C and
// CB rows into the CU again for every head, ~100 of the ~165 KB it reads per
// head, and waits for each of its loads in the wavefront that uses them.
// Here the group's C and CB rows are loaded once per workgroup, into
// registers, and the heads stream through LDS:
//
// Workgroup = 8 compute wavefronts + 4 load wavefronts.  Per head, x
// [128 x 64] and the state [64 x N] (fp32), dA, dt and D arrive in a ring of
// R LDS slots through direct global -> LDS loads (global_load_lds_dwordx4)
// issued by the load wavefronts R - 1 heads ahead; once a head's loads have
// landed, each load wavefront rewrites the rows it loaded, in place, as bf16
// hi / lo planes (v = hi + lo) and only then joins the barrier that hands the
// head to the compute wavefronts:
//   * x rows (256 bytes): a 128-byte hi and a 128-byte lo plane, their order
//     alternating with the row's parity, 16-byte pieces XOR-swizzled by row,
//     read through ds_read_b64_tr_b16 (8 positions of one head-dim column per
//     lane) with every bank hit once per 16 lanes;
//   * state rows (4 N bytes): a hi and a lo plane of 2 N bytes, 16-byte pieces
//     XOR-swizzled by row (and, at N = 64, the plane order alternating every
//     8 rows), read 16 bytes per lane by 16 consecutive rows, conflict-free.
//
// Compute wavefront w owns row tile t = w (w < 4) or 11 - w: the two
// wavefronts of a SIMD (w, w + 4) hold tiles t and 7 - t, whose causal work
// adds up to the same on every SIMD.  It computes the transposed product
//   y^T [64 p x 16 m] = state [p x n] C^T [n x m] + x^T [p x k] W^T [k x m],
//   W[m, k] = CB[m, k] exp(dA[m] - dA[k]) dt[k]   (k <= m),
// whose B operands (lane = output row m, 8 consecutive n or k) are the lane's
// own C row (split into hi / lo once) and CB row (kept as floats, weighted
// and split per head), and whose accumulators hold 4 consecutive head-dim
// columns of the lane's row: the carried-state factor exp(dA[m]) is one
// scalar per lane and the output leaves as 16-byte stores.  A product of two
// split operands is three 16x16x32 bf16 MFMAs (hi.hi + hi.lo + lo.hi, ~2^-16
// relative); the decay is evaluated per element (never factored through
// exp(dA[m]) exp(-dA[k]), which overflows once |dA| inside a chunk exceeds
// ~88).
//
// Follows reference ops/ssd_naive.py:189-318 (math), kernels/chunk_scan_fwd.py
// :294-322 (seq_idx rule for the carried-state term) and :545-570 (epilogue),
// kernels/bmm_chunk_fwd.py:353-372 (seq_idx mask of CB).
#include <math.h>

#include "m2_internal.h"

namespace {

constexpr int NWAVES = 8;                  // compute wavefronts
constexpr int NLOAD = 4;                   // load wavefronts
constexpr int THREADS = (NWAVES + NLOAD) * 64;
constexpr int P = 64;                      // head dim
constexpr int Q = 128;                     // chunk
constexpr int XROW = P * 4;                // bytes of an fp32 x row
constexpr float LOG2E = 1.4426950408889634f;
constexpr int LDS_BYTES = 160 * 1024;

template <int NS>
struct GCfg {
    static constexpr int N = 32 * NS;
    static constexpr int SROW = N * 4;                 // bytes of an fp32 state row
    static constexpr int CPP = N / 8;                  // 16-byte pieces per plane row
    static constexpr int PB = N * 2;                   // plane bytes per row
    static constexpr int XB = Q * XROW, SB = P * SROW;
    static constexpr int AUXB = 2 * Q * 4 + P * 4;     // dA, dt, D
    static constexpr int SLOT = XB + SB + AUXB;
    static constexpr int R = 3 * SLOT <= LDS_BYTES ? 3 : 2;
    // 1 KB direct loads per head and load wavefront: x, state
    static constexpr int XI = XB / 1024 / NLOAD, SI = SB / 1024 / NLOAD;
    static constexpr int SRPI = 1024 / SROW;           // state rows per direct load
    static constexpr int SPR = SROW / 16;              // 16-byte pieces per fp32 state row
    static constexpr int BI = Q * SROW / 1024 / NLOAD; // CBB: direct loads of B rows per load wavefront
    // loads of one load wavefront that may still be in flight when head i
    // must have landed: those of the R - 2 later heads (+ one aux load for the
    // wavefronts that bring dA, dt or D)
    static constexpr int WAITA = (R - 2) * (XI + SI + 1), WAITB = (R - 2) * (XI + SI);
    static_assert(XB % (1024 * NLOAD) == 0 && SB % (1024 * NLOAD) == 0, "even load split");
    static_assert(XI * 4 * NLOAD == Q && SI * SRPI * NLOAD == P, "rows per load wavefront");
    static_assert(WAITA <= 63, "vmcnt range");
    static_assert(R * SLOT <= LDS_BYTES, "LDS budget");
    static_assert(Q * SROW <= XB + SB && BI * SRPI * NLOAD == Q, "B rows fit a slot");
};

// x plane piece layout: byte offset in row r of the 4 bf16 of columns
// 4 ch .. 4 ch + 3 in plane pl (0 hi, 1 lo)
M2_DEV int xswz(int r) { return ((r >> 1) & 3) << 1; }
M2_DEV int xoff(int r, int pl, int ch) {
    return ((pl ^ (r & 1)) << 7) + ((((ch >> 1) ^ xswz(r))) << 4) + ((ch & 1) << 3);
}
// state plane piece layout: byte offset in row p of the 16-byte piece cc
// (columns 8 cc .. 8 cc + 7) of plane pl
template <int NS> M2_DEV int soff(int p, int pl, int cc) {
    typedef GCfg<NS> Cf;
    return ((pl ^ ((p / Cf::CPP) & 1)) * Cf::PB) + ((cc ^ (p % Cf::CPP)) << 4);
}

M2_DEV f32x4 mma3(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
}
M2_DEV void split8(const float* v, bf16x8& hi, bf16x8& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) split2(v[2 * i], v[2 * i + 1], h[i], l[i]);
    hi = as_bf16x8(h[0], h[1], h[2], h[3]);
    lo = as_bf16x8(l[0], l[1], l[2], l[3]);
}
M2_DEV float ex2(float v) { return __builtin_amdgcn_exp2f(v); }

struct GArgs {
    const float* x;
    const float* C;
    const float* B;         // [b, L, G, N] (CBB: CB built here)
    const float* cb;        // [b, nc, G, Q, Q] (given CB)
    const float* states;    // [b, nc, H, P, N]
    const float* dt;        // [b, H, nc, Q]
    const float* dA;        // [b, H, nc, Q]
    const float* D;
    const float* z;
    const int32_t* seq_idx;
    float* out;
    float* out_x;
    int D_has_hdim;
    int L, H, G, nc, hpg, hps, nslice, nwork;
};

template <bool NT> M2_DEV void store_f4(const f32x4& v, float* p) {
    if constexpr (NT) __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(p));
    else *reinterpret_cast<f32x4*>(p) = v;
}

// CBB: CB = C B^T (seq_idx-masked) is built here from the group's B rows,
// which pass through the second ring slot (as hi / lo planes laid out like
// the state rows) before the second head is loaded: the layer then needs no
// bmm_chunk launch and no CB buffer.  NT: non-temporal output stores; without
// them, x and the state rows are loaded non-temporally.
template <int NS, bool HASZ, bool CBB, bool NT>
__global__ void __launch_bounds__(THREADS) k_scan_f32g(GArgs a) {
    typedef GCfg<NS> Cf;
    constexpr int N = Cf::N, SROW = Cf::SROW, XB = Cf::XB, SB = Cf::SB, SLOT = Cf::SLOT;
    constexpr int R = Cf::R, XI = Cf::XI, SI = Cf::SI;
    __shared__ __align__(16) char ring[R * SLOT];

    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int sl = work % a.nslice;
    int rest = work / a.nslice;
    const int g = rest % a.G;
    rest /= a.G;
    const int c = rest % a.nc, bi = rest / a.nc;
    const int h0 = g * a.hpg + sl * a.hps;
    const int nh = min(a.hps, a.hpg - sl * a.hps);
    const int L = a.L, H = a.H, nc = a.nc;
    const int valid = min(Q, L - c * Q);
    const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;

    if (w >= NWAVES) {
        // ---- load wavefront li: x rows 32 li .. 32 li + 31 and state rows
        // 16 li .. 16 li + 15 of every head (direct load u brings x rows
        // 4 u .. 4 u + 3 / state rows SRPI u ..: lane l's 16 bytes land at
        // 16 l, so both tiles sit row-major as loaded); wavefronts 0 / 1 / 2
        // also bring dA / dt / D
        const int li = w - NWAVES;
        const uint32_t ring_lds = lds_addr(ring);
        const bool hasD = a.D != nullptr;
        auto issue = [&](int i, int k) {
            const int h = h0 + i;
            const uint32_t sb = ring_lds + k * SLOT;
            const float* xsrc = a.x + (tok0 * H + h) * P;
#pragma unroll
            for (int uu = 0; uu < XI; ++uu) {
                const int u = li * XI + uu;
                const int r = min(4 * u + (lane >> 4), valid - 1);   // past the end: weight 0
                if constexpr (!NT) dma16nt(xsrc + (int64_t)r * H * P + 4 * (lane & 15), sb + 1024 * u);
                else dma16(xsrc + (int64_t)r * H * P + 4 * (lane & 15), sb + 1024 * u);
            }
            const float* ssrc = a.states + (((int64_t)bi * nc + c) * H + h) * (int64_t)P * N;
#pragma unroll
            for (int uu = 0; uu < SI; ++uu) {
                const int u = li * SI + uu;
                if constexpr (!NT) dma16nt(ssrc + (int64_t)(Cf::SRPI * u) * N + 4 * lane, sb + XB + 1024 * u);
                else dma16(ssrc + (int64_t)(Cf::SRPI * u) * N + 4 * lane, sb + XB + 1024 * u);
            }
            const int64_t q0 = (((int64_t)bi * H + h) * nc + c) * Q;
            const uint32_t ab = sb + XB + SB;
            if (li == 0 && lane < 32) dma16(a.dA + q0 + 4 * lane, ab);
            if (li == 1 && lane < 32) dma16(a.dt + q0 + 4 * lane, ab + Q * 4);
            if (li == 2 && hasD) {
                if (a.D_has_hdim) {
                    if (lane < 16) dma16(a.D + (int64_t)h * P + 4 * lane, ab + 2 * Q * 4);
                } else if (lane == 0) {
                    dma4(a.D + h, ab + 2 * Q * 4);
                }
            }
        };
        // this wavefront's rows of slot k as bf16 hi / lo planes, in place; no
        // other wavefront touches these rows before the barrier that follows
        auto split = [&](int k) {
            char* const sbase = ring + k * SLOT;
            float4 xv[XI], sv[SI];
#pragma unroll
            for (int uu = 0; uu < XI; ++uu)
                xv[uu] = *reinterpret_cast<const float4*>(sbase + 1024 * (li * XI + uu) + 16 * lane);
#pragma unroll
            for (int uu = 0; uu < SI; ++uu)
                sv[uu] = *reinterpret_cast<const float4*>(sbase + XB + 1024 * (li * SI + uu) + 16 * lane);
            // the rows other lanes read are written below: every read has
            // returned (and the compiler keeps them all above) before the
            // first write
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
#pragma unroll
            for (int uu = 0; uu < XI; ++uu) {
                const int r = 4 * (li * XI + uu) + (lane >> 4), ch = lane & 15;
                uint32_t h0_, l0_, h1_, l1_;
                split2(xv[uu].x, xv[uu].y, h0_, l0_);
                split2(xv[uu].z, xv[uu].w, h1_, l1_);
                *reinterpret_cast<u2*>(sbase + r * XROW + xoff(r, 0, ch)) = u2{h0_, h1_};
                *reinterpret_cast<u2*>(sbase + r * XROW + xoff(r, 1, ch)) = u2{l0_, l1_};
            }
#pragma unroll
            for (int uu = 0; uu < SI; ++uu) {
                const int r = Cf::SRPI * (li * SI + uu) + lane / Cf::SPR, fc = lane % Cf::SPR;
                uint32_t h0_, l0_, h1_, l1_;
                split2(sv[uu].x, sv[uu].y, h0_, l0_);
                split2(sv[uu].z, sv[uu].w, h1_, l1_);
                char* const rp = sbase + XB + r * SROW + ((fc & 1) << 3);
                *reinterpret_cast<u2*>(rp + soff<NS>(r, 0, fc >> 1)) = u2{h0_, h1_};
                *reinterpret_cast<u2*>(rp + soff<NS>(r, 1, fc >> 1)) = u2{l0_, l1_};
            }
        };
        const bool aux = li < 2 || (li == 2 && hasD);
        if constexpr (CBB) {
            // the group's B rows 32 li .. 32 li + 31 (clamped like x) into the
            // second slot beside head 0, both split, then two barriers: B
            // ready, B consumed (the compute wavefronts' CB tiles are built)
            issue(0, 0);
            char* const bb = ring + SLOT;
            const float* bsrc = a.B + (tok0 * a.G + g) * N;
#pragma unroll
            for (int uu = 0; uu < Cf::BI; ++uu) {
                const int u = li * Cf::BI + uu;
                const int r = min(Cf::SRPI * u + lane / Cf::SPR, valid - 1);
                dma16(bsrc + (int64_t)r * a.G * N + 4 * (lane % Cf::SPR), ring_lds + SLOT + 1024 * u);
            }
            wait_vmem<0>();
            split(0);
            {
                float4 bv[Cf::BI];
#pragma unroll
                for (int uu = 0; uu < Cf::BI; ++uu)
                    bv[uu] = *reinterpret_cast<const float4*>(bb + 1024 * (li * Cf::BI + uu) + 16 * lane);
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
#pragma unroll
                for (int uu = 0; uu < Cf::BI; ++uu) {
                    const int r = Cf::SRPI * (li * Cf::BI + uu) + lane / Cf::SPR, fc = lane % Cf::SPR;
                    uint32_t h0_, l0_, h1_, l1_;
                    split2(bv[uu].x, bv[uu].y, h0_, l0_);
                    split2(bv[uu].z, bv[uu].w, h1_, l1_);
                    char* const rp = bb + r * SROW + ((fc & 1) << 3);
                    *reinterpret_cast<u2*>(rp + soff<NS>(r, 0, fc >> 1)) = u2{h0_, h1_};
                    *reinterpret_cast<u2*>(rp + soff<NS>(r, 1, fc >> 1)) = u2{l0_, l1_};
                }
            }
            lds_barrier();                // B planes and head 0 ready
            lds_barrier();                // B consumed: slots 1 .. R - 1 free
#pragma unroll
            for (int i = 1; i < R; ++i)
                if (R > 2 || i < nh) issue(min(i, nh - 1), i);
        } else {
#pragma unroll
            for (int i = 0; i < R - 1; ++i) issue(min(i, nh - 1), i);
        }
        for (int i = 0; i < nh; ++i) {
            if (!CBB || i > 0) {
                // head i complete (later heads may be in flight)
                if (aux) wait_vmem<Cf::WAITA>();
                else wait_vmem<Cf::WAITB>();
                split(i % R);
            }
            lds_barrier();                // slot i % R ready, slot (i - 1) % R free
            // past the last head the last one is loaded again into the free
            // slot (never read), so that every wait above counts the same
            // loads; with two slots every wait is for all loads (CBB: heads
            // 1 .. R - 1 went out after the B barriers)
            if ((!CBB || i > 0) && (R > 2 || i + 1 < nh))
                issue(min(i + R - 1, nh - 1), (i + R - 1) % R);
        }
        wait_vmem<0>();                   // nothing may land after the workgroup ends
        return;
    }

    // ---- compute wavefronts
    const int t = w < 4 ? w : 11 - w;     // row tile
    const int m = 16 * t + ln;            // the lane's output row
    const int mc = min(m, valid - 1);
    const int nks = t / 2 + 1;            // K steps of 32 positions up to the diagonal
    bool keep = true;                     // carried-state term of row m (seq_idx rule)
    if (a.seq_idx) {
        const int sp = c > 0 ? a.seq_idx[tok0 - 1] : 0;
        keep = a.seq_idx[tok0 + mc] == sp;
    }
    // C^T operand: C[m, 32 ks + 8 kg .. + 7] as hi / lo
    bf16x8 ch[NS], cl[NS];
    {
        const float* crow = a.C + ((tok0 + mc) * a.G + g) * N + 8 * kg;
        float4 cv[NS][2];
#pragma unroll
        for (int ks = 0; ks < NS; ++ks) {
            cv[ks][0] = *reinterpret_cast<const float4*>(crow + 32 * ks);
            cv[ks][1] = *reinterpret_cast<const float4*>(crow + 32 * ks + 4);
        }
#pragma unroll
        for (int ks = 0; ks < NS; ++ks) {
            const float v[8] = {cv[ks][0].x, cv[ks][0].y, cv[ks][0].z, cv[ks][0].w,
                                cv[ks][1].x, cv[ks][1].y, cv[ks][1].z, cv[ks][1].w};
            split8(v, ch[ks], cl[ks]);
        }
    }
    // W^T operand: CB[m, k] at MFMA k index j of K step ks, k = 32 ks + 4 kg +
    // (j & 3) + 16 (j >> 2) (the positions the transposed x reads give this
    // lane group)
    float cbv[4][8];
    if constexpr (CBB) {
        // CB^T tiles [16 k x 16 m] = B[k, :] C[m, :]^T: A operand B rows from
        // the planes in slot 1, B operand the C fragments above; the
        // accumulator (lane = m, 4 consecutive k of a 16-row k tile) is the
        // W^T layout: k tile 2 ks gives j < 4, k tile 2 ks + 1 gives j >= 4.
        // seq_idx: CB[m, k] = 0 where the sequences of m and k differ.
        int sq[4][8];
        if (a.seq_idx) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int k = 32 * ks + 4 * kg + (j & 3) + 16 * (j >> 2);
                    sq[ks][j] = ks < nks ? a.seq_idx[tok0 + min(k, valid - 1)] : 0;
                }
        }
        const int sm = a.seq_idx ? a.seq_idx[tok0 + mc] : 0;
        lds_barrier();                    // B planes ready
        const char* const bb = ring + SLOT;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            f32x4 t0 = zero4(), t1 = zero4();
            if (ks < nks) {
#pragma unroll
                for (int ns = 0; ns < NS; ++ns) {
                    const int r0 = 32 * ks + ln, r1 = r0 + 16;
                    const char* const p0 = bb + r0 * SROW;
                    const char* const p1 = bb + r1 * SROW;
                    t0 = mma3(*reinterpret_cast<const bf16x8*>(p0 + soff<NS>(r0, 0, 4 * ns + kg)),
                              *reinterpret_cast<const bf16x8*>(p0 + soff<NS>(r0, 1, 4 * ns + kg)),
                              ch[ns], cl[ns], t0);
                    t1 = mma3(*reinterpret_cast<const bf16x8*>(p1 + soff<NS>(r1, 0, 4 * ns + kg)),
                              *reinterpret_cast<const bf16x8*>(p1 + soff<NS>(r1, 1, 4 * ns + kg)),
                              ch[ns], cl[ns], t1);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                cbv[ks][j] = t0[j];
                cbv[ks][4 + j] = t1[j];
            }
            if (a.seq_idx)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (sq[ks][j] != sm) cbv[ks][j] = 0.f;
        }
        lds_barrier();                    // B consumed
    } else {
        const float* cbrow = a.cb + (((int64_t)bi * nc + c) * a.G + g) * (int64_t)Q * Q + (int64_t)m * Q;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo;
            if (ks < nks) {
                lo = *reinterpret_cast<const float4*>(cbrow + 32 * ks + 4 * kg);
                hi = *reinterpret_cast<const float4*>(cbrow + 32 * ks + 16 + 4 * kg);
            }
            cbv[ks][0] = lo.x; cbv[ks][1] = lo.y; cbv[ks][2] = lo.z; cbv[ks][3] = lo.w;
            cbv[ks][4] = hi.x; cbv[ks][5] = hi.y; cbv[ks][6] = hi.z; cbv[ks][7] = hi.w;
        }
    }
    // transposed x reads of K step ks, head-dim tile pt: rows 32 ks + 4 kg +
    // (ln >> 2) (+ 16), columns 16 pt + 4 (ln & 3) .. + 3
    const int rA = 4 * kg + (ln >> 2);
    int xo_h[4], xo_l[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
        xo_h[pt] = rA * XROW + xoff(rA, 0, 4 * pt + (ln & 3));
        xo_l[pt] = rA * XROW + xoff(rA, 1, 4 * pt + (ln & 3));
    }
    const bool hasD = a.D != nullptr;

    for (int i = 0; i < nh; ++i) {
        const int h = h0 + i;
        lds_barrier();                    // head i's slot landed and split
        const char* const slot = ring + (i % R) * SLOT;
        const char* const ss = slot + XB;
        const float* const dAs = reinterpret_cast<const float*>(slot + XB + SB);
        const float* const dts = dAs + Q;
        const float* const Ds = dts + Q;

        // 1. carried state: y^T = state C^T, scaled by exp(dA[m])
        f32x4 acc[4];
#pragma unroll
        for (int pt = 0; pt < 4; ++pt) acc[pt] = zero4();
#pragma unroll
        for (int ks = 0; ks < NS; ++ks) {
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const int p = 16 * pt + ln;
                const char* const sr = ss + p * SROW;
                const bf16x8 sh = *reinterpret_cast<const bf16x8*>(sr + soff<NS>(p, 0, 4 * ks + kg));
                const bf16x8 sl_ = *reinterpret_cast<const bf16x8*>(sr + soff<NS>(p, 1, 4 * ks + kg));
                acc[pt] = mma3(sh, sl_, ch[ks], cl[ks], acc[pt]);
            }
        }
        const float dAm = dAs[m];
        const float f = keep ? ex2(dAm * LOG2E) : 0.f;
#pragma unroll
        for (int pt = 0; pt < 4; ++pt)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[pt][r] *= f;

        // 2. intra chunk: y^T += x^T W^T over the K steps up to the diagonal
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks >= nks) break;
            __builtin_amdgcn_sched_barrier(0);           // one K step's operands live at a time
            const float4 a0 = *reinterpret_cast<const float4*>(dAs + 32 * ks + 4 * kg);
            const float4 a1 = *reinterpret_cast<const float4*>(dAs + 32 * ks + 16 + 4 * kg);
            const float4 d0 = *reinterpret_cast<const float4*>(dts + 32 * ks + 4 * kg);
            const float4 d1 = *reinterpret_cast<const float4*>(dts + 32 * ks + 16 + 4 * kg);
            const float dAk[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const float dtk[8] = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int k = 32 * ks + 4 * kg + (j & 3) + 16 * (j >> 2);
                v[j] = k <= m ? cbv[ks][j] * ex2((dAm - dAk[j]) * LOG2E) * dtk[j] : 0.f;
            }
            bf16x8 wh, wl;
            split8(v, wh, wl);
            const char* const xs = slot + ks * 32 * XROW;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const char* const ph = xs + xo_h[pt];
                const char* const pl = xs + xo_l[pt];
                const bf16x8 xh = __builtin_shufflevector(ds_read_tr(ph), ds_read_tr(ph + 16 * XROW), 0, 1, 2, 3, 4, 5, 6, 7);
                const bf16x8 xl = __builtin_shufflevector(ds_read_tr(pl), ds_read_tr(pl + 16 * XROW), 0, 1, 2, 3, 4, 5, 6, 7);
                acc[pt] = mma3(xh, xl, wh, wl, acc[pt]);
            }
        }

        // 3. epilogue: + D x, out_x, z gate, 16-byte stores of row m
        if (m < valid) {
            const int64_t orow = ((tok0 + m) * H + h) * (int64_t)P;
#pragma unroll
            for (int pt = 0; pt < 4; ++pt) {
                const int p0 = 16 * pt + 4 * kg;
                f32x4 v = acc[pt];
                if (hasD) {
                    typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
                    const u2 hv = *reinterpret_cast<const u2*>(slot + m * XROW + xoff(m, 0, 4 * pt + kg));
                    const u2 lv = *reinterpret_cast<const u2*>(slot + m * XROW + xoff(m, 1, 4 * pt + kg));
                    const float xv[4] = {bf16_lo(hv[0]) + bf16_lo(lv[0]), bf16_hi(hv[0]) + bf16_hi(lv[0]),
                                         bf16_lo(hv[1]) + bf16_lo(lv[1]), bf16_hi(hv[1]) + bf16_hi(lv[1])};
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] += (a.D_has_hdim ? Ds[p0 + r] : Ds[0]) * xv[r];
                }
                float* const op = a.out + orow + p0;
                if (a.out_x) store_f4<NT>(v, a.out_x + orow + p0);
                if (HASZ) {
                    const float4 zv = *reinterpret_cast<const float4*>(a.z + orow + p0);
                    v[0] *= silu_f(zv.x); v[1] *= silu_f(zv.y); v[2] *= silu_f(zv.z); v[3] *= silu_f(zv.w);
                }
                store_f4<NT>(v, op);
            }
        }
    }
}

}  // namespace

namespace m2 {

static bool shape_ok(int64_t headdim, int64_t chunk, int64_t dstate, int64_t H, int64_t G) {
    return headdim == P && chunk == Q && (dstate == 64 || dstate == 128) && G > 0 && H % G == 0 &&
           dispatch_override(M2_KNOB_F32_SCAN) != 1;
}

bool scan_f32g_supported(const m2_chunk_scan_args& a) {
    return a.dtype == M2_F32 && a.states_dtype == M2_F32 && a.cb_dtype == M2_F32 &&
           shape_ok(a.headdim, a.chunk_size, a.dstate, a.nheads, a.ngroups);
}

bool scan_f32g_layer_supported(const m2_ssd_combined_args& a) {
    return a.dtype == M2_F32 && shape_ok(a.headdim, a.chunk_size, a.dstate, a.nheads, a.ngroups);
}

// Heads per workgroup: one workgroup per CU (the ring takes 130-148 KB of
// LDS), so a launch takes ceil(workgroups / CUs) rounds, each as long as a
// workgroup's C and CB (or B) rows plus its heads' x and state tiles take to
// arrive (the bytes a CU pulls in: C and the causal half of CB, or B, against
// x + state per head).  The smallest cost over slices of at most 8 heads
// wins: measured at the nemotron-h-8b shape (16 heads per group, CB given),
// two rounds of 8-head slices take 91 us against 95 for one round of whole
// groups (every workgroup of a single round starts and stops its loads in
// step with the others) and 103.5 for four rounds of 4; at mamba2-130m (24
// heads, 16 chunks) slices of 1 / 2 / 3 / 4 heads take 21.5 / 16.6 / 19.7 /
// 23.2 us, as the cost predicts.  The M2_KNOB_F32_SCAN override (tests)
// forces value - 1 heads per workgroup.
int scan_f32g_heads_per_wg(int64_t batch, int64_t nc, int64_t G, int64_t hpg, int64_t N, bool cbb) {
    const int forced = dispatch_override(M2_KNOB_F32_SCAN);
    if (forced >= 2) return (int)(forced - 1 < hpg ? forced - 1 : hpg);
    const double cbytes = cbb ? (double)(Q * N * 4) : (double)(Q * Q * 4 * 9 / 16);
    const double pro = ((double)(Q * N * 4) + cbytes) / (double)(Q * P * 4 + P * N * 4);
    const int64_t cus = cu_count();
    double best = 1e300;
    int hps = 1;
    for (int64_t s = 1; s <= (hpg < 8 ? hpg : 8); ++s) {
        const int64_t nslice = (hpg + s - 1) / s;
        if (s > 1 && (hpg + s - 2) / (s - 1) == nslice) continue;   // same slices as s - 1
        const int64_t nwg = batch * nc * G * nslice;
        const double cost = (double)((nwg + cus - 1) / cus) * (pro + (double)s);
        if (cost < best) { best = cost; hps = (int)s; }
    }
    return hps;
}

static int launch_common(GArgs& k, int64_t batch, int64_t dstate, bool cbb, hipStream_t s) {
    // The output is written once and not read again here.  Where the rows the
    // scan reads (x and the states entering each chunk) fit the 256 MiB
    // Infinity Cache with room for the rest (at most 7/8 of it), non-temporal
    // output stores keep them there and leave no dirty output lines for the
    // end of the kernel (A/B on one box, mamba2-130m shape at batch 1 / 2 / 4 /
    // 8, rows 24-192 MiB: layer 36.7 -> 35.3, 52.7 -> 50.6, 84.9 -> 84.5,
    // 157.8 -> 152.1 us); where they do not (the nemotron-h-8b shape in fp32:
    // rows of 256 MiB), ordinary ones measure better (0.1886 against 0.1924 ms).
    // The non-temporal 64-byte row pieces reach HBM unmerged (c0: 18.6 instead
    // of 12.6 MB written); staging the tiles in LDS so that whole lines leave
    // measured slower (c0 scan 16.3 -> 16.8 us, batch 8: 76.7 -> 79.5 us).
    // Where the rows do not fit, the kernel instead loads x and the states
    // non-temporally (read once here): nemotron-h-8b shape in fp32 0.1920 ->
    // 0.1886 ms (A/B on one box).
    const double rows = (double)batch * k.L * k.H * P * 4 + (double)batch * k.nc * k.H * P * dstate * 4;
    const bool nt = rows <= 224.0 * (1 << 20);
    k.hps = scan_f32g_heads_per_wg(batch, k.nc, k.G, k.hpg, dstate, cbb);
    k.nslice = (k.hpg + k.hps - 1) / k.hps;
    const int64_t nwork = batch * k.nc * k.G * k.nslice;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_scan: too many workgroups");
    k.nwork = (int)nwork;
    void (*kern)(GArgs) = nullptr;
    const bool z = k.z != nullptr;
#define M2_F32G(NSV, NTV) \
    kern = cbb ? (z ? k_scan_f32g<NSV, true, true, NTV> : k_scan_f32g<NSV, false, true, NTV>) \
               : (z ? k_scan_f32g<NSV, true, false, NTV> : k_scan_f32g<NSV, false, false, NTV>);
    if (dstate == 64) {
        if (nt) { M2_F32G(2, true) } else { M2_F32G(2, false) }
    } else {
        if (nt) { M2_F32G(4, true) } else { M2_F32G(4, false) }
    }
#undef M2_F32G
    kern<<<(unsigned)k.nwork, THREADS, 0, s>>>(k);
    return check_launch("chunk_scan (fp32 group kernel)");
}

int launch_scan_f32g(const m2_chunk_scan_args& a, hipStream_t s) {
    M2_REQUIRE(scan_f32g_supported(a), M2_ERR_UNSUPPORTED,
               "chunk_scan: unsupported shape / dtype for the fp32 group kernel");
    GArgs k{};
    k.x = (const float*)a.x; k.C = (const float*)a.C; k.cb = (const float*)a.cb;
    k.states = (const float*)a.states; k.dt = a.dt; k.dA = a.dA_cumsum; k.D = a.D;
    k.z = (const float*)a.z; k.seq_idx = a.seq_idx; k.out = a.out; k.out_x = a.out_x;
    k.D_has_hdim = a.D_has_hdim;
    k.L = (int)a.seqlen; k.H = (int)a.nheads; k.G = (int)a.ngroups;
    k.nc = (int)((a.seqlen + Q - 1) / Q);
    k.hpg = (int)(a.nheads / a.ngroups);
    return launch_common(k, a.batch, a.dstate, false, s);
}

int launch_scan_f32g_layer(const m2_ssd_combined_args& a, const float* dA, const float* dt_out,
                           const void* states_passed, hipStream_t s) {
    M2_REQUIRE(scan_f32g_layer_supported(a), M2_ERR_UNSUPPORTED,
               "ssd_combined: unsupported shape / dtype for the fp32 group scan");
    GArgs k{};
    k.x = (const float*)a.x; k.C = (const float*)a.C; k.B = (const float*)a.B;
    k.states = (const float*)states_passed; k.dt = dt_out; k.dA = dA; k.D = a.D;
    k.z = (const float*)a.z; k.seq_idx = a.seq_idx; k.out = a.out;
    k.D_has_hdim = a.D_has_hdim;
    k.L = (int)a.seqlen; k.H = (int)a.nheads; k.G = (int)a.ngroups;
    k.nc = (int)((a.seqlen + Q - 1) / Q);
    k.hpg = (int)(a.nheads / a.ngroups);
    return launch_common(k, a.batch, a.dstate, true, s);
}

}  // namespace m2
