// ssd_states_f32: chunk_state + state_passing of the combined forward in one
// pass, for fp32 inputs.
//
//   S_c = sum_q w[q] x[q, :]^T B[q, :]                              (chunk_state)
//   h_0 = initial state (or 0),  passed[c] = h_c,
//   h_{c+1} = scl[c] h_c + S_c                                     (state_passing)
//
// with the weights w[q] = exp(min(dA[last] - dA[q], 0)) dt'[q] and the decay
// scl[c] = exp(dA[Q-1]) (seq_idx rules applied) precomputed by chunk_cumsum.
// The staged fp32 kernels write the fp32 chunk states S_c to HBM, read them
// back, and write the passed states: here one workgroup walks the chunks of a
// (batch, head, 64-column dstate block) in order with the running state in
// MFMA accumulators, and HBM sees only x, B, w, the fp32 states entering each
// chunk and the final states.
//
// Workgroup = 8 compute wavefronts + 4 load wavefronts, as the bf16 pass
// (ssd_states.hip), with stages of 64 positions through a ring of 3 LDS
// slots.  Each slot holds the stage's fp32 x rows [64 x 64] and B rows
// [64 x 64] (256-byte rows), the weights and the chunk's decay.  The load
// wavefronts fill it with direct global -> LDS loads two stages ahead; once a
// stage's loads have landed, each load wavefront rewrites the B rows it
// loaded itself in place as bf16 hi / lo planes, and only then joins the
// barrier that hands the stage to the compute wavefronts.  A 256-byte B row
// becomes a 128-byte hi plane and a 128-byte lo plane, whose order alternates
// with the row's parity, with the 16-byte pieces of each plane XOR-swizzled
// by row, so that the transposed reads below hit every bank once per half
// wavefront.  The x rows stay fp32 (16-byte chunks XOR-swizzled by row).
//
// Compute wavefront w owns head-dim rows 16 (w & 3) .. +15, all 64 columns
// and the position half 32 (w >> 2) .. +31 of every stage; the halves meet at
// chunk starts through an exchange buffer (one barrier per stage).  The
// product is computed transposed, h^T[n, p] += B^T[n, q] (w x)[q, p]: the B
// operand from ds_read_b64_tr_b16 on the planes, the x operand read per lane
// (8 positions of one column), weighted and split into hi / lo in registers
// (as the bf16 pass does), and three MFMAs per tile (B_hi (wx)_hi +
// B_hi (wx)_lo + B_lo (wx)_hi: ~2^-16 relative per product).  The fp32 state
// entering each chunk is staged in LDS by the compute wavefronts and stored
// by the load wavefronts as whole 256-byte rows (chunks of 64: stored by the
// compute wavefronts, 4 consecutive columns per lane).
//
// Measured at the BASELINE c2 shape with fp32 inputs: with both operands split
// by the load wavefronts and the states stored 4 columns per lane by the
// compute wavefronts the pass took 92 us, of which timing-only builds that
// drop one part put ~19 us on the split and ~13 us on those stores; this form
// takes 79 us.
//
// Follows reference kernels/chunk_state_fwd.py:104-187 (product),
// kernels/state_passing_fwd.py:108-151 (recurrence) and ops/ssd_naive.py:77-182.
#include <stdlib.h>
#include <string.h>

#include "m2_internal.h"

namespace {

constexpr int NWAVES = 8;                  // compute wavefronts
constexpr int NLOAD = 4;                   // load wavefronts
constexpr int THREADS = (NWAVES + NLOAD) * 64;
constexpr int P = 64;                      // head dim
constexpr int NB = 64;                     // dstate columns per workgroup
constexpr int KB = 64;                     // positions per stage
constexpr int ROW = 256;                   // bytes of a 64-element fp32 row
constexpr int XB = KB * ROW, BB = KB * ROW;
constexpr int AUXB = KB * 4 + 256;         // weights, 64 copies of the decay
constexpr int SLOT = XB + BB + AUXB;
constexpr int TL = KB * ROW / 1024 / NLOAD;   // 1 KB direct loads per tile, stage and load wavefront
static_assert(TL == 4, "each load wavefront owns 16 rows of each tile");

// 16-byte piece swizzle of a plane row: 8 consecutive rows read at one piece
// pair land on disjoint banks (together with the plane order by parity)
M2_DEV int swz(int r) { return ((r >> 1) & 3) << 1; }
// byte offset in row r of the 4 bf16 of fp32 chunk ch (columns 4 ch .. 4 ch + 3)
// in plane pl (0 hi, 1 lo)
M2_DEV int plane_off(int r, int pl, int ch) {
    return ((pl ^ (r & 1)) << 7) + ((((ch >> 1) ^ swz(r))) << 4) + ((ch & 1) << 3);
}

struct StatesF32Args {
    const float* x;
    const float* B;
    const float* wts;      // [b, H, nc, Q]
    const float* scl;      // [b, H, nc]
    const float* init;
    float* passed;         // [b, nc, H, P, N]
    float* fin;
    int L, H, G, N, Q, nc, nblk, nwork;
    int ntx;               // x rows loaded non-temporally
};

// 16-byte chunk swizzle of an fp32 x row: chunk c of row r sits at c ^ xsw(r),
// so that the per-lane reads of four rows 4 apart hit disjoint banks
M2_DEV int xsw(int r) { return ((r >> 2) & 3) << 2; }

// DEPTH LDS stage slots (DEPTH - 1 stages in flight).  LS (chunks of two or
// more stages): the state entering each chunk goes through an LDS staging
// tile and leaves as whole 256-byte rows stored by the load wavefronts, and
// the exchange and staging buffers are single (a chunk's parts are taken one
// stage after they are given, and the next are given at least one barrier
// later).  Otherwise (chunks of one stage) the exchange is double-buffered by
// chunk parity and the compute wavefronts store the states themselves.
template <int DEPTH, bool LS>
__global__ void __launch_bounds__(THREADS) k_ssd_states_f32(StatesF32Args a) {
    constexpr int NPAR = LS ? 1 : 2;
    // loads of one load wavefront per stage: TL each of x and B, its weights,
    // and (load wavefront 1) the decay; stage s is complete when only the
    // DEPTH - 2 later stages' loads may still be in flight (output stores
    // issued in between only lengthen the wait)
    constexpr int WAIT1 = (DEPTH - 2) * (2 * TL + 2), WAIT0 = (DEPTH - 2) * (2 * TL + 1);
    static_assert(WAIT1 <= 63, "vmcnt range");
    __shared__ __align__(16) char ring[DEPTH * SLOT];
    // partial states at chunk starts (as in the bf16 pass): the first half
    // sums column tiles 0, 1, the second half 2, 3, each taking the other
    // half's part from xchg[parity][the other's wavefront]
    __shared__ __align__(16) f32x4 xchg[NPAR][NWAVES][2][64];
    // LS: the state entering a chunk on its way to HBM, 64 head-dim rows of
    // the 64 columns (+ 16 bytes of padding)
    __shared__ __align__(16) float pst[LS ? P : 1][NB + 4];

    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int nb = work % a.nblk;
    const int bh = work / a.nblk;
    const int h = bh % a.H, bi = bh / a.H;
    const int g = h / (a.H / a.G);
    const int L = a.L, Q = a.Q, nc = a.nc, N = a.N, H = a.H;
    const int SPC = Q / KB, S = nc * SPC;
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    const int pw = w & 3, kh = w >> 2;          // row tile, position half

    // ---- running (partial) state h^T tiles: acc[j][i] = h[p][n],
    // p = 16 pw + ln, n = NB nb + 16 j + 4 kg + i; the initial state goes to
    // the first half.  Loaded before any direct load is issued.
    f32x4 acc[4];
    const int64_t hoff = ((int64_t)bi * H + h) * P * N;
    const int prow = 16 * pw + ln;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = NB * nb + 16 * j + 4 * kg;
        if (a.init && kh == 0 && w < NWAVES) {
            const float4 v = *reinterpret_cast<const float4*>(a.init + hoff + (int64_t)prow * N + n);
            acc[j][0] = v.x; acc[j][1] = v.y; acc[j][2] = v.z; acc[j][3] = v.w;
        } else {
            acc[j] = zero4();
        }
        asm volatile("" ::"v"(acc[j]));
    }

    if (w >= NWAVES) {
        // ---- load wavefront li: rows 16 li .. 16 li + 15 of the x and B tiles
        // of every stage.  Direct load u (1 KB) brings rows 4 u .. 4 u + 3:
        // lane l fills 16-byte chunk slot l & 15 of row r = 4 u + (l >> 4),
        // with chunk (l & 15) ^ xsw(r) of the x row and chunk l & 15 of the B row.
        const int li = w - NWAVES;
        const float* xsrc = a.x + ((int64_t)bi * L * H + h) * P;
        const int64_t xstr = (int64_t)H * P;
        const float* bsrc = a.B + ((int64_t)bi * L * a.G + g) * N + nb * NB;
        const int64_t bstr = (int64_t)a.G * N;
        const int64_t bhc = ((int64_t)bi * H + h) * nc;
        const uint32_t ring_lds = lds_addr(ring);
        const int ch = lane & 15;
        auto issue = [&](int st, int k) {
            const uint32_t sb = ring_lds + k * SLOT;
#pragma unroll
            for (int uu = 0; uu < TL; ++uu) {
                const int u = li * TL + uu;
                const int r = 4 * u + (lane >> 4);
                const int64_t t = min(st * KB + r, L - 1);   // past the end: weight 0
                if (a.ntx) dma16nt(xsrc + t * xstr + 4 * (ch ^ xsw(r)), sb + 1024 * u);
                else dma16(xsrc + t * xstr + 4 * (ch ^ xsw(r)), sb + 1024 * u);
                dma16(bsrc + t * bstr + 4 * ch, sb + XB + 1024 * u);
            }
            const int c = st / SPC;
            const float* wsrc = a.wts + (bhc + c) * Q + (st - c * SPC) * KB + 16 * li;
            if (lane < 4) dma16(wsrc + 4 * lane, sb + XB + BB + 64 * li);
            if (li == 1) dma4(a.scl + bhc + c, sb + XB + BB + KB * 4);
        };
        // this wavefront's B rows of slot k as hi / lo planes, in place; no
        // other wavefront touches these rows before the barrier that follows
        auto split = [&](int k) {
            char* sl = ring + k * SLOT + XB;
            float4 bv[TL];
#pragma unroll
            for (int uu = 0; uu < TL; ++uu)
                bv[uu] = *reinterpret_cast<const float4*>(sl + 1024 * (li * TL + uu) + 16 * lane);
            // the rows other lanes read are written below: every read has
            // returned (and the compiler keeps them all above) before the
            // first write
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int uu = 0; uu < TL; ++uu) {
                const int r = 4 * (li * TL + uu) + (lane >> 4);
                uint32_t h0, l0, h1, l1;
                split2(bv[uu].x, bv[uu].y, h0, l0);
                split2(bv[uu].z, bv[uu].w, h1, l1);
                typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
                *reinterpret_cast<u2*>(sl + r * ROW + plane_off(r, 0, ch)) = u2{h0, h1};
                *reinterpret_cast<u2*>(sl + r * ROW + plane_off(r, 1, ch)) = u2{l0, l1};
            }
        };
        // LS: the state entering chunk c (staged by the compute wavefronts in
        // the chunk's first stage) to HBM: rows 16 li .. 16 li + 15, 4 rows of
        // 256 bytes per store
        auto store_pst = [&](int c) {
            float* pp = a.passed + (((int64_t)bi * nc + c) * H + h) * P * N + NB * nb;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * li + 4 * i + (lane >> 4);
                const float4 v = *reinterpret_cast<const float4*>(&pst[row][4 * ch]);
                *reinterpret_cast<float4*>(pp + (int64_t)row * N + 4 * ch) = v;
            }
        };
#pragma unroll
        for (int i = 0; i < DEPTH - 1; ++i) issue(min(i, S - 1), i);
        for (int s = 0; s < S; ++s) {
            // stage s complete (the next stage may be in flight)
            if (li == 1) wait_vmem<WAIT1>();
            else wait_vmem<WAIT0>();
            split(s % DEPTH);
            lds_barrier();               // slot s % DEPTH ready, slot (s-1) % DEPTH free
            issue(min(s + DEPTH - 1, S - 1), (s + DEPTH - 1) % DEPTH);
            if (LS && s % SPC == 1) store_pst(s / SPC);
        }
        wait_vmem<0>();                  // the tail stages re-loaded into unused slots
        __syncthreads();                 // the final exchange
        return;
    }

    // B operands: rows of this half's MFMA k indices 0..3 (+16: 4..7); the
    // row swizzle and plane order repeat every 8 rows
    const int rA = (KB / 2) * kh + 4 * kg + (ln >> 2);
    const int c1 = ln & 3;                        // 4-column group of the read
    int bo_h[4], bo_l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        bo_h[j] = XB + rA * ROW + plane_off(rA, 0, 4 * j + c1);
        bo_l[j] = XB + rA * ROW + plane_off(rA, 1, 4 * j + c1);
    }
    // x operand: k index j of the lane is position 32 kh + 4 kg + (j & 3) +
    // 16 (j >> 2) (the rows of the B operand's k index j), column 16 pw + ln;
    // every such row has xsw = kg << 2.  Lane j < 8 of each row reads the
    // weight of k index j; the row shares them.
    const int xo = (KB / 2 * kh + 4 * kg) * ROW + ((((4 * pw + (ln >> 2)) ^ (kg << 2))) << 4) +
                   ((ln & 3) << 2);
    const int wpos = (KB / 2) * kh + (ln & 4 ? 16 : 0) + 4 * kg + (ln & 3);
    constexpr int R16 = 16 * ROW;
    auto give = [&](int par) {
        par %= NPAR;
        if (kh == 0) {
            xchg[par][w][0][lane] = acc[2];
            xchg[par][w][1][lane] = acc[3];
        } else {
            xchg[par][w][0][lane] = acc[0];
            xchg[par][w][1][lane] = acc[1];
        }
    };
    auto take = [&](int par, f32x4& s0, f32x4& s1) {
        par %= NPAR;
        const f32x4 o0 = xchg[par][w ^ 4][0][lane], o1 = xchg[par][w ^ 4][1][lane];
        s0 = (kh == 0 ? acc[0] : acc[2]) + o0;
        s1 = (kh == 0 ? acc[1] : acc[3]) + o1;
    };
    const int ncol = NB * nb + 32 * kh + 4 * kg;  // first column of this lane's summed tiles
    give(0);                                      // the parts of h_0
    for (int s = 0; s < S; ++s) {
        const int k = s % DEPTH;
        const int c = s / SPC, kb = s - c * SPC;
        lds_barrier();                            // slot k ready; at chunk starts the
                                                  // second half's part
        const char* slot = ring + k * SLOT;
        const float* aux = reinterpret_cast<const float*>(slot + XB + BB);
        f32x4 h0, h1;
        if (kb == 0) {
            take(c & 1, h0, h1);
            const float sc = aux[KB];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[j][r] *= sc;
        }
        // every operand of the stage read first (their latencies overlap)
        const float w0 = aux[wpos];
        float xv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j)
            xv[j] = *reinterpret_cast<const float*>(slot + xo + ((j & 3) + 16 * (j >> 2)) * ROW);
        bf16x4 bh0[4], bh1[4], bl0[4], bl1[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            bh0[j] = ds_read_tr(slot + bo_h[j]);
            bh1[j] = ds_read_tr(slot + bo_h[j] + R16);
            bl0[j] = ds_read_tr(slot + bo_l[j]);
            bl1[j] = ds_read_tr(slot + bo_l[j] + R16);
        }
        __builtin_amdgcn_sched_barrier(0);
        // w x of the lane's 8 k indices as bf16 hi / lo parts
        const float wv[8] = {row_bcast<0>(w0), row_bcast<1>(w0), row_bcast<2>(w0), row_bcast<3>(w0),
                             row_bcast<4>(w0), row_bcast<5>(w0), row_bcast<6>(w0), row_bcast<7>(w0)};
        uint32_t xhp[4], xlp[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) split2(xv[2 * i] * wv[2 * i], xv[2 * i + 1] * wv[2 * i + 1], xhp[i], xlp[i]);
        const bf16x8 xh = as_bf16x8(xhp[0], xhp[1], xhp[2], xhp[3]);
        const bf16x8 xl = as_bf16x8(xlp[0], xlp[1], xlp[2], xlp[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x8 bh = __builtin_shufflevector(bh0[j], bh1[j], 0, 1, 2, 3, 4, 5, 6, 7);
            const bf16x8 bl = __builtin_shufflevector(bl0[j], bl1[j], 0, 1, 2, 3, 4, 5, 6, 7);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, xh, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bh, xl, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bl, xh, acc[j], 0, 0, 0);
        }
        if (kb == 0) {
            // h_c, the state entering chunk c: this half's two summed tiles
            if (LS) {
                float* pr = &pst[prow][32 * kh + 4 * kg];
                *reinterpret_cast<f32x4*>(pr) = h0;
                *reinterpret_cast<f32x4*>(pr + 16) = h1;
            } else {
                float* pp = a.passed + ((((int64_t)bi * nc + c) * H + h) * P + prow) * N + ncol;
                *reinterpret_cast<float4*>(pp) = make_float4(h0[0], h0[1], h0[2], h0[3]);
                *reinterpret_cast<float4*>(pp + 16) = make_float4(h1[0], h1[1], h1[2], h1[3]);
            }
        }
        if ((s + 1) % SPC == 0) give((c + 1) & 1);   // the end of chunk c: parts of h_{c+1}
    }
    __syncthreads();
    if (a.fin) {
        f32x4 s0, s1;
        take(nc & 1, s0, s1);
        float* fp = a.fin + hoff + (int64_t)prow * N + ncol;
        *reinterpret_cast<float4*>(fp) = make_float4(s0[0], s0[1], s0[2], s0[3]);
        *reinterpret_cast<float4*>(fp + 16) = make_float4(s1[0], s1[1], s1[2], s1[3]);
    }
}

}  // namespace

namespace m2 {

// fp32 inputs take this pass where it fills the CUs (one workgroup per (batch,
// head, 64 dstate columns), at least 256 of them); below that the staged
// kernels spread the same work over more workgroups.  The M2_KNOB_F32_STATES
// override (tests) forces either where the shape allows it.
bool states_fused_f32_supported(const m2_ssd_combined_args& a) {
    if (!(a.dtype == M2_F32 && a.headdim == P && a.dstate % NB == 0 && a.chunk_size % KB == 0 &&
          a.chunk_size <= 256 && a.ngroups > 0 && a.nheads % a.ngroups == 0))
        return false;
    switch (dispatch_override(M2_KNOB_F32_STATES)) {
        case 1: return true;
        case 2: return false;
        default: break;
    }
    return a.batch * a.nheads * (a.dstate / NB) >= 256;
}

int launch_states_fused_f32(const m2_ssd_combined_args& a, const float* wts, const float* scl,
                            void* passed, hipStream_t s) {
    M2_REQUIRE(states_fused_f32_supported(a), M2_ERR_UNSUPPORTED,
               "ssd_states_f32: unsupported shape / dtype");
    StatesF32Args sa{};
    sa.x = (const float*)a.x; sa.B = (const float*)a.B; sa.wts = wts; sa.scl = scl;
    sa.init = a.initial_states; sa.passed = (float*)passed; sa.fin = a.final_states;
    sa.L = (int)a.seqlen; sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.N = (int)a.dstate;
    sa.Q = (int)a.chunk_size; sa.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    sa.nblk = (int)(a.dstate / NB);
    const int64_t nwork = a.batch * a.nheads * sa.nblk;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "ssd_states_f32: too many workgroups");
    sa.nwork = (int)nwork;
    // Where x and the passed states (the rows the scan reads after this pass)
    // do not fit the cache with room to spare, x is loaded non-temporally, so
    // that the states this pass writes stay cached for the scan (the
    // nemotron-h-8b shape in fp32, 256 MiB of rows: layer 0.1859 -> 0.1833 ms,
    // A/B on one box); the scan then loads both non-temporally as well.
    sa.ntx = (double)a.batch * a.seqlen * a.nheads * a.headdim * 4 +
             (double)a.batch * sa.nc * a.nheads * a.headdim * a.dstate * 4 > 224.0 * (1 << 20);
    if (sa.Q / KB >= 2) k_ssd_states_f32<3, true><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
    else k_ssd_states_f32<3, false><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
    return check_launch("ssd_states_f32");
}

}  // namespace m2
