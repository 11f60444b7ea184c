// ssd_states: chunk_state + state_passing of the combined forward in one pass.
//
//   S_c = sum_q w[q] x[q, :]^T B[q, :]                              (chunk_state)
//   h_0 = initial state (or 0),  passed[c] = h_c,
//   h_{c+1} = scl[c] h_c + S_c                                     (state_passing)
//
// with the weights w[q] = exp(min(dA[last] - dA[q], 0)) dt'[q] and the decay
// scl[c] = exp(dA[Q-1]) (seq_idx rules applied) precomputed by chunk_cumsum.
// Two kernels: k_ssd_states (a head's 64-column dstate block per workgroup,
// below) and k_ssd_pair (two heads of a group per workgroup, further down);
// launch_states_fused picks one per shape.
// The unfused stages write the fp32 chunk states S_c to HBM and read them
// back; here the running state h stays in the MFMA accumulators of one
// workgroup that walks the chunks of a (batch, head, 64-column dstate block) in
// order, so HBM sees only x, B, w, the bf16 states entering each chunk and the
// final states.
//
// Workgroup = 8 compute wavefronts (two per SIMD, so that one hides the
// other's LDS and MFMA latency) + 4 load wavefronts.  Positions stream through
// a ring of DEPTH LDS slots in stages of KB = 64 or 128: each slot holds the x
// rows [KB x 64], the B rows [KB x 64] and the stage's weights (+ the chunk's
// decay).  Compute wavefront w owns head-dim rows 16 (w & 3) .. +15, all 64
// dstate columns of the block (four 16 x 16 tiles) and the positions
// (KB/2) (w >> 2) .. +KB/2-1 of every stage: the two halves accumulate
// separate partial states (the recurrence is linear), which are summed
// through LDS only where the state is written (chunk starts and the end):
// the second half leaves its part in a chunk-parity double buffer at the end
// of a chunk, and the stage barrier that follows also hands it over, so the
// exchange costs no barrier of its own.  Each stage has one barrier.
// The load wavefronts fill the slots with direct global -> LDS loads
// (global_load_lds_dwordx4), DEPTH - 1 stages ahead of use, and wait for them
// with explicit vmcnt waits: no load result passes through VGPRs, so nothing
// forces the compiler to drain the loads in flight, and the compute
// wavefronts' stores never hold up those waits.  Tiles are dense in LDS with
// the 16-byte chunks of each row XOR-swizzled so that the transposed reads
// below hit 64 distinct banks per 32 lanes.
//
// MFMA operands need 8 consecutive positions per lane for a fixed row / column:
// they come straight from the row-major tiles through the gfx950 LDS transpose
// read (ds_read_b64_tr_b16: lane i of a 16-lane group receives column i of the
// 4 x 16 block the group addresses).  The product is computed transposed,
// h^T[n, p] += B^T[n, q] (w x)[q, p], so that each lane holds 4 consecutive
// dstate columns of one head-dim row (8-byte bf16 and 16-byte fp32 stores).
// w x is split into hi + lo bf16 parts (two MFMAs): the weighted operand keeps
// near-fp32 accuracy as in the fp32 einsum of the reference.
//
// Follows reference kernels/chunk_state_fwd.py:104-187 (product),
// kernels/state_passing_fwd.py:108-151 (recurrence) and ops/ssd_naive.py:77-182.
#include <stdlib.h>
#include <string.h>
#include <type_traits>

#include "m2_internal.h"

namespace {

constexpr int NWAVES = 8;                  // compute wavefronts
constexpr int NLOAD = 4;                   // load wavefronts: each keeps only so many
                                           // direct loads in flight
constexpr int THREADS = (NWAVES + NLOAD) * 64;
constexpr int P = 64;        // head dim
constexpr int NB = 64;       // dstate columns per workgroup
constexpr int CPR = 8;       // 16-byte chunks per 128-byte tile row

// Stages of KB positions (64 or 128): each half of the compute wavefronts
// takes KB/2 positions (KS MFMA K steps of 32).
template <int KB>
struct StCfg {
    // LDS stage slots, DEPTH - 1 stages in flight.  128-position stages: one
    // in flight measures faster than two (c2: 42.7-43.6 against 44.6-45.2 us by
    // events, A/B on one box), and three in flight (an early slot release) is
    // slower again; 64-position stages with three or four slots: 50.9-51.7 us
    static constexpr int DEPTH = KB == 64 ? 6 : 2;
    static constexpr int XB = KB * P * 2, BB = KB * NB * 2;   // tile bytes
    static constexpr int AUXB = KB * 4 + 256;        // weights, 64 copies of the decay
    static constexpr int SLOT = XB + BB + AUXB;
    static constexpr int TI = KB * CPR / 64;         // 1 KB loads per tile and stage
    static constexpr int TL = TI / NLOAD;            // ... per load wavefront
    static constexpr int KS = KB / 64;               // K steps per half
    // loads of one load wavefront that may still be in flight when stage s is
    // needed: DEPTH - 2 later stages of 2 TL tile loads (+ weights / decay for
    // load wavefronts 0 and 1)
    static constexpr int WAIT01 = (DEPTH - 2) * (2 * TL + 1), WAIT23 = (DEPTH - 2) * 2 * TL;
    static_assert(TI % NLOAD == 0, "tiles split evenly over the load wavefronts");
    static_assert(WAIT01 <= 63, "vmcnt range");
};

// 16-byte chunk swizzle of tile row R (128-byte rows): 8 consecutive rows read
// at one chunk pair land on disjoint banks.
M2_DEV int swz(int R) { return ((R >> 1) & 3) << 1; }

struct StatesArgs {
    const bf16* x;
    const bf16* B;
    const float* wts;      // [b, H, nc, Q]
    const float* scl;      // [b, H, nc]
    const float* init;
    bf16* passed;
    float* fin;
    int L, H, G, N, Q, nc, nblk, nwork;
};

template <int KB>
__global__ void __launch_bounds__(THREADS) k_ssd_states(StatesArgs a) {
    typedef StCfg<KB> C;
    constexpr int DEPTH = C::DEPTH, XB = C::XB, BB = C::BB, SLOT = C::SLOT, TL = C::TL;
    __shared__ __align__(16) char ring[DEPTH * SLOT];
    // partial states at chunk starts: the first half sums column tiles 0, 1,
    // the second half 2, 3, each taking the other half's part of them from
    // xchg[parity][the other's wavefront], double-buffered by chunk parity:
    // written at the end of a chunk, read after the next stage's barrier, and
    // not written again before the barrier after that
    __shared__ __align__(16) f32x4 xchg[2][NWAVES][2][64];
    // the bf16 states entering a chunk on their way to HBM (stored by the load
    // wavefronts after the next barrier), double-buffered by chunk parity: per
    // row tile 16 rows of 64 columns + 8 pad (144 bytes)
    __shared__ __align__(16) bf16 pst[2][4][16][72];

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
    // p = 16 pw + ln, n = NB nb + 16 j + 4 kg + i.  The initial state goes to
    // the first half.  Loaded (and consumed) before any direct load is issued,
    // so the compiler's own waits never cover those.
    f32x4 acc[4];
    const int64_t hoff = ((int64_t)bi * H + h) * P * N;
    const int prow = 16 * pw + ln;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int n = NB * nb + 16 * j + 4 * kg;
        if (a.init && kh == 0) {
            const float4 v = *reinterpret_cast<const float4*>(a.init + hoff + (int64_t)prow * N + n);
            acc[j][0] = v.x; acc[j][1] = v.y; acc[j][2] = v.z; acc[j][3] = v.w;
        } else {
            acc[j] = zero4();
        }
        asm volatile("" ::"v"(acc[j]));
    }

    // ---- the load wavefronts: stage st -> slot k.  Lane l of load u brings
    // 16-byte chunk 64 u + l of the x / B tile (row, swizzled column); load
    // wavefront li takes loads u in [li TL, li TL + TL), wavefront 0 also the
    // stage's weights (64 words), wavefront 1 64 copies of the chunk's decay.
    const bf16* xsrc = a.x + ((int64_t)bi * L * H + h) * P;
    const int64_t xstr = (int64_t)H * P;
    const bf16* bsrc = a.B + ((int64_t)bi * L * a.G + g) * N + nb * NB;
    const int64_t bstr = (int64_t)a.G * N;
    const int64_t bhc = ((int64_t)bi * H + h) * nc;
    const uint32_t ring_lds = lds_addr(ring);
    const int li = w - NWAVES;
    auto issue = [&](int st, int k) {
        const uint32_t sb = ring_lds + k * SLOT;
#pragma unroll
        for (int uu = 0; uu < TL; ++uu) {
            const int u = li * TL + uu;
            const int gi = 64 * u + lane, r = gi / CPR;
            const int64_t t = min(st * KB + r, L - 1);   // past the end: weight 0
            const int col = ((gi % CPR) ^ swz(r)) * 8;
            dma16(xsrc + t * xstr + col, sb + 1024 * u);
            dma16(bsrc + t * bstr + col, sb + XB + 1024 * u);
        }
        const int c = st / SPC;
        const float* wsrc = a.wts + (bhc + c) * Q + (st - c * SPC) * KB;
        if (li == 0) {
            if (KB == 64) dma4(wsrc + lane, sb + XB + BB);
            else if (lane < KB / 4) dma16(wsrc + 4 * lane, sb + XB + BB);
        }
        if (li == 1) dma4(a.scl + bhc + c, sb + XB + BB + KB * 4);
    };
    if (w >= NWAVES) {
        // the bf16 state entering chunk c (pst[c & 1], complete one barrier after
        // the chunk's first stage) to HBM: load wavefront li stores row tile li,
        // whole 128-byte rows, two 16-byte pieces per lane.  These stores only
        // make the vmcnt waits below longer (those count the loads issued after
        // the awaited ones); they are ordinary stores, so the compiler keeps
        // their address and data registers intact until the hardware has read
        // them (two wait states after a 16-byte store on gfx950).
        auto store_pst = [&](int c) {
            const bf16* pr = &pst[c & 1][li][0][0];
            bf16* pp = a.passed + ((((int64_t)bi * nc + c) * H + h) * P + 16 * li) * N + NB * nb;
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int row = 8 * half + (lane >> 3), col = 8 * (lane & 7);
                const u32x4 v = *reinterpret_cast<const u32x4*>(pr + row * 72 + col);
                *reinterpret_cast<u32x4*>(pp + (int64_t)row * N + col) = v;
            }
        };
#pragma unroll
        for (int i = 0; i < DEPTH - 1; ++i) issue(min(i, S - 1), i);
        for (int s = 0; s < S; ++s) {
            // stage s complete (later stages may be in flight)
            if (li < 2) wait_vmem<C::WAIT01>();
            else wait_vmem<C::WAIT23>();
            lds_barrier();               // slot s % DEPTH complete, slot (s-1) % DEPTH free
            issue(min(s + DEPTH - 1, S - 1), (s + DEPTH - 1) % DEPTH);
            if (s > 0 && (s - 1) % SPC == 0) store_pst((s - 1) / SPC);
        }
        wait_vmem<0>();                  // the tail stages re-loaded into unused slots
        __syncthreads();                 // the final exchange
        if (SPC == 1) store_pst(nc - 1);
        return;
    }

    // The compute path, instantiated per position half (kh is uniform in a
    // wavefront; as a compile-time constant the exchange's selects go away).
    auto compute_half = [&](auto KHC) {
        constexpr int kh = decltype(KHC)::value;
        // this half's K steps ks: tile rows (KB/2) kh + 32 ks + ...; the row swizzle
        // repeats every 8 rows, so step ks is step 0 moved by 32 rows
        const int rA = (KB / 2) * kh + 4 * kg + (ln >> 2);   // rows of MFMA k = 0..3 (+16: 4..7)
        const int c1 = ln & 3;                         // 8-byte column group of the read
        const int cb = 8 * (c1 & 1);
        const int wk = (KB / 2) * kh + 4 * kg;      // weight of k index 0 (4..7: 16 more)
        const int xo0 = rA * (2 * P) + (((2 * pw + (c1 >> 1)) ^ swz(rA)) * 16) + cb;
        const int xo1 = (rA + 16) * (2 * P) + (((2 * pw + (c1 >> 1)) ^ swz(rA + 16)) * 16) + cb;
        int bo0[4], bo1[4];
    #pragma unroll
        for (int j = 0; j < 4; ++j) {
            bo0[j] = XB + rA * (2 * NB) + (((2 * j + (c1 >> 1)) ^ swz(rA)) * 16) + cb;
            bo1[j] = XB + (rA + 16) * (2 * NB) + (((2 * j + (c1 >> 1)) ^ swz(rA + 16)) * 16) + cb;
        }
        // this wavefront's part of the tiles the other half sums; the sums of its
        // own two tiles (columns 32 kh .. 32 kh + 31)
        auto give = [&](int par) {
            if (kh == 0) {
                xchg[par][w][0][lane] = acc[2];
                xchg[par][w][1][lane] = acc[3];
            } else {
                xchg[par][w][0][lane] = acc[0];
                xchg[par][w][1][lane] = acc[1];
            }
        };
        auto take = [&](int par, f32x4& s0, f32x4& s1) {
            const f32x4 o0 = xchg[par][w ^ 4][0][lane], o1 = xchg[par][w ^ 4][1][lane];
            s0 = (kh == 0 ? acc[0] : acc[2]) + o0;
            s1 = (kh == 0 ? acc[1] : acc[3]) + o1;
        };
        give(0);                                         // the parts of h_0
        for (int s = 0; s < S; ++s) {
            const int k = s % DEPTH;
            const int c = s / SPC, kb = s - c * SPC;
            lds_barrier();                               // slot k complete (load wavefront),
                                                         // at chunk starts the second half's part
            const char* slot = ring + k * SLOT;
            const float* aux = reinterpret_cast<const float*>(slot + XB + BB);
            // h_c (sum of the halves) is the state entering chunk c: this half's
            // two tiles of it are summed, rounded to bf16 and staged after the
            // stage's MFMA steps are issued (whose latency hides the reads of the
            // other half's part); both halves continue with h <- scl[c] h
            f32x4 h0, h1;
            if (kb == 0) {
                take(c & 1, h0, h1);
                const float sc = aux[KB];
    #pragma unroll
                for (int j = 0; j < 4; ++j)
    #pragma unroll
                    for (int r = 0; r < 4; ++r) acc[j][r] *= sc;
            }
            // acc += B^T (w x) over this half's KB/2 positions.  In step ks, MFMA k
            // index j < 4 is position (KB/2) kh + 32 ks + 4 kg + j, j >= 4 is 16 more.
            // Lane j < 8 of each row reads the weight of k index j; the row shares them.
            // every LDS operand of the stage is read first, so that the reads'
            // latencies overlap (left to itself the scheduler reuses one register
            // set and waits for each B fragment before its MFMAs)
            float4 wa[C::KS], wb[C::KS];
            bf16x4 xa[C::KS], xb[C::KS], ba[C::KS][4], bb[C::KS][4];
    #pragma unroll
            for (int ks = 0; ks < C::KS; ++ks) {
                // the weights of the lane's k indices 0..3 and 4..7 (16 lanes read
                // each address: broadcast reads, no lane moves)
                wa[ks] = *reinterpret_cast<const float4*>(aux + wk + 32 * ks);
                wb[ks] = *reinterpret_cast<const float4*>(aux + wk + 32 * ks + 16);
                xa[ks] = ds_read_tr(slot + xo0 + ks * 32 * (2 * P));
                xb[ks] = ds_read_tr(slot + xo1 + ks * 32 * (2 * P));
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    ba[ks][j] = ds_read_tr(slot + bo0[j] + ks * 32 * (2 * NB));
                    bb[ks][j] = ds_read_tr(slot + bo1[j] + ks * 32 * (2 * NB));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
    #pragma unroll
            for (int ks = 0; ks < C::KS; ++ks) {
                const float wv[8] = {wa[ks].x, wa[ks].y, wa[ks].z, wa[ks].w, wb[ks].x, wb[ks].y, wb[ks].z, wb[ks].w};
                // w x of the lane's 8 k indices as packed bf16 hi / lo pairs
                typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
                const u2 pa = __builtin_bit_cast(u2, xa[ks]), pb = __builtin_bit_cast(u2, xb[ks]);
                uint32_t h[4], l[4];
                split2(bf16_lo(pa[0]) * wv[0], bf16_hi(pa[0]) * wv[1], h[0], l[0]);
                split2(bf16_lo(pa[1]) * wv[2], bf16_hi(pa[1]) * wv[3], h[1], l[1]);
                split2(bf16_lo(pb[0]) * wv[4], bf16_hi(pb[0]) * wv[5], h[2], l[2]);
                split2(bf16_lo(pb[1]) * wv[6], bf16_hi(pb[1]) * wv[7], h[3], l[3]);
                const bf16x8 xh = as_bf16x8(h[0], h[1], h[2], h[3]), xl = as_bf16x8(l[0], l[1], l[2], l[3]);
    #pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const bf16x8 bf = __builtin_shufflevector(ba[ks][j], bb[ks][j], 0, 1, 2, 3, 4, 5, 6, 7);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, xh, acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, xl, acc[j], 0, 0, 0);
                }
            }
            if (kb == 0) {
                // lane (ln, kg): 4 columns of staging row ln
                bf16* pr = &pst[c & 1][pw][ln][32 * kh + 4 * kg];
                const bf16x4 o0 = {(bf16)h0[0], (bf16)h0[1], (bf16)h0[2], (bf16)h0[3]};
                const bf16x4 o1 = {(bf16)h1[0], (bf16)h1[1], (bf16)h1[2], (bf16)h1[3]};
                *reinterpret_cast<bf16x4*>(pr) = o0;
                *reinterpret_cast<bf16x4*>(pr + 16) = o1;
            }
            if ((s + 1) % SPC == 0) give((c + 1) & 1);  // the end of chunk c: parts of h_{c+1}
        }
        __syncthreads();
        if (a.fin) {
            f32x4 s0, s1;
            take(nc & 1, s0, s1);
            const int n = NB * nb + 32 * kh + 4 * kg;
            *reinterpret_cast<float4*>(a.fin + hoff + (int64_t)prow * N + n) = make_float4(s0[0], s0[1], s0[2], s0[3]);
            *reinterpret_cast<float4*>(a.fin + hoff + (int64_t)prow * N + n + 16) = make_float4(s1[0], s1[1], s1[2], s1[3]);
        }
    };
    if (kh == 0) compute_half(std::integral_constant<int, 0>());
    else compute_half(std::integral_constant<int, 1>());
}

// 16-byte chunk swizzle of a tile row R: 128-byte rows read at one chunk pair
// by 8 consecutive rows, 256-byte rows likewise (each repeats every 8 rows)
template <int RB> M2_DEV int rswz(int R) { return RB == 128 ? ((R >> 1) & 3) << 1 : (R & 7) << 1; }

// ---------------------------------------------------------------------------
// k_ssd_pair: the same pass with one workgroup per (batch, pair of heads of a
// group, NB-column dstate block), for shapes with enough such workgroups to
// fill the CUs.  Two heads share each B row the CU brings in, and 128-column
// blocks bring x in once per 128 columns, so a pair moves 16 (NB 128) or 24
// (NB 64) KB into the CU per head, 64 columns and 128 positions, against 32 KB
// for the kernel above, and does twice a head's MFMA work per stage.  At c3
// the pass is HBM-bound (a build without MFMAs takes the same 218 us: 866 MB
// at 4.0 TB/s, against ~5-6 TB/s for plain HBM streams); at c1, with 160
// workgroups on 160 CUs, the compute alone takes 42.5 us, the memory 34 us.
// Compute wavefront w owns head (w >> 2) of the pair, head-dim rows
// 16 (w & 3) .. +15 and all NB columns, and takes every position of a stage
// (no position halves, so no exchange): each x element is weighted by one
// wavefront.  The bf16 state entering a chunk leaves through the wavefront's
// own staging rows in LDS, CW columns at a time, so that every store writes
// whole CW-column row pieces (128 bytes at NB 128): stored straight from the
// accumulators, 32-byte pieces of 16 rows per store, the states took 70 of
// the 257 us of the pass at c3 (1.37x).
//
// A slot holds the stage's x rows of both heads [KB x 2 P] (the heads are
// adjacent in memory: 256 contiguous bytes per row), the B rows [KB x NB],
// the heads' weights [2][KB] and their chunk decays.
template <int NB, int KB>
struct PairCfg {
    static constexpr int HP = 2;
    static constexpr int XROW = HP * P * 2, XCPR = XROW / 16;     // x row bytes, 16-byte chunks
    static constexpr int BROW = NB * 2, BCPR = BROW / 16;
    static constexpr int XB = KB * XROW, BB = KB * BROW;
    static constexpr int AUXB = HP * KB * 4 + 256;
    static constexpr int SLOT = XB + BB + AUXB;
    static constexpr int DEPTH = 150 * 1024 / SLOT < 8 ? 150 * 1024 / SLOT : 8;
    static constexpr int XL = XB / 1024 / NLOAD, BL = BB / 1024 / NLOAD;
    static constexpr int KS = KB / 32;                            // K steps per stage
    static constexpr int NT = NB / 16;                            // column tiles per wavefront
    // state staging: CW columns per pass, rows of CW + 8 bf16 (16 bytes of pad),
    // LPR lanes of 16 bytes per row, RPI rows per store
    static constexpr int CW = NB == 128 ? 64 : 32, SROW = CW + 8;
    static constexpr int LPR = CW / 8, RPI = 64 / LPR;
    // loads of one load wavefront that may still be in flight when stage s is
    // needed: DEPTH - 2 later stages (+ weights / decay for load wavefronts 0, 1)
    static constexpr int WAIT01 = (DEPTH - 2) * (XL + BL + 1), WAIT23 = (DEPTH - 2) * (XL + BL);
    static_assert(XB % (1024 * NLOAD) == 0 && BB % (1024 * NLOAD) == 0, "even load split");
    static_assert(DEPTH >= 3 && WAIT01 <= 63, "ring depth / vmcnt range");
    static_assert(HP * KB / 4 <= 64, "weights: one 16-byte load per lane");
    static_assert(DEPTH * SLOT + NWAVES * 16 * SROW * 2 <= 160 * 1024, "LDS budget");
};

template <int NB, int KB, bool NTS>
__global__ void __launch_bounds__(THREADS) k_ssd_pair(StatesArgs a) {
    typedef PairCfg<NB, KB> C;
    constexpr int HP = C::HP;
    constexpr int DEPTH = C::DEPTH, XB = C::XB, BB = C::BB, SLOT = C::SLOT, NT = C::NT;
    __shared__ __align__(16) char ring[DEPTH * SLOT];
    __shared__ __align__(16) bf16 stg[NWAVES][16][C::SROW];   // per compute wavefront

    // work = head pair x nblk + column block: the column blocks of a pair and
    // the pairs of a group, which read the same x and B rows, share an XCD
    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int nb = work % a.nblk;
    const int hq = work / a.nblk;                             // (b H + h0) / 2
    const int H = a.H, L = a.L, Q = a.Q, nc = a.nc, N = a.N;
    const int h0 = (hq * HP) % H, bi = (hq * HP) / H;
    const int g = h0 / (H / a.G);
    const int SPC = Q / KB;
    const int NST = nc * SPC;                                 // stages
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;

    if (w >= NWAVES) {
        // ---- the load wavefronts: stage i -> slot i % DEPTH.  Lane l of
        // load u brings 16-byte chunk 64 u + l of the x / B tile (row, swizzled
        // column); load wavefront li takes its XL x and BL B loads, wavefront 0
        // also the heads' weights of the stage, wavefront 1 their chunk decays.
        const bf16* xsrc = a.x + ((int64_t)bi * L * H + h0) * P;
        const int64_t xstr = (int64_t)H * P;
        const bf16* bsrc = a.B + ((int64_t)bi * L * a.G + g) * N + nb * NB;
        const int64_t bstr = (int64_t)a.G * N;
        const int64_t bhc = ((int64_t)bi * H + h0) * nc;
        const uint32_t ring_lds = lds_addr(ring);
        const int li = w - NWAVES;
        auto issue = [&](int st, int k) {
            const uint32_t sb = ring_lds + k * SLOT;
#pragma unroll
            for (int uu = 0; uu < C::XL; ++uu) {
                const int u = li * C::XL + uu;
                const int gi = 64 * u + lane, r = gi / C::XCPR;
                const int64_t t = min(st * KB + r, L - 1);    // past the end: weight 0
                dma16(xsrc + t * xstr + ((gi % C::XCPR) ^ rswz<C::XROW>(r)) * 8, sb + 1024 * u);
            }
#pragma unroll
            for (int uu = 0; uu < C::BL; ++uu) {
                const int u = li * C::BL + uu;
                const int gi = 64 * u + lane, r = gi / C::BCPR;
                const int64_t t = min(st * KB + r, L - 1);
                dma16(bsrc + t * bstr + ((gi % C::BCPR) ^ rswz<C::BROW>(r)) * 8, sb + XB + 1024 * u);
            }
            const int c = st / SPC, off = (st - c * SPC) * KB;
            if (li == 0 && lane < HP * KB / 4) {
                const int hh = lane / (KB / 4), q = 4 * (lane % (KB / 4));
                dma16(a.wts + (bhc + (int64_t)hh * nc + c) * Q + off + q, sb + XB + BB);
            }
            if (li == 1 && lane < HP) dma4(a.scl + bhc + (int64_t)lane * nc + c, sb + XB + BB + HP * KB * 4);
        };
#pragma unroll
        for (int i = 0; i < DEPTH - 1; ++i) issue(min(i, NST - 1), i);
        for (int i = 0; i < NST; ++i) {
            // stage i complete (later stages may be in flight)
            if (li < 2) wait_vmem<C::WAIT01>();
            else wait_vmem<C::WAIT23>();
            lds_barrier();               // slot i % DEPTH complete, slot (i-1) % DEPTH free
            issue(min(i + DEPTH - 1, NST - 1), (i + DEPTH - 1) % DEPTH);
        }
        wait_vmem<0>();                  // the tail stages re-loaded into unused slots
        return;
    }

    const int pw = w & 3, hh = w >> 2;
    const int h = h0 + hh;
    const int64_t hoff = ((int64_t)bi * H + h) * P * N;
    const int64_t bhc = ((int64_t)bi * H + h) * nc;

    // ---- running state h^T tiles: acc[j][i] = h[p][n], p = 16 pw + ln,
    // n = NB nb + 16 j + 4 kg + i
    f32x4 acc[NT];
    const int prow = 16 * pw + ln;
    const int ncol = NB * nb + 4 * kg;
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        if (a.init) {
            const float4 v = *reinterpret_cast<const float4*>(a.init + hoff + (int64_t)prow * N + ncol + 16 * j);
            acc[j][0] = v.x; acc[j][1] = v.y; acc[j][2] = v.z; acc[j][3] = v.w;
        } else {
            acc[j] = zero4();
        }
    }
    // the bf16 state entering chunk c (pk[j]: this lane's 4 columns of tile j)
    // into passed[c], rows 16 pw .. 16 pw + 15 of head h: per pass the lanes
    // write their pieces of CW columns into the staging rows and read them
    // back as 16-byte pieces of whole row segments.  The staging rows are this
    // wavefront's alone; its LDS operations complete in order, and the waits
    // keep the compiler from moving the accesses across each other.
    typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
    auto store_state = [&](int c, const u2* pk) {
        constexpr int CW = C::CW, SROW = C::SROW, LPR = C::LPR, RPI = C::RPI;
        bf16* pp = a.passed + ((((int64_t)bi * nc + c) * H + h) * P + 16 * pw) * N + NB * nb;
        bf16* sw = &stg[w][0][0];
#pragma unroll
        for (int ps = 0; ps < NB / CW; ++ps) {
#pragma unroll
            for (int jj = 0; jj < CW / 16; ++jj)
                *reinterpret_cast<u2*>(sw + ln * SROW + 16 * jj + 4 * kg) = pk[(CW / 16) * ps + jj];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            u32x4 v[16 / RPI];
#pragma unroll
            for (int q = 0; q < 16 / RPI; ++q)
                v[q] = *reinterpret_cast<const u32x4*>(sw + (RPI * q + lane / LPR) * SROW + 8 * (lane % LPR));
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int q = 0; q < 16 / RPI; ++q) {
                u32x4* dst = reinterpret_cast<u32x4*>(pp + (int64_t)(RPI * q + lane / LPR) * N + CW * ps + 8 * (lane % LPR));
                if constexpr (NTS) __builtin_nontemporal_store(v[q], dst);
                else *dst = v[q];
            }
        }
    };

    // MFMA operand offsets.  K step ks covers stage rows 32 ks .. 32 ks + 31:
    // MFMA k index j < 4 is row 32 ks + 4 kg + j, j >= 4 is 16 more; the row
    // swizzles repeat every 8 rows, so step ks is step 0 moved by 32 rows.
    // hT[n, p] += B^T[n, q] (w x)[q, p]: the lane reads B column n and x column
    // p through the gfx950 LDS transpose read (4 rows per lane group).
    const int rA = 4 * kg + (ln >> 2);
    const int c1 = ln & 3;                           // 8-byte column group of the read
    const int cb = 8 * (c1 & 1);
    const int wk = 4 * kg;                           // row of k index 0 (4..7: 16 more)
    const int xch = 8 * hh + 2 * pw + (c1 >> 1);     // 16-byte chunk of the x row
    const int xo0 = rA * C::XROW + ((xch ^ rswz<C::XROW>(rA)) * 16) + cb;
    const int xo1 = (rA + 16) * C::XROW + ((xch ^ rswz<C::XROW>(rA + 16)) * 16) + cb;
    int bo0[NT], bo1[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        bo0[j] = XB + rA * C::BROW + (((2 * j + (c1 >> 1)) ^ rswz<C::BROW>(rA)) * 16) + cb;
        bo1[j] = XB + (rA + 16) * C::BROW + (((2 * j + (c1 >> 1)) ^ rswz<C::BROW>(rA + 16)) * 16) + cb;
    }
    for (int s = 0; s < NST; ++s) {
        const int c = s / SPC, kb = s - c * SPC;
        const int i = s;
        lds_barrier();                               // slot i % DEPTH complete
        const char* slot = ring + (i % DEPTH) * SLOT;
        const float* aux = reinterpret_cast<const float*>(slot + XB + BB);
        // every LDS operand of the stage is read first, so that the reads'
        // latencies overlap
        float4 wa[C::KS], wb[C::KS];
        bf16x4 xa[C::KS], xb[C::KS], ba[C::KS][NT], bb[C::KS][NT];
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
            // the weights of the lane's k indices 0..3 and 4..7 (broadcast reads)
            wa[ks] = *reinterpret_cast<const float4*>(aux + hh * KB + wk + 32 * ks);
            wb[ks] = *reinterpret_cast<const float4*>(aux + hh * KB + wk + 32 * ks + 16);
            xa[ks] = ds_read_tr(slot + xo0 + ks * 32 * C::XROW);
            xb[ks] = ds_read_tr(slot + xo1 + ks * 32 * C::XROW);
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                ba[ks][j] = ds_read_tr(slot + bo0[j] + ks * 32 * C::BROW);
                bb[ks][j] = ds_read_tr(slot + bo1[j] + ks * 32 * C::BROW);
            }
        }
        u2 pk[NT];                                   // h_c in bf16 (chunk starts)
        if (kb == 0) {
            // acc = h_c, the state entering chunk c (stored after the stage's
            // MFMAs are issued); then h <- scl[c] h
            const float sc = aux[HP * KB + hh];
#pragma unroll
            for (int j = 0; j < NT; ++j) pk[j] = u2{pk_bf16(acc[j][0], acc[j][1]), pk_bf16(acc[j][2], acc[j][3])};
#pragma unroll
            for (int j = 0; j < NT; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[j][r] *= sc;
        }
        __builtin_amdgcn_sched_barrier(0);
        // acc += B^T (w x): w x split into packed bf16 hi / lo pairs (two MFMAs),
        // so the weighted operand keeps near-fp32 accuracy
#pragma unroll
        for (int ks = 0; ks < C::KS; ++ks) {
            const float wv[8] = {wa[ks].x, wa[ks].y, wa[ks].z, wa[ks].w, wb[ks].x, wb[ks].y, wb[ks].z, wb[ks].w};
            typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
            const u2 pa = __builtin_bit_cast(u2, xa[ks]), pb = __builtin_bit_cast(u2, xb[ks]);
            uint32_t hi[4], lo[4];
            split2(bf16_lo(pa[0]) * wv[0], bf16_hi(pa[0]) * wv[1], hi[0], lo[0]);
            split2(bf16_lo(pa[1]) * wv[2], bf16_hi(pa[1]) * wv[3], hi[1], lo[1]);
            split2(bf16_lo(pb[0]) * wv[4], bf16_hi(pb[0]) * wv[5], hi[2], lo[2]);
            split2(bf16_lo(pb[1]) * wv[6], bf16_hi(pb[1]) * wv[7], hi[3], lo[3]);
            const bf16x8 xh = as_bf16x8(hi[0], hi[1], hi[2], hi[3]), xl = as_bf16x8(lo[0], lo[1], lo[2], lo[3]);
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const bf16x8 bf = __builtin_shufflevector(ba[ks][j], bb[ks][j], 0, 1, 2, 3, 4, 5, 6, 7);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, xh, acc[j], 0, 0, 0);
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, xl, acc[j], 0, 0, 0);
            }
        }
        if (kb == 0) store_state(c, pk);
    }

    if (a.fin) {
        float* fp = a.fin + hoff + (int64_t)prow * N + ncol;
#pragma unroll
        for (int j = 0; j < NT; ++j)
            *reinterpret_cast<float4*>(fp + 16 * j) = make_float4(acc[j][0], acc[j][1], acc[j][2], acc[j][3]);
    }
}

}  // namespace

namespace m2 {

bool states_fused_supported(const m2_ssd_combined_args& a) {
    if (a.dtype == M2_F32) return states_fused_f32_supported(a);
    return a.dtype == M2_BF16 && a.headdim == P && a.dstate % NB == 0 &&
           a.chunk_size % 64 == 0 && a.chunk_size <= 256 && a.ngroups > 0 &&
           a.nheads % a.ngroups == 0;
}

// Work split of the pass (see k_ssd_pair): the time of a workgroup's chunk
// (128 positions) measured with every CU busy at the BASELINE shapes (1.36 us
// for a head in 64-column halves, 2.2 for a pair of heads x 64 columns, 3.0
// for a pair x 128 columns), times the rounds of workgroups over the CUs (one
// per CU) and the chunks.  The M2_KNOB_STATES_SPLIT override (tests) forces a split
// where the shape allows it.
enum StatesSplit { SPLIT_HALVES, SPLIT_PAIR64, SPLIT_PAIR128 };

StatesSplit states_split(const m2_ssd_combined_args& a) {
    const bool pair = (a.nheads / a.ngroups) % 2 == 0 && a.chunk_size % 128 == 0;
    const int64_t nc = (a.seqlen + a.chunk_size - 1) / a.chunk_size;
    const int64_t bh = a.batch * a.nheads;
    const int64_t cus = cu_count();
    auto rounds = [cus](int64_t wg) { return (double)((wg + cus - 1) / cus); };
    const double t_halves = rounds(bh * (a.dstate / 64)) * nc * 1.36;
    const double t_p64 = pair ? rounds(bh / 2 * (a.dstate / 64)) * nc * 2.2 : 1e30;
    const double t_p128 = pair && a.dstate % 128 == 0 ? rounds(bh / 2 * (a.dstate / 128)) * nc * 3.0 : 1e30;
    switch (dispatch_override(M2_KNOB_STATES_SPLIT)) {
        case 1: return SPLIT_HALVES;
        case 2: if (t_p64 < 1e30) return SPLIT_PAIR64; break;
        case 3: if (t_p128 < 1e30) return SPLIT_PAIR128; break;
        default: break;
    }
    if (t_p128 < t_halves && t_p128 <= t_p64) return SPLIT_PAIR128;
    if (t_p64 < t_halves) return SPLIT_PAIR64;
    return SPLIT_HALVES;
}

int launch_states_fused(const m2_ssd_combined_args& a, const float* wts, const float* scl,
                        void* passed, hipStream_t s) {
    if (a.dtype == M2_F32) return launch_states_fused_f32(a, wts, scl, passed, s);
    M2_REQUIRE(states_fused_supported(a), M2_ERR_UNSUPPORTED,
               "ssd_states: unsupported shape / dtype");
    StatesArgs sa{};
    sa.x = (const bf16*)a.x; sa.B = (const bf16*)a.B; sa.wts = wts; sa.scl = scl;
    sa.init = a.initial_states; sa.passed = (bf16*)passed; sa.fin = a.final_states;
    sa.L = (int)a.seqlen; sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.N = (int)a.dstate;
    sa.Q = (int)a.chunk_size; sa.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    const StatesSplit sp = states_split(a);
    const int nbw = sp == SPLIT_PAIR128 ? 128 : 64;
    sa.nblk = (int)(a.dstate / nbw);
    const int64_t nwork = a.batch * a.nheads / (sp == SPLIT_HALVES ? 1 : 2) * sa.nblk;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "ssd_states: too many workgroups");
    sa.nwork = (int)nwork;
    // The head-pair kernels store states larger than the 256 MB Infinity Cache
    // (c3: 537 MB) non-temporally: the scan that reads them then starts
    // without the pass's dirty lines in the cache, and its time drops by more
    // than the pass's grows (A/B on one box at c3: pass 194 -> 200 us, scan
    // 326 -> 302 us, layer 0.570 -> 0.554 ms).  Smaller ones (c1: 84 MB) stay
    // ordinary, as the scan then reads them from the cache (c1 0.110 against
    // 0.113 ms with non-temporal ones).
    const bool nts = (double)a.batch * sa.nc * a.nheads * a.headdim * a.dstate * 2 > 256.0 * (1 << 20);
    if (sp == SPLIT_PAIR128) {
        if (nts) k_ssd_pair<128, 64, true><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
        else k_ssd_pair<128, 64, false><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
    } else if (sp == SPLIT_PAIR64) {
        if (nts) k_ssd_pair<64, 128, true><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
        else k_ssd_pair<64, 128, false><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
    } else if (sa.Q % 128 == 0) {
        k_ssd_states<128><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
    } else {
        k_ssd_states<64><<<(unsigned)sa.nwork, THREADS, 0, s>>>(sa);
    }
    return check_launch("ssd_states");
}

}  // namespace m2
