// One-shot state sums for bf16 inputs, head dim 64 and dstate a multiple of
// 64, in two modes that share the kernel:
//
// chunk_state: the state of every chunk c of every batch row,
//   out[b, c, h] = sum_{q < qhi} w[q] x[q, :]^T B[q, :],  qhi = min(Q, L - c Q)
//   w[q]         = exp(min(dA[qhi - 1] - dA[q], 0)) dt[q],
// 0 where seq_idx[q] differs from seq_idx at the chunk's last position (all of
// the chunk if that is negative);
//
// chunk_state_varlen: the final state of each packed sequence s (batch 1)
// over the chunk c that holds its last token,
//   out[s, h] = sum_{q in [qlo, qhi)} w[q] x[q, :]^T B[q, :]  (+ carry)
//   w[q]      = exp(min(dA[qhi - 1] - dA[q], 0)) dt[q]
//   carry     = exp(dA[qhi - 1]) states[c, h]   when s started before chunk c
// with q the positions of chunk c, [qlo, qhi) the part of s in it, and
// states[c] the state entering chunk c.
//
// One workgroup per (chunk or sequence, HPW heads of a group, NB-column dstate
// block), NB = 128 when dstate allows (x then enters the CU once per 128
// columns instead of once per 64), else 64; HPW = 2 when a group has an even
// number of heads and the chunk is at most 128 positions (the two heads share
// every B row the CU brings in: 32 instead of 48 KB per head, 128 columns and
// 128 positions), else 1.  4096 chunk states at the nemotron-h-8b shape
// (2048 workgroups of two heads), 3072 varlen states at the packed 47b shape,
// several workgroups per CU, so a one-shot kernel hides its latency by
// occupancy.  The x rows [Q x HPW 64] (the heads are adjacent in memory) and
// the block's B rows [Q x NB] arrive by direct global -> LDS loads (16-byte
// chunks of each row XOR-swizzled, so the transposed reads hit distinct
// banks); the weights are computed from dA / dt while they are in flight.
// Wavefront w owns head w / 4 of the workgroup, head-dim rows 16 (w % 4) ..
// +15 and all NB columns (NB / 16 tiles of 16 x 16): it computes
// h^T[n, p] += B^T[n, q] (w x)[q, p] with MFMA operands read through the
// gfx950 LDS transpose read, w x split into hi + lo bf16 parts (near-fp32
// accuracy, as the reference's fp32 einsum).  The result goes through LDS so
// that each output row of NB fp32 (and its carry row) moves as NB / 4 lanes x
// 16 bytes.
//
// Follows reference kernels/chunk_state_fwd.py:104-187 (product), :239-269
// (weights, seq_idx rule) and :448-597 (varlen states).
#include <stdlib.h>
#include <string.h>

#include "m2_internal.h"

namespace {

constexpr int P = 64;        // head dim

// 16-byte chunk swizzle of tile row R: for 128-byte rows (x of one head, and
// B blocks of 64 columns) 8 consecutive rows read at one chunk pair land on
// disjoint banks; 256-byte rows (x of two heads, B blocks of 128 columns)
// start on the same bank, so 8 consecutive rows are spread by their low bits.
template <int RB> M2_DEV int swz(int R) { return RB == 128 ? ((R >> 1) & 3) << 1 : (R & 7) << 1; }

// LDS bytes of the x and B tiles, which the output staging [HPW 64][NB + 4]
// fp32 later reuses
__host__ __device__ inline int tiles_bytes(int Q, int NB, int HPW) {
    const int t = Q * (HPW * P + NB) * 2, o = HPW * P * (NB + 4) * 4;
    return t > o ? t : o;
}

struct VarlenArgs {
    const bf16* x;
    const bf16* B;
    const float* dt;        // [b, H, nc, Q]
    const float* dA;        // [b, H, nc, Q]
    const int32_t* cu;      // varlen: [nseq + 1]
    const void* states;     // varlen: [nc, H, P, N]
    const int32_t* seq;     // chunk mode: [b, L] or NULL
    float* out;             // varlen: [nseq, H, P, N]; chunk mode: [b, nc, H, P, N]
    int L, H, G, N, Q, nc, nblk, nwork, states_bf16;
};

template <bool CHUNK, int NB, int HPW>
__global__ void __launch_bounds__(256 * HPW) k_varlen_states(VarlenArgs a) {
    constexpr int THREADS = 256 * HPW;
    constexpr int OS = NB + 4;                                  // output staging row stride (floats)
    constexpr int NT = NB / 16;                                 // 16-column tiles per wavefront
    constexpr int XROW = HPW * P * 2;                           // x row bytes (the heads adjacent)
    constexpr int XCPR = XROW / 16;                             // 16-byte chunks per x row
    constexpr int BCPR = NB / 8;                                // 16-byte chunks per B row
    extern __shared__ __align__(16) char smem[];
    const int Q = a.Q, H = a.H, N = a.N;
    const int XB = Q * XROW;                                    // x tile bytes
    char* xs = smem;                                            // [Q][HPW 64] bf16, then B
    float* ot = reinterpret_cast<float*>(smem);                 // [HPW 64][OS], after the tiles
    float* wq = reinterpret_cast<float*>(smem + tiles_bytes(Q, NB, HPW)); // [HPW][Q]

    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int nb = work % a.nblk;
    const int HG = H / HPW;                    // head groups of HPW
    const int sp = work / a.nblk;              // (sequence or batch row x chunk) x HG + head group
    const int h0 = (sp % HG) * HPW;
    const int unit = sp / HG;                  // sequence, or batch row x chunk
    const int g = h0 / (H / a.G);
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    const int hh = w >> 2, wr = w & 3;         // head of the workgroup, row tile
    const int h = h0 + hh;
    float* const ob = a.out + ((int64_t)unit * H + h0) * P * N + NB * nb;   // head h0, row 0
    float* const op = ob + (int64_t)hh * P * N;                           // this wavefront's head

    int c, bi = 0, qlo = 0, qhi;
    bool carry = false;
    if (CHUNK) {
        c = unit % a.nc;
        bi = unit / a.nc;
        qhi = min(Q, a.L - c * Q);
    } else {
        const int s = unit;
        // clamp malformed boundaries into [0, L] so every access stays in bounds
        const int end = min(max(a.cu[s + 1], 0), a.L);
        const int start = min(max(a.cu[s], 0), end);
        if (end <= start) {                     // empty sequence: zero state
            for (int i = threadIdx.x; i < HPW * P * NB / 4; i += THREADS) {
                const int r = i / (NB / 4), c4 = 4 * (i % (NB / 4));   // r: head x P + row
                *reinterpret_cast<float4*>(ob + (int64_t)r * N + c4) = make_float4(0.f, 0.f, 0.f, 0.f);
            }
            return;
        }
        c = (end - 1) / Q;
        qlo = max(start - c * Q, 0);
        qhi = end - c * Q;
        carry = start < c * Q;
    }

    // ---- direct loads of the chunk's x rows and the block's B rows: load u
    // (64 lanes x 16 bytes = 1 KB) goes to tile bytes [1024 u, 1024 u + 1024);
    // rows past the end of the batch row are clamped (their weight is 0)
    const int64_t t0 = (int64_t)bi * a.L + (int64_t)c * Q, tend = (int64_t)bi * a.L + a.L - 1;
    const bf16* xsrc = a.x + (int64_t)h0 * P;
    const bf16* bsrc = a.B + (int64_t)g * N + NB * nb;
    const uint32_t xl = lds_addr(xs);
    // only the 32-position K steps that hold [qlo, qhi) (the varlen sequence's
    // part of the chunk) are loaded and multiplied; their other rows are
    // loaded as usual and weighted 0
    const int ks_lo = qlo / 32, ks_hi = (qhi + 31) / 32;
    for (int u = w + ks_lo * 32 * XCPR / 64; u < ks_hi * 32 * XCPR / 64; u += THREADS / 64) {
        const int gi = 64 * u + lane, r = gi / XCPR;
        const int64_t t = min(t0 + r, tend);
        const int col = ((gi % XCPR) ^ swz<XROW>(r)) * 8;
        dma16(xsrc + t * H * P + col, xl + 1024 * u);
    }
    for (int u = w + ks_lo * 32 * BCPR / 64; u < ks_hi * 32 * BCPR / 64; u += THREADS / 64) {
        const int gi = 64 * u + lane, r = gi / BCPR;
        const int64_t t = min(t0 + r, tend);
        const int col = ((gi % BCPR) ^ swz<2 * NB>(r)) * 8;
        dma16(bsrc + t * a.G * N + col, xl + XB + 1024 * u);
    }

    // ---- the carry rows of this lane's outputs (head h, rows 16 wr + RPI it +
    // lane / (NB / 4), columns 4 (lane % (NB / 4)) + i), loaded now so that
    // their latency overlaps the tiles'
    constexpr int LPR = NB / 4;                       // lanes per output row
    constexpr int RPI = 64 / LPR;                     // rows per store instruction
    constexpr int NIT = 16 / RPI;
    const int64_t soff = (((int64_t)c * H + h) * P) * N + NB * nb;
    const int orr = 16 * wr + lane / LPR, occ = 4 * (lane % LPR);
    bf16x4 cv16[NIT];
    float4 cv32[NIT];
    if (!CHUNK && carry) {
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
            const int64_t e = soff + (int64_t)(orr + RPI * it) * N + occ;
            if (a.states_bf16)
                cv16[it] = *reinterpret_cast<const bf16x4*>(reinterpret_cast<const bf16*>(a.states) + e);
            else
                cv32[it] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.states) + e);
        }
    }

    // ---- weights of the workgroup's heads (while the tiles are in flight)
    const int32_t* seq = CHUNK && a.seq ? a.seq + t0 : nullptr;
    const int se = seq ? seq[qhi - 1] : 0;
    for (int i = threadIdx.x; i < HPW * Q; i += THREADS) {
        const int ih = i / Q, q = i - ih * Q;
        const int64_t row = (((int64_t)bi * H + h0 + ih) * a.nc + c) * Q;
        float v = (q >= qlo && q < qhi) ? expf(fminf(a.dA[row + qhi - 1] - a.dA[row + q], 0.f)) * a.dt[row + q] : 0.f;
        if (seq && q < qhi && (se < 0 || seq[q] != se)) v = 0.f;
        wq[i] = v;
    }
    const float dA_ref = a.dA[(((int64_t)bi * H + h) * a.nc + c) * Q + qhi - 1];
    wait_vmem<0>();
    __syncthreads();

    // ---- acc[j] = h^T tile: lane (ln, kg) holds row p = 16 wr + ln of head h,
    // columns n = 16 j + 4 kg + i.  K step ks covers positions 32 ks .. 32 ks + 31:
    // MFMA k index j < 4 is position 32 ks + 4 kg + j, j >= 4 is 16 more.
    const int rA = 4 * kg + (ln >> 2);                // rows read by this lane (+16)
    const int c1 = ln & 3;                            // 8-byte column group of the read
    const int cb = 8 * (c1 & 1);
    const int wpos = (ln & 4 ? 16 : 0) + 4 * kg + (ln & 3);   // k index ln & 7
    const int xch = 8 * hh + 2 * wr + (c1 >> 1);     // 16-byte chunk of the x row
    const int xo0 = rA * XROW + ((xch ^ swz<XROW>(rA)) * 16) + cb;
    const int xo1 = (rA + 16) * XROW + ((xch ^ swz<XROW>(rA + 16)) * 16) + cb;
    int bo0[NT], bo1[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        bo0[j] = XB + rA * (2 * NB) + (((2 * j + (c1 >> 1)) ^ swz<2 * NB>(rA)) * 16) + cb;
        bo1[j] = XB + (rA + 16) * (2 * NB) + (((2 * j + (c1 >> 1)) ^ swz<2 * NB>(rA + 16)) * 16) + cb;
    }
    f32x4 acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = zero4();
    // the row swizzle repeats every 8 rows, so step ks is step 0 moved by 32 rows
    for (int ks = ks_lo; ks < ks_hi; ++ks) {
        const float wl = wq[hh * Q + wpos + 32 * ks];
        const float wv[8] = {row_bcast<0>(wl), row_bcast<1>(wl), row_bcast<2>(wl), row_bcast<3>(wl),
                             row_bcast<4>(wl), row_bcast<5>(wl), row_bcast<6>(wl), row_bcast<7>(wl)};
        bf16x8 xh, xlo;
        const bf16x4 x0 = ds_read_tr(xs + xo0 + ks * 32 * XROW);
        const bf16x4 x1 = ds_read_tr(xs + xo1 + ks * 32 * XROW);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float v = (float)(j < 4 ? x0[j] : x1[j - 4]) * wv[j];
            const bf16 hi = (bf16)v;
            xh[j] = hi;
            xlo[j] = (bf16)(v - (float)hi);
        }
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const bf16x4 b0 = ds_read_tr(xs + bo0[j] + ks * 32 * (2 * NB));
            const bf16x4 b1 = ds_read_tr(xs + bo1[j] + ks * 32 * (2 * NB));
            const bf16x8 bf = __builtin_shufflevector(b0, b1, 0, 1, 2, 3, 4, 5, 6, 7);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, xh, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, xlo, acc[j], 0, 0, 0);
        }
    }

    // ---- through LDS (in place of the tiles, once every wavefront is done
    // with them; each wavefront its own 16 rows), then whole rows
    lds_barrier();
    float* const oth = ot + (64 * hh) * OS;          // this head's staging rows
    float* orow = oth + (16 * wr) * OS;
#pragma unroll
    for (int j = 0; j < NT; ++j)
        *reinterpret_cast<f32x4*>(orow + ln * OS + 16 * j + 4 * kg) = acc[j];
    const float cs = !CHUNK && carry ? expf(dA_ref) : 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int r = orr + RPI * it;
        float4 v = *reinterpret_cast<const float4*>(oth + r * OS + occ);
        if (!CHUNK && carry) {
            float cv[4];
            if (a.states_bf16) {
#pragma unroll
                for (int i = 0; i < 4; ++i) cv[i] = (float)cv16[it][i];
            } else {
                cv[0] = cv32[it].x; cv[1] = cv32[it].y; cv[2] = cv32[it].z; cv[3] = cv32[it].w;
            }
            v.x += cs * cv[0]; v.y += cs * cv[1]; v.z += cs * cv[2]; v.w += cs * cv[3];
        }
        // the varlen states are final outputs: non-temporal, so that they
        // leave no dirty lines for the scan that follows them in the combined
        // forward (c3: scan 280 against 262 us)
        if constexpr (CHUNK) *reinterpret_cast<float4*>(op + (int64_t)r * N + occ) = v;
        else __builtin_nontemporal_store(f32x4{v.x, v.y, v.z, v.w}, reinterpret_cast<f32x4*>(op + (int64_t)r * N + occ));
    }
}

// the dstate block width of a launch: 128 columns when dstate allows
int block_cols(int64_t N) { return N % 128 == 0 ? 128 : 64; }

// heads per workgroup: two (sharing the B rows) when a group's heads pair up
// and the tiles of two heads leave room for two workgroups per CU (Q <= 128),
// else one; the M2_KNOB_ONESHOT_HEADS override forces one head (tests)
int heads_per_wg(const VarlenArgs& k) {
    if (m2::dispatch_override(M2_KNOB_ONESHOT_HEADS) == 1) return 1;
    return (k.H / k.G) % 2 == 0 && k.Q <= 128 ? 2 : 1;
}

template <bool CHUNK>
int launch_k(VarlenArgs k, int64_t units, hipStream_t s, const char* who) {
    const int NB = block_cols(k.N);
    const int HPW = heads_per_wg(k);
    const int64_t nwork = units * (k.H / HPW) * k.nblk;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "%s: too many workgroups", who);
    k.nwork = (int)nwork;
    const size_t shm = (size_t)tiles_bytes(k.Q, NB, HPW) + (size_t)HPW * k.Q * 4;
    void (*kern)(VarlenArgs) =
        HPW == 2 ? (NB == 128 ? k_varlen_states<CHUNK, 128, 2> : k_varlen_states<CHUNK, 64, 2>)
                 : (NB == 128 ? k_varlen_states<CHUNK, 128, 1> : k_varlen_states<CHUNK, 64, 1>);
    if (shm > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "%s: cannot reserve %zu B of LDS", who, shm);
    kern<<<(unsigned)k.nwork, 256 * HPW, shm, s>>>(k);
    return m2::check_launch(who);
}

}  // namespace

namespace m2 {

bool varlen_states_fast_supported(const m2_chunk_state_varlen_args& a) {
    return a.dtype == M2_BF16 && a.headdim == P && a.dstate % 64 == 0 &&
           a.chunk_size % 32 == 0 && a.chunk_size <= 256;
}

int launch_varlen_states(const m2_chunk_state_varlen_args& a, hipStream_t s) {
    M2_REQUIRE(varlen_states_fast_supported(a), M2_ERR_UNSUPPORTED,
               "varlen_states: unsupported shape / dtype");
    VarlenArgs k{};
    k.x = (const bf16*)a.x; k.B = (const bf16*)a.B; k.dt = a.dt; k.dA = a.dA_cumsum;
    k.cu = a.cu_seqlens; k.states = a.chunk_states; k.out = a.out;
    k.states_bf16 = a.states_dtype == M2_BF16;
    k.L = (int)a.seqlen; k.H = (int)a.nheads; k.G = (int)a.ngroups; k.N = (int)a.dstate;
    k.Q = (int)a.chunk_size; k.nc = (int)a.nchunks; k.nblk = (int)(a.dstate / block_cols(a.dstate));
    return launch_k<false>(k, a.nseq, s, "varlen_states");
}

bool chunk_state_fast_supported(const m2_chunk_state_args& a) {
    return a.dtype == M2_BF16 && a.headdim == P && a.dstate % 64 == 0 &&
           a.chunk_size % 32 == 0 && a.chunk_size <= 256;
}

int launch_chunk_state_fast(const m2_chunk_state_args& a, hipStream_t s) {
    M2_REQUIRE(chunk_state_fast_supported(a), M2_ERR_UNSUPPORTED,
               "chunk_state: unsupported shape / dtype for the one-shot kernel");
    VarlenArgs k{};
    k.x = (const bf16*)a.x; k.B = (const bf16*)a.B; k.dt = a.dt; k.dA = a.dA_cumsum;
    k.seq = a.seq_idx; k.out = a.states;
    k.L = (int)a.seqlen; k.H = (int)a.nheads; k.G = (int)a.ngroups; k.N = (int)a.dstate;
    k.Q = (int)a.chunk_size; k.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    k.nblk = (int)(a.dstate / block_cols(a.dstate));
    M2_REQUIRE(a.batch * a.seqlen < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_state: too many positions");
    return launch_k<true>(k, a.batch * k.nc, s, "chunk_state");
}

}  // namespace m2
