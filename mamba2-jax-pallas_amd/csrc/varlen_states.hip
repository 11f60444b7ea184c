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
// One workgroup per (chunk or sequence, head, NB-column dstate block), NB =
// 128 when dstate allows (x then enters the CU once per 128 columns instead
// of once per 64), else 64: 4096 chunk states at the nemotron-h-8b shape,
// 3072 varlen states at the packed 47b shape, several per CU, so a one-shot
// kernel hides its latency by occupancy.  The x rows [Q x 64] and the block's B rows [Q x 64] arrive by
// direct global -> LDS loads (16-byte chunks of each 128-byte row
// XOR-swizzled, so the transposed reads hit distinct banks); the weights are
// computed from dA / dt while they are in flight.  Wavefront w owns head-dim
// rows 16 w .. 16 w + 15 and all NB columns (NB / 16 tiles of 16 x 16): it computes
// h^T[n, p] += B^T[n, q] (w x)[q, p] with MFMA operands read through the
// gfx950 LDS transpose read, w x split into hi + lo bf16 parts (near-fp32
// accuracy, as the reference's fp32 einsum).  The result goes through LDS so
// that each output row of NB fp32 (and its carry row) moves as NB / 4 lanes x
// 16 bytes.
//
// Follows reference kernels/chunk_state_fwd.py:104-187 (product), :239-269
// (weights, seq_idx rule) and :448-597 (varlen states).
#include "m2_internal.h"

namespace {

constexpr int THREADS = 256;
constexpr int P = 64;        // head dim
constexpr int CPR = 8;       // 16-byte chunks per 128-byte x row

// 16-byte chunk swizzle of tile row R: for 128-byte rows (x, and B blocks of
// 64 columns) 8 consecutive rows read at one chunk pair land on disjoint
// banks; 256-byte rows (B blocks of 128 columns) start on the same bank, so
// 8 consecutive rows are spread by their low bits.
template <int RB> M2_DEV int swz(int R) { return RB == 128 ? ((R >> 1) & 3) << 1 : (R & 7) << 1; }

// LDS bytes of the x and B tiles, which the output staging [64][NB + 4] fp32
// later reuses
__host__ __device__ inline int tiles_bytes(int Q, int NB) {
    return Q * (P + NB) * 2 > P * (NB + 4) * 4 ? Q * (P + NB) * 2 : P * (NB + 4) * 4;
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

template <bool CHUNK, int NB>
__global__ void __launch_bounds__(THREADS) k_varlen_states(VarlenArgs a) {
    constexpr int OS = NB + 4;                                  // output staging row stride (floats)
    constexpr int NT = NB / 16;                                 // 16-column tiles per wavefront
    constexpr int BCPR = NB / 8;                                // 16-byte chunks per B row
    extern __shared__ __align__(16) char smem[];
    const int Q = a.Q, H = a.H, N = a.N;
    const int XB = Q * P * 2;                                   // x tile bytes
    char* xs = smem;                                            // [Q][64] bf16, then B
    float* ot = reinterpret_cast<float*>(smem);                 // [64][OS], after the tiles
    float* wq = reinterpret_cast<float*>(smem + tiles_bytes(Q, NB)); // [Q]

    const int work = xcd_remap(blockIdx.x, a.nwork);
    const int nb = work % a.nblk;
    const int sh = work / a.nblk;              // (sequence or batch row x chunk) x H + h
    const int h = sh % H;
    const int g = h / (H / a.G);
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    float* op = a.out + ((int64_t)sh * P) * N + NB * nb;

    int c, bi = 0, qlo = 0, qhi;
    bool carry = false;
    if (CHUNK) {
        c = (sh / H) % a.nc;
        bi = (sh / H) / a.nc;
        qhi = min(Q, a.L - c * Q);
    } else {
        const int s = sh / H;
        // clamp malformed boundaries into [0, L] so every access stays in bounds
        const int end = min(max(a.cu[s + 1], 0), a.L);
        const int start = min(max(a.cu[s], 0), end);
        if (end <= start) {                     // empty sequence: zero state
            for (int i = threadIdx.x; i < P * NB / 4; i += THREADS) {
                const int r = i / (NB / 4), c4 = 4 * (i % (NB / 4));
                *reinterpret_cast<float4*>(op + (int64_t)r * N + c4) = make_float4(0.f, 0.f, 0.f, 0.f);
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
    const bf16* xsrc = a.x + (int64_t)h * P;
    const bf16* bsrc = a.B + (int64_t)g * N + NB * nb;
    const uint32_t xl = lds_addr(xs);
    for (int u = w; u < Q * CPR / 64; u += THREADS / 64) {
        const int gi = 64 * u + lane, r = gi / CPR;
        const int64_t t = min(t0 + r, tend);
        const int col = ((gi % CPR) ^ swz<128>(r)) * 8;
        dma16(xsrc + t * H * P + col, xl + 1024 * u);
    }
    for (int u = w; u < Q * BCPR / 64; u += THREADS / 64) {
        const int gi = 64 * u + lane, r = gi / BCPR;
        const int64_t t = min(t0 + r, tend);
        const int col = ((gi % BCPR) ^ swz<2 * NB>(r)) * 8;
        dma16(bsrc + t * a.G * N + col, xl + XB + 1024 * u);
    }

    // ---- the carry rows of this lane's outputs (rows 16 w + RPI it + lane /
    // (NB / 4), columns 4 (lane % (NB / 4)) + i), loaded now so that their
    // latency overlaps the tiles'
    constexpr int LPR = NB / 4;                       // lanes per output row
    constexpr int RPI = 64 / LPR;                     // rows per store instruction
    constexpr int NIT = 16 / RPI;
    const int64_t soff = (((int64_t)c * H + h) * P) * N + NB * nb;
    const int orr = 16 * w + lane / LPR, occ = 4 * (lane % LPR);
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

    // ---- weights (while the tiles are in flight)
    const float* dAp = a.dA + (((int64_t)bi * H + h) * a.nc + c) * Q;
    const float* dtp = a.dt + (((int64_t)bi * H + h) * a.nc + c) * Q;
    const float dA_ref = dAp[qhi - 1];
    const int32_t* seq = CHUNK && a.seq ? a.seq + t0 : nullptr;
    const int se = seq ? seq[qhi - 1] : 0;
    for (int q = threadIdx.x; q < Q; q += THREADS) {
        float v = (q >= qlo && q < qhi) ? expf(fminf(dA_ref - dAp[q], 0.f)) * dtp[q] : 0.f;
        if (seq && q < qhi && (se < 0 || seq[q] != se)) v = 0.f;
        wq[q] = v;
    }
    wait_vmem<0>();
    __syncthreads();

    // ---- acc[j] = h^T tile: lane (ln, kg) holds row p = 16 w + ln, columns
    // n = 16 j + 4 kg + i.  K step ks covers positions 32 ks .. 32 ks + 31:
    // MFMA k index j < 4 is position 32 ks + 4 kg + j, j >= 4 is 16 more.
    const int rA = 4 * kg + (ln >> 2);                // rows read by this lane (+16)
    const int c1 = ln & 3;                            // 8-byte column group of the read
    const int cb = 8 * (c1 & 1);
    const int wpos = (ln & 4 ? 16 : 0) + 4 * kg + (ln & 3);   // k index ln & 7
    const int xo0 = rA * (2 * P) + (((2 * w + (c1 >> 1)) ^ swz<128>(rA)) * 16) + cb;
    const int xo1 = (rA + 16) * (2 * P) + (((2 * w + (c1 >> 1)) ^ swz<128>(rA + 16)) * 16) + cb;
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
    for (int ks = 0; ks < Q / 32; ++ks) {
        const float wl = wq[wpos + 32 * ks];
        const float wv[8] = {row_bcast<0>(wl), row_bcast<1>(wl), row_bcast<2>(wl), row_bcast<3>(wl),
                             row_bcast<4>(wl), row_bcast<5>(wl), row_bcast<6>(wl), row_bcast<7>(wl)};
        bf16x8 xh, xlo;
        const bf16x4 x0 = ds_read_tr(xs + xo0 + ks * 32 * (2 * P));
        const bf16x4 x1 = ds_read_tr(xs + xo1 + ks * 32 * (2 * P));
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
    float* orow = ot + (16 * w) * OS;
#pragma unroll
    for (int j = 0; j < NT; ++j)
        *reinterpret_cast<f32x4*>(orow + ln * OS + 16 * j + 4 * kg) = acc[j];
    const float cs = !CHUNK && carry ? expf(dA_ref) : 0.f;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
        const int r = orr + RPI * it;
        float4 v = *reinterpret_cast<const float4*>(ot + r * OS + occ);
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
        *reinterpret_cast<float4*>(op + (int64_t)r * N + occ) = v;
    }
}

// the dstate block width of a launch: 128 columns when dstate allows
int block_cols(int64_t N) { return N % 128 == 0 ? 128 : 64; }

template <bool CHUNK>
int launch_k(const VarlenArgs& k, hipStream_t s, const char* who) {
    const int NB = block_cols(k.N);
    const size_t shm = (size_t)tiles_bytes(k.Q, NB) + (size_t)k.Q * 4;
    void (*kern)(VarlenArgs) = NB == 128 ? k_varlen_states<CHUNK, 128> : k_varlen_states<CHUNK, 64>;
    if (shm > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "%s: cannot reserve %zu B of LDS", who, shm);
    kern<<<(unsigned)k.nwork, THREADS, shm, s>>>(k);
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
    const int64_t nwork = a.nseq * a.nheads * k.nblk;
    M2_REQUIRE(nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "varlen_states: too many workgroups");
    k.nwork = (int)nwork;
    return launch_k<false>(k, s, "varlen_states");
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
    const int64_t nwork = a.batch * k.nc * a.nheads * k.nblk;
    M2_REQUIRE(nwork < (1ll << 31) && a.batch * a.seqlen < (1ll << 31), M2_ERR_UNSUPPORTED,
               "chunk_state: too many workgroups");
    k.nwork = (int)nwork;
    return launch_k<true>(k, s, "chunk_state");
}

}  // namespace m2
