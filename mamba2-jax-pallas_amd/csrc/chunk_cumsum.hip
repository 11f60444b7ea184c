// chunk_cumsum: dt processing + per-chunk inclusive cumsum of dt' * A, and
// (for the fused state pass of the combined forward) the chunk-state weights
//   w[q]  = exp(min(dA[last] - dA[q], 0)) dt'[q]    (0 where seq_idx differs
//           from the chunk's last position, or that id is negative)
//   scl   = exp(dA[Q-1]), 0 where the chunk-end seq_idx differs from the
//           previous chunk's (the previous id of chunk 0 is 0)
// which are the chunk_state scale and the state_passing decay.
//
// One workgroup per (batch, chunk, block of 16 heads), 256 threads: thread
// & 15 is a head, thread >> 4 one of 16 position segments of the chunk.  Each
// thread loads its segment's dt (coalesced across the 16 heads: dt is
// [b, L, H], so one head's positions are H elements apart), processes it
// and sums it sequentially in registers; segment totals meet in
// LDS and each thread adds the totals of the segments before it.  Outputs are
// transposed through LDS so that each row [b, h, c, :] is written by
// consecutive lanes.
//
// Follows reference kernels/chunk_cumsum_fwd.py:213-235 (bias -> softplus ->
// clip -> zero pad) and ops/ssd_naive.py:67-68 (dA = dt' * A, then cumsum);
// the weights and decay follow kernels/chunk_state_fwd.py:239-269 and
// kernels/state_passing_fwd.py:108-151, :208-225.
#include "m2_internal.h"

namespace {

constexpr int HB = 16;                 // heads per workgroup (256 workgroups at H 128, 32 chunks)
constexpr int NSEG = 16;               // position segments per chunk
constexpr int THREADS = HB * NSEG;
constexpr int QMAX = 256;
constexpr int TS = QMAX + 4;          // LDS tile row stride (16-byte rows)

struct CumsumArgs {
    const void* dt;
    const float* A;
    const float* bias;
    const int32_t* seq;       // [b, L] or NULL (weights / decay only)
    float* dA;
    float* dto;
    float* wts;               // [b, H, nc, Q] or NULL
    float* scl;               // [b, H, nc] or NULL
    int L, H, Q, nc, softplus, nhb, nblocks;
    float lo, hi;
};

// QS: positions per segment rounded up to a power of two (>= ceil(Q / 16)).
// Every load is issued unconditionally (addresses clamped into the chunk's
// valid range, results selected afterwards): loads under per-position
// branches would each be waited for on their own.
template <typename TD, int QS, bool VEC>
__global__ void __launch_bounds__(THREADS) k_chunk_cumsum(CumsumArgs a) {
    __shared__ float tot[NSEG][HB];
    __shared__ __align__(16) float tile[3][HB][TS];
    // the head blocks of one (batch, chunk) read the same dt rows: they share
    // an XCD (and its L2)
    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int hb = work % a.nhb, c = (work / a.nhb) % a.nc, bi = work / (a.nhb * a.nc);
    const int hh = threadIdx.x % HB, seg = threadIdx.x / HB;
    const int h = hb * HB + hh;
    const bool hok = h < a.H;
    const int Q = a.Q, L = a.L;
    const int qs = (Q + NSEG - 1) / NSEG;
    const int q0 = seg * qs;
    const int qe = min(q0 + qs, Q);                 // this segment: [q0, qe)
    const int qhi = min(Q, L - c * Q);              // valid positions of the chunk
    const int qv = min(qe, qhi);                    // valid positions of the segment: [q0, qv)
    const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;
    const TD* dtp = reinterpret_cast<const TD*>(a.dt) + tok0 * a.H + min(h, a.H - 1);

    TD raw[QS];
    int sq[QS];
#pragma unroll
    for (int j = 0; j < QS; ++j) raw[j] = dtp[(int64_t)min(q0 + j, qhi - 1) * a.H];
    int se = 0, sprev = 0;
    if (a.seq) {
#pragma unroll
        for (int j = 0; j < QS; ++j) sq[j] = a.seq[tok0 + min(q0 + j, qhi - 1)];
        se = a.seq[tok0 + qhi - 1];
        if (c > 0) sprev = a.seq[tok0 - 1];
    }
    const float Ah = a.A[min(h, a.H - 1)];
    const float bias = a.bias ? a.bias[min(h, a.H - 1)] : 0.f;

    float v[QS], dA[QS];
    float run = 0.f;
#pragma unroll
    for (int j = 0; j < QS; ++j) {
        float d = to_f32(raw[j]);
        if (a.bias) d += bias;
        if (a.softplus) d = softplus_f(d);
        d = fminf(fmaxf(d, a.lo), a.hi);
        v[j] = (hok && q0 + j < qv) ? d : 0.f;
        run += v[j] * Ah;
        dA[j] = run;
    }
    tot[seg][hh] = run;
    __syncthreads();
    // totals summed in segment order: off + (last segment's total) is the
    // same sum as `total`, so dA[Q - 1] == total exactly
    float off = 0.f, total = 0.f;
#pragma unroll
    for (int k = 0; k < NSEG; ++k) {
        const float t = tot[k][hh];
        if (k < seg) off += t;
        total += t;
    }
    // outputs go through LDS [head][position] so that the rows [b, h, c, :]
    // are written by consecutive lanes (16 bytes per lane when VEC)
    const int nout = a.wts ? 3 : 2;
#pragma unroll
    for (int j = 0; j < QS; ++j) {
        const int q = q0 + j;
        if (j < qs && q < qe) {
            const float d = off + dA[j];
            tile[0][hh][q] = d;
            tile[1][hh][q] = v[j];
            if (a.wts) {
                float wv = expf(fminf(total - d, 0.f)) * v[j];
                if (a.seq && (q >= qhi || se < 0 || sq[j] != se)) wv = 0.f;
                tile[2][hh][q] = wv;
            }
        }
    }
    __syncthreads();
    float* outs[3] = {a.dA, a.dto, a.wts};
    const int nh = min(HB, a.H - (int)hb * HB);
    const int64_t row0 = (((int64_t)bi * a.H + hb * HB) * a.nc + c) * Q;
    const int64_t hstride = (int64_t)a.nc * Q;       // between heads' rows
    if (VEC) {
        const int q4n = Q / 4;
        for (int idx = threadIdx.x; idx < nout * nh * q4n; idx += THREADS) {
            const int o = idx / (nh * q4n), rem = idx - o * (nh * q4n);
            const int r = rem / q4n, q = 4 * (rem - r * q4n);
            *reinterpret_cast<float4*>(outs[o] + row0 + r * hstride + q) =
                *reinterpret_cast<const float4*>(&tile[o][r][q]);
        }
    } else {
        for (int idx = threadIdx.x; idx < nout * nh * Q; idx += THREADS) {
            const int o = idx / (nh * Q), rem = idx - o * (nh * Q);
            const int r = rem / Q, q = rem - r * Q;
            outs[o][row0 + r * hstride + q] = tile[o][r][q];
        }
    }
    if (a.scl && seg == 0 && hok) {
        const bool keep = !a.seq || se == sprev;
        a.scl[((int64_t)bi * a.H + h) * a.nc + c] = keep ? expf(total) : 0.f;
    }
}

}  // namespace

namespace m2 {

int launch_chunk_cumsum_ex(const m2_chunk_cumsum_args& a, const int32_t* seq_idx, float* wts,
                           float* scl, hipStream_t s) {
    M2_REQUIRE(a.dt && a.A && a.dA_cumsum && a.dt_out, M2_ERR_INVALID,
               "chunk_cumsum: dt, A, dA_cumsum and dt_out are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.nheads > 0 && a.chunk_size > 0, M2_ERR_INVALID,
               "chunk_cumsum: sizes must be positive");
    M2_REQUIRE(a.chunk_size <= QMAX, M2_ERR_UNSUPPORTED, "chunk_cumsum: chunk_size %lld > %d",
               (long long)a.chunk_size, QMAX);
    CumsumArgs k{};
    k.dt = a.dt; k.A = a.A; k.bias = a.dt_bias; k.seq = seq_idx;
    k.dA = a.dA_cumsum; k.dto = a.dt_out; k.wts = wts; k.scl = scl;
    k.L = (int)a.seqlen; k.H = (int)a.nheads; k.Q = (int)a.chunk_size;
    k.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    k.softplus = a.dt_softplus; k.lo = a.dt_min; k.hi = a.dt_max;
    k.nhb = (int)((a.nheads + HB - 1) / HB);
    const int64_t nblocks = (int64_t)k.nhb * k.nc * a.batch;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_cumsum: too many blocks");
    k.nblocks = (int)nblocks;
    const dim3 grid((unsigned)nblocks);
    if (a.dt_dtype != M2_F32 && a.dt_dtype != M2_BF16)
        return set_error(M2_ERR_UNSUPPORTED, "chunk_cumsum: dt dtype %d", a.dt_dtype);
    const int qs = (k.Q + NSEG - 1) / NSEG;
    const bool f32 = a.dt_dtype == M2_F32;
    // 16-byte row stores need 16-byte aligned outputs and chunk_size % 4 == 0
    const bool vec = k.Q % 4 == 0 && ((uintptr_t)k.dA % 16 == 0) && ((uintptr_t)k.dto % 16 == 0) &&
                     ((uintptr_t)k.wts % 16 == 0);
#define M2_CUMSUM_LAUNCH(QS)                                                          \
    if (vec) {                                                                        \
        if (f32) k_chunk_cumsum<float, QS, true><<<grid, THREADS, 0, s>>>(k);         \
        else k_chunk_cumsum<bf16, QS, true><<<grid, THREADS, 0, s>>>(k);              \
    } else {                                                                          \
        if (f32) k_chunk_cumsum<float, QS, false><<<grid, THREADS, 0, s>>>(k);        \
        else k_chunk_cumsum<bf16, QS, false><<<grid, THREADS, 0, s>>>(k);             \
    }
    if (qs <= 2) { M2_CUMSUM_LAUNCH(2) }
    else if (qs <= 4) { M2_CUMSUM_LAUNCH(4) }
    else if (qs <= 8) { M2_CUMSUM_LAUNCH(8) }
    else { M2_CUMSUM_LAUNCH(16) }
#undef M2_CUMSUM_LAUNCH
    return check_launch("chunk_cumsum");
}

int launch_chunk_cumsum(const m2_chunk_cumsum_args& a, hipStream_t s) {
    return launch_chunk_cumsum_ex(a, nullptr, nullptr, nullptr, s);
}

}  // namespace m2
