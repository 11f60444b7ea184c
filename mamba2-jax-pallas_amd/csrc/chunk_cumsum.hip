// chunk_cumsum: dt processing + per-chunk inclusive cumsum of dt' * A, and
// (for the fused state pass of the combined forward) the chunk-state weights
//   w[q]  = exp(min(dA[last] - dA[q], 0)) dt'[q]    (0 where seq_idx differs
//           from the chunk's last position, or that id is negative)
//   scl   = exp(dA[Q-1]), 0 where the chunk-end seq_idx differs from the
//           previous chunk's (the previous id of chunk 0 is 0)
// which are the chunk_state scale and the state_passing decay.
//
// One workgroup per (batch, chunk, block of 16 heads), 16 wavefronts.  The
// chunk's dt rows for the 16 heads (32 contiguous bytes per position for
// bf16) are loaded coalesced into an LDS tile [position][head]; then
// wavefront w processes head w of the block alone: lane l takes positions
// l, l + 64, ... (PPL = ceil(Q / 64) of them), processes dt, and the
// chunk cumsum is a wavefront prefix scan (one per 64 positions, carried from
// one to the next).  The outputs leave lanes-along-positions, so each store
// instruction writes 256 contiguous bytes of a row [b, h, c, :].  A
// wavefront thus runs a few dozen instructions per position batch instead of
// a serial loop, and 16 wavefronts per CU hide each other's latencies.
//
// Follows reference kernels/chunk_cumsum_fwd.py:213-235 (bias -> softplus ->
// clip -> zero pad) and ops/ssd_naive.py:67-68 (dA = dt' * A, then cumsum);
// the weights and decay follow kernels/chunk_state_fwd.py:239-269 and
// kernels/state_passing_fwd.py:108-151, :208-225.
#include "m2_internal.h"

namespace {

constexpr int HB = 16;                 // heads per workgroup: one wavefront each
constexpr int THREADS = HB * 64;
constexpr int QMAX = 256;

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

// PPL: positions per lane (Q <= 64 PPL); CPW: chunks per workgroup (1, or 2
// where one chunk per workgroup would need more than one round of the CUs:
// all loads of both chunks go out before the first wait, so the two load
// round trips overlap instead of following each other)
template <typename TD, int PPL, int CPW>
__global__ void __launch_bounds__(THREADS) k_chunk_cumsum(CumsumArgs a) {
    __shared__ float tile[CPW][QMAX][HB + 1];  // dt of the chunks, [position][head]
    // the head blocks of one (batch, chunk) read the same dt rows: they share
    // an XCD (and its L2)
    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int ncw = (a.nc + CPW - 1) / CPW;
    const int hb = work % a.nhb, cw = (work / a.nhb) % ncw, bi = work / (a.nhb * ncw);
    const int Q = a.Q, L = a.L, H = a.H;
    const int lane = threadIdx.x & 63, w = wave_id();
    const int h = hb * HB + w;
    // every global load of the workgroup is issued before the first wait:
    // the head's A / bias and the chunks' seq ids, then the dt tiles
    const float Ah = a.A[min(h, H - 1)];
    const float bias = a.bias ? a.bias[min(h, H - 1)] : 0.f;
    int sq[CPW][PPL];
    int se[CPW], sprev[CPW];
    const int hh = threadIdx.x % HB, r0 = threadIdx.x / HB;
    TD raw[CPW][PPL];
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
        // a workgroup's second chunk past the last one repeats the last (its
        // loads stay in bounds; it stores nothing)
        const int c = min(cw * CPW + k, a.nc - 1);
        const int qhi = min(Q, L - c * Q);          // valid positions of the chunk
        const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;
        se[k] = 0; sprev[k] = 0;
        if (a.seq) {
#pragma unroll
            for (int j = 0; j < PPL; ++j) sq[k][j] = a.seq[tok0 + min(lane + 64 * j, qhi - 1)];
            se[k] = a.seq[tok0 + qhi - 1];
            if (c > 0) sprev[k] = a.seq[tok0 - 1];
        }
        // ---- coalesced tile load: thread t -> head t % 16, rows t / 16 + 64 i;
        // addresses clamped into the valid rows / heads (masked below)
        const TD* dtp = reinterpret_cast<const TD*>(a.dt) + tok0 * H + min(hb * HB + hh, H - 1);
#pragma unroll
        for (int i = 0; i < PPL; ++i) raw[k][i] = dtp[(int64_t)min(r0 + 64 * i, qhi - 1) * H];
    }
#pragma unroll
    for (int k = 0; k < CPW; ++k)
#pragma unroll
        for (int i = 0; i < PPL; ++i)
            if (r0 + 64 * i < Q) tile[k][r0 + 64 * i][hh] = to_f32(raw[k][i]);
    __syncthreads();
    if (h >= H) return;                             // no barrier follows
#pragma unroll
    for (int k = 0; k < CPW; ++k) {
    const int c = cw * CPW + k;
    if (c >= a.nc) break;
    const int qhi = min(Q, L - c * Q);

    float v[PPL], dA[PPL];
    float carry = 0.f;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int q = lane + 64 * j;
        float d = q < Q ? tile[k][q][w] : 0.f;
        if (a.bias) d += bias;
        if (a.softplus) d = softplus_f(d);
        d = fminf(fmaxf(d, a.lo), a.hi);
        v[j] = q < qhi ? d : 0.f;
        dA[j] = wave_scan(v[j] * Ah) + carry;
        carry = lane63(dA[j]);
    }
    const float total = carry;                      // == dA[Q - 1] exactly
    float* const rowp = a.dA + (((int64_t)bi * H + h) * a.nc + c) * Q;
    const int64_t off = rowp - a.dA;
#pragma unroll
    for (int j = 0; j < PPL; ++j) {
        const int q = lane + 64 * j;
        if (q >= Q) continue;
        a.dA[off + q] = dA[j];
        a.dto[off + q] = v[j];
        if (a.wts) {
            float wv = expf(fminf(total - dA[j], 0.f)) * v[j];
            if (a.seq && (q >= qhi || se[k] < 0 || sq[k][j] != se[k])) wv = 0.f;
            a.wts[off + q] = wv;
        }
    }
    if (a.scl && lane == 0) {
        const bool keep = !a.seq || se[k] == sprev[k];
        a.scl[((int64_t)bi * H + h) * a.nc + c] = keep ? expf(total) : 0.f;
    }
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
    // two chunks per workgroup where one per workgroup needs more than one
    // round of the CUs (two 16-wavefront workgroups on each of MI355X's 256)
    const int cpw = (int64_t)k.nhb * k.nc * a.batch > 2 * 256 ? 2 : 1;
    const int64_t nblocks = (int64_t)k.nhb * ((k.nc + cpw - 1) / cpw) * a.batch;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_cumsum: too many blocks");
    k.nblocks = (int)nblocks;
    const dim3 grid((unsigned)nblocks);
    if (a.dt_dtype != M2_F32 && a.dt_dtype != M2_BF16)
        return set_error(M2_ERR_UNSUPPORTED, "chunk_cumsum: dt dtype %d", a.dt_dtype);
    const bool f32 = a.dt_dtype == M2_F32;
#define M2_CUMSUM_LAUNCH(PPL)                                                              \
    if (cpw == 2) {                                                                        \
        if (f32) k_chunk_cumsum<float, PPL, 2><<<grid, THREADS, 0, s>>>(k);                \
        else k_chunk_cumsum<bf16, PPL, 2><<<grid, THREADS, 0, s>>>(k);                     \
    } else {                                                                               \
        if (f32) k_chunk_cumsum<float, PPL, 1><<<grid, THREADS, 0, s>>>(k);                \
        else k_chunk_cumsum<bf16, PPL, 1><<<grid, THREADS, 0, s>>>(k);                     \
    }
    if (k.Q <= 64) { M2_CUMSUM_LAUNCH(1) }
    else if (k.Q <= 128) { M2_CUMSUM_LAUNCH(2) }
    else { M2_CUMSUM_LAUNCH(4) }
#undef M2_CUMSUM_LAUNCH
    return check_launch("chunk_cumsum");
}

int launch_chunk_cumsum(const m2_chunk_cumsum_args& a, hipStream_t s) {
    return launch_chunk_cumsum_ex(a, nullptr, nullptr, nullptr, s);
}

}  // namespace m2
