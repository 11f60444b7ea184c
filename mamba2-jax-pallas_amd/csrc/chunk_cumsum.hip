// chunk_cumsum: dt processing + per-chunk inclusive cumsum of dt' * A.
//
// One workgroup per (batch, chunk, block of 32 heads).  The [Q x 32] dt tile
// is read row by row (coalesced along heads), processed (bias, softplus,
// clamp; 0 past the end of the sequence) into LDS, then each wavefront scans
// whole heads: 64 lanes take 64 consecutive positions, a 6-step shuffle scan
// per 64-position segment plus a carried running sum.  Stores of dA_cumsum and
// dt_out are contiguous along positions.
//
// Follows reference kernels/chunk_cumsum_fwd.py:213-235 (bias -> softplus ->
// clip -> zero pad) and ops/ssd_naive.py:67-68 (dA = dt' * A, then cumsum).
#include "m2_internal.h"

namespace {

constexpr int HB = 32;        // heads per workgroup
constexpr int THREADS = 256;

template <typename TD>
__global__ void __launch_bounds__(THREADS)
k_chunk_cumsum(const TD* __restrict__ dt, const float* __restrict__ A,
               const float* __restrict__ bias, float* __restrict__ dA_cs,
               float* __restrict__ dt_out, int L, int H, int Q, int nc,
               int softplus, float lo, float hi) {
    extern __shared__ float tile[];  // [Q][HB + 1]
    const int hb = blockIdx.x * HB, c = blockIdx.y, bi = blockIdx.z;
    const int nh = min(HB, H - hb);
    for (int idx = threadIdx.x; idx < Q * HB; idx += THREADS) {
        const int q = idx / HB, hh = idx % HB;
        const int t = c * Q + q;
        float v = 0.f;
        if (hh < nh && t < L) {
            v = to_f32(dt[((size_t)bi * L + t) * H + hb + hh]);
            if (bias) v += bias[hb + hh];
            if (softplus) v = softplus_f(v);
            v = fminf(fmaxf(v, lo), hi);
        }
        tile[q * (HB + 1) + hh] = v;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int hh = w; hh < nh; hh += THREADS / 64) {
        const float a = A[hb + hh];
        const size_t base = (((size_t)bi * H + hb + hh) * nc + c) * Q;
        float carry = 0.f;
        for (int q0 = 0; q0 < Q; q0 += 64) {
            const int q = q0 + lane;
            const float v = q < Q ? tile[q * (HB + 1) + hh] : 0.f;
            float incl = v * a;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float o = __shfl_up(incl, off, 64);
                if (lane >= off) incl += o;
            }
            if (q < Q) {
                dA_cs[base + q] = carry + incl;
                dt_out[base + q] = v;
            }
            carry += __shfl(incl, 63, 64);
        }
    }
}

}  // namespace

namespace m2 {

int launch_chunk_cumsum(const m2_chunk_cumsum_args& a, hipStream_t s) {
    M2_REQUIRE(a.dt && a.A && a.dA_cumsum && a.dt_out, M2_ERR_INVALID,
               "chunk_cumsum: dt, A, dA_cumsum and dt_out are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.nheads > 0 && a.chunk_size > 0, M2_ERR_INVALID,
               "chunk_cumsum: sizes must be positive");
    M2_REQUIRE(a.chunk_size <= 256, M2_ERR_UNSUPPORTED, "chunk_cumsum: chunk_size %lld > 256",
               (long long)a.chunk_size);
    const int Q = (int)a.chunk_size;
    const int nc = (int)((a.seqlen + Q - 1) / Q);
    dim3 grid((unsigned)((a.nheads + HB - 1) / HB), (unsigned)nc, (unsigned)a.batch);
    const size_t shm = (size_t)Q * (HB + 1) * sizeof(float);
    if (a.dt_dtype == M2_F32) {
        k_chunk_cumsum<float><<<grid, THREADS, shm, s>>>(
            (const float*)a.dt, a.A, a.dt_bias, a.dA_cumsum, a.dt_out, (int)a.seqlen,
            (int)a.nheads, Q, nc, a.dt_softplus, a.dt_min, a.dt_max);
    } else if (a.dt_dtype == M2_BF16) {
        k_chunk_cumsum<bf16><<<grid, THREADS, shm, s>>>(
            (const bf16*)a.dt, a.A, a.dt_bias, a.dA_cumsum, a.dt_out, (int)a.seqlen,
            (int)a.nheads, Q, nc, a.dt_softplus, a.dt_min, a.dt_max);
    } else {
        return set_error(M2_ERR_UNSUPPORTED, "chunk_cumsum: dt dtype %d", a.dt_dtype);
    }
    return check_launch("chunk_cumsum");
}

}  // namespace m2
