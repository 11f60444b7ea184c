// Skinny GEMM for the decode step's projections: y[M, N] = x[M, K] W^T (+ bias),
// M <= 64 (the decode batch), bf16 operands, float32 accumulation.
//
// A decode step reads every projection weight once per token, so these
// products are HBM-bound on the weights (M * K * N MACs for 2 * K * N bytes).
// The weights are K-contiguous ([N, K], the layout torch.nn.functional.linear
// takes), so each lane loads 8 consecutive k of one output column as one
// 16-byte access, which is exactly a 16x16x32 bf16 MFMA's B-operand fragment.
// One workgroup per 16 output columns; its 4, 8 or 16 wavefronts (enough for
// ~2048 over the chip) split K and meet in LDS, so every weight byte is read
// once; x (a few KB) comes from the cache.
// MT = ceil(M / 16) row tiles share each weight fragment.
#include "m2_internal.h"

namespace {

constexpr int UNROLL = 4;          // k steps of 32 per load batch (two batches in flight)

struct GemmArgs {
    const bf16* x;
    const bf16* w;
    const void* bias;
    void* y;
    int64_t ldx, ldw, ldy;
    int M, N, K;
    int bias_bf16, y_bf16;
};

// MT 16-row tiles of x, NW wavefronts splitting K
template <int MT, int NW>
__global__ void __launch_bounds__(NW * 64) k_skinny_gemm(GemmArgs a) {
    __shared__ f32x4 red[NW - 1][MT][64];
    const int lane = threadIdx.x & 63, w = wave_id();
    const int n0 = blockIdx.x * 16;
    const int col = lane & 15, kq = (lane >> 4) * 8;   // fragment column / k offset
    const int nb = min(n0 + col, a.N - 1);             // clamped: tail columns are masked on store
    const bf16* wr = a.w + (int64_t)nb * a.ldw;
    // this wavefront's k range, in steps of 32
    const int nsteps = (a.K + 31) / 32;
    const int per = (nsteps + NW - 1) / NW;
    const int s0 = w * per, s1 = min(nsteps, s0 + per);

    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = zero4();
    const bf16x8 zf = {};
    // two load batches (named arrays: register indices must be constants)
    bf16x8 ba[UNROLL], aa[UNROLL][MT], bb[UNROLL], ab[UNROLL][MT];
    auto load = [&](bf16x8 (&bf)[UNROLL], bf16x8 (&af)[UNROLL][MT], int s) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int k = (s + u) * 32 + kq;
            const bool ok = s + u < s1 && k < a.K;
            bf[u] = ok ? *reinterpret_cast<const bf16x8*>(wr + k) : zf;
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const int m = 16 * t + col;
                af[u][t] = ok && m < a.M ? *reinterpret_cast<const bf16x8*>(a.x + (int64_t)m * a.ldx + k)
                                         : zf;
            }
        }
    };
    auto mma = [&](const bf16x8 (&bf)[UNROLL], const bf16x8 (&af)[UNROLL][MT]) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
#pragma unroll
            for (int t = 0; t < MT; ++t)
                acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[u][t], bf[u], acc[t], 0, 0, 0);
    };
    // the next batch's loads are issued before the current batch's MFMAs
    load(ba, aa, s0);
    for (int s = s0; s < s1; s += 2 * UNROLL) {
        if (s + UNROLL < s1) load(bb, ab, s + UNROLL);
        mma(ba, aa);
        if (s + UNROLL >= s1) break;
        if (s + 2 * UNROLL < s1) load(ba, aa, s + 2 * UNROLL);
        mma(bb, ab);
    }
    // K-split partial sums meet in wavefront 0
    if (w > 0) {
#pragma unroll
        for (int t = 0; t < MT; ++t) red[w - 1][t][lane] = acc[t];
    }
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int j = 0; j < NW - 1; ++j) {
            const f32x4 o = red[j][t][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[t][i] += o[i];
        }
    // D layout: lane holds column n0 + (lane & 15), rows 16 t + 4 (lane >> 4) + i
    const int n = n0 + col;
    if (n >= a.N) return;
    float bv = 0.f;
    if (a.bias)
        bv = a.bias_bf16 ? (float)reinterpret_cast<const bf16*>(a.bias)[n]
                         : reinterpret_cast<const float*>(a.bias)[n];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int m = 16 * t + 4 * (lane >> 4) + i;
            if (m < a.M) {
                const float v = acc[t][i] + bv;
                if (a.y_bf16) reinterpret_cast<bf16*>(a.y)[(int64_t)m * a.ldy + n] = (bf16)v;
                else reinterpret_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
            }
        }
}

template <int MT>
void launch_mt(const GemmArgs& k, int64_t ngroups, hipStream_t s) {
    // enough wavefronts to keep the weight stream in flight: >= ~2048 over the
    // chip, each with at least two load batches of k steps
    const int nsteps = (k.K + 31) / 32;
    const dim3 grid((unsigned)ngroups);
    // (16 wavefronts of 1024 threads only for one row tile: more row tiles
    // need more than the 128 registers such a workgroup leaves a lane)
    if (ngroups * 4 >= 2048 || nsteps < 8 * 2 * UNROLL) {
        hipLaunchKernelGGL((k_skinny_gemm<MT, 4>), grid, dim3(4 * 64), 0, s, k);
    } else if constexpr (MT == 1) {
        if (ngroups * 8 >= 2048 || nsteps < 16 * 2 * UNROLL)
            hipLaunchKernelGGL((k_skinny_gemm<1, 8>), grid, dim3(8 * 64), 0, s, k);
        else
            hipLaunchKernelGGL((k_skinny_gemm<1, 16>), grid, dim3(16 * 64), 0, s, k);
    } else {
        hipLaunchKernelGGL((k_skinny_gemm<MT, 8>), grid, dim3(8 * 64), 0, s, k);
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

namespace m2 {

int launch_skinny_gemm(const m2_skinny_gemm_args& a, hipStream_t s) {
    const char* who = "skinny_gemm";
    M2_REQUIRE(a.x && a.w && a.y, M2_ERR_INVALID, "%s: x, w and y are required", who);
    M2_REQUIRE(a.M >= 1 && a.M <= 64 && a.N >= 1 && a.K >= 8, M2_ERR_INVALID,
               "%s: need 1 <= M <= 64, N >= 1, K >= 8 (got %lld, %lld, %lld)", who,
               (long long)a.M, (long long)a.N, (long long)a.K);
    M2_REQUIRE(a.K % 8 == 0 && a.ldx % 8 == 0 && a.ldw % 8 == 0 && a.ldx >= a.K && a.ldw >= a.K &&
                   a.ldy >= a.N && aligned16(a.x) && aligned16(a.w),
               M2_ERR_UNSUPPORTED,
               "%s: K and the x / w row strides must be multiples of 8 elements on 16-byte "
               "aligned bases", who);
    M2_REQUIRE(a.x_dtype == M2_BF16 && a.w_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "%s: x and w must be bf16", who);
    M2_REQUIRE(a.y_dtype == M2_BF16 || a.y_dtype == M2_F32, M2_ERR_UNSUPPORTED, "%s: y dtype %d",
               who, a.y_dtype);
    M2_REQUIRE(!a.bias || a.bias_dtype == M2_BF16 || a.bias_dtype == M2_F32, M2_ERR_UNSUPPORTED,
               "%s: bias dtype %d", who, a.bias_dtype);
    M2_REQUIRE(a.N < (1ll << 35) && a.K < (1 << 30), M2_ERR_UNSUPPORTED, "%s: too large", who);
    GemmArgs k{};
    k.x = reinterpret_cast<const bf16*>(a.x);
    k.w = reinterpret_cast<const bf16*>(a.w);
    k.bias = a.bias; k.y = a.y;
    k.ldx = a.ldx; k.ldw = a.ldw; k.ldy = a.ldy;
    k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
    k.bias_bf16 = a.bias_dtype == M2_BF16; k.y_bf16 = a.y_dtype == M2_BF16;
    const int64_t ng = (a.N + 15) / 16;
    if (a.M <= 16) launch_mt<1>(k, ng, s);
    else if (a.M <= 32) launch_mt<2>(k, ng, s);
    else launch_mt<4>(k, ng, s);
    return check_launch(who);
}

}  // namespace m2
