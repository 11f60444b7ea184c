// Skinny GEMM for the decode step's projections: y[M, N] = x[M, K] W^T (+ bias),
// M <= 64 (the decode batch), bf16 operands, float32 accumulation.
//
// A decode step reads every projection weight once per token, so these
// products are HBM-bound on the weights (M * K * N MACs for 2 * K * N bytes).
// The weights are K-contiguous ([N, K], the layout torch.nn.functional.linear
// takes), so each lane loads 8 consecutive k of one output column as one
// 16-byte access, which is exactly a 16x16x32 bf16 MFMA's B-operand fragment.
// One workgroup per 16 output columns (fewer where that leaves CUs idle); its
// 4, 8 or 16 wavefronts (enough for ~2048 over the chip) split K and meet in
// LDS, so every weight byte is read once; x (a few KB) comes from the cache.
// MT = ceil(M / 16) row tiles share each weight fragment.
//
// k_skinny_gemm_norm is the same product for a decode step's first rows
// (M <= 16, M * K <= 32768) whose x is the output of an RMSNorm (optionally SiLU-gated, over
// groups): every workgroup normalises the rows itself into LDS (bf16; a few
// KB read from L2) while its first weight fragments load, so the norm costs no
// launch and no HBM round trip of its output; the epilogue can add the
// (output-dtype rounded) result into a float32 residual stream instead of, or
// besides, storing it -- each output column belongs to one workgroup, so the
// add needs no synchronisation.
#include "conv_ops.h"
#include "norm_ops.h"

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
    int cw;                 // output columns per workgroup (<= 16)
};

// MT 16-row tiles of x, NW wavefronts splitting K
template <int MT, int NW>
__global__ void __launch_bounds__(NW * 64) k_skinny_gemm(GemmArgs a) {
    __shared__ f32x4 red[NW - 1][MT][64];
    const int lane = threadIdx.x & 63, w = wave_id();
    const int n0 = blockIdx.x * a.cw;
    const int col = lane & 15, kq = (lane >> 4) * 8;   // fragment column / k offset
    const bool colok = col < a.cw;                     // lanes past cw load and store nothing
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
            bf[u] = ok && colok ? *reinterpret_cast<const bf16x8*>(wr + k) : zf;
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
    if (!colok || n >= a.N) return;
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

constexpr int NORM_MAXM = 16;       // rows of the normalising GEMM (one row tile)
constexpr int NORM_MAXG = 8;        // norm groups per row
constexpr int NORM_MAXX = 32768;    // normalised elements (M x K) held in LDS

struct NormGemmArgs {
    m2conv::UpdArgs cv;     // conv update of columns [conv_lo, conv_lo + cv.D) (CONV)
    int64_t conv_lo;
    m2norm::NormArgs n;     // the rows to normalise (out unused: they go to LDS)
    const bf16* w;
    const void* bias;
    void* y;
    float* res;
    int64_t ldw, ldy, r_rs;
    int M, N, K;
    int bias_bf16, y_bf16;
    int cw;                 // output columns per workgroup (<= 16)
};

template <int NW, bool CONV>
__global__ void __launch_bounds__(NW * 64) k_skinny_gemm_norm(NormGemmArgs a) {
    extern __shared__ __align__(16) bf16 xs[];          // [M][K] normalised rows
    __shared__ f32x4 red[NW - 1][64];
    __shared__ float part[NW][NORM_MAXM * NORM_MAXG];    // per-wavefront sums of squares
    const int lane = threadIdx.x & 63, w = wave_id();
    const int n0 = blockIdx.x * a.cw;
    const int col = lane & 15, kq = (lane >> 4) * 8;
    const bool colok = col < a.cw;                     // lanes past cw load and store nothing
    const int nb = min(n0 + col, a.N - 1);
    const bf16* wr = a.w + (int64_t)nb * a.ldw;
    const int K = a.K, M = a.M;
    const int nsteps = (K + 31) / 32;
    const int per = (nsteps + NW - 1) / NW;
    const int s0 = w * per, s1 = min(nsteps, s0 + per);
    const bf16x8 zf = {};
    bf16x8 ba[UNROLL], bb[UNROLL];
    // the weights are read once per decode step: non-temporal loads leave the
    // cache to the rows and the states (LM decode at batch 1, A/B on one box:
    // 130m 0.506 -> 0.465 ms, 2.7b 2.550 -> 2.517 ms per token; the same in
    // k_skinny_gemm took the 2.7b step at batch 16 from 5.15 to 5.33 ms)
    auto loadw = [&](bf16x8 (&bf)[UNROLL], int s) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int k = (s + u) * 32 + kq;
            bf[u] = s + u < s1 && k < K && colok
                        ? __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(wr + k)) : zf;
        }
    };
    // the first two weight batches are in flight while the rows are normalised
    // (LM decode at batch 1, A/B on one box: 130m 0.467 -> 0.448 ms per token,
    // 2.7b 2.522 -> 2.533; with only the first batch early the 130m step keeps
    // most of its prologue wait)
    loadw(ba, s0);
    loadw(bb, s0 + UNROLL);

    // ---- the rows' RMSNorm (as k_rms_norm: same operand / output rounding)
    const m2norm::NormArgs& na = a.n;
    const int G = (int)na.ngroups, gs = (int)na.gs, n4 = gs / 4, NT = NW * 64;
    auto rows = [&](int m, int g, const char*& xr, const char*& zr) {
        xr = reinterpret_cast<const char*>(na.x) + ((int64_t)m * na.x_rs + (int64_t)g * gs) * (na.x_bf16 ? 2 : 4);
        zr = na.z ? reinterpret_cast<const char*>(na.z) + ((int64_t)m * na.z_rs + (int64_t)g * gs) * (na.z_bf16 ? 2 : 4)
                  : nullptr;
    };
    for (int m = 0; m < M; ++m)
        for (int g = 0; g < G; ++g) {
            const char *xr, *zr;
            rows(m, g, xr, zr);
            float ss = 0.f;
            for (int c = threadIdx.x; c < n4; c += NT) {
                float v[4], sz[4];
                m2norm::operand<4>(na, xr, zr, nullptr, 4 * c, v, sz);
#pragma unroll
                for (int k = 0; k < 4; ++k) ss += na.r_x ? m2norm::rbf(v[k] * v[k]) : v[k] * v[k];
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off);
            if (lane == 0) part[w][m * G + g] = ss;
        }
    __syncthreads();
    for (int m = 0; m < M; ++m)
        for (int g = 0; g < G; ++g) {
            float tot = 0.f;
#pragma unroll
            for (int j = 0; j < NW; ++j) tot += part[j][m * G + g];
            float ms = tot / (float)gs;
            if (na.r_x) ms = m2norm::rbf(ms);
            float den = ms + na.eps;
            if (na.r_x) den = m2norm::rbf(den);
            float rms = sqrtf(den);
            if (na.r_x) rms = m2norm::rbf(rms);
            const float inv = 1.f / rms;
            const char *xr, *zr;
            rows(m, g, xr, zr);
            for (int c = threadIdx.x; c < n4; c += NT) {
                float v[4], sz[4], wt[4];
                m2norm::ldc<4>(na.w, (int64_t)g * gs + 4 * c, na.w_bf16, na.vec, wt);
                m2norm::operand<4>(na, xr, zr, nullptr, 4 * c, v, sz);
                m2norm::output<4>(na, xs + m * K + g * gs, 4 * c, inv, v, sz, wt);
            }
        }
    __syncthreads();

    // ---- y = x' W^T: A fragments from LDS (rows >= M are zero)
    f32x4 acc = zero4();
    auto mma = [&](const bf16x8 (&bf)[UNROLL], int s) {
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int k = (s + u) * 32 + kq;
            const bf16x8 af = s + u < s1 && k < K && col < M
                                  ? *reinterpret_cast<const bf16x8*>(xs + col * K + k) : zf;
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bf[u], acc, 0, 0, 0);
        }
    };
    for (int s = s0; s < s1; s += 2 * UNROLL) {
        if (s > s0 && s + UNROLL < s1) loadw(bb, s + UNROLL);
        mma(ba, s);
        if (s + UNROLL >= s1) break;
        if (s + 2 * UNROLL < s1) loadw(ba, s + 2 * UNROLL);
        mma(bb, s + UNROLL);
    }
    if (w > 0) red[w - 1][lane] = acc;
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int j = 0; j < NW - 1; ++j) {
        const f32x4 o = red[j][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += o[i];
    }
    const int n = n0 + col;
    if (!colok || n >= a.N) return;
    float bv = 0.f;
    if (a.bias)
        bv = a.bias_bf16 ? (float)reinterpret_cast<const bf16*>(a.bias)[n]
                         : reinterpret_cast<const float*>(a.bias)[n];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = 4 * (lane >> 4) + i;
        if (m < M) {
            float v = acc[i] + bv;
            if (a.y_bf16) v = (float)(bf16)v;        // the output dtype, also for the residual add
            if (CONV && n >= a.conv_lo && n < a.conv_lo + a.cv.D) {
                // the decode conv update of this column's channel (width 4, f32
                // state in place): each (row, channel) belongs to this lane only
                const int64_t c = n - a.conv_lo;
                float* st = reinterpret_cast<float*>(a.cv.nstate) + ((int64_t)m * a.cv.D + c) * 4;
                const float4 o = *reinterpret_cast<const float4*>(st);
                const float sv[4] = {o.y, o.z, o.w, v};
                *reinterpret_cast<float4*>(st) = make_float4(sv[0], sv[1], sv[2], sv[3]);
                m2conv::conv_store(a.cv, m, c, m2conv::conv_channel<4>(a.cv, sv, c));
                continue;
            }
            if (a.y) {
                if (a.y_bf16) reinterpret_cast<bf16*>(a.y)[(int64_t)m * a.ldy + n] = (bf16)v;
                else reinterpret_cast<float*>(a.y)[(int64_t)m * a.ldy + n] = v;
            }
            if (a.res) a.res[(int64_t)m * a.r_rs + n] += v;
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

// Output columns per workgroup: 16 (a full MFMA tile) when that gives at
// least one workgroup per CU, else as few as spread the columns over every CU
// (at least 4): the weight stream then comes in through all the CUs instead
// of a few, e.g. the 2.7b out-projection (N 2560: 160 workgroups of 16
// columns) as 256 workgroups of 10.  MFMA lanes past cw carry zeros.
int cols_per_wg(int64_t N) {
    const int64_t cus = m2::cu_count();
    if ((N + 15) / 16 >= cus) return 16;
    const int64_t cw = (N + cus - 1) / cus;
    return (int)(cw < 4 ? 4 : cw > 16 ? 16 : cw);
}

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
    k.cw = cols_per_wg(a.N);
    const int64_t ng = (a.N + k.cw - 1) / k.cw;
    if (a.M <= 16) launch_mt<1>(k, ng, s);
    else if (a.M <= 32) launch_mt<2>(k, ng, s);
    else launch_mt<4>(k, ng, s);
    return check_launch(who);
}

int launch_skinny_gemm_norm(const m2_skinny_gemm_norm_args& a, hipStream_t s) {
    const char* who = "skinny_gemm_norm";
    M2_REQUIRE(a.x && a.norm_weight && a.w && (a.y || a.residual), M2_ERR_INVALID,
               "%s: x, norm_weight, w and y or residual are required", who);
    M2_REQUIRE(a.M >= 1 && a.M <= NORM_MAXM && a.N >= 1 && a.K >= 8 && a.M * a.K <= NORM_MAXX,
               M2_ERR_UNSUPPORTED, "%s: need 1 <= M <= %d, M * K <= %d (got %lld, %lld)", who,
               NORM_MAXM, NORM_MAXX, (long long)a.M, (long long)a.K);
    M2_REQUIRE(a.group_size > 0 && a.K % a.group_size == 0 && a.K / a.group_size <= NORM_MAXG,
               M2_ERR_UNSUPPORTED, "%s: K / group_size must be a whole number <= %d", who, NORM_MAXG);
    M2_REQUIRE(a.K % 8 == 0 && a.ldw % 8 == 0 && a.ldw >= a.K && aligned16(a.w) && a.w_dtype == M2_BF16,
               M2_ERR_UNSUPPORTED, "%s: w must be bf16 [N, K] with 16-byte aligned rows", who);
    M2_REQUIRE(!a.y || ((a.y_dtype == M2_BF16 || a.y_dtype == M2_F32) && a.ldy >= a.N),
               M2_ERR_UNSUPPORTED, "%s: y dtype %d", who, a.y_dtype);
    M2_REQUIRE(!a.bias || a.bias_dtype == M2_BF16 || a.bias_dtype == M2_F32, M2_ERR_UNSUPPORTED,
               "%s: bias dtype %d", who, a.bias_dtype);
    M2_REQUIRE(!a.residual || a.residual_row_stride >= a.N, M2_ERR_INVALID,
               "%s: residual row stride", who);
    M2_REQUIRE(a.N < (1ll << 31), M2_ERR_UNSUPPORTED, "%s: too large", who);
    // the norm as m2_rms_norm_gated sees it, storing bf16 (the LDS rows)
    m2_rms_norm_gated_args na{};
    na.x = a.x; na.z = a.z; na.weight = a.norm_weight;
    na.x_row_stride = a.x_row_stride; na.z_row_stride = a.z_row_stride; na.out_row_stride = a.K;
    na.rows = a.M; na.hidden = a.K; na.group_size = a.group_size; na.eps = a.eps;
    na.x_dtype = a.x_dtype; na.z_dtype = a.z_dtype; na.w_dtype = a.norm_weight_dtype;
    na.out_dtype = M2_BF16; na.norm_before_gate = a.norm_before_gate;
    NormGemmArgs k{};
    bool c4;
    if (int rc = prepare_norm(na, k.n, c4, true)) return rc;
    M2_REQUIRE(c4 && k.n.vec, M2_ERR_UNSUPPORTED,
               "%s: the rows need 4-element aligned groups, strides and bases", who);
    k.n.out = nullptr;
    k.w = reinterpret_cast<const bf16*>(a.w); k.bias = a.bias; k.y = a.y; k.res = a.residual;
    k.ldw = a.ldw; k.ldy = a.ldy; k.r_rs = a.residual_row_stride;
    k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
    // y_dtype is the rounding of the result also when only the residual is written
    M2_REQUIRE(a.y_dtype == M2_BF16 || a.y_dtype == M2_F32, M2_ERR_UNSUPPORTED, "%s: y dtype %d",
               who, a.y_dtype);
    k.bias_bf16 = a.bias_dtype == M2_BF16; k.y_bf16 = a.y_dtype == M2_BF16;
    k.cw = cols_per_wg(a.N);
    const int64_t ng = (a.N + k.cw - 1) / k.cw;
    const int nsteps = (int)((a.K + 31) / 32);
    k.conv_lo = -1;
    if (a.with_conv) {
        const m2_causal_conv1d_update_args& c = a.conv;
        M2_REQUIRE(c.width == 4 && c.state_dtype == M2_F32 && c.new_state == c.conv_state &&
                       c.batch == a.M && a.conv_begin >= 0 && a.conv_begin + c.dim <= a.N &&
                       c.x_dtype == a.y_dtype && aligned16(c.conv_state),
                   M2_ERR_UNSUPPORTED, "%s: the conv update needs width 4, an f32 state updated in "
                   "place, batch M, x_dtype == y_dtype and columns inside N", who);
        if (int rc = prepare_conv_update(c, k.cv, true)) return rc;
        k.conv_lo = a.conv_begin;
    }
    const size_t shm = (size_t)a.M * a.K * 2;
    const dim3 grid((unsigned)ng);
    const bool cv = a.with_conv;
    // as the plain product: enough wavefronts to keep the weight stream in flight
    if (ng * 4 >= 2048 || nsteps < 8 * 2 * UNROLL) {
        if (cv) hipLaunchKernelGGL((k_skinny_gemm_norm<4, true>), grid, dim3(4 * 64), shm, s, k);
        else hipLaunchKernelGGL((k_skinny_gemm_norm<4, false>), grid, dim3(4 * 64), shm, s, k);
    } else if (ng * 8 >= 2048 || nsteps < 16 * 2 * UNROLL) {
        if (cv) hipLaunchKernelGGL((k_skinny_gemm_norm<8, true>), grid, dim3(8 * 64), shm, s, k);
        else hipLaunchKernelGGL((k_skinny_gemm_norm<8, false>), grid, dim3(8 * 64), shm, s, k);
    } else {
        if (cv) hipLaunchKernelGGL((k_skinny_gemm_norm<16, true>), grid, dim3(16 * 64), shm, s, k);
        else hipLaunchKernelGGL((k_skinny_gemm_norm<16, false>), grid, dim3(16 * 64), shm, s, k);
    }
    return check_launch(who);
}

}  // namespace m2
