// rms_norm_gated: RMSNorm over groups of the last dimension with an optional
// SiLU gate, the step after the SSD in a Mamba2 layer:
//   x' = x * silu(z)              (gate before the norm: z given, !norm_before_gate)
//   out = x' / sqrt(mean(x'^2) + eps) * weight
//   out *= silu(z)                (gate after the norm: z given, norm_before_gate)
// per row and group of `group_size` consecutive elements.
//
// HBM-bound (x, z read once, out written once).  One workgroup per (row,
// group): NT threads hold E chunks of CW elements each in registers (CW = 4:
// 16- / 8-byte accesses; CW = 1 for sizes that are not multiples of 4),
// the sum of squares is reduced over the wavefronts in LDS, and the scaled
// values are written from the registers.  Groups longer than NT * E are
// processed in passes (the second pass re-reads x and z from cache).
// With a residual stream (plain RMSNorm of a pre-norm block) the kernel also
// does the block's residual add: res = res + x in float32, stored back, and
// normalises that sum -- one kernel instead of an add and a norm.
// Rounding follows the reference's array dtypes: every intermediate whose
// JAX dtype is bfloat16 is rounded to bf16 (bf16 only when all its operands
// are bf16); silu(z) has z's dtype.
//
// Follows reference ops/rms_norm.py:15-92.
#include "norm_ops.h"

namespace {

using namespace m2norm;

template <int NT>
M2_DEV float block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
    if (NT == 64) return v;
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NT / 64; ++j) s += red[j];
    return s;
}

// NT threads, E CW-element chunks per thread in registers
template <int NT, int E, int CW>
__global__ void __launch_bounds__(NT) k_rms_norm(NormArgs a) {
    __shared__ float red[NT / 64];
    const int64_t blk = blockIdx.x;
    const int64_t row = blk / a.ngroups, g = blk % a.ngroups;
    const int64_t gofs = g * a.gs;
    const char* xr = reinterpret_cast<const char*>(a.x) + (row * a.x_rs + gofs) * (a.x_bf16 ? 2 : 4);
    const char* zr = a.z ? reinterpret_cast<const char*>(a.z) + (row * a.z_rs + gofs) * (a.z_bf16 ? 2 : 4)
                         : nullptr;
    char* orow = reinterpret_cast<char*>(a.out) + (row * a.o_rs + gofs) * (a.o_bf16 ? 2 : 4);
    float* rr = a.res ? a.res + row * a.r_rs + gofs : nullptr;
    const int t = threadIdx.x;
    const int64_t n4 = a.gs / CW;                // chunks in the group
    const bool resident = n4 <= (int64_t)NT * E;

    float v[E][CW], sz[E][CW], wt[E][CW];
    float ss = 0.f;
    if (resident) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int64_t c = (int64_t)e * NT + t;
            if (c < n4) {
                // the weights load with the operands: no second round trip
                ldc<CW>(a.w, gofs + CW * c, a.w_bf16, a.vec, wt[e]);
                operand<CW>(a, xr, zr, rr, CW * c, v[e], sz[e]);
#pragma unroll
                for (int k = 0; k < CW; ++k) ss += a.r_x ? rbf(v[e][k] * v[e][k]) : v[e][k] * v[e][k];
            }
        }
    } else {
        for (int64_t c = t; c < n4; c += NT) {
            float vv[CW], zz[CW];
            operand<CW>(a, xr, zr, rr, CW * c, vv, zz);
#pragma unroll
            for (int k = 0; k < CW; ++k) ss += a.r_x ? rbf(vv[k] * vv[k]) : vv[k] * vv[k];
        }
    }
    const float tot = block_sum<NT>(ss, red);
    float ms = tot / (float)a.gs;
    if (a.r_x) ms = rbf(ms);
    float den = ms + a.eps;
    if (a.r_x) den = rbf(den);
    float rms = sqrtf(den);
    if (a.r_x) rms = rbf(rms);
    const float inv = 1.f / rms;
    if (resident) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
            const int64_t c = (int64_t)e * NT + t;
            if (c < n4) output<CW>(a, orow, CW * c, inv, v[e], sz[e], wt[e]);
        }
    } else {
        for (int64_t c = t; c < n4; c += NT) {
            float vv[CW], zz[CW], ww[CW];
            ldc<CW>(a.w, gofs + CW * c, a.w_bf16, a.vec, ww);
            operand<CW>(a, xr, zr, rr, CW * c, vv, zz, true);
            output<CW>(a, orow, CW * c, inv, vv, zz, ww);
        }
    }
}

}  // namespace

namespace m2 {

using m2norm::NormArgs;

static bool aligned_to(const void* p, int bytes) { return ((uintptr_t)p % bytes) == 0; }


int prepare_norm(const m2_rms_norm_gated_args& a, NormArgs& k, bool& c4, bool to_lds) {
    const char* who = "rms_norm_gated";
    M2_REQUIRE(a.x && a.weight && (a.out || to_lds), M2_ERR_INVALID,
               "%s: x, weight and out are required", who);
    M2_REQUIRE(a.rows > 0 && a.hidden > 0 && a.group_size > 0 && a.hidden % a.group_size == 0,
               M2_ERR_INVALID, "%s: bad sizes (hidden %% group_size must be 0)", who);
    for (int d : {a.x_dtype, a.w_dtype, a.out_dtype})
        M2_REQUIRE(d == M2_F32 || d == M2_BF16, M2_ERR_UNSUPPORTED, "%s: dtype %d", who, d);
    M2_REQUIRE(!a.z || a.z_dtype == M2_F32 || a.z_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "%s: z dtype %d", who, a.z_dtype);
    M2_REQUIRE(!a.residual || !a.z, M2_ERR_INVALID, "%s: a residual stream needs z == NULL", who);
    const bool zb = a.z && a.z_dtype == M2_BF16;
    const bool gate_first = a.z && !a.norm_before_gate, gate_after = a.z && a.norm_before_gate;
    // dtypes of the reference's intermediates (bf16 only when all operands are)
    const bool xdt_bf = a.x_dtype == M2_BF16 && (!gate_first || zb) && !a.residual;
    const bool wdt_bf = xdt_bf && a.w_dtype == M2_BF16;
    const bool odt_bf = wdt_bf && (!gate_after || zb);
    M2_REQUIRE(a.out_dtype == (odt_bf ? M2_BF16 : M2_F32) || a.out_dtype == M2_BF16, M2_ERR_INVALID,
               "%s: out_dtype must be the result dtype %d or bf16", who, odt_bf ? M2_BF16 : M2_F32);
    k = NormArgs{};
    k.x = a.x; k.z = a.z; k.w = a.weight; k.out = a.out;
    k.x_rs = a.x_row_stride; k.z_rs = a.z_row_stride; k.o_rs = a.out_row_stride;
    k.hidden = a.hidden; k.gs = a.group_size; k.ngroups = a.hidden / a.group_size; k.eps = a.eps;
    k.x_bf16 = a.x_dtype == M2_BF16; k.z_bf16 = zb; k.w_bf16 = a.w_dtype == M2_BF16;
    k.o_bf16 = a.out_dtype == M2_BF16;
    k.gate_first = gate_first; k.gate_after = gate_after;
    k.r_x = xdt_bf; k.r_w = wdt_bf; k.r_o = odt_bf;
    k.res = a.residual; k.r_rs = a.residual_row_stride;
    // 4-element chunks: every row and group start a multiple of 4 elements on
    // a 4-element-aligned base, as one access each when also aligned
    const int xs = a.x_dtype == M2_BF16 ? 2 : 4, os = k.o_bf16 ? 2 : 4, ws = a.w_dtype == M2_BF16 ? 2 : 4;
    c4 = a.group_size % 4 == 0 && a.x_row_stride % 4 == 0 && a.out_row_stride % 4 == 0 &&
         (!a.z || a.z_row_stride % 4 == 0) && (!a.residual || a.residual_row_stride % 4 == 0);
    bool vec = c4 && aligned_to(a.x, 4 * xs) && (to_lds || aligned_to(a.out, 4 * os)) &&
               aligned_to(a.weight, 4 * ws) &&
               (!a.residual || aligned_to(a.residual, 16));
    if (a.z) vec = vec && aligned_to(a.z, 4 * (zb ? 2 : 4));
    k.vec = vec;
    return M2_OK;
}

int launch_rms_norm_gated(const m2_rms_norm_gated_args& a, hipStream_t s) {
    const char* who = "rms_norm_gated";
    NormArgs k;
    bool c4;
    if (int rc = prepare_norm(a, k, c4, false)) return rc;
    const int64_t nblocks = a.rows * (a.hidden / a.group_size);
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "%s: too many rows", who);
    const dim3 grid((unsigned)nblocks);
    if (c4) {
        const int64_t n4 = a.group_size / 4;
        if (n4 <= 64 * 4) hipLaunchKernelGGL((k_rms_norm<64, 4, 4>), grid, dim3(64), 0, s, k);
        else if (n4 <= 256 * 2) hipLaunchKernelGGL((k_rms_norm<256, 2, 4>), grid, dim3(256), 0, s, k);
        else if (n4 <= 256 * 4) hipLaunchKernelGGL((k_rms_norm<256, 4, 4>), grid, dim3(256), 0, s, k);
        else hipLaunchKernelGGL((k_rms_norm<256, 8, 4>), grid, dim3(256), 0, s, k);
    } else {
        if (a.group_size <= 64 * 8) hipLaunchKernelGGL((k_rms_norm<64, 8, 1>), grid, dim3(64), 0, s, k);
        else hipLaunchKernelGGL((k_rms_norm<256, 16, 1>), grid, dim3(256), 0, s, k);
    }
    return check_launch(who);
}

}  // namespace m2
