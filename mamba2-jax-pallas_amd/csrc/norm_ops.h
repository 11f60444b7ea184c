// Element operations of rms_norm_gated, shared by the norm kernel and the
// skinny GEMM whose prologue normalises its input rows: the normalised operand
// (x, x * silu(z), or x + residual) and the scaled / gated output of CW
// consecutive elements, with the bf16 rounding points of the reference's
// array dtypes (ops/rms_norm.py:15-92).
#pragma once

#include "m2_internal.h"

namespace m2norm {

struct NormArgs {
    const void* x;
    const void* z;
    const void* w;
    void* out;
    int64_t x_rs, z_rs, o_rs;     // row strides (elements)
    int64_t hidden, gs, ngroups;  // ngroups per row
    float eps;
    int x_bf16, z_bf16, w_bf16, o_bf16;
    int gate_first, gate_after;
    int r_x;                      // the normalised operand (x or x * silu(z)) is bf16
    int r_w;                      // x_normed * weight is bf16
    int r_o;                      // the gated output is bf16
    int vec;                      // 4-element accesses
    float* res;                   // residual stream (x += res; res = x), or NULL
    int64_t r_rs;
};

M2_DEV inline float rbf(float v) { return (float)(bf16)v; }

// silu(v) = v / (1 + e^-v) from the hardware exp2 / reciprocal (~1 ulp each)
M2_DEV inline float silu_fast(float v) {
    const float e = __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.f + e);
}

// CW consecutive elements at i (one 16- / 8-byte access when CW == 4 and vec)
template <int CW> M2_DEV void ldc(const void* p, int64_t i, int is_bf16, int vec, float (&o)[CW]) {
    if constexpr (CW == 1) {
        o[0] = is_bf16 ? (float)reinterpret_cast<const bf16*>(p)[i] : reinterpret_cast<const float*>(p)[i];
        return;
    } else if (is_bf16) {
        const bf16* q = reinterpret_cast<const bf16*>(p) + i;
        if (vec) {
            const bf16x4 r = *reinterpret_cast<const bf16x4*>(q);
            o[0] = (float)r[0]; o[1] = (float)r[1]; o[2] = (float)r[2]; o[3] = (float)r[3];
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = (float)q[k];
        }
    } else {
        const float* q = reinterpret_cast<const float*>(p) + i;
        if (vec) {
            const float4 r = *reinterpret_cast<const float4*>(q);
            o[0] = r.x; o[1] = r.y; o[2] = r.z; o[3] = r.w;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) o[k] = q[k];
        }
    }
}

template <int CW> M2_DEV void stc(void* p, int64_t i, int is_bf16, int vec, const float (&v)[CW]) {
    if constexpr (CW == 1) {
        if (is_bf16) reinterpret_cast<bf16*>(p)[i] = (bf16)v[0];
        else reinterpret_cast<float*>(p)[i] = v[0];
        return;
    } else if (is_bf16) {
        bf16* q = reinterpret_cast<bf16*>(p) + i;
        bf16x4 r;
#pragma unroll
        for (int k = 0; k < 4; ++k) r[k] = (bf16)v[k];
        if (vec) {
            *reinterpret_cast<bf16x4*>(q) = r;
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = r[k];
        }
    } else {
        float* q = reinterpret_cast<float*>(p) + i;
        if (vec) {
            *reinterpret_cast<float4*>(q) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k) q[k] = v[k];
        }
    }
}

// the normalised operand of CW elements at group offset i; with a residual
// stream the first pass adds it in float32 and stores the sum back, a second
// pass (groups longer than the registers hold) reads that sum
template <int CW>
M2_DEV void operand(const NormArgs& a, const void* xr, const void* zr, float* rr, int64_t i,
                    float (&v)[CW], float (&sz)[CW], bool second = false) {
    if (rr && second) {
        ldc<CW>(rr, i, 0, a.vec, v);
    } else {
        ldc<CW>(xr, i, a.x_bf16, a.vec, v);
        if (rr) {
            float r[CW];
            ldc<CW>(rr, i, 0, a.vec, r);
#pragma unroll
            for (int k = 0; k < CW; ++k) v[k] += r[k];
            stc<CW>(rr, i, 0, a.vec, v);
        }
    }
    if (a.gate_first || a.gate_after) {
        ldc<CW>(zr, i, a.z_bf16, a.vec, sz);
#pragma unroll
        for (int k = 0; k < CW; ++k) sz[k] = a.z_bf16 ? rbf(silu_fast(sz[k])) : silu_fast(sz[k]);
    }
    if (a.gate_first) {
#pragma unroll
        for (int k = 0; k < CW; ++k) v[k] = a.r_x ? rbf(v[k] * sz[k]) : v[k] * sz[k];
    }
}

template <int CW>
M2_DEV void output(const NormArgs& a, void* orow, int64_t i, float inv, const float (&v)[CW],
                   const float (&sz)[CW], const float (&wt)[CW]) {
    float o[CW];
#pragma unroll
    for (int k = 0; k < CW; ++k) {
        float xn = v[k] * inv;
        if (a.r_x) xn = rbf(xn);
        float y = xn * wt[k];
        if (a.r_w) y = rbf(y);
        if (a.gate_after) {
            y *= sz[k];
            if (a.r_o) y = rbf(y);
        }
        o[k] = y;
    }
    stc<CW>(orow, i, a.o_bf16, a.vec, o);
}

}  // namespace m2norm

namespace m2 {
// The norm's arguments for these sizes and dtypes (rounding flags as the
// reference's dtype promotion gives them; k.vec set when every access can be
// 4 elements wide); c4: the sizes allow 4-element chunks.  Checks the
// arguments as m2_rms_norm_gated does; to_lds: the caller writes the rows to
// its own LDS (a.out is not used and may be NULL).
int prepare_norm(const m2_rms_norm_gated_args& a, m2norm::NormArgs& k, bool& c4, bool to_lds);
}  // namespace m2
