// The causal conv1d's shared element code: the split outputs, the dtype
// helpers and one channel's decode step (conv of the shifted state row, bias,
// SiLU, with the reference's bf16 rounding points), used by the conv kernels
// and by the in-projection whose epilogue runs a decode step's conv update.
// Follows reference ops/causal_conv1d.py:88-139.
#pragma once

#include "m2_internal.h"

namespace m2conv {

struct Outs {
    void* ptr[3];
    int64_t c_begin[3], sb[3], sd[3], st[3];
    int n;
};

M2_DEV inline float rbf(float v) { return (float)(bf16)v; }

// silu(v) = v / (1 + e^-v) from the hardware base-2 exponential and
// reciprocal (each ~1 ulp; the e^-v argument is rounded once, a relative
// error below |v| 2^-24): a few instructions instead of a full-precision exp
// and division, which dominated this HBM-bound kernel's issue time.  Limits:
// e^-v = inf gives v * 0 = 0, e^-v = 0 gives v.
M2_DEV inline float silu_fast(float v) {
    const float e = __builtin_amdgcn_exp2f(v * -1.4426950408889634f);
    return v * __builtin_amdgcn_rcpf(1.f + e);
}
M2_DEV inline float ldf(const void* p, int64_t i, int is_bf16) {
    return is_bf16 ? (float)reinterpret_cast<const bf16*>(p)[i] : reinterpret_cast<const float*>(p)[i];
}

struct UpdArgs {
    const void* x;
    int64_t xsb;
    const void* state;
    void* nstate;
    const void* w;
    const void* bias;
    Outs o;
    int64_t B, D;
    int x_bf16, w_bf16, bias_bf16, out_bf16;
    int round_prod;             // products and their sum are bf16
    int round_bias;
    int silu;
};

// the conv output of channel c from its new state row s (already rounded to
// the new state's dtype)
template <int K> M2_DEV inline float conv_channel(const UpdArgs& a, const float (&s)[K], int64_t c) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const float p = s[i] * ldf(a.w, c * K + i, a.w_bf16);
        acc += a.round_prod ? rbf(p) : p;
    }
    if (a.round_prod) acc = rbf(acc);
    if (a.bias) acc += ldf(a.bias, c, a.bias_bf16);
    if (a.round_bias) acc = rbf(acc);
    if (a.silu) acc = silu_fast(acc);
    return acc;
}

// output element (b, c) into the split output its channel belongs to
M2_DEV inline void conv_store(const UpdArgs& a, int64_t b, int64_t c, float v) {
    int r = 0;
#pragma unroll
    for (int j = 1; j < 3; ++j)
        if (j < a.o.n && c >= a.o.c_begin[j]) r = j;
    const int64_t o = b * a.o.sb[r] + (c - a.o.c_begin[r]);
    if (a.out_bf16) reinterpret_cast<bf16*>(a.o.ptr[r])[o] = (bf16)v;
    else reinterpret_cast<float*>(a.o.ptr[r])[o] = v;
}

}  // namespace m2conv

namespace m2 {
// The decode conv update's arguments (dtype flags as the reference's
// promotion gives them), checked as m2_causal_conv1d_update does; x_given:
// the caller supplies the new inputs itself (a.x is not used, may be NULL).
int prepare_conv_update(const m2_causal_conv1d_update_args& a, m2conv::UpdArgs& k, bool x_given);
}  // namespace m2
