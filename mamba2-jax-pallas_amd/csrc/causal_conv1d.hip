// causal_conv1d (prefill) and causal_conv1d_update (decode): depthwise causal
// convolution over time with optional bias and SiLU, as in Mamba2's xBC path.
//
//   xm[s] = x[s], zeroed (seq_idx given) when seq_idx[s + j] != seq_idx[s + j - 1]
//           for some 1 <= j < width with s + j < L
//   y[t]  = sum_{i < width} w[c, i] xm[t - width + 1 + i]      (xm = 0 for s < 0)
//   out   = silu?(round(y) + bias[c])
//
// Both kernels are HBM-bound streams (width multiply-adds per element read).
//
// Prefill, channels-last (x[b, t, c] with unit channel stride: the layout the
// in-projection produces): k_conv_walk.  Lane -> a 16-byte vector of
// channels, wavefront -> a run of TT tokens; the thread walks its run keeping
// the last width - 1 inputs in registers, so each input is read once (plus a
// width - 1 token halo per run) and every wavefront access is 64 x 16 bytes
// contiguous.  The output channels may go to up to three tensors (x, B and C
// of the SSD in their own contiguous layouts), chosen per thread.
// Prefill, channels-first (x[b, c, t] with unit time stride: the reference
// tests' layout): k_conv_cf.  Wavefront -> one channel (its weights are
// scalar loads), lane -> a 16-byte vector of tokens; the width - 1 halo
// inputs are the tail of the previous vector (a cache hit).
// Any other strides run k_conv_walk with one channel per lane.
//
// Decode: k_conv_update, one thread per (batch, channel): the state row
// (width elements, contiguous) is read and written once.
//
// Follows reference ops/causal_conv1d.py:18-85 (causal_conv1d), :88-139
// (causal_conv1d_update) and :142-193 (the sequence-boundary mask).
#include <type_traits>

#include "conv_ops.h"

namespace {

using namespace m2conv;

constexpr int THREADS = 256;
constexpr int TT = 16;          // tokens per wavefront in k_conv_walk
constexpr int GRP = 4;          // tokens per load group (two groups in flight)
constexpr int MAXW = 8;         // largest conv width


struct ConvArgs {
    const void* x;
    int64_t xsb, xsd, xst;
    const void* w;
    const void* bias;
    const int32_t* seq;
    Outs o;
    int64_t B, D, L;
    int w_bf16, bias_bf16;
    int round_conv;             // the conv result is bf16 (x and weight bf16)
    int round_bias;             // the bias sum is bf16 (x, weight and bias bf16)
    int silu;
    int w_vec, bias_vec;        // a thread's weights / bias load as 16-byte vectors
    int64_t nwork, ncv, nrun;   // work decomposition
};



// the reference's mask: keep x[s] iff seq[s] == seq[s + 1] == ... == seq[s + K - 1]
// (positions past the end compare equal)
template <int K> M2_DEV bool keep_pos(const int32_t* sq, int64_t s, int64_t L) {
    bool k = true;
#pragma unroll
    for (int j = 1; j < K; ++j)
        if (s + j < L) k = k && sq[s + j] == sq[s + j - 1];
    return k;
}

// conv sums -> outputs: rounding of a bf16 conv result, bias, rounding of a
// bf16 sum, silu (flags uniform over the launch)
template <int N> M2_DEV void finish(float (&y)[N], const float (&bias)[N], const ConvArgs& a) {
    if (a.round_conv) {
#pragma unroll
        for (int v = 0; v < N; ++v) y[v] = rbf(y[v]);
    }
#pragma unroll
    for (int v = 0; v < N; ++v) y[v] += bias[v];
    if (a.round_bias) {
#pragma unroll
        for (int v = 0; v < N; ++v) y[v] = rbf(y[v]);
    }
    if (a.silu) {
#pragma unroll
        for (int v = 0; v < N; ++v) y[v] = silu_fast(y[v]);
    }
}

// N consecutive f32 / bf16 values at element offset `off` of p, as 16-byte
// loads when `vec` (the host sets it only when every such row is 16-byte
// aligned and a whole number of vectors)
template <int N> M2_DEV void load_row(const void* p, int64_t off, int is_bf16, int vec, float (&o)[N]) {
    if (vec && is_bf16) {
        if constexpr (N % 8 == 0) {
            const bf16x8* q = reinterpret_cast<const bf16x8*>(reinterpret_cast<const bf16*>(p) + off);
#pragma unroll
            for (int j = 0; j < N / 8; ++j) {
                const bf16x8 r = q[j];
#pragma unroll
                for (int i = 0; i < 8; ++i) o[8 * j + i] = (float)r[i];
            }
            return;
        }
    } else if (vec) {
        if constexpr (N % 4 == 0) {
            const f32x4* q = reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(p) + off);
#pragma unroll
            for (int j = 0; j < N / 4; ++j) {
                const f32x4 r = q[j];
#pragma unroll
                for (int i = 0; i < 4; ++i) o[4 * j + i] = r[i];
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = ldf(p, off + i, is_bf16);
}

// VEC values of type T, loaded as one 16-byte access when VEC > 1 and kept in
// the loaded form until used
template <typename T, int VEC> struct Vec { typedef T type; };
template <> struct Vec<bf16, 8> { typedef bf16x8 type; };
template <> struct Vec<float, 4> { typedef f32x4 type; };

template <typename T, int VEC> M2_DEV typename Vec<T, VEC>::type load_raw(const T* p) {
    static_assert(VEC == 1 || VEC * sizeof(T) == 16, "16-byte vectors");
    return *reinterpret_cast<const typename Vec<T, VEC>::type*>(p);
}
template <typename R> M2_DEV float elem(const R& r, int i) {
    if constexpr (std::is_same<R, bf16>::value || std::is_same<R, float>::value) return to_f32(r);
    else return (float)r[i];
}
template <typename T, int VEC> M2_DEV void load_vec(const T* p, float (&v)[VEC]) {
    const auto r = load_raw<T, VEC>(p);
#pragma unroll
    for (int i = 0; i < VEC; ++i) v[i] = elem(r, i);
}

template <typename TO, int VEC> M2_DEV void store_vec(TO* p, const float (&v)[VEC]) {
    if constexpr (VEC == 1) {
        p[0] = from_f32<TO>(v[0]);
    } else if constexpr (std::is_same<TO, bf16>::value) {
        bf16x8 r;
#pragma unroll
        for (int i = 0; i < 8; ++i) r[i] = (bf16)v[i];
        *reinterpret_cast<bf16x8*>(p) = r;
    } else {
#pragma unroll
        for (int i = 0; i < VEC; i += 4)
            *reinterpret_cast<float4*>(p + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
    }
}

// ---------------------------------------------------------------------------
// prefill, channel-vector lanes walking a token run
// ---------------------------------------------------------------------------
template <typename T, typename TO, int VEC, int K, bool SEQ>
__global__ void __launch_bounds__(THREADS) k_conv_walk(ConvArgs a) {
    // work id -> (batch, 64-lane channel block, 4 x TT token block), token
    // blocks of one channel block on one XCD (their halos stay in its L2)
    const int64_t wid = xcd_remap(blockIdx.x, (int)a.nwork);
    const int64_t run = wid % a.nrun;
    const int64_t rest = wid / a.nrun;
    const int64_t cblk = rest % a.ncv;
    const int64_t b = rest / a.ncv;
    const int lane = threadIdx.x & 63;
    const int64_t c0 = (cblk * 64 + lane) * VEC;
    const int64_t t_begin = (run * (THREADS / 64) + wave_id()) * TT;
    if (t_begin >= a.L) return;                         // uniform over the wavefront
    const int64_t t_end = min(t_begin + TT, a.L);
    const int32_t* sq = SEQ ? a.seq + b * a.L : nullptr;
    // keep mask of positions t_begin - K + 1 .. t_begin + TT - 1 (bit s - t_begin + K - 1)
    uint64_t keepm = ~0ull;
    if (SEQ) {
        const int64_t s = t_begin - (K - 1) + lane;
        const bool kp = lane >= TT + K - 1 || s < 0 || s >= a.L || keep_pos<K>(sq, s, a.L);
        keepm = __ballot(kp);
    }
    if (c0 >= a.D) return;

    float wl[VEC * K], w[K][VEC], bs[VEC];
    load_row<VEC * K>(a.w, c0 * K, a.w_bf16, a.w_vec, wl);
#pragma unroll
    for (int v = 0; v < VEC; ++v)
#pragma unroll
        for (int i = 0; i < K; ++i) w[i][v] = wl[v * K + i];
    if (a.bias) {
        load_row<VEC>(a.bias, c0, a.bias_bf16, a.bias_vec, bs);
    } else {
#pragma unroll
        for (int v = 0; v < VEC; ++v) bs[v] = 0.f;
    }
    int r = 0;
#pragma unroll
    for (int j = 1; j < 3; ++j)
        if (j < a.o.n && c0 >= a.o.c_begin[j]) r = j;
    TO* op = reinterpret_cast<TO*>(a.o.ptr[r]) + b * a.o.sb[r] + (c0 - a.o.c_begin[r]) * a.o.sd[r];
    const int64_t ost = a.o.st[r];
    const T* xp = reinterpret_cast<const T*>(a.x) + b * a.xsb + c0 * a.xsd;

    // window: inputs at t - K + 1 .. t - 1 (masked)
    float win[K > 1 ? K - 1 : 1][VEC];
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
        const int64_t s = t_begin - (K - 1) + i;
        const bool kp = s >= 0 && (!SEQ || ((keepm >> i) & 1));
        if (s >= 0) load_vec<T, VEC>(xp + s * a.xst, win[i]);
#pragma unroll
        for (int v = 0; v < VEC; ++v) win[i][v] = kp ? win[i][v] : 0.f;
    }
    // groups of GRP tokens, the next group's loads in flight during the
    // current group's arithmetic and stores
    typedef typename Vec<T, VEC>::type RawT;
    RawT raw[GRP], nxt[GRP];
#pragma unroll
    for (int g = 0; g < GRP; ++g)
        if (t_begin + g < t_end) raw[g] = load_raw<T, VEC>(xp + (t_begin + g) * a.xst);
    for (int64_t t0 = t_begin; t0 < t_end; t0 += GRP) {
#pragma unroll
        for (int g = 0; g < GRP; ++g)
            if (t0 + GRP + g < t_end) nxt[g] = load_raw<T, VEC>(xp + (t0 + GRP + g) * a.xst);
#pragma unroll
        for (int g = 0; g < GRP; ++g) {
            if (t0 + g >= t_end) break;
            float cur[VEC];
            const bool kp = !SEQ || ((keepm >> (t0 + g - t_begin + K - 1)) & 1);
#pragma unroll
            for (int v = 0; v < VEC; ++v) cur[v] = kp ? elem(raw[g], v) : 0.f;
            float y[VEC];
#pragma unroll
            for (int v = 0; v < VEC; ++v) {
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < K - 1; ++i) acc = fmaf(w[i][v], win[i][v], acc);
                y[v] = fmaf(w[K - 1][v], cur[v], acc);
            }
            finish(y, bs, a);
            store_vec<TO, VEC>(op + (t0 + g) * ost, y);
#pragma unroll
            for (int i = 0; i + 1 < K - 1; ++i)
#pragma unroll
                for (int v = 0; v < VEC; ++v) win[i][v] = win[i + 1][v];
            if (K > 1) {
#pragma unroll
                for (int v = 0; v < VEC; ++v) win[K > 1 ? K - 2 : 0][v] = cur[v];
            }
        }
#pragma unroll
        for (int g = 0; g < GRP; ++g) raw[g] = nxt[g];
    }
}

// ---------------------------------------------------------------------------
// prefill, channels-first: wavefront -> one (batch, channel) and NV steps of
// 64 consecutive token vectors (one 64 x 16-byte access per step); the
// channel's weights and bias are wavefront-uniform (scalar loads); the halo
// of a vector is the tail of the previous one (loaded again: a cache hit)
// ---------------------------------------------------------------------------
constexpr int NV = 4;

template <typename T, typename TO, int VT, int K, bool SEQ>
__global__ void __launch_bounds__(THREADS) k_conv_cf(ConvArgs a) {
    constexpr int NP = K > 1 ? (K - 2) / VT + 1 : 0;   // previous vectors the halo spans
    const int64_t nvec = (a.L + VT - 1) / VT;
    const int64_t wv = (int64_t)blockIdx.x * (THREADS / 64) + wave_id();
    if (wv >= a.nwork) return;                         // uniform over the wavefront
    const int64_t seg = wv % a.nrun, rest = wv / a.nrun;
    const int64_t c = rest % a.D, b = rest / a.D;
    const int lane = threadIdx.x & 63;
    const T* xp = reinterpret_cast<const T*>(a.x) + b * a.xsb + c * a.xsd;
    const int32_t* sq = SEQ ? a.seq + b * a.L : nullptr;
    int r = 0;
#pragma unroll
    for (int j = 1; j < 3; ++j)
        if (j < a.o.n && c >= a.o.c_begin[j]) r = j;
    TO* op = reinterpret_cast<TO*>(a.o.ptr[r]) + b * a.o.sb[r] + (c - a.o.c_begin[r]) * a.o.sd[r];
    float w[K];
#pragma unroll
    for (int i = 0; i < K; ++i) w[i] = ldf(a.w, c * K + i, a.w_bf16);
    float bs[VT];
    const float b1 = a.bias ? ldf(a.bias, c, a.bias_bf16) : 0.f;
#pragma unroll
    for (int j = 0; j < VT; ++j) bs[j] = b1;

#pragma unroll
    for (int step = 0; step < NV; ++step) {
        const int64_t vi = (seg * NV + step) * 64 + lane;
        if (vi >= nvec) break;
        const int64_t t0 = vi * VT;
        // e[0 .. K-2]: inputs t0 - K + 1 .. t0 - 1; e[K-1 ..]: the vector's tokens
        float e[K - 1 + VT];
        const bool full = t0 + VT <= a.L;
        if (full) {
            float v[VT];
            load_vec<T, VT>(xp + t0, v);
#pragma unroll
            for (int i = 0; i < VT; ++i) e[K - 1 + i] = v[i];
        } else {
#pragma unroll
            for (int i = 0; i < VT; ++i) e[K - 1 + i] = t0 + i < a.L ? to_f32(xp[t0 + i]) : 0.f;
        }
#pragma unroll
        for (int pv = 0; pv < NP; ++pv) {
            // previous vector vi - 1 - pv covers e[K-1 - VT (pv + 1) ..]
            float v[VT];
            if (t0 - VT * (pv + 1) >= 0) {
                load_vec<T, VT>(xp + t0 - VT * (pv + 1), v);
            } else {
#pragma unroll
                for (int i = 0; i < VT; ++i) v[i] = 0.f;
            }
#pragma unroll
            for (int i = 0; i < VT; ++i) {
                const int ei = K - 1 - VT * (pv + 1) + i;
                if (ei >= 0 && ei < K - 1) e[ei] = v[i];
            }
        }
        if (SEQ) {
#pragma unroll
            for (int i = 0; i < K - 1 + VT; ++i) {
                const int64_t s = t0 - (K - 1) + i;
                if (s >= 0 && s < a.L && !keep_pos<K>(sq, s, a.L)) e[i] = 0.f;
            }
        }
        float y[VT];
#pragma unroll
        for (int j = 0; j < VT; ++j) {
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < K; ++i) acc = fmaf(w[i], e[j + i], acc);
            y[j] = acc;
        }
        finish(y, bs, a);
        if (full) {
            store_vec<TO, VT>(op + t0, y);
        } else {
#pragma unroll
            for (int j = 0; j < VT; ++j)
                if (t0 + j < a.L) op[t0 + j] = from_f32<TO>(y[j]);
        }
    }
}

// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------

template <typename TS, typename TN, int K>
__global__ void __launch_bounds__(THREADS) k_conv_update(UpdArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * THREADS + threadIdx.x;
    if (idx >= a.B * a.D) return;
    const int64_t c = idx % a.D, b = idx / a.D;
    const TS* sp = reinterpret_cast<const TS*>(a.state) + idx * K;
    float s[K];
#pragma unroll
    for (int i = 0; i + 1 < K; ++i) s[i] = to_f32(sp[i + 1]);
    s[K - 1] = ldf(a.x, b * a.xsb + c, a.x_bf16);
    // every read of the row is done before the (possibly in-place) write
    TN* np = reinterpret_cast<TN*>(a.nstate) + idx * K;
#pragma unroll
    for (int i = 0; i < K; ++i) {
        const TN v = from_f32<TN>(s[i]);
        s[i] = to_f32(v);
        np[i] = v;
    }
    conv_store(a, b, c, conv_channel<K>(a, s, c));
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

int result_dtype(int x, int w, int bias_or_neg) {
    const bool bf = x == M2_BF16 && w == M2_BF16 && (bias_or_neg < 0 || bias_or_neg == M2_BF16);
    return bf ? M2_BF16 : M2_F32;
}

// checks the output ranges; fills o
int take_outs(const m2_conv_out* out, int nout, int64_t D, Outs& o, const char* who) {
    M2_REQUIRE(nout >= 1 && nout <= 3, M2_ERR_INVALID, "%s: nout must be 1..3 (got %d)", who, nout);
    M2_REQUIRE(out[0].c_begin == 0, M2_ERR_INVALID, "%s: out[0].c_begin must be 0", who);
    o.n = nout;
    for (int j = 0; j < 3; ++j) {
        const int jj = j < nout ? j : nout - 1;
        M2_REQUIRE(out[jj].ptr, M2_ERR_INVALID, "%s: out[%d].ptr is NULL", who, jj);
        if (j > 0 && j < nout)
            M2_REQUIRE(out[j].c_begin > out[j - 1].c_begin && out[j].c_begin < D, M2_ERR_INVALID,
                       "%s: out[%d].c_begin must be ascending and < dim", who, j);
        o.ptr[j] = out[jj].ptr;
        o.c_begin[j] = out[jj].c_begin;
        o.sb[j] = out[jj].stride_batch;
        o.sd[j] = out[jj].stride_dim;
        o.st[j] = out[jj].stride_time;
    }
    return M2_OK;
}

template <typename T, typename TO, int VEC, bool SEQ, int K>
void go_walk(const ConvArgs& a, hipStream_t s) {
    hipLaunchKernelGGL((k_conv_walk<T, TO, VEC, K, SEQ>), dim3(a.nwork), dim3(THREADS), 0, s, a);
}
template <typename T, typename TO, int VT, bool SEQ, int K>
void go_cf(const ConvArgs& a, hipStream_t s) {
    const int64_t waves_per_block = THREADS / 64;
    hipLaunchKernelGGL((k_conv_cf<T, TO, VT, K, SEQ>),
                       dim3((unsigned)((a.nwork + waves_per_block - 1) / waves_per_block)),
                       dim3(THREADS), 0, s, a);
}

#define M2_CONV_WIDTHS(fn, T, TO, V, SEQ)                          \
    switch (width) {                                               \
        case 1: fn<T, TO, V, SEQ, 1>(a, s); break;                 \
        case 2: fn<T, TO, V, SEQ, 2>(a, s); break;                 \
        case 3: fn<T, TO, V, SEQ, 3>(a, s); break;                 \
        case 4: fn<T, TO, V, SEQ, 4>(a, s); break;                 \
        case 5: fn<T, TO, V, SEQ, 5>(a, s); break;                 \
        case 6: fn<T, TO, V, SEQ, 6>(a, s); break;                 \
        case 7: fn<T, TO, V, SEQ, 7>(a, s); break;                 \
        default: fn<T, TO, V, SEQ, 8>(a, s); break;                \
    }

enum Path { WALK_VEC, WALK_1, CF_VEC, CF_1 };

template <typename T, typename TO, bool SEQ>
void dispatch(Path p, int width, const ConvArgs& a, hipStream_t s) {
    constexpr int V = 16 / sizeof(T);
    switch (p) {
        case WALK_VEC: M2_CONV_WIDTHS(go_walk, T, TO, V, SEQ); break;
        case WALK_1: M2_CONV_WIDTHS(go_walk, T, TO, 1, SEQ); break;
        case CF_VEC: M2_CONV_WIDTHS(go_cf, T, TO, V, SEQ); break;
        case CF_1: M2_CONV_WIDTHS(go_cf, T, TO, 1, SEQ); break;
    }
}

template <typename T, typename TO>
void dispatch_seq(bool seq, Path p, int width, const ConvArgs& a, hipStream_t s) {
    if (seq) dispatch<T, TO, true>(p, width, a, s);
    else dispatch<T, TO, false>(p, width, a, s);
}

}  // namespace

namespace m2 {

int launch_causal_conv1d(const m2_causal_conv1d_args& a, hipStream_t s) {
    const char* who = "causal_conv1d";
    M2_REQUIRE(a.x && a.weight, M2_ERR_INVALID, "%s: x and weight are required", who);
    M2_REQUIRE(a.batch > 0 && a.dim > 0 && a.seqlen > 0, M2_ERR_INVALID, "%s: bad sizes", who);
    M2_REQUIRE(a.width >= 1 && a.width <= MAXW, M2_ERR_UNSUPPORTED,
               "%s: width must be 1..%d (got %lld)", who, MAXW, (long long)a.width);
    M2_REQUIRE(a.x_dtype == M2_F32 || a.x_dtype == M2_BF16, M2_ERR_UNSUPPORTED, "%s: x dtype %d", who, a.x_dtype);
    M2_REQUIRE(a.w_dtype == M2_F32 || a.w_dtype == M2_BF16, M2_ERR_UNSUPPORTED, "%s: weight dtype %d", who, a.w_dtype);
    M2_REQUIRE(!a.bias || a.bias_dtype == M2_F32 || a.bias_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "%s: bias dtype %d", who, a.bias_dtype);
    const int rdt = result_dtype(a.x_dtype, a.w_dtype, a.bias ? a.bias_dtype : -1);
    M2_REQUIRE(a.out_dtype == rdt, M2_ERR_INVALID,
               "%s: out_dtype must be the result dtype %d (bf16 only when x, weight and bias are bf16)",
               who, rdt);
    ConvArgs k{};
    int rc = take_outs(a.out, a.nout, a.dim, k.o, who);
    if (rc) return rc;
    k.x = a.x; k.xsb = a.x_stride_batch; k.xsd = a.x_stride_dim; k.xst = a.x_stride_time;
    k.w = a.weight; k.bias = a.bias; k.seq = a.seq_idx;
    k.B = a.batch; k.D = a.dim; k.L = a.seqlen;
    k.w_bf16 = a.w_dtype == M2_BF16; k.bias_bf16 = a.bias_dtype == M2_BF16;
    k.round_conv = a.x_dtype == M2_BF16 && a.w_dtype == M2_BF16;
    k.round_bias = a.bias && rdt == M2_BF16;
    k.silu = a.silu != 0;

    const int xs = (int)m2_dtype_size(a.x_dtype), os = (int)m2_dtype_size(rdt);
    const int V = 16 / xs;
    // path: channel vectors (unit channel stride everywhere), token vectors
    // (unit time stride everywhere), or one channel per lane (any strides)
    bool cl = a.x_stride_dim == 1 && a.dim % V == 0 && a.x_stride_batch % V == 0 &&
              a.x_stride_time % V == 0 && aligned16(a.x);
    bool cf = a.x_stride_time == 1 && a.x_stride_batch % V == 0 && a.x_stride_dim % V == 0 &&
              aligned16(a.x);
    for (int j = 0; j < a.nout; ++j) {
        const m2_conv_out& o = a.out[j];
        cl = cl && o.stride_dim == 1 && o.c_begin % V == 0 && o.stride_batch % V == 0 &&
             o.stride_time % V == 0 && aligned16(o.ptr) && (V * os) % 16 == 0;
        cf = cf && o.stride_time == 1 && o.stride_batch % V == 0 && o.stride_dim % V == 0 &&
             aligned16(o.ptr) && (V * os) % 16 == 0;
    }
    bool unit_time = a.x_stride_time == 1;
    for (int j = 0; j < a.nout; ++j) unit_time = unit_time && a.out[j].stride_time == 1;
    Path p;
    if (cl) p = WALK_VEC;
    else if (cf) p = CF_VEC;
    else if (unit_time) p = CF_1;
    else p = WALK_1;
    if (p == WALK_VEC || p == WALK_1) {
        // workgroups over (batch, 64 channel vectors, 4 x TT tokens)
        const int vec = p == WALK_VEC ? V : 1;
        const int64_t ncv = ((a.dim + vec - 1) / vec + 63) / 64;
        const int64_t nrun = (a.seqlen + (THREADS / 64) * TT - 1) / ((THREADS / 64) * TT);
        k.nwork = a.batch * ncv * nrun; k.ncv = ncv; k.nrun = nrun;
        M2_REQUIRE(k.nwork < (1ll << 31), M2_ERR_UNSUPPORTED, "%s: too many workgroups", who);
        // a thread's vec * width weights / vec biases as 16-byte vectors
        const int ws = (int)m2_dtype_size(a.w_dtype), bsz = (int)m2_dtype_size(a.bias_dtype);
        k.w_vec = aligned16(a.weight) && (vec * a.width * ws) % 16 == 0;
        k.bias_vec = a.bias && aligned16(a.bias) && (vec * bsz) % 16 == 0;
    } else {
        // wavefronts over (batch, channel, NV x 64 token vectors)
        const int vt = p == CF_VEC ? V : 1;
        const int64_t nvec = (a.seqlen + vt - 1) / vt;
        k.nrun = (nvec + 64 * NV - 1) / (64 * NV);
        k.nwork = a.batch * a.dim * k.nrun;
        M2_REQUIRE(k.nwork / (THREADS / 64) < (1ll << 31), M2_ERR_UNSUPPORTED,
                   "%s: too many workgroups", who);
    }
    const int width = (int)a.width;
    const bool seq = a.seq_idx != nullptr;
    if (a.x_dtype == M2_BF16) {
        if (rdt == M2_BF16) dispatch_seq<bf16, bf16>(seq, p, width, k, s);
        else dispatch_seq<bf16, float>(seq, p, width, k, s);
    } else {
        dispatch_seq<float, float>(seq, p, width, k, s);
    }
    return check_launch(who);
}

int prepare_conv_update(const m2_causal_conv1d_update_args& a, UpdArgs& k, bool x_given) {
    const char* who = "causal_conv1d_update";
    M2_REQUIRE((a.x || x_given) && a.conv_state && a.new_state && a.weight, M2_ERR_INVALID,
               "%s: x, conv_state, new_state and weight are required", who);
    M2_REQUIRE(a.batch > 0 && a.dim > 0, M2_ERR_INVALID, "%s: bad sizes", who);
    M2_REQUIRE(a.width >= 1 && a.width <= MAXW, M2_ERR_UNSUPPORTED,
               "%s: width must be 1..%d (got %lld)", who, MAXW, (long long)a.width);
    for (int d : {a.x_dtype, a.state_dtype, a.w_dtype})
        M2_REQUIRE(d == M2_F32 || d == M2_BF16, M2_ERR_UNSUPPORTED, "%s: dtype %d", who, d);
    M2_REQUIRE(!a.bias || a.bias_dtype == M2_F32 || a.bias_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "%s: bias dtype %d", who, a.bias_dtype);
    const int nsdt = a.state_dtype == M2_BF16 && a.x_dtype == M2_BF16 ? M2_BF16 : M2_F32;
    M2_REQUIRE(a.new_state_dtype == nsdt, M2_ERR_INVALID,
               "%s: new_state_dtype must be %d (bf16 only when conv_state and x are bf16)", who, nsdt);
    M2_REQUIRE(a.new_state != a.conv_state || nsdt == a.state_dtype, M2_ERR_INVALID,
               "%s: in-place update needs new_state_dtype == state_dtype", who);
    const int pdt = nsdt == M2_BF16 && a.w_dtype == M2_BF16 ? M2_BF16 : M2_F32;
    const int rdt = pdt == M2_BF16 && (!a.bias || a.bias_dtype == M2_BF16) ? M2_BF16 : M2_F32;
    M2_REQUIRE(a.out_dtype == rdt, M2_ERR_INVALID, "%s: out_dtype must be the result dtype %d",
               who, rdt);
    k = UpdArgs{};
    int rc = take_outs(a.out, a.nout, a.dim, k.o, who);
    if (rc) return rc;
    for (int j = 0; j < a.nout; ++j)
        M2_REQUIRE(a.out[j].stride_dim == 1, M2_ERR_INVALID, "%s: out[%d].stride_dim must be 1", who, j);
    k.x = a.x; k.xsb = a.x_stride_batch; k.state = a.conv_state; k.nstate = a.new_state;
    k.w = a.weight; k.bias = a.bias; k.B = a.batch; k.D = a.dim;
    k.x_bf16 = a.x_dtype == M2_BF16; k.w_bf16 = a.w_dtype == M2_BF16;
    k.bias_bf16 = a.bias_dtype == M2_BF16; k.out_bf16 = rdt == M2_BF16;
    k.round_prod = pdt == M2_BF16; k.round_bias = a.bias && rdt == M2_BF16; k.silu = a.silu != 0;
    return M2_OK;
}

int launch_causal_conv1d_update(const m2_causal_conv1d_update_args& a, hipStream_t s) {
    const char* who = "causal_conv1d_update";
    UpdArgs k;
    if (int rc = prepare_conv_update(a, k, false)) return rc;
    const int nsdt = a.state_dtype == M2_BF16 && a.x_dtype == M2_BF16 ? M2_BF16 : M2_F32;
    const int64_t n = a.batch * a.dim;
    M2_REQUIRE((n + THREADS - 1) / THREADS < (1ll << 31), M2_ERR_UNSUPPORTED, "%s: too many workgroups", who);
    const dim3 grid((unsigned)((n + THREADS - 1) / THREADS));
#define M2_UPD(TS, TN)                                                                             \
    switch (a.width) {                                                                             \
        case 1: hipLaunchKernelGGL((k_conv_update<TS, TN, 1>), grid, dim3(THREADS), 0, s, k); break; \
        case 2: hipLaunchKernelGGL((k_conv_update<TS, TN, 2>), grid, dim3(THREADS), 0, s, k); break; \
        case 3: hipLaunchKernelGGL((k_conv_update<TS, TN, 3>), grid, dim3(THREADS), 0, s, k); break; \
        case 4: hipLaunchKernelGGL((k_conv_update<TS, TN, 4>), grid, dim3(THREADS), 0, s, k); break; \
        case 5: hipLaunchKernelGGL((k_conv_update<TS, TN, 5>), grid, dim3(THREADS), 0, s, k); break; \
        case 6: hipLaunchKernelGGL((k_conv_update<TS, TN, 6>), grid, dim3(THREADS), 0, s, k); break; \
        case 7: hipLaunchKernelGGL((k_conv_update<TS, TN, 7>), grid, dim3(THREADS), 0, s, k); break; \
        default: hipLaunchKernelGGL((k_conv_update<TS, TN, 8>), grid, dim3(THREADS), 0, s, k); break; \
    }
    if (a.state_dtype == M2_BF16) {
        if (nsdt == M2_BF16) { M2_UPD(bf16, bf16) } else { M2_UPD(bf16, float) }
    } else {
        M2_UPD(float, float)
    }
#undef M2_UPD
    return check_launch(who);
}

}  // namespace m2
