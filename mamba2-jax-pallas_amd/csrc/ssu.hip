// selective_state_update: one decode token on an fp32 state
//   dt' = softplus?(dt + dt_bias)
//   new[p,n] = state[p,n] * exp(dt' A) + dt' x[p] B[n]
//   y[p] = sum_n new[p,n] C[n] + D x[p];   y *= silu(z[p])
// new goes to a separate tensor or back into state (in place).
//
// HBM-bound: the state (b*H*P*N fp32) is read and written exactly once.  One
// workgroup per (batch, head), or per slice of its rows for small batches
// (enough workgroups to fill the chip); each thread owns 4 consecutive n
// (16-byte accesses) of RPT rows p, issuing all RPT state loads before any
// arithmetic so that RPT x 16 B stay in flight per thread.  The per-row
// operands (dt', x, D x, silu(z)) of the workgroup's rows are loaded and
// prepared into LDS while the state loads are in flight: vmcnt is one in-order
// counter, so a small load issued per row after the state loads would cost a
// memory round trip per row.  The readout over n is a butterfly reduction
// across the N/4 lanes that share a row (a power of two: lanes past N idle).
// dstate that is not a multiple of 4 or above 256 takes k_ssu_gen: one
// wavefront per row, its lanes striding over n.
//
// Follows reference ops/selective_state_update.py:68-123.
#include "m2_internal.h"

namespace {

constexpr int THREADS = 256;

struct SsuArgs {
    const float* state;         // read
    float* new_state;           // written (may equal state)
    const void* x;
    const void* dt;
    const float* A;
    const void* B;
    const void* C;
    const float* D;
    const void* z;
    const float* dt_bias;
    float* out;
    int H, G, P, N;
    int nsl;                    // workgroups (row slices) per (batch, head)
    int64_t rows;               // batch * H * P (k_ssu_gen)
    int dt_bf16, dt_has_hdim, A_full, D_has_hdim, bias_has_hdim, softplus;
};

template <typename T> M2_DEV float ld(const void* p, int64_t i) {
    return to_f32(reinterpret_cast<const T*>(p)[i]);
}

// TPR = threads per row (N / 4), RPT = rows per thread
template <typename T, int TPR, int RPT>
__global__ void __launch_bounds__(THREADS) k_ssu(SsuArgs a) {
    constexpr int ROWS_PER_PASS = THREADS / TPR;
    const int bh = blockIdx.x / a.nsl;
    const int p0 = (blockIdx.x % a.nsl) * (RPT * ROWS_PER_PASS);   // first row of the slice
    const int bi = bh / a.H, h = bh % a.H;
    const int g = h / (a.H / a.G);
    const int P = a.P, N = a.N;
    const int tr = threadIdx.x / TPR;           // row within a pass
    const int n0 = (threadIdx.x % TPR) * 4;
    const bool act = n0 < N;                    // lanes past N (TPR > N / 4) idle
    const float* st = a.state + (int64_t)bh * P * N;
    float* nst = a.new_state + (int64_t)bh * P * N;

    float Bv[4] = {0.f, 0.f, 0.f, 0.f}, Cv[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            Bv[j] = ld<T>(a.B, ((int64_t)bi * a.G + g) * N + n0 + j);
            Cv[j] = ld<T>(a.C, ((int64_t)bi * a.G + g) * N + n0 + j);
        }
    }
    float4 s[RPT];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int p = p0 + r * ROWS_PER_PASS + tr;
        s[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p < P && act) s[r] = *reinterpret_cast<const float4*>(st + (int64_t)p * N + n0);
    }
    // per-row operands of this workgroup's rows, while the state loads are in
    // flight: one memory round trip for the workgroup instead of one per row
    constexpr int NROWS = RPT * ROWS_PER_PASS;
    __shared__ float sd[NROWS], sx[NROWS], sy0[NROWS], sz[NROWS];
    for (int lr = threadIdx.x; lr < NROWS; lr += THREADS) {
        const int p = min(p0 + lr, P - 1);
        const int64_t hp = (int64_t)bh * P + p;
        float d = a.dt_has_hdim ? (a.dt_bf16 ? ld<bf16>(a.dt, hp) : ld<float>(a.dt, hp))
                                : (a.dt_bf16 ? ld<bf16>(a.dt, bh) : ld<float>(a.dt, bh));
        if (a.dt_bias) d += a.bias_has_hdim ? a.dt_bias[h * P + p] : a.dt_bias[h];
        if (a.softplus) d = softplus_f(d);
        const float xv = ld<T>(a.x, hp);
        sd[lr] = d;
        sx[lr] = xv;
        sy0[lr] = a.D ? (a.D_has_hdim ? a.D[h * P + p] : a.D[h]) * xv : 0.f;
        // silu(z) in z's dtype, as the reference (ops/selective_state_update.py:121)
        sz[lr] = a.z ? to_f32(from_f32<T>(silu_f(ld<T>(a.z, hp)))) : 1.f;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        const int p = p0 + r * ROWS_PER_PASS + tr;
        if (p >= P) continue;
        const int64_t hp = (int64_t)bh * P + p;       // (batch, head, p) index
        const int lr = r * ROWS_PER_PASS + tr;
        const float d = sd[lr];
        const float xv = sx[lr];
        const float dx = d * xv;
        float v[4] = {s[r].x, s[r].y, s[r].z, s[r].w};
        float part = 0.f;
        if (a.A_full) {
            const float* Ar = a.A + ((int64_t)h * P + p) * N + (act ? n0 : 0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = v[j] * expf(d * (act ? Ar[j] : 0.f)) + dx * Bv[j];
                part += v[j] * Cv[j];
            }
        } else {
            const float dA = expf(d * a.A[h]);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                v[j] = v[j] * dA + dx * Bv[j];
                part += v[j] * Cv[j];
            }
        }
        if (act)
            *reinterpret_cast<float4*>(nst + (int64_t)p * N + n0) = make_float4(v[0], v[1], v[2], v[3]);
#pragma unroll
        for (int off = TPR / 2; off > 0; off >>= 1) part += __shfl_xor(part, off, TPR);
        if (threadIdx.x % TPR == 0) a.out[hp] = (part + sy0[lr]) * sz[lr];
    }
}

// Any dstate: one wavefront per (batch, head, row p), its lanes striding
// over n (coalesced scalar accesses), the readout a wavefront reduction.  The
// per-row operands are wavefront-uniform loads.
template <typename T>
__global__ void __launch_bounds__(THREADS) k_ssu_gen(SsuArgs a) {
    const int64_t row = (int64_t)blockIdx.x * (THREADS / 64) + threadIdx.x / 64;  // (b, h, p)
    if (row >= a.rows) return;                  // whole wavefronts only
    const int lane = threadIdx.x & 63;
    const int P = a.P, N = a.N;
    const int p = (int)(row % P);
    const int64_t bh = row / P;
    const int h = (int)(bh % a.H), bi = (int)(bh / a.H);
    const int g = h / (a.H / a.G);
    float d = a.dt_has_hdim ? (a.dt_bf16 ? ld<bf16>(a.dt, row) : ld<float>(a.dt, row))
                            : (a.dt_bf16 ? ld<bf16>(a.dt, bh) : ld<float>(a.dt, bh));
    if (a.dt_bias) d += a.bias_has_hdim ? a.dt_bias[h * P + p] : a.dt_bias[h];
    if (a.softplus) d = softplus_f(d);
    const float xv = ld<T>(a.x, row);
    const float dx = d * xv;
    const float dA = a.A_full ? 0.f : expf(d * a.A[h]);
    const float* st = a.state + row * N;
    float* nst = a.new_state + row * N;
    const int64_t bc = ((int64_t)bi * a.G + g) * N;
    const float* Ar = a.A + ((int64_t)h * P + p) * N;
    float part = 0.f;
    for (int n = lane; n < N; n += 64) {
        const float decay = a.A_full ? expf(d * Ar[n]) : dA;
        const float v = st[n] * decay + dx * ld<T>(a.B, bc + n);
        nst[n] = v;
        part += v * ld<T>(a.C, bc + n);
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) part += __shfl_xor(part, off, 64);
    if (lane == 0) {
        const float y0 = a.D ? (a.D_has_hdim ? a.D[h * P + p] : a.D[h]) * xv : 0.f;
        const float sz = a.z ? to_f32(from_f32<T>(silu_f(ld<T>(a.z, row)))) : 1.f;
        a.out[row] = (part + y0) * sz;
    }
}

template <typename T>
int launch_gen(SsuArgs sa, int64_t nblocks, hipStream_t s) {
    sa.rows = nblocks * sa.P;
    const int64_t nwg = (sa.rows + THREADS / 64 - 1) / (THREADS / 64);
    M2_REQUIRE(nwg < (1ll << 31), M2_ERR_UNSUPPORTED, "selective_state_update: too many blocks");
    k_ssu_gen<T><<<(unsigned)nwg, THREADS, 0, s>>>(sa);
    return m2::check_launch("selective_state_update");
}

template <typename T>
int launch_typed(SsuArgs sa, int64_t nblocks, hipStream_t s) {
    // 16-byte rows of <= 64 lanes: dstate a multiple of 4, at most 256
    if (sa.N % 4 != 0 || sa.N > 256) return launch_gen<T>(sa, nblocks, s);
    void (*kern)(SsuArgs) = nullptr;
    int tpr = 1;                                // lanes per row: N / 4 rounded up to 2^k
    while (tpr * 4 < sa.N) tpr *= 2;
    const int rows_per_pass = THREADS / tpr;
    const int rpt_full = (sa.P + rows_per_pass - 1) / rows_per_pass;
    // small batches: split each head's rows over several workgroups so that
    // the step fills the chip (>= 512 workgroups where the rows allow)
    int nsl = 1;
    while (nsl * 2 <= rpt_full && nblocks * nsl < 512) nsl *= 2;
    const int rpt = (rpt_full + nsl - 1) / nsl;
    sa.nsl = nsl;
#define M2_SSU_CASE(TPRV, RPTV) \
    if (tpr == TPRV && rpt <= RPTV && !kern) kern = k_ssu<T, TPRV, RPTV>;
    M2_SSU_CASE(1, 1) M2_SSU_CASE(1, 2) M2_SSU_CASE(1, 4)                        // N <= 4
    M2_SSU_CASE(2, 1) M2_SSU_CASE(2, 2) M2_SSU_CASE(2, 4)                        // N <= 8
    M2_SSU_CASE(4, 1) M2_SSU_CASE(4, 2) M2_SSU_CASE(4, 4)                        // N <= 16
    M2_SSU_CASE(8, 1) M2_SSU_CASE(8, 2) M2_SSU_CASE(8, 4)                        // N <= 32
    M2_SSU_CASE(16, 1) M2_SSU_CASE(16, 2) M2_SSU_CASE(16, 4) M2_SSU_CASE(16, 8)  // N <= 64
    M2_SSU_CASE(32, 1) M2_SSU_CASE(32, 2) M2_SSU_CASE(32, 4) M2_SSU_CASE(32, 8)
    M2_SSU_CASE(32, 16)                                                          // N <= 128
    M2_SSU_CASE(64, 1) M2_SSU_CASE(64, 2) M2_SSU_CASE(64, 4) M2_SSU_CASE(64, 8)
    M2_SSU_CASE(64, 16) M2_SSU_CASE(64, 32)                                      // N <= 256
#undef M2_SSU_CASE
    if (!kern) return launch_gen<T>(sa, nblocks, s);
    const int64_t nwg = nblocks * nsl;
    M2_REQUIRE(nwg < (1ll << 31), M2_ERR_UNSUPPORTED, "selective_state_update: too many blocks");
    kern<<<(unsigned)nwg, THREADS, 0, s>>>(sa);
    return m2::check_launch("selective_state_update");
}

}  // namespace

namespace m2 {

int launch_ssu(const m2_ssu_args& a, hipStream_t s) {
    M2_REQUIRE(a.state && a.x && a.dt && a.A && a.B && a.C && a.out, M2_ERR_INVALID,
               "selective_state_update: state, x, dt, A, B, C and out are required");
    M2_REQUIRE(a.batch > 0 && a.nheads > 0 && a.ngroups > 0 && a.nheads % a.ngroups == 0 &&
                   a.headdim > 0 && a.dstate > 0 && a.headdim * a.dstate < (1ll << 31),
               M2_ERR_INVALID, "selective_state_update: bad sizes");
    M2_REQUIRE(a.dt_dtype == M2_F32 || a.dt_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "selective_state_update: dt dtype %d", a.dt_dtype);
    const int64_t nblocks = a.batch * a.nheads;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "selective_state_update: too many blocks");
    SsuArgs sa{};
    sa.state = a.state; sa.new_state = a.new_state ? a.new_state : a.state;
    sa.x = a.x; sa.dt = a.dt; sa.A = a.A; sa.B = a.B; sa.C = a.C; sa.D = a.D;
    sa.z = a.z; sa.dt_bias = a.dt_bias; sa.out = a.out;
    sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.P = (int)a.headdim; sa.N = (int)a.dstate;
    sa.dt_bf16 = a.dt_dtype == M2_BF16; sa.dt_has_hdim = a.dt_has_hdim; sa.A_full = a.A_full;
    sa.D_has_hdim = a.D_has_hdim; sa.bias_has_hdim = a.dt_bias_has_hdim; sa.softplus = a.dt_softplus;
    if (a.dtype == M2_BF16) return launch_typed<bf16>(sa, nblocks, s);
    if (a.dtype == M2_F32) return launch_typed<float>(sa, nblocks, s);
    return set_error(M2_ERR_UNSUPPORTED, "selective_state_update: dtype %d", a.dtype);
}

}  // namespace m2
