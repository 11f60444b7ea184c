// chunk_state: per-chunk SSM states
//   states[b,c,h][p,n] = sum_q w[q] x[q,p] B[q,n],  w[q] = exp(min(dA[last]-dA[q],0)) dt[q]
// and its variable-length twin (the final state of each packed sequence).
//
// One workgroup per (b, c, h) (per (sequence, h) for varlen), 8 wavefronts.
// The contraction runs over chunk positions q, the outer (row) dimension of
// both x [.., L, H, P] and B [.., L, G, N] in HBM, so x and B rows are staged
// through LDS with coalesced 16-byte loads and the MFMA fragments (8
// consecutive positions per lane for bf16) are gathered from LDS; the decay
// weight w[q] is applied to the x operand as it is gathered, and for bf16 the
// weighted operand is split into hi + lo bf16 parts (two MFMAs) so that the
// states keep near-fp32 accuracy, as the reference's fp32 einsum does.  Positions are
// processed in blocks of KB rows to bound LDS.  Wavefront w owns half of the
// P/16 row tiles (w >> 2) and N/64 of the 16-column tiles (w & 3): the
// [P x N] fp32 accumulators live in VGPRs and are written once.
//
// Follows reference kernels/chunk_state_fwd.py:104-187 (product), :239-269
// (scale and seq_idx rule), :448-597 (varlen) and ops/ssd_naive.py:77-128.
#include "m2_internal.h"

namespace {

constexpr int THREADS = 512;         // 8 wavefronts: two per SIMD

// LDS row padding (elements) so that the 4 k-groups of a fragment gather hit
// different banks.
template <typename T> struct Pad;
template <> struct Pad<bf16> { static constexpr int v = 2; static constexpr int KB = 128; };
template <> struct Pad<float> { static constexpr int v = 16; static constexpr int KB = 64; };

// Copy `nrows` rows of W elements (row r at src + r * stride) into LDS rows of
// stride S; rows >= valid are zero.  16-byte global loads, 4-byte LDS stores.
template <typename T>
M2_DEV void stage_rows(T* __restrict__ dst, int S, const T* __restrict__ src,
                       int64_t stride, int nrows, int valid, int W) {
    constexpr int VE = 16 / sizeof(T);
    const int vpr = W / VE;
    const int total = nrows * vpr;
    for (int base = threadIdx.x; base < total; base += 4 * THREADS) {
        uint4 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = base + u * THREADS;
            const int r = idx / vpr, cv = idx % vpr;
            v[u] = make_uint4(0, 0, 0, 0);
            if (idx < total && r < valid)
                v[u] = *reinterpret_cast<const uint4*>(src + r * stride + cv * VE);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int idx = base + u * THREADS;
            if (idx < total) {
                const int r = idx / vpr, cv = idx % vpr;
                uint32_t* d = reinterpret_cast<uint32_t*>(dst + r * S + cv * VE);
                d[0] = v[u].x; d[1] = v[u].y; d[2] = v[u].z; d[3] = v[u].w;
            }
        }
    }
}

struct StateArgs {
    const void* x;
    const void* B;
    const float* dt;
    const float* dA;
    const int32_t* seq_idx;
    const int32_t* cu_seqlens;   // varlen only
    const void* chunk_states;    // varlen only
    int states_bf16;             // varlen only: dtype of chunk_states
    float* out;
    int L, H, G, P, N, Q, nc, nblocks;
    // chunk_cumsum folded in (k_chunk_state_f32<..., true>): the raw dt, its
    // processing, and where dA_cumsum / dt' go (written by the first dstate
    // block of each chunk and head; dA / dt above are not read)
    const void* dt_raw;
    int dt_bf16, softplus;
    const float* A;
    const float* dt_bias;
    float dt_lo, dt_hi;
    float* dA_out;
    float* dt_out;
};

template <typename T, int PT, int CTW, bool VARLEN>
__global__ void __launch_bounds__(THREADS) k_chunk_state(StateArgs a) {
    typedef MF<T> M;
    constexpr int PAD = Pad<T>::v;
    extern __shared__ __align__(16) char smem[];
    const int P = PT * 16, N = CTW * 64;
    const int Q = a.Q, L = a.L, H = a.H, nc = a.nc;
    const int KB = min(Pad<T>::KB, Q);
    const int SX = P + PAD, SB = N + PAD;
    T* xs = reinterpret_cast<T*>(smem);               // [KB][SX]
    T* bs = xs + KB * SX;                              // [KB][SB]
    float* wq = reinterpret_cast<float*>(bs + KB * SB); // [Q]

    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int h = work % H;
    const int g = h / (H / a.G);
    int bi = 0, c, s = 0, qlo = 0, qhi, start = 0;
    if (!VARLEN) {
        const int rest = work / H;
        c = rest % nc;
        bi = rest / nc;
        qhi = min(Q, L - c * Q);
    } else {
        s = work / H;
        // clamp malformed boundaries into [0, L] so every access stays in bounds
        const int end = min(max(a.cu_seqlens[s + 1], 0), L);
        start = min(max(a.cu_seqlens[s], 0), end);
        if (end <= start) {          // empty sequence: zero state
            float* op = a.out + ((int64_t)s * H + h) * a.P * a.N;
            for (int i = threadIdx.x; i < a.P * a.N; i += THREADS) op[i] = 0.f;
            return;
        }
        c = (end - 1) / Q;
        qlo = max(start - c * Q, 0);
        qhi = end - c * Q;
    }
    const float* dAp = a.dA + (((int64_t)bi * H + h) * nc + c) * Q;
    const float* dtp = a.dt + (((int64_t)bi * H + h) * nc + c) * Q;
    const float dA_ref = dAp[qhi - 1];
    int se = 0;
    if (!VARLEN && a.seq_idx) se = a.seq_idx[(int64_t)bi * L + c * Q + qhi - 1];
    for (int q = threadIdx.x; q < Q; q += THREADS) {
        float v = 0.f;
        if (q >= qlo && q < qhi) {
            v = expf(fminf(dA_ref - dAp[q], 0.f)) * dtp[q];
            if (!VARLEN && a.seq_idx &&
                (se < 0 || a.seq_idx[(int64_t)bi * L + c * Q + q] != se))
                v = 0.f;
        }
        wq[q] = v;
    }

    const int lane = threadIdx.x & 63, w8 = wave_id();
    // wavefront w8: column tiles of group w = w8 & 3, row tiles of half w8 >> 2
    const int w = w8 & 3, pr0 = (w8 >> 2) * (PT / 2);
    const int ln = lane & 15, kg = lane >> 4;
    const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;   // token of position 0
    const int valid = min(Q, L - c * Q);
    const T* xsrc = reinterpret_cast<const T*>(a.x) + (tok0 * H + h) * P;
    const T* bsrc = reinterpret_cast<const T*>(a.B) + (tok0 * a.G + g) * N;

    constexpr int PTH = PT / 2;          // row tiles per wavefront
    f32x4 acc[PTH][CTW];
#pragma unroll
    for (int pt = 0; pt < PTH; ++pt)
#pragma unroll
        for (int j = 0; j < CTW; ++j) acc[pt][j] = zero4();

    for (int kb = 0; kb < Q; kb += KB) {
        if (kb) __syncthreads();
        stage_rows<T>(xs, SX, xsrc + (int64_t)kb * H * P, (int64_t)H * P, KB, valid - kb, P);
        stage_rows<T>(bs, SB, bsrc + (int64_t)kb * a.G * N, (int64_t)a.G * N, KB, valid - kb, N);
        __syncthreads();
        for (int k0 = 0; k0 < KB; k0 += M::K) {
            // x[q,p] * w[q] is split into bf16 hi + lo parts (x and B are exact
            // in their dtype, so two MFMAs give near-fp32 weighted sums)
            typename M::frag af[PTH], al[PTH], bfr[CTW];
#pragma unroll
            for (int j = 0; j < M::KPL; ++j) {
                const int kl = k0 + kg * M::KPL + j;      // position within the block
                const bool kok = kl < KB && kb + kl < Q;
                const float wk = kok ? wq[kb + kl] : 0.f;
#pragma unroll
                for (int pt = 0; pt < PTH; ++pt) {
                    const float xv = kok ? to_f32(xs[kl * SX + (pr0 + pt) * 16 + ln]) : 0.f;
                    M::set_split(af[pt], al[pt], j, xv * wk);
                }
#pragma unroll
                for (int jj = 0; jj < CTW; ++jj) {
                    const int n = (w * CTW + jj) * 16 + ln;
                    M::set_raw(bfr[jj], j, kok ? bs[kl * SB + n] : T(0.f));
                }
            }
#pragma unroll
            for (int pt = 0; pt < PTH; ++pt)
#pragma unroll
                for (int jj = 0; jj < CTW; ++jj) {
                    acc[pt][jj] = M::mma(af[pt], bfr[jj], acc[pt][jj]);
                    if constexpr (M::kSplit) acc[pt][jj] = M::mma(al[pt], bfr[jj], acc[pt][jj]);
                }
        }
    }

    float* op;
    float carry_scale = 0.f;
    const bf16* cs16 = nullptr;
    const float* cs32 = nullptr;
    if (!VARLEN) {
        op = a.out + ((((int64_t)bi * nc + c) * H + h) * P) * N;
    } else {
        op = a.out + (((int64_t)s * H + h) * P) * N;
        if (start < c * Q) {
            carry_scale = expf(dA_ref);
            const int64_t off = (((int64_t)c * H + h) * P) * N;
            if (a.states_bf16) cs16 = reinterpret_cast<const bf16*>(a.chunk_states) + off;
            else cs32 = reinterpret_cast<const float*>(a.chunk_states) + off;
        }
    }
#pragma unroll
    for (int pt = 0; pt < PTH; ++pt)
#pragma unroll
        for (int jj = 0; jj < CTW; ++jj) {
            const int n = (w * CTW + jj) * 16 + ln;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = (pr0 + pt) * 16 + kg * 4 + i;
                float v = acc[pt][jj][i];
                if (VARLEN) {
                    if (cs16) v += carry_scale * to_f32(cs16[p * N + n]);
                    else if (cs32) v += carry_scale * cs32[p * N + n];
                }
                op[p * N + n] = v;
            }
        }
}

// ---------------------------------------------------------------------------
// k_chunk_state_f32: chunk mode for fp32 x / B.  One workgroup per (b, c,
// HP heads of a group, 128-column dstate block): the weighted rows w[q] x[q, :]
// of the HP heads and the block's B rows are staged once as bf16 hi / lo
// planes, row-major with the 16-byte chunks of each row XOR-swizzled, and
// the MFMA operands (8 consecutive positions of one column) come through the
// gfx950 LDS transpose read; a product of two split operands is three
// 16x16x32 bf16 MFMAs (~2^-16 relative).  With two heads the block's B rows
// serve both.  The product is computed transposed, h^T[n, p] = B^T[n, q]
// (w x)[q, p], so each lane holds 4 consecutive dstate columns of one
// head-dim row (16-byte stores).  Wavefront w: with two heads, head w >> 2,
// p-row tiles 2 ((w >> 1) & 1) .. +1; with one head, p-row tile w >> 1; n
// tiles 4 (w & 1) .. +3.
// The x and B rows are loaded into registers before the weights are formed,
// so the two overlap.  With CS the workgroup also does chunk_cumsum for its
// heads (the combined forward's fp32 path): wavefront hh processes head
// h0 + hh's dt column (bias, softplus, clamp, zero past the end) and scans
// dt' A over the chunk exactly as k_chunk_cumsum does, and the first dstate
// block writes dA_cumsum and dt' for the kernels that follow.
// ---------------------------------------------------------------------------
constexpr float LOG2E_CS = 1.4426950408889634f;
constexpr int F32_NB = 128;                            // dstate columns per workgroup
__host__ __device__ inline size_t cs_f32_lds(int Q, int HP) {
    return (size_t)2 * Q * (HP * 64 + F32_NB) * 2 + (size_t)HP * Q * 4;
}
// 16-byte chunk swizzle of plane row R (128- or 256-byte rows): the 8 rows a
// transpose read touches at one chunk pair land on distinct banks
template <int RB> M2_DEV int cswz(int R) { return RB == 128 ? ((R >> 1) & 3) << 1 : (R & 7) << 1; }

M2_DEV f32x4 mma3cs(const bf16x8& ah, const bf16x8& al, const bf16x8& bh, const bf16x8& bl, f32x4 c) {
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
}
// 8 k of one column: rows r and r + 16 of the transpose read
M2_DEV bf16x8 tr8(const char* p0, const char* p1) {
    return __builtin_shufflevector(ds_read_tr(p0), ds_read_tr(p1), 0, 1, 2, 3, 4, 5, 6, 7);
}

template <int HP, int QT, bool CS, bool NT>
__global__ void __launch_bounds__(THREADS) k_chunk_state_f32(StateArgs a) {
    constexpr int P = 64, Q = 32 * QT;
    constexpr int XROW = HP * P * 2, BROW = F32_NB * 2;     // plane row bytes
    extern __shared__ __align__(16) char smem[];
    char* xh = smem;                                     // [Q] rows of XROW: (w x) hi
    char* xl = xh + Q * XROW;                            // (w x) lo
    char* bh = xl + Q * XROW;                            // [Q] rows of BROW: B hi
    char* bl = bh + Q * BROW;                            // B lo
    float* wq = reinterpret_cast<float*>(bl + Q * BROW); // [HP][Q]

    const int H = a.H, L = a.L, N = a.N, nc = a.nc;
    const int nblk = N / F32_NB;
    const int work = xcd_remap(blockIdx.x, a.nblocks);
    const int nb = work % nblk;
    const int hq = (work / nblk) % (H / HP);
    const int rest = work / (nblk * (H / HP));
    const int c = rest % nc, bi = rest / nc;
    const int h0 = hq * HP;
    const int g = h0 / (H / a.G);
    const int qhi = min(Q, L - c * Q);                   // valid positions
    const int64_t tok0 = (int64_t)bi * L + (int64_t)c * Q;

    // ---- x and B rows into registers (all loads in flight first)
    typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
    constexpr int XV = HP * P / 4, XI = Q * XV / THREADS;   // float4 per x row, per thread
    constexpr int BV = F32_NB / 4, BI = Q * BV / THREADS;
    static_assert(Q * XV % THREADS == 0 && Q * BV % THREADS == 0, "even staging split");
    static_assert(!NT || 2 * Q * (XROW + BROW) >= (THREADS / 64) * 4096, "output staging fits the planes");
    float4 xf[XI], bf[BI];
    {
        const float* xsrc = reinterpret_cast<const float*>(a.x) + (tok0 * H + h0) * P;
        const float* bsrc = reinterpret_cast<const float*>(a.B) + (tok0 * a.G + g) * N + nb * F32_NB;
#pragma unroll
        for (int it = 0; it < XI; ++it) {
            const int idx = threadIdx.x + it * THREADS, q = idx / XV, v = idx % XV;
            xf[it] = *reinterpret_cast<const float4*>(xsrc + (int64_t)min(q, qhi - 1) * H * P + 4 * v);
        }
#pragma unroll
        for (int it = 0; it < BI; ++it) {
            const int idx = threadIdx.x + it * THREADS, q = idx / BV, v = idx % BV;
            bf[it] = *reinterpret_cast<const float4*>(bsrc + (int64_t)min(q, qhi - 1) * a.G * N + 4 * v);
        }
    }

    // ---- weights w[q] = exp(min(dA[last] - dA[q], 0)) dt[q], 0 past the end
    // and where seq_idx differs from the chunk's last position (or that id < 0)
    const int se = a.seq_idx ? a.seq_idx[tok0 + qhi - 1] : 0;
    if constexpr (CS) {
        constexpr int PPL = Q / 64;
        const int lane = threadIdx.x & 63, hh = wave_id();
        if (hh < HP) {
            const int h = h0 + hh;
            const float Ah = a.A[h];
            const float bias = a.dt_bias ? a.dt_bias[h] : 0.f;
            int sq[PPL];
            float d[PPL];
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const int64_t t = tok0 + min(lane + 64 * j, qhi - 1);
                d[j] = a.dt_bf16 ? to_f32(reinterpret_cast<const bf16*>(a.dt_raw)[t * H + h])
                                 : reinterpret_cast<const float*>(a.dt_raw)[t * H + h];
                sq[j] = a.seq_idx ? a.seq_idx[t] : 0;
            }
            float v[PPL], dA[PPL], carry = 0.f;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const int q = lane + 64 * j;
                float dd = d[j];
                if (a.dt_bias) dd += bias;
                if (a.softplus) dd = softplus_f(dd);
                dd = fminf(fmaxf(dd, a.dt_lo), a.dt_hi);
                v[j] = q < qhi ? dd : 0.f;
                dA[j] = wave_scan(v[j] * Ah) + carry;
                carry = lane63(dA[j]);
            }
            const float total = carry;                  // dA at the chunk's last position
            const int64_t row = (((int64_t)bi * H + h) * nc + c) * Q;
#pragma unroll
            for (int j = 0; j < PPL; ++j) {
                const int q = lane + 64 * j;
                if (nb == 0) {
                    a.dA_out[row + q] = dA[j];
                    a.dt_out[row + q] = v[j];
                }
                float wv = q < qhi ? __builtin_amdgcn_exp2f(fminf(total - dA[j], 0.f) * LOG2E_CS) * v[j] : 0.f;
                if (a.seq_idx && (se < 0 || sq[j] != se)) wv = 0.f;
                wq[hh * Q + q] = wv;
            }
        }
    } else {
        for (int i = threadIdx.x; i < HP * Q; i += THREADS) {
            const int hh = i / Q, q = i % Q;
            const int64_t row = (((int64_t)bi * H + h0 + hh) * nc + c) * Q;
            float v = 0.f;
            if (q < qhi) {
                v = __builtin_amdgcn_exp2f(fminf(a.dA[row + qhi - 1] - a.dA[row + q], 0.f) * LOG2E_CS) * a.dt[row + q];
                if (a.seq_idx && (se < 0 || a.seq_idx[tok0 + q] != se)) v = 0.f;
            }
            wq[i] = v;
        }
    }
    __syncthreads();

    // ---- staging: weighted / split and written as 8-byte halves of
    // swizzled 16-byte chunks
    {
#pragma unroll
        for (int it = 0; it < XI; ++it) {
            const int idx = threadIdx.x + it * THREADS, q = idx / XV, v = idx % XV;
            const float wv = wq[(4 * v / P) * Q + q];    // zero past the end
            uint32_t h01, l01, h23, l23;
            split2(xf[it].x * wv, xf[it].y * wv, h01, l01);
            split2(xf[it].z * wv, xf[it].w * wv, h23, l23);
            const int off = q * XROW + (((v >> 1) ^ cswz<XROW>(q)) * 16) + 8 * (v & 1);
            *reinterpret_cast<u2*>(xh + off) = u2{h01, h23};
            *reinterpret_cast<u2*>(xl + off) = u2{l01, l23};
        }
#pragma unroll
        for (int it = 0; it < BI; ++it) {
            const int idx = threadIdx.x + it * THREADS, q = idx / BV, v = idx % BV;
            uint32_t h01, l01, h23, l23;
            split2(bf[it].x, bf[it].y, h01, l01);
            split2(bf[it].z, bf[it].w, h23, l23);
            const int off = q * BROW + (((v >> 1) ^ cswz<BROW>(q)) * 16) + 8 * (v & 1);
            *reinterpret_cast<u2*>(bh + off) = u2{h01, h23};
            *reinterpret_cast<u2*>(bl + off) = u2{l01, l23};
        }
    }
    __syncthreads();

    // ---- h^T[n, p] over the chunk's positions.  K step ks covers rows
    // 32 ks .. +31: MFMA k index j < 4 is row 32 ks + 4 kg + j, j >= 4 is 16
    // more; the swizzles repeat every 8 rows
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    constexpr int PTW = HP == 2 ? 2 : 1;                 // p-row tiles per wavefront
    const int pt0 = HP == 2 ? 4 * (w >> 2) + 2 * ((w >> 1) & 1) : (w >> 1);   // over the HP heads
    const int nt0 = 4 * (w & 1);                         // first n tile
    const int rA = 4 * kg + (ln >> 2), c1 = ln & 3, cb = 8 * (c1 & 1);
    int xo[PTW], bo[4];
#pragma unroll
    for (int i = 0; i < PTW; ++i)
        xo[i] = rA * XROW + (((2 * (pt0 + i) + (c1 >> 1)) ^ cswz<XROW>(rA)) * 16) + cb;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        bo[j] = rA * BROW + (((2 * (nt0 + j) + (c1 >> 1)) ^ cswz<BROW>(rA)) * 16) + cb;
    f32x4 acc[4][PTW];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i = 0; i < PTW; ++i) acc[j][i] = zero4();
#pragma unroll
    for (int ks = 0; ks < QT; ++ks) {
        const int xs = ks * 32 * XROW, bs = ks * 32 * BROW;
        bf16x8 ph[PTW], pl[PTW];
#pragma unroll
        for (int i = 0; i < PTW; ++i) {
            ph[i] = tr8(xh + xs + xo[i], xh + xs + xo[i] + 16 * XROW);
            pl[i] = tr8(xl + xs + xo[i], xl + xs + xo[i] + 16 * XROW);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x8 nh = tr8(bh + bs + bo[j], bh + bs + bo[j] + 16 * BROW);
            const bf16x8 nlo = tr8(bl + bs + bo[j], bl + bs + bo[j] + 16 * BROW);
#pragma unroll
            for (int i = 0; i < PTW; ++i) acc[j][i] = mma3cs(nh, nlo, ph[i], pl[i], acc[j][i]);
        }
    }
    // lane: p-tile pt0 + i, p = 16 (pt0 + i) + ln over the heads, n = 16 (nt0 + j) + 4 kg .. + 3
    if constexpr (NT) {
        // non-temporal stores of whole row pieces (64 columns, 256 bytes): each
        // wavefront stages the 16 rows of its p-tile in 4 KB of the (no longer
        // read) plane LDS, 16-byte piece 4 j + kg of row ln XOR-swizzled by the
        // row, and reads them back 16 lanes per row.  The region is this
        // wavefront's alone; its LDS operations complete in order, and the
        // waits keep the compiler from moving the accesses across each other.
        __syncthreads();
        char* sw = smem + w * 4096;
#pragma unroll
        for (int i = 0; i < PTW; ++i) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<f32x4*>(sw + ln * 256 + 16 * ((4 * j + kg) ^ ln)) = acc[j][i];
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            f32x4 v[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int r = 4 * q + (lane >> 4);
                v[q] = *reinterpret_cast<const f32x4*>(sw + r * 256 + 16 * ((lane & 15) ^ r));
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int pr = 16 * (pt0 + i) + 4 * q + (lane >> 4);
                const int hh = pr / P, pp = pr % P;
                float* const dst = a.out + ((((int64_t)bi * nc + c) * H + h0 + hh) * P + pp) * N +
                                   nb * F32_NB + 16 * nt0 + 4 * (lane & 15);
                __builtin_nontemporal_store(v[q], reinterpret_cast<f32x4*>(dst));
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < PTW; ++i) {
            const int pr = 16 * (pt0 + i) + ln;
            const int hh = pr / P, pp = pr % P;
            float* op = a.out + ((((int64_t)bi * nc + c) * H + h0 + hh) * P + pp) * N + nb * F32_NB;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *reinterpret_cast<float4*>(op + 16 * (nt0 + j) + 4 * kg) =
                    make_float4(acc[j][i][0], acc[j][i][1], acc[j][i][2], acc[j][i][3]);
        }
    }
}

// fp32 chunk mode: head dim 64, dstate a multiple of 128, chunk 64 / 128,
// the plane LDS in budget; two heads per workgroup when the group's head
// count is even.  cs: chunk_cumsum folded in (the StateArgs cumsum fields set)
int launch_chunk_state_f32(const StateArgs& sa, int64_t bhc, hipStream_t s, bool cs = false) {
    if (sa.P != 64 || sa.N % F32_NB || (sa.Q != 64 && sa.Q != 128))
        return m2::set_error(M2_ERR_UNSUPPORTED,
                             "chunk_state (fp32 planes): headdim 64, dstate %% %d == 0 and chunk 64 "
                             "/ 128 only (got %d / %d / %d)", F32_NB, sa.P, sa.N, sa.Q);
    const int HP = (sa.H / sa.G) % 2 == 0 ? 2 : 1;
    const size_t shm = cs_f32_lds(sa.Q, HP);
    if (shm > 160 * 1024)
        return m2::set_error(M2_ERR_UNSUPPORTED, "chunk_state (fp32 planes): %zu B of LDS", shm);
    // The combined forward's chunk states (cumsum folded in) leave
    // non-temporally, as whole row pieces staged in LDS, when they are small (at most 16 MiB; the fp32 mamba2-130m
    // layer: 12 MiB): this kernel 10.6 against 11.6 us, the layer 33.8 against
    // 34.4 us (A/B on one box), no dirty lines remaining in L2 for the end of
    // the kernel; at 24 / 48 MiB the state passing that reads them next lost
    // more than this kernel gained.
    const bool nt = cs && (double)bhc * sa.P * sa.N * 4 <= 16.0 * (1 << 20);
    void (*kern)(StateArgs) = nullptr;
#define M2_CSF_CASE(HPV, QV, CSV, NTV) \
    if (HP == HPV && sa.Q == QV && cs == CSV && nt == NTV) kern = k_chunk_state_f32<HPV, QV / 32, CSV, NTV>;
    M2_CSF_CASE(2, 64, false, false) M2_CSF_CASE(2, 128, false, false)
    M2_CSF_CASE(1, 64, false, false) M2_CSF_CASE(1, 128, false, false)
    M2_CSF_CASE(2, 64, true, false) M2_CSF_CASE(2, 128, true, false)
    M2_CSF_CASE(1, 64, true, false) M2_CSF_CASE(1, 128, true, false)
    M2_CSF_CASE(2, 64, true, true) M2_CSF_CASE(2, 128, true, true)
    M2_CSF_CASE(1, 64, true, true) M2_CSF_CASE(1, 128, true, true)
#undef M2_CSF_CASE
    if (shm > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "chunk_state: cannot reserve %zu B of LDS", shm);
    StateArgs k = sa;
    const int64_t nblocks = bhc / HP * (sa.N / F32_NB);
    if (nblocks >= (1ll << 31))
        return m2::set_error(M2_ERR_UNSUPPORTED, "chunk_state (fp32 planes): too many blocks");
    k.nblocks = (int)nblocks;
    kern<<<(unsigned)nblocks, THREADS, shm, s>>>(k);
    return m2::check_launch("chunk_state");
}

template <typename T, bool VARLEN>
int launch_typed(const StateArgs& sa, int64_t nblocks, hipStream_t s) {
    const int KB = Pad<T>::KB < sa.Q ? Pad<T>::KB : sa.Q;
    const size_t shm = (size_t)KB * ((sa.P + Pad<T>::v) + (sa.N + Pad<T>::v)) * sizeof(T) +
                       (size_t)sa.Q * sizeof(float);
    const void* fn = nullptr;
    void (*kern)(StateArgs) = nullptr;
#define M2_CS_CASE(PTV, CTWV)                                       \
    if (sa.P == PTV * 16 && sa.N == CTWV * 64) kern = k_chunk_state<T, PTV, CTWV, VARLEN>;
    M2_CS_CASE(2, 1) M2_CS_CASE(2, 2) M2_CS_CASE(2, 4)
    M2_CS_CASE(4, 1) M2_CS_CASE(4, 2) M2_CS_CASE(4, 4)
    M2_CS_CASE(8, 1) M2_CS_CASE(8, 2) M2_CS_CASE(8, 4)
#undef M2_CS_CASE
    if (!kern)
        return m2::set_error(M2_ERR_UNSUPPORTED,
                             "chunk_state: headdim %d / dstate %d not supported "
                             "(headdim in {32, 64, 128}, dstate in {64, 128, 256})",
                             sa.P, sa.N);
    fn = reinterpret_cast<const void*>(kern);
    if (shm > 65536) {
        if (hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) !=
            hipSuccess)
            return m2::set_error(M2_ERR_LAUNCH, "chunk_state: cannot reserve %zu B of LDS", shm);
    }
    kern<<<(unsigned)nblocks, THREADS, shm, s>>>(sa);
    return m2::check_launch(VARLEN ? "chunk_state_varlen" : "chunk_state");
}

}  // namespace

namespace m2 {

int launch_chunk_state(const m2_chunk_state_args& a, hipStream_t s) {
    M2_REQUIRE(a.x && a.B && a.dt && a.dA_cumsum && a.states, M2_ERR_INVALID,
               "chunk_state: x, B, dt, dA_cumsum and states are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.nheads > 0 && a.ngroups > 0 &&
                   a.nheads % a.ngroups == 0 && a.chunk_size > 0,
               M2_ERR_INVALID, "chunk_state: bad sizes (nheads must be a multiple of ngroups)");
    M2_REQUIRE(a.chunk_size % 16 == 0 && a.chunk_size <= 256, M2_ERR_UNSUPPORTED,
               "chunk_state: chunk_size must be a multiple of 16 and <= 256");
    if (chunk_state_fast_supported(a)) return launch_chunk_state_fast(a, s);
    StateArgs sa{};
    sa.x = a.x; sa.B = a.B; sa.dt = a.dt; sa.dA = a.dA_cumsum; sa.seq_idx = a.seq_idx;
    sa.out = a.states;
    sa.L = (int)a.seqlen; sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.P = (int)a.headdim;
    sa.N = (int)a.dstate; sa.Q = (int)a.chunk_size;
    sa.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    const int64_t nblocks = a.batch * sa.nc * a.nheads;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_state: too many blocks");
    sa.nblocks = (int)nblocks;
    if (a.dtype == M2_BF16) return launch_typed<bf16, false>(sa, nblocks, s);
    if (a.dtype == M2_F32) {
        const int rc = launch_chunk_state_f32(sa, nblocks, s);
        if (rc != M2_ERR_UNSUPPORTED) return rc;
        return launch_typed<float, false>(sa, nblocks, s);
    }
    return set_error(M2_ERR_UNSUPPORTED, "chunk_state: dtype %d", a.dtype);
}

// chunk_cumsum + chunk_state of the combined forward's fp32 path in one
// kernel: c1's outputs (dA_cumsum, dt_out) are written as chunk_cumsum
// writes them.  For the shapes chunk_state_cumsum_supported accepts; the
// caller runs the two stages separately for the others.
bool chunk_state_cumsum_supported(const m2_chunk_cumsum_args& c1, const m2_chunk_state_args& a) {
    return a.dtype == M2_F32 && (c1.dt_dtype == M2_F32 || c1.dt_dtype == M2_BF16) &&
           a.chunk_size == c1.chunk_size && a.dt == c1.dt_out && a.dA_cumsum == c1.dA_cumsum &&
           a.headdim == 64 && a.dstate % F32_NB == 0 && (a.chunk_size == 64 || a.chunk_size == 128) &&
           a.ngroups > 0 && a.nheads % a.ngroups == 0 &&
           cs_f32_lds((int)a.chunk_size, (a.nheads / a.ngroups) % 2 == 0 ? 2 : 1) <= 160 * 1024;
}

int launch_chunk_state_cumsum(const m2_chunk_cumsum_args& c1, const m2_chunk_state_args& a,
                              hipStream_t s) {
    M2_REQUIRE(chunk_state_cumsum_supported(c1, a), M2_ERR_UNSUPPORTED,
               "chunk_state: shape / dtype not covered with chunk_cumsum folded in");
    M2_REQUIRE(c1.dt && c1.A && a.x && a.B && a.dt && a.dA_cumsum && a.states, M2_ERR_INVALID,
               "chunk_state: x, B, dt, A and the outputs are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.nheads > 0 && a.ngroups > 0 &&
                   a.nheads % a.ngroups == 0,
               M2_ERR_INVALID, "chunk_state: bad sizes (nheads must be a multiple of ngroups)");
    StateArgs sa{};
    sa.x = a.x; sa.B = a.B; sa.dt = a.dt; sa.dA = a.dA_cumsum; sa.seq_idx = a.seq_idx;
    sa.out = a.states;
    sa.L = (int)a.seqlen; sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.P = (int)a.headdim;
    sa.N = (int)a.dstate; sa.Q = (int)a.chunk_size;
    sa.nc = (int)((a.seqlen + a.chunk_size - 1) / a.chunk_size);
    sa.dt_raw = c1.dt; sa.dt_bf16 = c1.dt_dtype == M2_BF16; sa.softplus = c1.dt_softplus;
    sa.A = c1.A; sa.dt_bias = c1.dt_bias; sa.dt_lo = c1.dt_min; sa.dt_hi = c1.dt_max;
    sa.dA_out = c1.dA_cumsum; sa.dt_out = c1.dt_out;
    const int64_t nblocks = a.batch * sa.nc * a.nheads;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_state: too many blocks");
    return launch_chunk_state_f32(sa, nblocks, s, true);
}

int launch_chunk_state_varlen(const m2_chunk_state_varlen_args& a, hipStream_t s) {
    M2_REQUIRE(a.x && a.B && a.dt && a.dA_cumsum && a.cu_seqlens && a.chunk_states && a.out,
               M2_ERR_INVALID, "chunk_state_varlen: all pointers are required");
    M2_REQUIRE(a.seqlen > 0 && a.nseq > 0 && a.nheads > 0 && a.ngroups > 0 &&
                   a.nheads % a.ngroups == 0 && a.chunk_size > 0 &&
                   a.nchunks == (a.seqlen + a.chunk_size - 1) / a.chunk_size,
               M2_ERR_INVALID, "chunk_state_varlen: bad sizes");
    M2_REQUIRE(a.chunk_size % 16 == 0 && a.chunk_size <= 256, M2_ERR_UNSUPPORTED,
               "chunk_state_varlen: chunk_size must be a multiple of 16 and <= 256");
    M2_REQUIRE(a.states_dtype == M2_F32 || a.states_dtype == M2_BF16, M2_ERR_UNSUPPORTED,
               "chunk_state_varlen: states dtype %d", a.states_dtype);
    if (varlen_states_fast_supported(a)) return launch_varlen_states(a, s);
    StateArgs sa{};
    sa.x = a.x; sa.B = a.B; sa.dt = a.dt; sa.dA = a.dA_cumsum; sa.cu_seqlens = a.cu_seqlens;
    sa.chunk_states = a.chunk_states; sa.states_bf16 = a.states_dtype == M2_BF16; sa.out = a.out;
    sa.L = (int)a.seqlen; sa.H = (int)a.nheads; sa.G = (int)a.ngroups; sa.P = (int)a.headdim;
    sa.N = (int)a.dstate; sa.Q = (int)a.chunk_size; sa.nc = (int)a.nchunks;
    const int64_t nblocks = a.nseq * a.nheads;
    M2_REQUIRE(nblocks < (1ll << 31), M2_ERR_UNSUPPORTED, "chunk_state_varlen: too many blocks");
    sa.nblocks = (int)nblocks;
    if (a.dtype == M2_BF16) return launch_typed<bf16, true>(sa, nblocks, s);
    if (a.dtype == M2_F32) return launch_typed<float, true>(sa, nblocks, s);
    return set_error(M2_ERR_UNSUPPORTED, "chunk_state_varlen: dtype %d", a.dtype);
}

}  // namespace m2
