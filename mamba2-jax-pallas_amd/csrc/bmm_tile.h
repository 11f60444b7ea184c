// One 64 x (16 CT) output tile of bmm_chunk, CB[b, c, g] = a_c b_c^T
// (Q x Q, contraction over K), for the tiled kernel of bmm_chunk.hip and for
// the launch that runs bmm_chunk beside state_passing (state_passing.hip).
// Both operands are K-contiguous in HBM ([.., L, G, K] rows), which is the
// per-lane layout MFMA wants: every fragment is one load straight into VGPRs.
// Each of the 4 wavefronts of the 256-thread block owns one 16-row tile and
// the block's column tiles; causal and seq_idx masks in the epilogue.
// Follows reference kernels/bmm_chunk_fwd.py:87-154 (product), :348-372
// (masks; positions past the end carry seq id -1) and ops/ssd_naive.py:189-216.
#pragma once

#include "m2ssd.h"
#include "m2_common.h"

namespace m2 {

struct BmmTileArgs {
    const void* a;
    const void* b;
    const int32_t* seq_idx;
    void* out;
    int L, G, K, Q, nc, causal, rowblocks, colblocks, nblocks;
};

template <typename T, typename TO, int CT>
M2_DEV void bmm_tile(const BmmTileArgs& p, int work) {
    typedef MF<T> M;
    const T* __restrict__ a = static_cast<const T*>(p.a);
    const T* __restrict__ b = static_cast<const T*>(p.b);
    const int32_t* __restrict__ seq_idx = p.seq_idx;
    TO* __restrict__ out = static_cast<TO*>(p.out);
    const int L = p.L, G = p.G, K = p.K, Q = p.Q, nc = p.nc, causal = p.causal;
    const int rowblocks = p.rowblocks, colblocks = p.colblocks;
    const int cb = work % colblocks;                     // (16 CT)-column block
    const int rb = (work / colblocks) % rowblocks;       // 64-row block
    int rest = work / (rowblocks * colblocks);
    const int g = rest % G;
    rest /= G;
    const int c = rest % nc;
    const int bi = rest / nc;
    const int lane = threadIdx.x & 63, w = wave_id();
    const int r0 = rb * 64 + w * 16;
    if (r0 >= Q) return;
    const int ln = lane & 15, kg = lane >> 4;

    const int arow = r0 + ln;
    const int64_t tbase = (int64_t)bi * L + (int64_t)c * Q;
    const bool arow_ok = (c * Q + arow) < L;
    const T* ap = a + ((tbase + arow) * G + g) * K + kg * M::KPL;
    const T* bp[CT];
    bool bok[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        const int col = cb * 16 * CT + ct * 16 + ln;
        bok[ct] = (c * Q + col) < L && col < Q;
        bp[ct] = b + ((tbase + min(col, Q - 1)) * G + g) * K + kg * M::KPL;
    }
    f32x4 acc[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) acc[ct] = zero4();

    typename M::frag zf;
#pragma unroll
    for (int j = 0; j < M::KPL; ++j) M::set(zf, j, 0.f);

#pragma unroll 8
    for (int k0 = 0; k0 < K; k0 += M::K) {
        const typename M::frag af = arow_ok ? load_frag(ap + k0) : zf;
        typename M::frag bf[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) bf[ct] = bok[ct] ? load_frag(bp[ct] + k0) : zf;
        // transposed product (A = b rows, B = a rows): lane (ln, kg) ends with
        // row r0 + ln, columns 16 ct + 4 kg + i -- four consecutive outputs
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) acc[ct] = M::mma(bf[ct], af, acc[ct]);
    }

    TO* op = out + ((((int64_t)bi * nc + c) * G + g) * Q) * Q;
    const int row = arow;
    int srow = 0;
    if (seq_idx) srow = (c * Q + row) < L ? seq_idx[tbase + row] : -1;
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
        const int col0 = cb * 16 * CT + ct * 16 + 4 * kg;
        if (col0 >= Q) continue;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int col = col0 + i;
            v[i] = acc[ct][i];
            if (causal && col > row) v[i] = 0.f;
            if (seq_idx) {
                const int scol = (c * Q + col) < L ? seq_idx[tbase + col] : -1;
                if (srow != scol) v[i] = 0.f;
            }
        }
        TO* dst = op + (int64_t)row * Q + col0;
        if constexpr (sizeof(TO) == 4) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
            const bf16x4 o = {(bf16)v[0], (bf16)v[1], (bf16)v[2], (bf16)v[3]};
            *reinterpret_cast<bf16x4*>(dst) = o;
        }
    }
}

// The tiled kernel's grid: 64 x (16 ct) tiles, narrower column blocks (more
// workgroups) while there are too few tiles to fill the CUs.  Returns ct.
inline int bmm_tile_plan(const m2_bmm_chunk_args& a, BmmTileArgs& p) {
    const int Q = (int)a.chunk_size;
    const int nc = (int)((a.seqlen + Q - 1) / Q);
    const int rowblocks = (Q + 63) / 64;
    int ct = Q < 64 ? Q / 16 : 4;
    const int64_t items = a.batch * nc * a.ngroups * rowblocks;
    while (ct > 1 && items * ((Q + 16 * ct - 1) / (16 * ct)) < 512 && Q % (16 * (ct / 2)) == 0) ct /= 2;
    const int colblocks = (Q + 16 * ct - 1) / (16 * ct);
    const int64_t nblocks = items * colblocks;
    p = BmmTileArgs{a.a, a.b, a.seq_idx, a.out, (int)a.seqlen, (int)a.ngroups, (int)a.k, Q, nc,
                    a.causal, rowblocks, colblocks, nblocks < (1ll << 31) ? (int)nblocks : -1};
    return ct;
}

}  // namespace m2
