// bmm_chunk: CB[b,c,g] = a_c @ b_c^T for every chunk c and group g
// (Q x Q output, contraction over K = dstate).
//
// bf16 operands at the usual sizes take k_bmm_chunk_lds (one workgroup per
// chunk and group, operands staged in LDS once), fp32 operands on shapes with
// enough (chunk, group) blocks k_bmm_chunk_lds_f32 (the same, operands staged
// as bf16 hi / lo planes, each product three MFMAs).  Otherwise k_bmm_chunk:
// 64 x (16 CT) output tiles with every fragment loaded straight into VGPRs
// (the tile is bmm_tile.h's, which the fp32 combined forward also runs beside
// state_passing in one launch).
//
// Follows reference kernels/bmm_chunk_fwd.py:87-154 (product), :348-372
// (masks; positions past the end carry seq id -1) and ops/ssd_naive.py:189-216.
#include "m2_internal.h"
#include "bmm_tile.h"

namespace {

constexpr int THREADS = 256;

template <typename T, typename TO, int CT>
__global__ void __launch_bounds__(THREADS) k_bmm_chunk(m2::BmmTileArgs p) {
    m2::bmm_tile<T, TO, CT>(p, xcd_remap(blockIdx.x, p.nblocks));
}

// One workgroup per (b, c, g) for bf16 operands whose two Q x K row blocks fit
// in LDS: both blocks are loaded once (coalesced 16-byte loads, 16-byte chunks
// XOR-swizzled by row so that the fragment reads of 16 rows at one chunk hit
// distinct banks), then wavefront w computes row tiles w, w + 8, ... against
// every column tile from LDS.  Every operand byte enters the CU once; the
// tiled kernel above reads each row block several times (once per column
// block, and the column rows once per wavefront).
constexpr int LDS_THREADS = 512;
template <typename TO, int QT, int KC>
__global__ void __launch_bounds__(LDS_THREADS)
k_bmm_chunk_lds(const bf16* __restrict__ a, const bf16* __restrict__ b,
                const int32_t* __restrict__ seq_idx, TO* __restrict__ out, int L, int G, int nc,
                int causal) {
    constexpr int Q = 16 * QT, K = 8 * KC;                 // KC 16-byte chunks per row
    __shared__ __align__(16) bf16 sa[Q * K], sb[Q * K];
    __shared__ int seqs[Q];
    const int work = blockIdx.x;
    const int g = work % G, c = (work / G) % nc, bi = work / (G * nc);
    const int64_t tbase = (int64_t)bi * L + (int64_t)c * Q;
    const int valid = min(Q, L - c * Q);
    // ---- both row blocks into LDS; rows past the end are zero
    {
        constexpr int NCH = Q * KC;                        // 16-byte chunks per block
        for (int i = threadIdx.x; i < NCH; i += LDS_THREADS) {
            const int r = i / KC, ch = i % KC;
            const int so = r * K + 8 * (ch ^ (r & (KC - 1) & 15));
            u32x4 va = {0u, 0u, 0u, 0u}, vb = {0u, 0u, 0u, 0u};
            if (r < valid) {
                const int64_t go = ((tbase + r) * G + g) * K + 8 * ch;
                va = *reinterpret_cast<const u32x4*>(a + go);
                vb = *reinterpret_cast<const u32x4*>(b + go);
            }
            *reinterpret_cast<u32x4*>(sa + so) = va;
            *reinterpret_cast<u32x4*>(sb + so) = vb;
        }
        for (int q = threadIdx.x; q < Q; q += LDS_THREADS)
            seqs[q] = (seq_idx && q < valid) ? seq_idx[tbase + q] : -1;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    TO* op = out + ((((int64_t)bi * nc + c) * G + g) * Q) * Q;
    for (int rt = w; rt < QT; rt += LDS_THREADS / 64) {
        const int row = 16 * rt + ln;                      // this lane's output row (a row)
        f32x4 acc[QT];
#pragma unroll
        for (int ct = 0; ct < QT; ++ct) acc[ct] = zero4();
#pragma unroll
        for (int ks = 0; ks < KC / 4; ++ks) {
            const int ch = 4 * ks + kg;
            const bf16x8 af = *reinterpret_cast<const bf16x8*>(sa + row * K + 8 * (ch ^ (row & (KC - 1) & 15)));
#pragma unroll
            for (int ct = 0; ct < QT; ++ct) {
                const int col = 16 * ct + ln;
                const bf16x8 bf = *reinterpret_cast<const bf16x8*>(sb + col * K + 8 * (ch ^ (col & (KC - 1) & 15)));
                // transposed product (A = b rows, B = a rows): lane (ln, kg)
                // ends with row 16 rt + ln, columns 16 ct + 4 kg + i
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf, af, acc[ct], 0, 0, 0);
            }
        }
        const int srow = seqs[row];
#pragma unroll
        for (int ct = 0; ct < QT; ++ct) {
            const int col0 = 16 * ct + 4 * kg;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int col = col0 + i;
                v[i] = acc[ct][i];
                if (causal && col > row) v[i] = 0.f;
                if (seq_idx && srow != seqs[col]) v[i] = 0.f;
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
}

// fp32 operands: one workgroup per (b, c, g) as above, both row blocks
// staged once as bf16 hi / lo planes (v = hi + lo; a product is
// hi.hi + hi.lo + lo.hi, ~2^-16 relative), rows row-major with the 16-byte
// chunks XOR-swizzled by row.  Every fp32 row is loaded into registers
// before the first is split, so one round trip brings the whole block in.
template <typename TO, int QT, int KC>
__global__ void __launch_bounds__(LDS_THREADS)
k_bmm_chunk_lds_f32(const float* __restrict__ a, const float* __restrict__ b,
                    const int32_t* __restrict__ seq_idx, TO* __restrict__ out, int L, int G, int nc,
                    int causal) {
    constexpr int Q = 16 * QT, K = 8 * KC;                 // KC 16-byte bf16 chunks per row
    extern __shared__ __align__(16) char smem[];
    bf16* ah = reinterpret_cast<bf16*>(smem);              // [Q][K] planes
    bf16* al = ah + Q * K;
    bf16* bh = al + Q * K;
    bf16* bl = bh + Q * K;
    int* seqs = reinterpret_cast<int*>(bl + Q * K);        // [Q]
    const int work = blockIdx.x;
    const int g = work % G, c = (work / G) % nc, bi = work / (G * nc);
    const int64_t tbase = (int64_t)bi * L + (int64_t)c * Q;
    const int valid = min(Q, L - c * Q);
    // ---- both row blocks into registers, then split into the planes; rows
    // past the end are zero
    {
        typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u2;
        constexpr int VPR = K / 4, NV = Q * VPR / LDS_THREADS;   // float4 per row, per thread
        static_assert(Q * VPR % LDS_THREADS == 0, "even staging split");
        float4 va[NV], vb[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = threadIdx.x + i * LDS_THREADS, r = idx / VPR, v = idx % VPR;
            const int64_t go = ((tbase + min(r, valid - 1)) * G + g) * K + 4 * v;
            va[i] = *reinterpret_cast<const float4*>(a + go);
            vb[i] = *reinterpret_cast<const float4*>(b + go);
        }
        for (int q = threadIdx.x; q < Q; q += LDS_THREADS)
            seqs[q] = (seq_idx && q < valid) ? seq_idx[tbase + q] : -1;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int idx = threadIdx.x + i * LDS_THREADS, r = idx / VPR, v = idx % VPR;
            const int so = r * K + 8 * ((v >> 1) ^ (r & (KC - 1) & 15)) + 4 * (v & 1);
            const float4 x = r < valid ? va[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            const float4 y = r < valid ? vb[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            uint32_t h01, l01, h23, l23;
            split2(x.x, x.y, h01, l01);
            split2(x.z, x.w, h23, l23);
            *reinterpret_cast<u2*>(ah + so) = u2{h01, h23};
            *reinterpret_cast<u2*>(al + so) = u2{l01, l23};
            split2(y.x, y.y, h01, l01);
            split2(y.z, y.w, h23, l23);
            *reinterpret_cast<u2*>(bh + so) = u2{h01, h23};
            *reinterpret_cast<u2*>(bl + so) = u2{l01, l23};
        }
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, w = wave_id();
    const int ln = lane & 15, kg = lane >> 4;
    TO* op = out + ((((int64_t)bi * nc + c) * G + g) * Q) * Q;
    for (int rt = w; rt < QT; rt += LDS_THREADS / 64) {
        const int row = 16 * rt + ln;                      // this lane's output row (a row)
        f32x4 acc[QT];
#pragma unroll
        for (int ct = 0; ct < QT; ++ct) acc[ct] = zero4();
#pragma unroll
        for (int ks = 0; ks < KC / 4; ++ks) {
            const int ch = 4 * ks + kg;
            const int ro = row * K + 8 * (ch ^ (row & (KC - 1) & 15));
            const bf16x8 afh = *reinterpret_cast<const bf16x8*>(ah + ro);
            const bf16x8 afl = *reinterpret_cast<const bf16x8*>(al + ro);
#pragma unroll
            for (int ct = 0; ct < QT; ++ct) {
                const int col = 16 * ct + ln;
                const int co = col * K + 8 * (ch ^ (col & (KC - 1) & 15));
                const bf16x8 bfh = *reinterpret_cast<const bf16x8*>(bh + co);
                const bf16x8 bfl = *reinterpret_cast<const bf16x8*>(bl + co);
                // transposed product (A = b rows, B = a rows): lane (ln, kg)
                // ends with row 16 rt + ln, columns 16 ct + 4 kg + i
                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfl, afh, acc[ct], 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfh, afl, t, 0, 0, 0);
                acc[ct] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfh, afh, t, 0, 0, 0);
            }
        }
        const int srow = seqs[row];
#pragma unroll
        for (int ct = 0; ct < QT; ++ct) {
            const int col0 = 16 * ct + 4 * kg;
            float v[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int col = col0 + i;
                v[i] = acc[ct][i];
                if (causal && col > row) v[i] = 0.f;
                if (seq_idx && srow != seqs[col]) v[i] = 0.f;
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
}

// the fp32 LDS kernel where it applies: chunk 64 / 128, K 64 / 128, and at
// least 128 (chunk, group) blocks (fewer leave most CUs idle: the tiled
// kernel spreads small problems wider)
template <typename TO>
bool launch_lds_f32(const m2_bmm_chunk_args& a, hipStream_t s) {
    const int Q = (int)a.chunk_size, K = (int)a.k;
    const int nc = (int)((a.seqlen + Q - 1) / Q);
    const int64_t nblocks = a.batch * nc * a.ngroups;
    if (nblocks < 128 || nblocks >= (1ll << 31)) return false;
    void (*kern)(const float*, const float*, const int32_t*, TO*, int, int, int, int) = nullptr;
#define M2_BMMF_CASE(QV, KV) if (Q == QV && K == KV) kern = k_bmm_chunk_lds_f32<TO, QV / 16, KV / 8>;
    M2_BMMF_CASE(64, 64) M2_BMMF_CASE(64, 128) M2_BMMF_CASE(128, 64) M2_BMMF_CASE(128, 128)
#undef M2_BMMF_CASE
    if (!kern) return false;
    const size_t shm = (size_t)8 * Q * K + (size_t)Q * 4;
    if (shm > 65536 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm) != hipSuccess)
        return false;
    kern<<<(unsigned)nblocks, LDS_THREADS, shm, s>>>((const float*)a.a, (const float*)a.b, a.seq_idx,
                                                      (TO*)a.out, (int)a.seqlen, (int)a.ngroups, nc,
                                                      a.causal);
    return true;
}

template <typename TO>
bool launch_lds(const m2_bmm_chunk_args& a, hipStream_t s) {
    const int Q = (int)a.chunk_size, K = (int)a.k;
    const int nc = (int)((a.seqlen + Q - 1) / Q);
    const int64_t nblocks = a.batch * nc * a.ngroups;
    if (nblocks >= (1ll << 31)) return false;
    void (*kern)(const bf16*, const bf16*, const int32_t*, TO*, int, int, int, int) = nullptr;
#define M2_BMML_CASE(QV, KV) if (Q == QV && K == KV) kern = k_bmm_chunk_lds<TO, QV / 16, KV / 8>;
    M2_BMML_CASE(64, 64) M2_BMML_CASE(64, 128) M2_BMML_CASE(64, 256)
    M2_BMML_CASE(128, 64) M2_BMML_CASE(128, 128) M2_BMML_CASE(128, 256)
#undef M2_BMML_CASE
    if (!kern) return false;
    kern<<<(unsigned)nblocks, LDS_THREADS, 0, s>>>((const bf16*)a.a, (const bf16*)a.b, a.seq_idx,
                                                    (TO*)a.out, (int)a.seqlen, (int)a.ngroups, nc,
                                                    a.causal);
    return true;
}

template <typename T, typename TO>
int launch_typed(const m2_bmm_chunk_args& a, hipStream_t s) {
    if constexpr (sizeof(T) == 2) {
        if (launch_lds<TO>(a, s)) return m2::check_launch("bmm_chunk");
    } else {
        if (launch_lds_f32<TO>(a, s)) return m2::check_launch("bmm_chunk");
    }
    m2::BmmTileArgs p;
    const int ct = m2::bmm_tile_plan(a, p);
    M2_REQUIRE(p.nblocks > 0, M2_ERR_UNSUPPORTED, "bmm_chunk: too many blocks");
    const int64_t nblocks = p.nblocks;
    const int Q = p.Q;
#define M2_BMM_CASE(CTV)                                                                  \
    case CTV:                                                                             \
        k_bmm_chunk<T, TO, CTV><<<(unsigned)nblocks, THREADS, 0, s>>>(p);                  \
        break;
    switch (ct) {
        M2_BMM_CASE(1) M2_BMM_CASE(2) M2_BMM_CASE(3) M2_BMM_CASE(4)
        default: return m2::set_error(M2_ERR_UNSUPPORTED, "bmm_chunk: chunk_size %d", Q);
    }
#undef M2_BMM_CASE
    return m2::check_launch("bmm_chunk");
}

}  // namespace

namespace m2 {

// launch_bmm_chunk takes the tiled kernel (the LDS kernels do not apply)
bool bmm_uses_tiles(const m2_bmm_chunk_args& a) {
    const int64_t Q = a.chunk_size, K = a.k;
    const int64_t nblocks = a.batch * ((a.seqlen + Q - 1) / Q) * a.ngroups;
    if (a.dtype == M2_BF16)
        return !((Q == 64 || Q == 128) && (K == 64 || K == 128 || K == 256) && nblocks < (1ll << 31));
    return !(nblocks >= 128 && nblocks < (1ll << 31) && (Q == 64 || Q == 128) && (K == 64 || K == 128));
}

int check_bmm_chunk_args(const m2_bmm_chunk_args& a) {
    M2_REQUIRE(a.a && a.b && a.out, M2_ERR_INVALID, "bmm_chunk: a, b and out are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.ngroups > 0 && a.k > 0 && a.chunk_size > 0,
               M2_ERR_INVALID, "bmm_chunk: sizes must be positive");
    M2_REQUIRE(a.chunk_size % 16 == 0 && a.chunk_size <= 256, M2_ERR_UNSUPPORTED,
               "bmm_chunk: chunk_size must be a multiple of 16 and <= 256 (got %lld)",
               (long long)a.chunk_size);
    M2_REQUIRE(a.k % 32 == 0, M2_ERR_UNSUPPORTED, "bmm_chunk: k %% 32 != 0");
    return M2_OK;
}

int launch_bmm_chunk(const m2_bmm_chunk_args& a, hipStream_t s) {
    M2_REQUIRE(a.a && a.b && a.out, M2_ERR_INVALID, "bmm_chunk: a, b and out are required");
    M2_REQUIRE(a.batch > 0 && a.seqlen > 0 && a.ngroups > 0 && a.k > 0 && a.chunk_size > 0,
               M2_ERR_INVALID, "bmm_chunk: sizes must be positive");
    M2_REQUIRE(a.chunk_size % 16 == 0 && a.chunk_size <= 256, M2_ERR_UNSUPPORTED,
               "bmm_chunk: chunk_size must be a multiple of 16 and <= 256 (got %lld)",
               (long long)a.chunk_size);
    if (a.dtype == M2_BF16) {
        M2_REQUIRE(a.k % 32 == 0, M2_ERR_UNSUPPORTED, "bmm_chunk: bf16 needs k %% 32 == 0");
        if (a.out_dtype == M2_F32) return launch_typed<bf16, float>(a, s);
        if (a.out_dtype == M2_BF16) return launch_typed<bf16, bf16>(a, s);
    } else if (a.dtype == M2_F32) {
        M2_REQUIRE(a.k % 32 == 0, M2_ERR_UNSUPPORTED, "bmm_chunk: f32 needs k %% 32 == 0");
        if (a.out_dtype == M2_F32) return launch_typed<float, float>(a, s);
        if (a.out_dtype == M2_BF16) return launch_typed<float, bf16>(a, s);
    }
    return set_error(M2_ERR_UNSUPPORTED, "bmm_chunk: dtype %d -> %d", a.dtype, a.out_dtype);
}

}  // namespace m2
