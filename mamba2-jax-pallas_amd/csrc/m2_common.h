// Shared device helpers for the gfx950 SSD kernels: element types, MFMA
// fragment traits, workgroup->XCD mapping and the error plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "m2ssd.h"

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

#define M2_DEV __device__ __forceinline__

// ---------------------------------------------------------------------------
// element conversion
// ---------------------------------------------------------------------------
M2_DEV float to_f32(float v) { return v; }
M2_DEV float to_f32(bf16 v) { return (float)v; }

template <typename T> M2_DEV T from_f32(float v);
template <> M2_DEV float from_f32<float>(float v) { return v; }
template <> M2_DEV bf16 from_f32<bf16>(float v) { return (bf16)v; }  // RNE

// softplus(v) = log(1 + exp(v)) = max(v, 0) + log1p(exp(-|v|)), stable for
// all v.  log1p(e) for e in (0, 1] is evaluated with Goldberg's compensated
// formula log(u) * e / (u - 1), u = 1 + e (D. Goldberg, "What every computer
// scientist should know about floating-point arithmetic", 1991, Thm. 4): the
// hardware exp / log are accurate to a few ulp and the rounding of 1 + e is
// cancelled exactly.
M2_DEV float softplus_f(float v) {
    const float e = __expf(-fabsf(v));
    const float u = 1.f + e;
    const float l = u == 1.f ? e : __logf(u) * __fdividef(e, u - 1.f);
    return fmaxf(v, 0.f) + l;
}
M2_DEV float silu_f(float v) { return v / (1.f + expf(-v)); }

// inclusive prefix sum over the 64 lanes of a wavefront, on DPP lane moves
// (no LDS round trips): a Hillis-Steele scan inside each row of 16 lanes
// (row_shr 1, 2, 4, 8; lanes shifted in from outside the row read 0), then
// the last lane of row 0 / 2 is added into row 1 / 3 (row_bcast:15) and
// lane 31 into rows 2 and 3 (row_bcast:31)
template <int CTRL, int ROWS = 0xf>
M2_DEV float dpp_add(float v) {
    const int t = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xf, true);
    return v + __int_as_float(t);
}
M2_DEV float wave_scan(float v) {
    v = dpp_add<0x111>(v);            // row_shr:1
    v = dpp_add<0x112>(v);            // row_shr:2
    v = dpp_add<0x114>(v);            // row_shr:4
    v = dpp_add<0x118>(v);            // row_shr:8
    v = dpp_add<0x142, 0xa>(v);       // row_bcast:15 into rows 1, 3
    v = dpp_add<0x143, 0xc>(v);       // row_bcast:31 into rows 2, 3
    return v;
}
M2_DEV float lane63(float v) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63)); }

// ---------------------------------------------------------------------------
// MFMA 16x16 traits.  One instruction computes D(16x16) += A(16xK) B(Kx16).
//   A operand: lane l holds row (l & 15), k = (l >> 4) * KPL + j, j < KPL
//   B operand: lane l holds col (l & 15), same k
//   D:         lane l holds col (l & 15), rows 4 * (l >> 4) + i, i < 4
// bf16 inputs use v_mfma_f32_16x16x32_bf16 (K = 32); fp32 inputs use the same
// instruction on bf16 hi / lo triples (MF<float> below).
// ---------------------------------------------------------------------------
template <typename T> struct MF;

template <> struct MF<bf16> {
    static constexpr int KPL = 8;
    static constexpr int K = 32;
    typedef bf16x8 frag;
    static M2_DEV f32x4 mma(const frag& a, const frag& b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static M2_DEV void set(frag& f, int j, float v) { f[j] = (bf16)v; }
    static M2_DEV void set_raw(frag& f, int j, bf16 v) { f[j] = v; }
    // v ~= hi + lo with both parts bf16 (relative error ~2^-17): a scaled
    // operand keeps near-fp32 accuracy through two bf16 MFMAs.
    static constexpr bool kSplit = true;
    static M2_DEV void set_split(frag& hi, frag& lo, int j, float v) {
        const bf16 h = (bf16)v;
        hi[j] = h;
        lo[j] = (bf16)(v - (float)h);
    }
};

// fp32 operands as bf16 triples: v = hi + lo (both bf16, |v - hi - lo| ~ 2^-17 |v|),
// a.b ~ hi.hi + hi.lo + lo.hi (the dropped lo.lo term is ~2^-16 of the
// product): three 16x16x32 bf16 MFMAs per K = 32 step, ~16x the fp32 MFMA
// rate at near-fp32 accuracy, and 8 consecutive k per lane (32-byte loads).
struct f32x3frag {
    bf16x8 hi, lo;
};

template <> struct MF<float> {
    static constexpr int KPL = 8;
    static constexpr int K = 32;
    typedef f32x3frag frag;
    static M2_DEV f32x4 mma(const frag& a, const frag& b, f32x4 c) {
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.lo, b.hi, c, 0, 0, 0);
        c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.lo, c, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.hi, b.hi, c, 0, 0, 0);
    }
    static M2_DEV void set(frag& f, int j, float v) {
        const bf16 h = (bf16)v;
        f.hi[j] = h;
        f.lo[j] = (bf16)(v - (float)h);
    }
    static M2_DEV void set_raw(frag& f, int j, float v) { set(f, j, v); }
    // the triple already carries the split: one fragment, no second MFMA pass
    static constexpr bool kSplit = false;
    static M2_DEV void set_split(frag& hi, frag& lo, int j, float v) {
        set(hi, j, v);
        set(lo, j, 0.f);
    }
};

// Load KPL consecutive elements (16 B for bf16, 32 B for fp32) as a fragment.
M2_DEV bf16x8 load_frag(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
M2_DEV f32x3frag load_frag(const float* p) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    f32x3frag f;
#pragma unroll
    for (int j = 0; j < 8; ++j) MF<float>::set(f, j, v[j]);
    return f;
}

// Two floats rounded to bf16 (RNE) and packed, a in the low half
// (v_cvt_pk_bf16_f32).
M2_DEV uint32_t pk_bf16(float a, float b) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    typedef float f2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf2));
}
// a ~= hi + lo, b likewise, each part bf16 (packed pairs); the hi values are
// unpacked with bit operations (a bf16 is the high half of its float)
M2_DEV void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
    hi = pk_bf16(a, b);
    lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}
M2_DEV bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u4;
    const u4 v = {a, b, c, d};
    return __builtin_bit_cast(bf16x8, v);
}
// the two bf16 of a packed pair as floats
M2_DEV float bf16_lo(uint32_t d) { return __uint_as_float(d << 16); }
M2_DEV float bf16_hi(uint32_t d) { return __uint_as_float(d & 0xffff0000u); }

M2_DEV f32x4 zero4() { f32x4 z = {0.f, 0.f, 0.f, 0.f}; return z; }

// Index of the calling wavefront in its workgroup, as a scalar: branches and
// selects on it (or on values derived from it) stay scalar instead of being
// treated as divergent per lane.
M2_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Workgroup barrier that orders LDS accesses only.  __syncthreads() is a
// workgroup release/acquire fence and waits for every outstanding global load
// and store (vmcnt(0)); barriers that only hand LDS tiles between wavefronts
// use this one so that prefetches and output stores stay in flight.
// The wait is also issued through the builtin (0xc07f: lgkmcnt(0), vmcnt and
// expcnt left at their maxima), which the compiler's wait insertion sees: the
// asm one alone leaves it believing that earlier scalar loads (which complete
// out of order) and LDS accesses are still pending past the barrier, so its
// next LDS wait drains every read in flight instead of waiting for the one it
// needs.  The asm wait stays next to the barrier, where it orders the LDS
// accesses.
M2_DEV void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// LDS transpose read (gfx950 ds_read_b64_tr_b16): lane i of each 16-lane group
// receives column i of the 4 x 16 block of 16-bit elements whose rows the
// group's lanes address (lane 4 r + c supplies row r, columns 4 c .. 4 c + 3).
M2_DEV bf16x4 ds_read_tr(const void* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(const_cast<void*>(p)));
}

// Direct global -> LDS loads: lane l's 16 (4) bytes land at LDS byte address
// M0 + 16 l (4 l); `lds` (an LDS byte address) must be the same in every lane
// of the wavefront.  They are counted by vmcnt like any vector load but are
// invisible to the compiler's wait insertion: kernels wait for them
// explicitly (wait_vmem) before the barrier that hands the data to other
// wavefronts, and keep their own vector loads out of loops that have these in
// flight (the compiler would wait for those with too small a count).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// The compiler cannot see that these read their address registers, so they
// keep the two wait states it puts between a VALU write of an address (a
// 64-bit add, say) and a global_load_lds reading it: the M0 write and an
// s_nop.
M2_DEV void dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g) : "memory", "m0");
}
// the same with a non-temporal hint: rows read once that should not displace
// cached data
M2_DEV void dma16nt(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off nt"
                 ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g) : "memory", "m0");
}
M2_DEV void dma4(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off"
                 ::"s"(__builtin_amdgcn_readfirstlane(lds)), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop
template <int N> M2_DEV void wait_vmem() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
// LDS byte address of a __shared__ object
M2_DEV uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }

// Lane J of each 16-lane row, broadcast to the row (DPP row_newbcast).
template <int J> M2_DEV float row_bcast(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + J, 0xf, 0xf, false));
}

// ---------------------------------------------------------------------------
// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2).  Remap the hardware block id so that each XCD receives a contiguous
// range of work ids: neighbouring work items (heads of one group, which share
// B / C / CB tiles) then share an L2.
// ---------------------------------------------------------------------------
M2_DEV int xcd_remap(int bid, int nblocks) {
    const int nx = 8;
    int per = nblocks / nx, rem = nblocks % nx;
    int xcd = bid % nx, local = bid / nx;
    return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// ---------------------------------------------------------------------------
// error plumbing (host side)
// ---------------------------------------------------------------------------
namespace m2 {
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int check_launch(const char* what);
}  // namespace m2

#define M2_REQUIRE(cond, code, ...)                              \
    do {                                                         \
        if (!(cond)) return ::m2::set_error((code), __VA_ARGS__); \
    } while (0)

// element size of an M2_* dtype code (0 if unknown)
static inline size_t m2_dtype_size(int32_t dt) {
    return dt == M2_F32 ? 4 : dt == M2_BF16 ? 2 : 0;
}
