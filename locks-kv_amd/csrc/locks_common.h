// Shared device/host helpers for the LOCKS gfx950 kernels.
//
// Everything here is CDNA4-specific: wave64, MFMA operand vector types, and
// the order-preserving fp32 <-> uint32 radix key used by the page selector
// (same key the reference's selector uses, selection/select_cuda.py:77-86).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace locks {

constexpr int kWave = 64;

// Workgroup barrier that orders LDS only: each wave waits for its own LDS
// accesses, not for its outstanding global stores (__syncthreads() also
// waits vmcnt(0) on gfx950, which stalls a barrier behind stores that no
// other thread of the workgroup reads).
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(((uint32_t)b) << 16);
}
// low / high bf16 of a packed 32-bit word -> fp32
__device__ __forceinline__ float bf16lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// fp32 -> bf16 bits, round to nearest even (NaN stays NaN)
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu))
        return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// order-preserving fp32 -> uint32 key (monotone for finite values and +-inf)
__device__ __forceinline__ uint32_t f2u(float f) {
    uint32_t u = __float_as_uint(f);
    uint32_t mask = (uint32_t)(-(int32_t)(u >> 31)) | 0x80000000u;
    return u ^ mask;
}
__device__ __forceinline__ float u2f(uint32_t x) {
    uint32_t mask = ((x >> 31) - 1u) | 0x80000000u;
    return __uint_as_float(x ^ mask);
}

// DPP row rotate (by N lanes inside each 16-lane row): a plain VALU move.
template <int N>
__device__ __forceinline__ int row_ror(int x) {
    return __builtin_amdgcn_update_dpp(0, x, 0x120 + N, 0xF, 0xF, false);
}
template <int N>
__device__ __forceinline__ float row_ror(float x) {
    return __int_as_float(row_ror<N>(__float_as_int(x)));
}

// Pair reductions across lanes l and l^16 / l^32 with the gfx950 permlane
// swaps (plain VALU, no LDS round trip).  Swapping a value with itself
// leaves {x[l], x[l^16]} (resp. {x[l], x[l^32]}) in the two results, in
// row order, so the pair sum / max equals x + shfl_xor(x, 16 / 32) bit for
// bit (fp32 add and max are commutative).
__device__ __forceinline__ float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Whole-wave max of unsigned keys, result in every lane (DPP row rotations,
// then the two pair swaps).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)row_ror<8>((int)v));
    v = max(v, (uint32_t)row_ror<4>((int)v));
    v = max(v, (uint32_t)row_ror<2>((int)v));
    v = max(v, (uint32_t)row_ror<1>((int)v));
    auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(r[0], r[1]);
    r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(r[0], r[1]);
}

// Whole-wave max / integer sum, result in every lane: row rotations, then
// the two pair swaps -- no LDS round trip.
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, row_ror<8>(v));
    v = fmaxf(v, row_ror<4>(v));
    v = fmaxf(v, row_ror<2>(v));
    v = fmaxf(v, row_ror<1>(v));
    return xor32_max(xor16_max(v));
}
__device__ __forceinline__ float wave_sum(float v) {
    v += row_ror<8>(v);
    v += row_ror<4>(v);
    v += row_ror<2>(v);
    v += row_ror<1>(v);
    return xor32_sum(xor16_sum(v));
}
__device__ __forceinline__ int wave_sum_i(int v) {
    v += row_ror<8>(v);
    v += row_ror<4>(v);
    v += row_ror<2>(v);
    v += row_ror<1>(v);
    const auto a = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = (int)a[0] + (int)a[1];
    const auto b = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return (int)b[0] + (int)b[1];
}

// Whole-wave inclusive integer prefix sum on DPP (no LDS crossbar trips):
// Hillis-Steele within each 16-lane row (row_shr 1, 2, 4, 8; lanes whose
// source falls outside the row keep 0), then row_bcast:15 adds row 0 / 2's
// totals to rows 1 / 3 and row_bcast:31 adds rows 0-1's total to rows 2-3.
__device__ __forceinline__ int wave_incl_scan_i(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);
    return v;
}

// Order LDS traffic between lanes of ONE wave (no cross-wave barrier).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__host__ __device__ __forceinline__ int cdiv(int a, int b) { return (a + b - 1) / b; }

// The six rki4 summary slabs of one layer as (base, row stride in bytes):
// field f of the (block, kv head) row i lives at base_f + i * stride_f.
// Contiguous slabs have the natural strides (8 d/2, 16, 8 page, 2 page, d,
// 2 bytes); a state that packs all six fields of a row together gives every
// field the same stride (the packed row size).
struct SlabRows {
    uint8_t* v4; uint8_t* vs; uint8_t* c8; uint8_t* cs; uint8_t* mu; uint8_t* mus;
    long sv4, svs, sc8, scs, smu, smus;
};

// Host side: the natural strides of geometry (d, page), or the caller's
// six (row_bytes != nullptr).
inline SlabRows slab_rows(const void* v4, const void* vs, const void* c8, const void* cs,
                          const void* mu, const void* mus, const int64_t* row_bytes, int d, int page) {
    SlabRows s;
    s.v4 = (uint8_t*)v4; s.vs = (uint8_t*)vs; s.c8 = (uint8_t*)c8;
    s.cs = (uint8_t*)cs; s.mu = (uint8_t*)mu; s.mus = (uint8_t*)mus;
    if (row_bytes) {
        s.sv4 = row_bytes[0]; s.svs = row_bytes[1]; s.sc8 = row_bytes[2];
        s.scs = row_bytes[3]; s.smu = row_bytes[4]; s.smus = row_bytes[5];
    } else {
        s.sv4 = 4L * d; s.svs = 16; s.sc8 = 8L * page; s.scs = 2L * page; s.smu = d; s.smus = 2;
    }
    return s;
}

// Host side: strides at least the field sizes, 16-byte aligned bases and
// strides for the fields read with 16-byte loads (all but mus), even mus.
inline bool slab_rows_ok(const SlabRows& s, int d, int page) {
    auto a16 = [](const void* p, long st) { return ((uintptr_t)p % 16 == 0) && (st % 16 == 0); };
    return s.sv4 >= 4L * d && s.svs >= 16 && s.sc8 >= 8L * page && s.scs >= 2L * page && s.smu >= d &&
           s.smus >= 2 && a16(s.v4, s.sv4) && a16(s.vs, s.svs) && a16(s.c8, s.sc8) &&
           a16(s.cs, s.scs) && a16(s.mu, s.smu) && ((uintptr_t)s.mus % 2 == 0) && (s.smus % 2 == 0);
}

// Largest byte offset a kernel forms into any slab for `rows` rows.
inline long slab_rows_extent(const SlabRows& s, long rows) {
    long m = s.sv4;
    for (long v : {s.svs, s.sc8, s.scs, s.smu, s.smus}) m = v > m ? v : m;
    return rows * m;
}

}  // namespace locks

// ---- host-side error plumbing for the C ABI -------------------------------
namespace locks {
void set_error(const char* fmt, ...);
int check_launch(const char* what);
}  // namespace locks

#define LOCKS_REQUIRE(cond, ...)                                              \
    do {                                                                      \
        if (!(cond)) {                                                        \
            ::locks::set_error(__VA_ARGS__);                                  \
            return -1;                                                        \
        }                                                                     \
    } while (0)
