// omh_device.h — device helpers shared by the GDN kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define OMH_WAVE 64

// Activations with the reference's definitions (engines/qwen.c:158-160):
// sigmoid = 1/(1+e^-z); silu = z*sigmoid(z); softplus thresholded at 20.
__device__ __forceinline__ float omh_sigmoid(float z) { return 1.f / (1.f + expf(-z)); }
__device__ __forceinline__ float omh_silu(float z) { return z * omh_sigmoid(z); }
__device__ __forceinline__ float omh_softplus(float z) { return z > 20.f ? z : log1pf(expf(z)); }
// SiLU with the hardware exp2 and reciprocal (a few ulp; used where it is
// evaluated for every channel of every token of a prefill chunk).
__device__ __forceinline__ float omh_silu_fast(float z) { return z * __builtin_amdgcn_rcpf(1.f + __expf(-z)); }

// Workgroup barrier that orders LDS only: outstanding global loads stay in
// flight across it (a plain __syncthreads also drains them).  Correct
// wherever threads communicate through LDS alone.
__device__ __forceinline__ void omh_lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Butterfly sum over the lanes whose index differs in the bits [lo, 64).
template <int LO>
__device__ __forceinline__ float omh_xor_sum_from(float v) {
#pragma unroll
    for (int off = LO; off < OMH_WAVE; off <<= 1) v += __shfl_xor(v, off, OMH_WAVE);
    return v;
}
// Butterfly sum over the lanes whose index differs in the bits [0, HI).
template <int HI>
__device__ __forceinline__ float omh_xor_sum_below(float v) {
#pragma unroll
    for (int off = 1; off < HI; off <<= 1) v += __shfl_xor(v, off, OMH_WAVE);
    return v;
}

// Lane sums on the VALU: DPP row operations within a 16-lane row and
// gfx950's permlane swaps across rows, instead of the LDS permutes that
// __shfl_xor compiles to (each of those waits for an LDS round trip).
// Layouts (checked on the device): quad_perm 0xB1 / 0x4E = lane ^ 1 / ^ 2;
// row_ror:8 = lane ^ 8; row_ror:4 = lane - 4 within the row; row_half_mirror
// = 7 - lane within 8; permlane16_swap / permlane32_swap of (v, v) return
// v[lane & ~16], v[lane | 16] / v[lane & ~32], v[lane | 32].  Every lane of a
// summed group gets the same bits: each step adds two values that the two
// partner lanes hold identically (fp addition commutes).
template <int CTRL>
__device__ __forceinline__ float omh_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
// The swap's two results pass through an empty asm that takes both in
// registers of their own: used directly, this compiler gave both results
// the first one's register (p[0] + p[1] became p[0] + p[0]; seen in the
// generated code and on the device).
__device__ __forceinline__ float omh_swap_add(unsigned a, unsigned b) {
    asm("" : "+v"(a), "+v"(b));
    return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}
__device__ __forceinline__ float omh_swap_max(unsigned a, unsigned b) {
    asm("" : "+v"(a), "+v"(b));
    return fmaxf(__builtin_bit_cast(float, a), __builtin_bit_cast(float, b));
}
// v + (v of lane ^ 16) and the same for 32, max likewise: the operands a
// plain xor exchange gives, in one order or the other (both operations commute)
__device__ __forceinline__ float omh_swap16_max(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return omh_swap_max(p[0], p[1]);
}
__device__ __forceinline__ float omh_swap32_max(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return omh_swap_max(p[0], p[1]);
}
__device__ __forceinline__ float omh_swap16_sum(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return omh_swap_add(p[0], p[1]);
}
__device__ __forceinline__ float omh_swap32_sum(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const auto p = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return omh_swap_add(p[0], p[1]);
}
// Sum over the lanes whose index differs in the bits [log2 LO, 6).
template <int LO>
__device__ __forceinline__ float omh_lane_sum_from(float v) {
    static_assert(LO >= 1 && LO <= 32 && (LO & (LO - 1)) == 0, "lane group");
    if constexpr (LO <= 1) v += omh_dpp<0xB1>(v);
    if constexpr (LO <= 2) v += omh_dpp<0x4E>(v);
    if constexpr (LO <= 8) v += omh_dpp<0x128>(v);
    // lanes i and i ^ 8 now agree, so the rotation by 4 adds the other pair
    // of the 4-lane group {i, i ^ 4, i ^ 8, i ^ 12}
    if constexpr (LO <= 4) v += omh_dpp<0x124>(v);
    if constexpr (LO <= 16) v = omh_swap16_sum(v);
    return omh_swap32_sum(v);
}
// Sum over the lanes whose index differs in the bits [0, log2 HI).
template <int HI>
__device__ __forceinline__ float omh_lane_sum_below(float v) {
    static_assert(HI >= 1 && HI <= OMH_WAVE && (HI & (HI - 1)) == 0, "lane group");
    if constexpr (HI >= 2) v += omh_dpp<0xB1>(v);
    if constexpr (HI >= 4) v += omh_dpp<0x4E>(v);
    // the lanes of a quad now agree, so the mirror adds the other quad
    if constexpr (HI >= 8) v += omh_dpp<0x141>(v);
    if constexpr (HI >= 16) v += omh_dpp<0x128>(v);
    if constexpr (HI >= 32) v = omh_swap16_sum(v);
    if constexpr (HI >= 64) v = omh_swap32_sum(v);
    return v;
}

// Maximum over all 64 lanes (every lane gets it; max is exact, so the
// order does not matter).
__device__ __forceinline__ float omh_lane_max(float v) {
    v = fmaxf(v, omh_dpp<0xB1>(v));
    v = fmaxf(v, omh_dpp<0x4E>(v));
    v = fmaxf(v, omh_dpp<0x141>(v));
    v = fmaxf(v, omh_dpp<0x128>(v));
    v = omh_swap16_max(v);
    return omh_swap32_max(v);
}

// Sum over aligned groups of N = 1, 2 or 4 consecutive lanes (DPP quad
// permutes: no LDS round trip).
template <int N>
__device__ __forceinline__ float omh_group_sum(float v) {
    static_assert(N == 1 || N == 2 || N == 4, "lane group");
    if constexpr (N >= 2)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    if constexpr (N >= 4)
        v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    return v;
}

// Streaming (nontemporal) 16-byte load/store for data touched once per launch.
typedef float omh_v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 omh_ld_stream(const float *p) {
    const omh_v4f v = __builtin_nontemporal_load(reinterpret_cast<const omh_v4f *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void omh_st_stream(float *p, float4 a) {
    omh_v4f v = {a.x, a.y, a.z, a.w};
    __builtin_nontemporal_store(v, reinterpret_cast<omh_v4f *>(p));
}

// The same streaming accesses through a buffer resource: the tile's base
// address lives in scalar registers and each lane passes a 32-bit byte
// offset.  Cache policy: the nontemporal bit only (kOmhNT).  On MI355X this
// form moves a decode step's state about 2% faster than the global-address
// form above (30 layers x B = 1: 22.9 against 23.4 us), with fewer
// registers spent on addresses.
constexpr int kOmhNT = 2;
typedef unsigned omh_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t omh_rsrc(const void *base, int bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, bytes, 0x00020000);
}
__device__ __forceinline__ float4 omh_ld_stream_buf(__amdgpu_buffer_rsrc_t r, int off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kOmhNT));
}
__device__ __forceinline__ void omh_st_stream_buf(__amdgpu_buffer_rsrc_t r, int off, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(omh_v4u, v), r, off, 0, kOmhNT);
}

__device__ __forceinline__ float4 f4_scale(float4 a, float s) { return make_float4(a.x * s, a.y * s, a.z * s, a.w * s); }
__device__ __forceinline__ float4 f4_sub(float4 a, float4 b) { return make_float4(a.x - b.x, a.y - b.y, a.z - b.z, a.w - b.w); }
// c + a*s, component-wise
__device__ __forceinline__ float4 f4_fma(float4 a, float s, float4 c) {
    return make_float4(fmaf(a.x, s, c.x), fmaf(a.y, s, c.y), fmaf(a.z, s, c.z), fmaf(a.w, s, c.w));
}
__device__ __forceinline__ float4 f4_zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// x split into three int8 planes at the power-of-two scale 2^E of its block
// (omh_internal.h, i8_off): p1 = rint(x 2^-E), then the remainder twice at
// 7 more bits each.  With |x| < 2^(E+6) every p lies in [-64, 64], and each
// remainder is exact in fp32 (it is a multiple of ulp(x) no wider than 23
// bits), so |x - 2^E (p1 + p2 2^-7 + p3 2^-14)| <= 2^(E-15).
__device__ __forceinline__ int omh_i8_exponent(float maxabs) {
    if (!(maxabs > 0.f)) return 0;                        // all-zero block: every plane value is 0
    const int e = ilogbf(maxabs) - 5;
    return e < -120 ? -120 : e;
}
__device__ __forceinline__ void omh_i8_split(float x, int E, int8_t &p1, int8_t &p2, int8_t &p3) {
    const float a = rintf(ldexpf(x, -E));
    const float r1 = x - ldexpf(a, E);
    const float b = rintf(ldexpf(r1, 7 - E));
    const float r2 = r1 - ldexpf(b, E - 7);
    const float c = rintf(ldexpf(r2, 14 - E));
    p1 = (int8_t)(int)a;
    p2 = (int8_t)(int)b;
    p3 = (int8_t)(int)c;
}
