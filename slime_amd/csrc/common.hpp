// common.hpp — shared device helpers for the gfx950 CA kernels.
//
// Storage types are fp32 or bf16 (raw 16-bit words); every kernel computes in
// fp32 (Jacobi in fp64). Wavefronts are 64 lanes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace slime {

typedef uint16_t bf16_t;  // raw bfloat16 bits
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_v;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_v;
typedef __attribute__((ext_vector_type(16))) float f32x16;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) unsigned int u32x4;
typedef __attribute__((ext_vector_type(2))) unsigned int u32x2;

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
    return __builtin_bit_cast(float, (uint32_t)v << 16);
}
__device__ __forceinline__ float bf16lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) {
    return __builtin_bit_cast(float, w & 0xffff0000u);
}
// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32 on gfx950).
__device__ __forceinline__ bf16_t f32_to_bf16(float f) {
    return __builtin_bit_cast(bf16_t, (__bf16)f);
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const bf16x2_v v = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, v);
}

// Storage-type traits: load/store pairs of adjacent channels as float2.
template <typename T> struct Store;
template <> struct Store<float> {
    static constexpr int kBytes = 4;
    __device__ static __forceinline__ float2 load2(const float* p) {
        return *reinterpret_cast<const float2*>(p);
    }
    __device__ static __forceinline__ void store2(float* p, float a, float b) {
        *reinterpret_cast<float2*>(p) = make_float2(a, b);
    }
    __device__ static __forceinline__ float round(float v) { return v; }
    __device__ static __forceinline__ float to_f32(float v) { return v; }
    __device__ static __forceinline__ float from_f32(float v) { return v; }
};
template <> struct Store<bf16_t> {
    static constexpr int kBytes = 2;
    __device__ static __forceinline__ float2 load2(const bf16_t* p) {
        const uint32_t w = *reinterpret_cast<const uint32_t*>(p);
        return make_float2(bf16lo(w), bf16hi(w));
    }
    __device__ static __forceinline__ void store2(bf16_t* p, float a, float b) {
        *reinterpret_cast<uint32_t*>(p) = pack_bf16x2(a, b);
    }
    __device__ static __forceinline__ float round(float v) { return bf16_to_f32(f32_to_bf16(v)); }
    __device__ static __forceinline__ float to_f32(bf16_t v) { return bf16_to_f32(v); }
    __device__ static __forceinline__ bf16_t from_f32(float v) { return f32_to_bf16(v); }
};

// ---- wave64 reductions -------------------------------------------------------
// DPP steps inside each 16-lane row (quad_perm 1,0,3,2; quad_perm 2,3,0,1;
// row_half_mirror; row_mirror) leave every lane holding its row's sum; the four
// row sums are then combined through v_readlane, so the result is uniform.
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    const int iv = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
    return (r0 + r1) + (r2 + r3);
}

// fp64 wave sum with the same DPP row steps and row order (each DPP move carries
// the two 32-bit halves of the value).
template <int kCtrl>
__device__ __forceinline__ double dpp_f64(double v) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)b, kCtrl, 0xf, 0xf, false);
    const unsigned hi = (unsigned)__builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), kCtrl, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double readlane_f64(double v, int l) {
    const unsigned long long b = __builtin_bit_cast(unsigned long long, v);
    const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, l);
    const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), l);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
__device__ __forceinline__ double wave_sum64(double v) {
    v += dpp_f64<0xB1>(v);
    v += dpp_f64<0x4E>(v);
    v += dpp_f64<0x141>(v);
    v += dpp_f64<0x140>(v);
    return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// Sum over aligned groups of kN consecutive lanes (kN = 1, 2, 4 or 8), every lane of
// the group receiving the group's sum (DPP quad_perm and row_half_mirror steps).
template <int kN>
__device__ __forceinline__ float group_sum_n(float v) {
    static_assert(kN == 1 || kN == 2 || kN == 4 || kN == 8, "group of 1, 2, 4 or 8 lanes");
    if constexpr (kN >= 2) v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (kN >= 4) v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (kN >= 8) v += dpp_f32<0x141>(v);  // row_half_mirror
    return v;
}

// ---- direct global->LDS loads -------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void_t;

// LDS byte address of a __shared__ object.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
    return (unsigned)(size_t)(const lds_void_t*)p;
}

// s_waitcnt vmcnt(0): this wave's vector-memory operations, direct loads included,
// have completed.
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// One direct global->LDS load (global_load_lds_dwordx4 with an SGPR base and a 32-bit
// lane offset): 16 bytes per lane from base + voff land at LDS byte address
// lds + 16 * lane. Issued through inline asm, so that the per-lane addresses stay
// 32-bit and the compiler does not make every later LDS read wait for all such loads
// in flight (it cannot tell which buffer they fill): each kernel waits for them
// itself (vmcnt) before the barrier that publishes them. base and lds are uniform.
__device__ __forceinline__ void dma16_lds(const void* base, unsigned voff, unsigned lds) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2"
        :
        : "s"(lds), "v"(voff), "s"(base)
        : "memory", "m0");
}

// As dma16_lds, with the nontemporal hint: for rows read once, so that they do not
// displace from L2 the lines that neighbouring workgroups share.
__device__ __forceinline__ void dma16_lds_nt(const void* base, unsigned voff, unsigned lds) {
    asm volatile(
        "s_mov_b32 m0, %0\n\t"
        "s_nop 0\n\t"
        "global_load_lds_dwordx4 %1, %2 nt"
        :
        : "s"(lds), "v"(voff), "s"(base)
        : "memory", "m0");
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float rcp_fast(float x) { return __builtin_amdgcn_rcpf(x); }

// tanh-GELU written as x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3):
// 0.5 x (1 + tanh u) = x / (1 + exp(-2u)). exp(-2u) = 2^(x (k0 + k1 x^2)).
constexpr float kGeluK0 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
constexpr float kGeluK1 = kGeluK0 * 0.044715f;
__device__ __forceinline__ float gelu_tanh(float x) {
    const float e = exp2_fast(x * __builtin_fmaf(kGeluK1, x * x, kGeluK0));
    return x * rcp_fast(1.0f + e);
}

// gelu_tanh of N independent values in place, one stage at a time over all of them,
// so that their transcendentals issue back to back. Per value the operations and
// their order are those of gelu_tanh, and so are the results.
template <int N>
__device__ __forceinline__ void gelu_tanh_n(float (&v)[N]) {
    float t[N];
#pragma unroll
    for (int e = 0; e < N; ++e) t[e] = v[e] * v[e];
#pragma unroll
    for (int e = 0; e < N; ++e) t[e] = __builtin_fmaf(kGeluK1, t[e], kGeluK0);
#pragma unroll
    for (int e = 0; e < N; ++e) t[e] = exp2_fast(v[e] * t[e]);
#pragma unroll
    for (int e = 0; e < N; ++e) t[e] = rcp_fast(1.0f + t[e]);
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = v[e] * t[e];
}

}  // namespace slime
