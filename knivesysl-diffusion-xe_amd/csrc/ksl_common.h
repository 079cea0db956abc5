// Shared device helpers for the gfx950 (CDNA4) kernels of the fused layer path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/ksl.h"

namespace ksl {

typedef _Float16 f16;
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// ---- scalar conversions -----------------------------------------------------
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// fp32 -> bf16 bits, round-to-nearest-even, NaN -> 0x7FC0 (torch's rule).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint16_t f16_bits(f16 h) { return __builtin_bit_cast(uint16_t, h); }

// Element access by storage dtype code.
template <int DT> struct Elem;
template <> struct Elem<KSL_DTYPE_F32> {
    typedef float T;
    static __device__ __forceinline__ float load(const T* p) { return *p; }
    static __device__ __forceinline__ void store(T* p, float v) { *p = v; }
};
template <> struct Elem<KSL_DTYPE_F16> {
    typedef f16 T;
    static __device__ __forceinline__ float load(const T* p) { return static_cast<float>(*p); }
    static __device__ __forceinline__ void store(T* p, float v) { *p = static_cast<f16>(v); }
};
template <> struct Elem<KSL_DTYPE_BF16> {
    typedef uint16_t T;
    static __device__ __forceinline__ float load(const T* p) { return bf16_bits_to_f32(*p); }
    static __device__ __forceinline__ void store(T* p, float v) { *p = f32_to_bf16_bits(v); }
};

// Load 8 consecutive elements (16-byte aligned for 2-byte types, 32-byte for fp32).
template <int DT> __device__ __forceinline__ void load8(const void* p, float (&v)[8]);
template <> __device__ __forceinline__ void load8<KSL_DTYPE_BF16>(const void* p, float (&v)[8]) {
    u32x4 q = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(q[i] << 16);
        v[2 * i + 1] = __uint_as_float(q[i] & 0xFFFF0000u);
    }
}
template <> __device__ __forceinline__ void load8<KSL_DTYPE_F16>(const void* p, float (&v)[8]) {
    f16x8 q = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(q[i]);
}
template <> __device__ __forceinline__ void load8<KSL_DTYPE_F32>(const void* p, float (&v)[8]) {
    const f32x4* q = reinterpret_cast<const f32x4*>(p);
    f32x4 a = q[0], b = q[1];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = a[i];
        v[4 + i] = b[i];
    }
}

// Store 8 consecutive values (already rounded as the caller wants).
template <int DT> __device__ __forceinline__ void store8(void* p, const float (&v)[8]);
template <> __device__ __forceinline__ void store8<KSL_DTYPE_BF16>(void* p, const float (&v)[8]) {
    u32x4 q;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        q[i] = static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i])) |
               (static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i + 1])) << 16);
    *reinterpret_cast<u32x4*>(p) = q;
}
template <> __device__ __forceinline__ void store8<KSL_DTYPE_F16>(void* p, const float (&v)[8]) {
    f16x8 q;
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = static_cast<f16>(v[i]);
    *reinterpret_cast<f16x8*>(p) = q;
}
template <> __device__ __forceinline__ void store8<KSL_DTYPE_F32>(void* p, const float (&v)[8]) {
    f32x4* q = reinterpret_cast<f32x4*>(p);
    q[0] = f32x4{v[0], v[1], v[2], v[3]};
    q[1] = f32x4{v[4], v[5], v[6], v[7]};
}

// ---- W4 nibble decode -------------------------------------------------------
// A 32-bit word of the packed format holds k0..k7 of one weight row, k_i in
// bits [4i, 4i+4) (byte j = q[2j] | q[2j+1] << 4). OR-ing a nibble into the
// mantissa of fp16 1024.0 (0x6400) gives exactly 1024 + q. The four pairs come
// out as (k0,k4), (k1,k5), (k2,k6), (k3,k7), so the MFMA K-slot order of one
// word is {0,4,1,5,2,6,3,7}; activations are stored in the same order.
// zc = 1024 + zero (exact for integer zero-points in [0, 15]); the result is
// q - zero, exact in fp16.
// fp16((q - zero) * scale) for the 8 nibbles of w, in K-slot order: the
// reference's dequantised weight (kernels/w4a16.py:47-48), exact: (q - zero)
// is an exact small integer and the product is rounded once to fp16.
__device__ __forceinline__ f16x8 nib8_dequant(uint32_t w, f16x2 zc, f16x2 sc) {
    const uint32_t m = 0x000F000Fu, magic = 0x64006400u;
    f16x2 h0 = (__builtin_bit_cast(f16x2, (w & m) | magic) - zc) * sc;
    f16x2 h1 = (__builtin_bit_cast(f16x2, ((w >> 4) & m) | magic) - zc) * sc;
    f16x2 h2 = (__builtin_bit_cast(f16x2, ((w >> 8) & m) | magic) - zc) * sc;
    f16x2 h3 = (__builtin_bit_cast(f16x2, ((w >> 12) & m) | magic) - zc) * sc;
    return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

__device__ __forceinline__ f16x8 nib8_minus_zero(uint32_t w, f16x2 zc) {
    const uint32_t m = 0x000F000Fu, magic = 0x64006400u;
    f16x2 h0 = __builtin_bit_cast(f16x2, (w & m) | magic) - zc;
    f16x2 h1 = __builtin_bit_cast(f16x2, ((w >> 4) & m) | magic) - zc;
    f16x2 h2 = __builtin_bit_cast(f16x2, ((w >> 8) & m) | magic) - zc;
    f16x2 h3 = __builtin_bit_cast(f16x2, ((w >> 12) & m) | magic) - zc;
    return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// Logical offset o within an 8-block -> storage index (inverse of {0,4,1,5,2,6,3,7}).
__device__ __forceinline__ int perm8_store_index(int n) {
    const int o = n & 7;
    return (n & ~7) | (o < 4 ? 2 * o : 2 * (o - 4) + 1);
}

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

}  // namespace ksl

#define KSL_LAUNCH_CHECK()                                   \
    do {                                                     \
        if (hipGetLastError() != hipSuccess) return KSL_ERR_LAUNCH; \
    } while (0)
