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

// Words between two counters of the one-launch expert FFN's ctl array (256
// bytes: no two counters share a cache line); the routing launch clears them.
constexpr int kCtlStride = 64;

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

// fp32 rounded to the nearest bf16 value (as a float).
__device__ __forceinline__ float bf16r(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }

// Wave-wide reductions of the ROCm device library (declared in the HIP
// headers, amd_warp_sync_functions.h): fixed DPP trees, deterministic; every
// lane of the wave receives the result.
extern "C" __device__ __attribute__((const)) float __ockl_wfred_max_f32(float);
extern "C" __device__ __attribute__((const)) float __ockl_wfred_add_f32(float);
extern "C" __device__ __attribute__((const)) unsigned long long __ockl_wfred_max_u64(unsigned long long);
extern "C" __device__ __attribute__((const)) int __ockl_wfred_max_i32(int);

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

// 8 consecutive elements kept as loaded (4 registers for 2-byte types): rows
// held across a reduction stay in this form and are widened on use.
template <int DT> struct Raw8 { u32x4 q[DT == KSL_DTYPE_F32 ? 2 : 1]; };
template <int DT> __device__ __forceinline__ Raw8<DT> raw_load8(const void* p) {
    Raw8<DT> r;
#pragma unroll
    for (int i = 0; i < (DT == KSL_DTYPE_F32 ? 2 : 1); ++i) r.q[i] = reinterpret_cast<const u32x4*>(p)[i];
    return r;
}
// The same load marked non-temporal (data read once: streamed past the caches).
template <int DT> __device__ __forceinline__ Raw8<DT> raw_load8_nt(const void* p) {
    Raw8<DT> r;
#pragma unroll
    for (int i = 0; i < (DT == KSL_DTYPE_F32 ? 2 : 1); ++i)
        r.q[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p) + i);
    return r;
}
template <int DT> __device__ __forceinline__ void raw_unpack8(const Raw8<DT>& r, float (&v)[8]) {
    if constexpr (DT == KSL_DTYPE_BF16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(r.q[0][i] << 16);
            v[2 * i + 1] = __uint_as_float(r.q[0][i] & 0xFFFF0000u);
        }
    } else if constexpr (DT == KSL_DTYPE_F16) {
        const f16x8 h = __builtin_bit_cast(f16x8, r.q[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = static_cast<float>(h[i]);
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = __uint_as_float(r.q[0][i]);
            v[4 + i] = __uint_as_float(r.q[1][i]);
        }
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

// store8 marked non-temporal (data written once, not read back soon).
template <int DT> __device__ __forceinline__ void store8_nt(void* p, const float (&v)[8]) {
    if constexpr (DT == KSL_DTYPE_BF16) {
        u32x4 q;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            q[i] = static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i])) |
                   (static_cast<uint32_t>(f32_to_bf16_bits(v[2 * i + 1])) << 16);
        __builtin_nontemporal_store(q, reinterpret_cast<u32x4*>(p));
    } else if constexpr (DT == KSL_DTYPE_F16) {
        f16x8 q;
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = static_cast<f16>(v[i]);
        __builtin_nontemporal_store(q, reinterpret_cast<f16x8*>(p));
    } else {
        __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]}, reinterpret_cast<f32x4*>(p));
        __builtin_nontemporal_store(f32x4{v[4], v[5], v[6], v[7]}, reinterpret_cast<f32x4*>(p) + 1);
    }
}

// ---- W4 nibble decode -------------------------------------------------------
// A 32-bit word of the packed format holds k0..k7 of one weight row, k_i in
// bits [4i, 4i+4) (byte j = q[2j] | q[2j+1] << 4). Each fp16 pair is built by
// one AND-OR into the mantissa of a power of two:
//   (w      & 0x000F000F) | 0x6400 6400 = (1024 + k0, 1024 + k4)   ulp 1
//   (w      & 0x00F000F0) | 0x5400 5400 = (  64 + k1,   64 + k5)   ulp 1/16
//   (w >> 8 & 0x000F000F) | 0x6400 6400 = (1024 + k2, 1024 + k6)
//   (w >> 8 & 0x00F000F0) | 0x5400 5400 = (  64 + k3,   64 + k7)
// so one word is 1 shift + 4 AND-ORs, and its MFMA K-slot order is
// {0,4,1,5,2,6,3,7}; activations are stored in the same order. Subtracting
// (1024 + zero) resp. (64 + zero) leaves q - zero, exact in fp16 for integer
// zero-points in [0, 15].
struct NibConsts {
    uint32_t m_lo, m_hi, b_lo, b_hi;
};

// The constants are laundered through empty asm so that the selector keeps
// them in registers and emits v_and_or_b32 (gfx9 VOP3 takes no literal).
__device__ __forceinline__ NibConsts nib_consts() {
    NibConsts c{0x000F000Fu, 0x00F000F0u, 0x64006400u, 0x54005400u};
    asm volatile("" : "+s"(c.m_lo), "+s"(c.m_hi));
    asm volatile("" : "+v"(c.b_lo), "+v"(c.b_hi));
    return c;
}

// Zero-point pairs for one weight row: (1024 + z, 1024 + z) and (64 + z, 64 + z).
struct ZeroPair {
    f16x2 lo, hi;
};
__device__ __forceinline__ ZeroPair zero_pair(f16 z) {
    const f16 a = z + static_cast<f16>(1024.0f), b = z + static_cast<f16>(64.0f);
    return ZeroPair{f16x2{a, a}, f16x2{b, b}};
}

__device__ __forceinline__ f16x8 nib8_minus_zero(uint32_t w, const ZeroPair& zc, const NibConsts& k) {
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = __builtin_bit_cast(f16x2, (w & k.m_lo) | k.b_lo) - zc.lo;
    const f16x2 h1 = __builtin_bit_cast(f16x2, (w & k.m_hi) | k.b_hi) - zc.hi;
    const f16x2 h2 = __builtin_bit_cast(f16x2, (w8 & k.m_lo) | k.b_lo) - zc.lo;
    const f16x2 h3 = __builtin_bit_cast(f16x2, (w8 & k.m_hi) | k.b_hi) - zc.hi;
    return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// fp16((q - zero) * scale) for the 8 nibbles of w, in K-slot order: the
// reference's dequantised weight (kernels/w4a16.py:47-48), exact: (q - zero)
// is an exact small integer and the product is rounded once to fp16.
__device__ __forceinline__ f16x8 nib8_dequant(uint32_t w, const ZeroPair& zc, f16x2 sc, const NibConsts& k) {
    const uint32_t w8 = w >> 8;
    const f16x2 h0 = (__builtin_bit_cast(f16x2, (w & k.m_lo) | k.b_lo) - zc.lo) * sc;
    const f16x2 h1 = (__builtin_bit_cast(f16x2, (w & k.m_hi) | k.b_hi) - zc.hi) * sc;
    const f16x2 h2 = (__builtin_bit_cast(f16x2, (w8 & k.m_lo) | k.b_lo) - zc.lo) * sc;
    const f16x2 h3 = (__builtin_bit_cast(f16x2, (w8 & k.m_hi) | k.b_hi) - zc.hi) * sc;
    return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

// Logical offset o within an 8-block -> storage index (inverse of {0,4,1,5,2,6,3,7}).
__device__ __forceinline__ int perm8_store_index(int n) {
    const int o = n & 7;
    return (n & ~7) | (o < 4 ? 2 * o : 2 * (o - 4) + 1);
}

// Activation storage order of the expert GEMMs. Within one quantisation group
// of GS elements (GS = 128 for gate/up over H, 64 for down over I), MFMA step
// i (GS/32 steps) of lane group c (4 groups) covers logical offsets
// c*(GS/4) + i*8 .. +8. Those 8-element chunks are stored step-major at
// i*32 + c*8, so one fragment block (fixed i, all 16 rows x 4 lane groups)
// reads 64 contiguous bytes per row; inside a chunk the K-slot order is
// {0,4,1,5,2,6,3,7}. Returns the storage index of logical column n.
template <int GS>
__device__ __forceinline__ int act_store_index(int n) {
    constexpr int Q = GS / 4;  // logical span of one lane group
    const int g0 = n & ~(GS - 1), o = n & (GS - 1);
    const int c = o / Q, i = (o % Q) >> 3;
    return g0 + i * 32 + c * 8 + (perm8_store_index(o) & 7);
}

// out2 (the down GEMM's activation) uses the 128-group order over its first
// i128 = I rounded down to a multiple of 128 columns, and the 64-group order
// over a trailing half group (I % 128 == 64).
__device__ __forceinline__ int out2_store_index(int n, int i128) {
    return n < i128 ? act_store_index<128>(n) : i128 + act_store_index<64>(n - i128);
}

__device__ __forceinline__ f32x4 mfma16x16x32(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---- RMSNorm arithmetic (kernels/fused_rmsnorm.py:10-21), shared by every
// kernel that normalises rows so that they all produce the same bits:
//   ss    = fma chain over the lane's 8-blocks in step order, then a fixed xor
//           tree over the row's lanes (rms_sumsq8, rms_scale);
//   r     = 1 / sqrt(ss / cols + eps)                      (rms_inv);
//   y     = bf16(x * r [* w]), returned as a float (rms_apply).
template <int XD>
__device__ __forceinline__ float rms_sumsq8(const Raw8<XD>& v, float ss) {
    float xf[8];
    raw_unpack8<XD>(v, xf);
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(xf[j], xf[j], ss);
    return ss;
}
// Sum over aligned groups of 2^lpr_log2 lanes (lpr_log2 <= 6) by the xor
// tree v += v[l ^ off], off = 2^(lpr_log2-1) .. 1 in that order: the bits of
// adding __shfl_xor(v, off) step by step (each step adds the same two values,
// and the addition commutes), with the partners fetched by cross-lane moves
// instead of LDS permutes: v_permlane32_swap / v_permlane16_swap for 32 and
// 16 (every lane then holds its half and the partner's, so their sum is the
// step's), DPP row_ror:8 for 8, quad_perm then row_half_mirror for 4
// (l ^ 3 ^ 7), quad_perm for 2 and 1. All lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}
__device__ __forceinline__ float xor_tree_sum(float v, int lpr_log2) {
    if (lpr_log2 >= 6) {
        const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if (lpr_log2 >= 5) {
        const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
    }
    if (lpr_log2 >= 4) v += dpp_mov<0x128>(v);                 // row_ror:8
    if (lpr_log2 >= 3) v += dpp_mov<0x141>(dpp_mov<0x1B>(v));  // quad_perm [3,2,1,0], row_half_mirror
    if (lpr_log2 >= 2) v += dpp_mov<0x4E>(v);                  // quad_perm [2,3,0,1]
    if (lpr_log2 >= 1) v += dpp_mov<0xB1>(v);                  // quad_perm [1,0,3,2]
    return v;
}
__device__ __forceinline__ float rms_inv(float ss, int cols, float eps) {
    const float ms = ss / static_cast<float>(cols) + eps;
    return 1.0f / __builtin_sqrtf(ms);
}
__device__ __forceinline__ float rms_scale(float ss, int lpr_log2, int cols, float eps) {
    return rms_inv(xor_tree_sum(ss, lpr_log2), cols, eps);
}
template <bool HAS_W>
__device__ __forceinline__ float rms_apply(float x, float r, float w) {
    float t = x * r;
    if constexpr (HAS_W) t = t * w;
    return bf16_bits_to_f32(f32_to_bf16_bits(t));  // the reference stores bf16
}

// RMSNorm of one row. The row is split over LPR = 1 << lpr_log2 lanes; lane
// sl owns 8 consecutive columns per step, NSTEP steps, so
// c0(s) = s*8*LPR + sl*8. x and w are loaded up front (one round trip, kept
// as loaded), and emit(s, c0, o) receives o[j] = bf16(x * r [* w]) as floats
// for every step with c0 < cols. Steps past the row end add exact zeros, so
// any NSTEP that covers the row gives the same bits.
template <int XD, int WD, int NSTEP, bool HAS_W, typename Emit>
__device__ __forceinline__ void rms_row(const typename Elem<XD>::T* __restrict__ xr,
                                        const typename Elem<WD>::T* __restrict__ w, int cols, float eps,
                                        int sl, int lpr_log2, bool row_ok, Emit&& emit) {
    const int stride_cols = 8 << lpr_log2;
    Raw8<XD> xv[NSTEP];
    Raw8<WD> wv[HAS_W ? NSTEP : 1];
    // loads not predicated (a step past the row end, or a row past the last,
    // reloads column 0 and drops it): predicated loads sit in branches, and the
    // compiler then waits for every load and store in flight (vmcnt(0)) before
    // each use instead of counting
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
        const int c0 = s * stride_cols + sl * 8;
        const int cc = row_ok && c0 < cols ? c0 : 0;
        xv[s] = raw_load8<XD>(xr + cc);
        if constexpr (HAS_W) wv[s] = raw_load8<WD>(w + cc);
    }
    __builtin_amdgcn_sched_barrier(0);  // all issued here, not sunk below the sum of squares
#pragma unroll
    for (int s = 0; s < NSTEP; ++s)
        if (!(row_ok && s * stride_cols + sl * 8 < cols)) xv[s] = Raw8<XD>{};  // zeros
    float ss = 0.0f;
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) ss = rms_sumsq8<XD>(xv[s], ss);
    const float r = rms_scale(ss, lpr_log2, cols, eps);
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
        const int c0 = s * stride_cols + sl * 8;
        if (c0 >= cols) continue;
        float xf[8], wf[8], o[8];
        // widen again here: keeping the first pass's floats live doubles the registers
#pragma unroll
        for (int i = 0; i < (XD == KSL_DTYPE_F32 ? 2 : 1); ++i) asm volatile("" : "+v"(xv[s].q[i]));
        raw_unpack8<XD>(xv[s], xf);
        if constexpr (HAS_W) raw_unpack8<WD>(wv[s], wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = rms_apply<HAS_W>(xf[j], r, HAS_W ? wf[j] : 1.0f);
        emit(s, c0, o);
    }
}


// ---- expert GEMM helpers shared by the kernels of moe_gemm.hip and moe_ffn.hip

template <int ACT>
__device__ __forceinline__ float act_times_up(float g, float u) {
    if (ACT == KSL_ACT_GELU_TANH) {
        // kernels/fused_moe_w4_v2.py:136-138
        const float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
        const float th = 2.0f / (1.0f + expf(-2.0f * inner)) - 1.0f;
        return 0.5f * g * (1.0f + th) * u;
    } else {
        return g / (1.0f + expf(-g)) * u;
    }
}

// act(g) * u with the hardware exp and reciprocal (v_exp_f32, v_rcp_f32,
// about 1 ulp each) instead of IEEE division: both forms are the logistic
// function, g * sigmoid(g) and, since 0.5 * (1 + tanh(x)) = 1 / (1 + e^(-2x)),
// the tanh-GELU. The fp32 differences are far below the fp16 rounding of
// the stored value. Used where the epilogue's arithmetic shows in the time
// (the row-block kernels of large routings).
template <int ACT>
__device__ __forceinline__ float act_times_up_fast(float g, float u) {
    float z;
    if (ACT == KSL_ACT_GELU_TANH)
        z = -2.0f * 0.7978845608028654f * (g + 0.044715f * g * g * g);
    else
        z = -g;
    return g * u * __builtin_amdgcn_rcpf(1.0f + __expf(z));
}

typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* gbl_vptr;

// Direct global -> LDS copy of one fragment block: lane L's 16 bytes land at
// lds_block + 16*L. lds_block must be wave-uniform. Completion is tracked by
// the issuing wave's vmcnt only.
__device__ __forceinline__ void dma16(const void* src, char* lds_block) {
    __builtin_amdgcn_global_load_lds((gbl_vptr)(const_cast<void*>(src)), (lds_vptr)lds_block, 16, 0, 0);
}

// s_waitcnt vmcnt(N), other counters left free (gfx9 encoding: vmcnt bits
// [3:0] and [15:14], expcnt [6:4], lgkmcnt [11:8]).
template <int N>
__device__ __forceinline__ void vm_wait() {
    static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Wait until at most n groups of k loads each are outstanding, n in [0, NMAX].
template <int K, int NMAX>
__device__ __forceinline__ void vm_wait_groups(int n) {
    if constexpr (NMAX > 0) {
        if (n >= NMAX) {
            vm_wait<NMAX * K>();
            return;
        }
        vm_wait_groups<K, NMAX - 1>(n);
    } else {
        vm_wait<0>();
    }
}

// Workgroup barrier of a wave whose only LDS writes are direct global->LDS
// loads that it has already waited for with vm_wait. __syncthreads() would
// add s_waitcnt vmcnt(0) for the still-pending loads of later groups and
// drain the ring; the asm statements keep the compiler from moving memory
// operations across the barrier.
__device__ __forceinline__ void dma_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// LDS position (16-byte unit) of MFMA lane (row, k-group c) within a fragment
// block of 16 rows x 64 bytes. Blocks are fetched row-major (4 consecutive
// lanes per 64-byte row: whole 64-byte segments per 4 lanes, which streams
// faster than 16 rows per 4 lanes), and chunk c of row r sits at
// r*4 + (c ^ swz(r)), swz(r) = (r/2 ^ 3*(r/8)) % 4, so that the 16 lanes of
// one k-group cover all 64 four-byte banks and each 8 of them (rows 0-7,
// 8-15) 32 distinct banks modulo 32.
__device__ __forceinline__ int frag_swz(int row) { return ((row >> 1) ^ (row >> 3) * 3) & 3; }
__device__ __forceinline__ int frag_pos(int row, int c) { return row * 4 + (c ^ frag_swz(row)); }
constexpr int kBlk = kWave * 16;                 // one fragment block: 64 lanes x 16 B

// Workgroup barrier after this wave's LDS reads (no wait on global memory).
__device__ __forceinline__ void lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}


// ---- launch geometry shared by the expert GEMM kernels

constexpr int kXcds = 8;

// Index of the calling wave in its workgroup, in a scalar register (branches
// on it are uniform).
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave); }

// blockIdx.x -> logical tile, placing consecutive logical tiles on one XCD
// (workgroups are dispatched round-robin over the XCDs).
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    if (nblocks % kXcds != 0) return bid;
    return (bid % kXcds) * (nblocks / kXcds) + bid / kXcds;
}

// Row blocks (large routings): the rows of each expert split into blocks of at
// most rb rows, numbered expert by expert (expert e has ceil(cnt_e / rb) of
// them). The block `blk` of a workgroup is found by wave 0 from the offsets
// (a wave scan of the per-expert block counts, 64 experts at a time) and
// broadcast through LDS; every thread gets the same (e, start, M), M = 0
// past the last block. One workgroup barrier, taken by every wave.
__device__ __forceinline__ void find_row_block(const int32_t* __restrict__ offsets, int E, int rb, int blk,
                                               int& e, int& start, int& M) {
    __shared__ int info[3];
    if (threadIdx.x < kWave) {
        const int lane = threadIdx.x;
        if (lane == 0) {
            info[0] = 0;
            info[1] = 0;
            info[2] = 0;
        }
        int base = 0;  // blocks of the experts before this batch
        for (int e0 = 0; e0 < E; e0 += kWave) {
            const int ex = e0 + lane;
            int o0 = 0, cnt = 0;
            if (ex < E) {
                o0 = offsets[ex];
                cnt = offsets[ex + 1] - o0;
            }
            const int nb = (cnt + rb - 1) / rb;
            int incl = nb;
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) {
                const int o = __shfl_up(incl, off, kWave);
                if (lane >= off) incl += o;
            }
            const int excl = base + incl - nb;
            if (ex < E && blk >= excl && blk < excl + nb) {
                const int b = blk - excl;
                info[0] = ex;
                info[1] = o0 + b * rb;
                info[2] = cnt - b * rb < rb ? cnt - b * rb : rb;
            }
            base += __shfl(incl, kWave - 1, kWave);
        }
    }
    __syncthreads();
    e = info[0];
    start = info[1];
    M = info[2];
}

// Buffer resource over `bytes` bytes at p (gfx9 raw buffer: stride 0, byte
// offsets; a store at an offset past the end is dropped by the hardware).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(p, 0, bytes, 0x00020000);
}
constexpr uint32_t kDropOffset = 0x80000000u;

}  // namespace ksl

#define KSL_LAUNCH_CHECK()                                   \
    do {                                                     \
        if (hipGetLastError() != hipSuccess) return KSL_ERR_LAUNCH; \
    } while (0)
