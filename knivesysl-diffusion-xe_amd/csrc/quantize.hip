// Asymmetric group-wise 4-bit quantisation of expert weights (load time).
//
// Replaces quantize_w4 (kernels/w4a16.py:19-32), which pack_experts_module /
// _pack_3d (kernels/pack_experts.py:34-41, 87-106) runs per expert on the
// bf16 weights. For each row r and group g of gs consecutive columns, in fp32:
//   wmin, wmax = min, max of the group
//   scale = max(wmax - wmin, 1e-8) / 15
//   zero  = clamp(rint(-wmin / scale), 0, 15)
//   q[k]  = clamp(rint(w[k] / scale + zero), 0, 15)
//   byte j of the row = q[2j] | q[2j+1] << 4;  scale, zero stored as fp16
// rint rounds half to even (torch.round); the divisions are IEEE divisions
// and w / scale + zero is a division then an addition (no fused form), so
// the bytes, scales and zero-points are those of the reference.
//
// One thread per pair of columns: a group of gs columns is gs/2 consecutive
// lanes of one wave (gs = 64: two groups per wave, gs = 128: one), reduced
// with xor shuffles inside the group.
#include "ksl_common.h"

namespace ksl {
namespace {

// Columns 2c and 2c+1 of a row as fp32 (exact for every storage type).
template <int DT>
__device__ __forceinline__ float2 load_pair(const void* p) {
    if constexpr (DT == KSL_DTYPE_F32) {
        return *reinterpret_cast<const float2*>(p);
    } else if constexpr (DT == KSL_DTYPE_F16) {
        const f16x2 v = *reinterpret_cast<const f16x2*>(p);
        return make_float2(static_cast<float>(v[0]), static_cast<float>(v[1]));
    } else {
        const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
        return make_float2(__uint_as_float(v << 16), __uint_as_float(v & 0xFFFF0000u));
    }
}

// clamp to [0, 15] by comparisons (torch.clamp's rule: a value equal to a
// bound, -0.0 included, is returned unchanged)
__device__ __forceinline__ float clamp15(float x) { return x < 0.0f ? 0.0f : (x > 15.0f ? 15.0f : x); }

template <int DT, int TG>
__global__ __launch_bounds__(256) void quantize_w4_kernel(const void* __restrict__ w, int64_t rows, int K,
                                                          uint8_t* __restrict__ q, f16* __restrict__ scale,
                                                          f16* __restrict__ zero) {
    const int64_t pair = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // global pair index
    const int kp = K / 2;
    const bool live = pair < rows * kp;
    const int64_t p = live ? pair : 0;
    const int64_t r = p / kp;
    const int c2 = static_cast<int>(p - r * kp);  // pair within the row
    constexpr int kEs = DT == KSL_DTYPE_F32 ? 4 : 2;
    const float2 v = load_pair<DT>(static_cast<const char*>(w) + (r * K + 2 * c2) * kEs);
    float mn = fminf(v.x, v.y), mx = fmaxf(v.x, v.y);
#pragma unroll
    for (int off = 1; off < TG; off <<= 1) {
        mn = fminf(mn, __shfl_xor(mn, off, kWave));
        mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    }
    const float d = mx - mn;
    const float s = __fdiv_rn(d < 1e-8f ? 1e-8f : d, 15.0f);
    const float z = clamp15(rintf(__fdiv_rn(-mn, s)));  // -0.0 stays -0.0, as torch.clamp keeps it
    const float q0 = clamp15(rintf(__fadd_rn(__fdiv_rn(v.x, s), z)));
    const float q1 = clamp15(rintf(__fadd_rn(__fdiv_rn(v.y, s), z)));
    if (!live) return;
    q[r * kp + c2] = static_cast<uint8_t>(static_cast<uint32_t>(q0) | (static_cast<uint32_t>(q1) << 4));
    if ((c2 & (TG - 1)) == 0) {
        const int64_t gi = r * (K / (2 * TG)) + c2 / TG;
        scale[gi] = static_cast<f16>(s);
        zero[gi] = static_cast<f16>(z);
    }
}

template <int DT>
int launch_quantize(const void* w, int64_t rows, int64_t K, int64_t gs, uint8_t* q, void* s, void* z,
                    hipStream_t st) {
    const int64_t pairs = rows * (K / 2);
    const int64_t grid = (pairs + 255) / 256;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    f16* sp = static_cast<f16*>(s);
    f16* zp = static_cast<f16*>(z);
    const int k = static_cast<int>(K);
    const dim3 g(static_cast<unsigned>(grid)), b(256);
    if (gs == 128) hipLaunchKernelGGL((quantize_w4_kernel<DT, 64>), g, b, 0, st, w, rows, k, q, sp, zp);
    else if (gs == 64) hipLaunchKernelGGL((quantize_w4_kernel<DT, 32>), g, b, 0, st, w, rows, k, q, sp, zp);
    else if (gs == 32) hipLaunchKernelGGL((quantize_w4_kernel<DT, 16>), g, b, 0, st, w, rows, k, q, sp, zp);
    else return KSL_ERR_SHAPE;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

// dequant_w4 (kernels/w4a16.py:35-48): W[n, k] = fp16((q - zero) * scale) with
// the difference and the product taken in fp32 (the reference promotes the
// fp16 nibble values against fp32 scale / zero), rounded once to fp16. One
// thread per 8 consecutive K of one row (4 packed bytes in, 16 bytes out);
// group_size % 8 == 0, so the 8 share one (scale, zero).
__global__ __launch_bounds__(256) void dequant_w4_kernel(const uint8_t* __restrict__ q, const f16* __restrict__ scale,
                                                         const f16* __restrict__ zero, int64_t rows, int K, int gs,
                                                         f16* __restrict__ out) {
    const int64_t per_row = K / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= rows * per_row) return;
    const int64_t r = i / per_row;
    const int c8 = static_cast<int>(i - r * per_row) * 8;
    const uint32_t w = *reinterpret_cast<const uint32_t*>(q + r * (K / 2) + c8 / 2);
    const int64_t gi = r * (K / gs) + c8 / gs;
    const float s = static_cast<float>(scale[gi]);
    const float z = static_cast<float>(zero[gi]);
    f16x8 v;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const float qj = static_cast<float>((w >> (4 * j)) & 15u);
        v[j] = static_cast<f16>(__fmul_rn(__fsub_rn(qj, z), s));
    }
    *reinterpret_cast<f16x8*>(out + r * K + c8) = v;
}

}  // namespace
}  // namespace ksl

extern "C" int ksl_dequant_w4(const uint8_t* qpacked, const void* scale, const void* zero, int64_t rows, int64_t K,
                              int64_t group_size, void* out, void* stream) {
    using namespace ksl;
    if (rows < 0 || K <= 0 || group_size <= 0) return KSL_ERR_SHAPE;
    if (group_size % 8 != 0 || K % group_size != 0 || K > (int64_t(1) << 30)) return KSL_ERR_SHAPE;
    if (rows == 0) return KSL_OK;
    if (!qpacked || !scale || !zero || !out) return KSL_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(qpacked) % 4 || reinterpret_cast<uintptr_t>(out) % 16 ||
        reinterpret_cast<uintptr_t>(scale) % 2 || reinterpret_cast<uintptr_t>(zero) % 2)
        return KSL_ERR_ALIGN;
    const int64_t n = rows * (K / 8);
    const int64_t grid = (n + 255) / 256;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipLaunchKernelGGL(dequant_w4_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), qpacked, static_cast<const f16*>(scale),
                       static_cast<const f16*>(zero), rows, static_cast<int>(K), static_cast<int>(group_size),
                       static_cast<f16*>(out));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

extern "C" int ksl_quantize_w4(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t group_size,
                               uint8_t* qpacked, void* scale, void* zero, void* stream) {
    using namespace ksl;
    if (rows < 0 || K <= 0 || group_size <= 0) return KSL_ERR_SHAPE;
    if (group_size != 32 && group_size != 64 && group_size != 128) return KSL_ERR_SHAPE;
    if (K % group_size != 0 || K > (int64_t(1) << 30)) return KSL_ERR_SHAPE;
    if (rows == 0) return KSL_OK;
    if (!w || !qpacked || !scale || !zero) return KSL_ERR_ARG;
    const int es = w_dtype == KSL_DTYPE_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(w) % (2 * es) || reinterpret_cast<uintptr_t>(scale) % 2 ||
        reinterpret_cast<uintptr_t>(zero) % 2)
        return KSL_ERR_ALIGN;
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (w_dtype) {
        case KSL_DTYPE_F32: return launch_quantize<KSL_DTYPE_F32>(w, rows, K, group_size, qpacked, scale, zero, st);
        case KSL_DTYPE_F16: return launch_quantize<KSL_DTYPE_F16>(w, rows, K, group_size, qpacked, scale, zero, st);
        case KSL_DTYPE_BF16: return launch_quantize<KSL_DTYPE_BF16>(w, rows, K, group_size, qpacked, scale, zero, st);
    }
    return KSL_ERR_ARG;
}
