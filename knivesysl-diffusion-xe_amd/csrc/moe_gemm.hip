// Grouped W4A16 expert GEMMs for gfx950: gate/up with the gated activation in
// the epilogue, and down. Bandwidth bound at a 256-token canvas: every packed
// weight byte is read from HBM once and decoded once in registers.
//
// Operand mapping onto v_mfma_f32_16x16x32_f16 (wave64):
//   A (16 x 32, activations): lane l holds row l%16, 8 K-slots of group l/16;
//   B (32 x 16, weights^T)  : lane l holds column l%16 (one weight row),
//                             8 K-slots of group l/16;
//   D (16 x 16, fp32)       : lane l holds column l%16, rows 4*(l/16)+0..3.
// A weight row's packed bytes load straight into B: one 32-bit word is 8
// consecutive K of that row, decoded by nib8_minus_zero into K-slot order
// {0,4,1,5,2,6,3,7}; the activations are stored in that same order, so
// activation and weight K match slot by slot.
//
// Dequantisation is factored per quantisation group: the MFMA consumes the
// exact integers (q - zero) in fp16, and the fp32 group partial is scaled once,
// acc += scale[n, g] * partial. That is two VALU ops per weight pair instead
// of the reference's three (q - z, * s, convert), with the same fp32
// accumulation. (Reference: fp16((q - z) * s) per weight then tl.dot,
// kernels/fused_moe_w4_v2.py:125-128, :172-175; the values agree within the
// fp16 rounding of the dequantised weight.)
//
// Work split: one workgroup per (expert, column block); the workgroup walks
// all rows routed to its expert (sorted slots offsets[e] .. offsets[e+1]) in
// chunks of 32 rows, one or two 16-row M tiles, so each weight byte is read
// once per 32 routed rows.
#include "ksl_common.h"

namespace ksl {
namespace {

// ---------------------------------------------------------------- gate / up
constexpr int kGuTiles = 2;                  // 16-column tiles of I per wave (x2: gate and up)
constexpr int kGuWaveCols = 16 * kGuTiles;   // 32
constexpr int kGuWaves = 2;
constexpr int kGuWgCols = kGuWaveCols * kGuWaves;  // 64 columns of I per workgroup
constexpr int kGuThreads = kGuWaves * kWave;
constexpr int kGuPrefetch = 2;               // quantisation groups in flight per wave

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

template <int ACT, int MT>
__device__ __forceinline__ void gateup_chunk(const f16* __restrict__ a16,
                                             const int32_t* __restrict__ rows, int mrows, int topk,
                                             int H, int G, const uint8_t* const (&wq)[2 * kGuTiles],
                                             const f16* const (&ws)[2 * kGuTiles],
                                             const f16* const (&wz)[2 * kGuTiles],
                                             f16* __restrict__ out2_rows, int I, int n0) {
    constexpr int NT = 2 * kGuTiles;  // gate tiles 0..kGuTiles-1, up tiles kGuTiles..
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;

    const f16* ap[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        int r = t * 16 + col;
        if (r >= mrows) r = mrows - 1;  // rows past the expert's last: loaded, never stored
        const int tok = rows[r] / topk;
        ap[t] = a16 + static_cast<int64_t>(tok) * H + c * 32;
    }

    f32x4 acc[NT][MT];
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wb[kGuPrefetch][NT];
#pragma unroll
    for (int p = 0; p < kGuPrefetch; ++p)
        if (p < G)
#pragma unroll
            for (int j = 0; j < NT; ++j) wb[p][j] = *reinterpret_cast<const u32x4*>(wq[j] + p * 64);

    for (int g0 = 0; g0 < G; g0 += kGuPrefetch) {
#pragma unroll
        for (int p = 0; p < kGuPrefetch; ++p) {
            const int g = g0 + p;
            if (g < G) {
                u32x4 w[NT];
#pragma unroll
                for (int j = 0; j < NT; ++j) w[j] = wb[p][j];
                if (g + kGuPrefetch < G) {
#pragma unroll
                    for (int j = 0; j < NT; ++j)
                        wb[p][j] = *reinterpret_cast<const u32x4*>(wq[j] + (g + kGuPrefetch) * 64);
                }
                f16x8 a[MT][4];
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        a[t][i] = *reinterpret_cast<const f16x8*>(ap[t] + g * 128 + i * 8);
                float s[NT];
                f16x2 zc[NT];
#pragma unroll
                for (int j = 0; j < NT; ++j) {
                    s[j] = static_cast<float>(ws[j][g]);
                    const f16 z = wz[j][g] + static_cast<f16>(1024.0f);
                    zc[j] = f16x2{z, z};
                }
                f32x4 part[NT][MT];
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
#pragma unroll
                    for (int j = 0; j < NT; ++j) {
                        const f16x8 b = nib8_minus_zero(w[j][i], zc[j]);
#pragma unroll
                        for (int t = 0; t < MT; ++t) part[j][t] = mfma16x16x32(a[t][i], b, part[j][t]);
                    }
                }
#pragma unroll
                for (int j = 0; j < NT; ++j)
#pragma unroll
                    for (int t = 0; t < MT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            acc[j][t][r] = __builtin_fmaf(s[j], part[j][t][r], acc[j][t][r]);
            }
        }
    }

#pragma unroll
    for (int j = 0; j < kGuTiles; ++j) {
        const int sc = perm8_store_index(n0 + 16 * j + col);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = t * 16 + 4 * c + r;
                if (row < mrows)
                    out2_rows[static_cast<int64_t>(row) * I + sc] =
                        static_cast<f16>(act_times_up<ACT>(acc[j][t][r], acc[kGuTiles + j][t][r]));
            }
    }
}

template <int ACT>
__global__ __launch_bounds__(kGuThreads) void gateup_act_kernel(
    const f16* __restrict__ a16, const int32_t* __restrict__ sorted_rows,
    const int32_t* __restrict__ offsets, int topk, const uint8_t* __restrict__ gu_q,
    const f16* __restrict__ gu_s, const f16* __restrict__ gu_z, int I, int H,
    f16* __restrict__ out2) {
    const int nb_per_e = I / kGuWgCols;
    const int e = blockIdx.x / nb_per_e;
    const int nb = blockIdx.x - e * nb_per_e;
    const int start = offsets[e];
    const int M = offsets[e + 1] - start;
    if (M <= 0) return;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int n0 = nb * kGuWgCols + wave * kGuWaveCols;
    const int G = H >> 7;
    const int64_t rb = H >> 1;

    const uint8_t* wq[2 * kGuTiles];
    const f16* ws[2 * kGuTiles];
    const f16* wz[2 * kGuTiles];
#pragma unroll
    for (int j = 0; j < kGuTiles; ++j) {
        const int64_t rg = static_cast<int64_t>(e) * 2 * I + n0 + 16 * j + col;  // gate row
        const int64_t ru = rg + I;                                               // up row
        wq[j] = gu_q + rg * rb + c * 16;
        wq[kGuTiles + j] = gu_q + ru * rb + c * 16;
        ws[j] = gu_s + rg * G;
        ws[kGuTiles + j] = gu_s + ru * G;
        wz[j] = gu_z + rg * G;
        wz[kGuTiles + j] = gu_z + ru * G;
    }
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mrows = M - m0 < 32 ? M - m0 : 32;
        f16* o = out2 + static_cast<int64_t>(start + m0) * I;
        if (mrows <= 16)
            gateup_chunk<ACT, 1>(a16, sorted_rows + start + m0, mrows, topk, H, G, wq, ws, wz, o, I, n0);
        else
            gateup_chunk<ACT, 2>(a16, sorted_rows + start + m0, mrows, topk, H, G, wq, ws, wz, o, I, n0);
    }
}

// --------------------------------------------------------------------- down
constexpr int kDnTiles = 4;                 // 16-column tiles of H per wave
constexpr int kDnWaveCols = 16 * kDnTiles;  // 64
constexpr int kDnWaves = 4;
constexpr int kDnWgCols = kDnWaveCols * kDnWaves;  // 256
constexpr int kDnThreads = kDnWaves * kWave;
constexpr int kDnPrefetch = 4;

template <int MT>
__device__ __forceinline__ void down_chunk(const f16* __restrict__ out2_rows, int mrows, int I, int G,
                                           const uint8_t* const (&wq)[kDnTiles],
                                           const f16* const (&ws)[kDnTiles],
                                           const f16* const (&wz)[kDnTiles],
                                           f16* __restrict__ out3_rows, int H, int n0) {
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const f16* ap[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        int r = t * 16 + col;
        if (r >= mrows) r = mrows - 1;
        ap[t] = out2_rows + static_cast<int64_t>(r) * I + c * 16;
    }
    f32x4 acc[kDnTiles][MT];
#pragma unroll
    for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x2 wb[kDnPrefetch][kDnTiles];
#pragma unroll
    for (int p = 0; p < kDnPrefetch; ++p)
        if (p < G)
#pragma unroll
            for (int j = 0; j < kDnTiles; ++j) wb[p][j] = *reinterpret_cast<const u32x2*>(wq[j] + p * 32);

    for (int g0 = 0; g0 < G; g0 += kDnPrefetch) {
#pragma unroll
        for (int p = 0; p < kDnPrefetch; ++p) {
            const int g = g0 + p;
            if (g < G) {
                u32x2 w[kDnTiles];
#pragma unroll
                for (int j = 0; j < kDnTiles; ++j) w[j] = wb[p][j];
                if (g + kDnPrefetch < G) {
#pragma unroll
                    for (int j = 0; j < kDnTiles; ++j)
                        wb[p][j] = *reinterpret_cast<const u32x2*>(wq[j] + (g + kDnPrefetch) * 32);
                }
                f16x8 a[MT][2];
#pragma unroll
                for (int t = 0; t < MT; ++t)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        a[t][i] = *reinterpret_cast<const f16x8*>(ap[t] + g * 64 + i * 8);
                float s[kDnTiles];
                f16x2 zc[kDnTiles];
#pragma unroll
                for (int j = 0; j < kDnTiles; ++j) {
                    s[j] = static_cast<float>(ws[j][g]);
                    const f16 z = wz[j][g] + static_cast<f16>(1024.0f);
                    zc[j] = f16x2{z, z};
                }
                f32x4 part[kDnTiles][MT];
#pragma unroll
                for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
                    for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int i = 0; i < 2; ++i) {
#pragma unroll
                    for (int j = 0; j < kDnTiles; ++j) {
                        const f16x8 b = nib8_minus_zero(w[j][i], zc[j]);
#pragma unroll
                        for (int t = 0; t < MT; ++t) part[j][t] = mfma16x16x32(a[t][i], b, part[j][t]);
                    }
                }
#pragma unroll
                for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
                    for (int t = 0; t < MT; ++t)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            acc[j][t][r] = __builtin_fmaf(s[j], part[j][t][r], acc[j][t][r]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < kDnTiles; ++j) {
        const int n = n0 + 16 * j + col;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = t * 16 + 4 * c + r;
                if (row < mrows) out3_rows[static_cast<int64_t>(row) * H + n] = static_cast<f16>(acc[j][t][r]);
            }
    }
}

__global__ __launch_bounds__(kDnThreads) void down_kernel(const f16* __restrict__ out2,
                                                         const int32_t* __restrict__ offsets,
                                                         const uint8_t* __restrict__ dn_q,
                                                         const f16* __restrict__ dn_s,
                                                         const f16* __restrict__ dn_z, int H, int I,
                                                         f16* __restrict__ out3) {
    const int nb_per_e = (H + kDnWgCols - 1) / kDnWgCols;
    const int e = blockIdx.x / nb_per_e;
    const int nb = blockIdx.x - e * nb_per_e;
    const int start = offsets[e];
    const int M = offsets[e + 1] - start;
    if (M <= 0) return;
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int n0 = nb * kDnWgCols + wave * kDnWaveCols;
    if (n0 >= H) return;  // whole wave (H % 64 == 0)
    const int G = I >> 6;
    const int64_t rb = I >> 1;
    const uint8_t* wq[kDnTiles];
    const f16* ws[kDnTiles];
    const f16* wz[kDnTiles];
#pragma unroll
    for (int j = 0; j < kDnTiles; ++j) {
        const int64_t rn = static_cast<int64_t>(e) * H + n0 + 16 * j + col;
        wq[j] = dn_q + rn * rb + c * 8;
        ws[j] = dn_s + rn * G;
        wz[j] = dn_z + rn * G;
    }
    for (int m0 = 0; m0 < M; m0 += 32) {
        const int mrows = M - m0 < 32 ? M - m0 : 32;
        const f16* a = out2 + static_cast<int64_t>(start + m0) * I;
        f16* o = out3 + static_cast<int64_t>(start + m0) * H;
        if (mrows <= 16)
            down_chunk<1>(a, mrows, I, G, wq, ws, wz, o, H, n0);
        else
            down_chunk<2>(a, mrows, I, G, wq, ws, wz, o, H, n0);
    }
}

}  // namespace

int launch_gateup(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                  const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H,
                  int64_t I, int act, void* out2, hipStream_t st) {
    if (!a16 || !sorted_rows || !offsets || !gu_q || !gu_s || !gu_z || !out2) return KSL_ERR_ARG;
    if (E <= 0 || H <= 0 || I <= 0 || topk <= 0) return KSL_ERR_SHAPE;
    if (H % 128 != 0 || I % kGuWgCols != 0) return KSL_ERR_SHAPE;
    if (E * 2 * I * (H / 2) >= (int64_t(1) << 40)) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(gu_q) % 16 || reinterpret_cast<uintptr_t>(a16) % 16 ||
        reinterpret_cast<uintptr_t>(gu_s) % 2 || reinterpret_cast<uintptr_t>(gu_z) % 2 ||
        reinterpret_cast<uintptr_t>(out2) % 2)
        return KSL_ERR_ALIGN;
    const unsigned grid = static_cast<unsigned>(E * (I / kGuWgCols));
    const f16* a = static_cast<const f16*>(a16);
    const f16* s = static_cast<const f16*>(gu_s);
    const f16* z = static_cast<const f16*>(gu_z);
    f16* o = static_cast<f16*>(out2);
    if (act == KSL_ACT_GELU_TANH)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_GELU_TANH>), dim3(grid), dim3(kGuThreads), 0, st, a,
                           sorted_rows, offsets, static_cast<int>(topk), gu_q, s, z, static_cast<int>(I),
                           static_cast<int>(H), o);
    else if (act == KSL_ACT_SILU)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_SILU>), dim3(grid), dim3(kGuThreads), 0, st, a,
                           sorted_rows, offsets, static_cast<int>(topk), gu_q, s, z, static_cast<int>(I),
                           static_cast<int>(H), o);
    else
        return KSL_ERR_ARG;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

int launch_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                const void* dn_z, int64_t E, int64_t H, int64_t I, void* out3, hipStream_t st) {
    if (!out2 || !offsets || !dn_q || !dn_s || !dn_z || !out3) return KSL_ERR_ARG;
    if (E <= 0 || H <= 0 || I <= 0) return KSL_ERR_SHAPE;
    if (H % 64 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (E * H * (I / 2) >= (int64_t(1) << 40)) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(dn_q) % 8 || reinterpret_cast<uintptr_t>(out2) % 16 ||
        reinterpret_cast<uintptr_t>(dn_s) % 2 || reinterpret_cast<uintptr_t>(dn_z) % 2 ||
        reinterpret_cast<uintptr_t>(out3) % 2)
        return KSL_ERR_ALIGN;
    const unsigned grid = static_cast<unsigned>(E * ((H + kDnWgCols - 1) / kDnWgCols));
    hipLaunchKernelGGL(down_kernel, dim3(grid), dim3(kDnThreads), 0, st, static_cast<const f16*>(out2),
                       offsets, dn_q, static_cast<const f16*>(dn_s), static_cast<const f16*>(dn_z),
                       static_cast<int>(H), static_cast<int>(I), static_cast<f16*>(out3));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

}  // namespace ksl

extern "C" int ksl_moe_gateup_act(const void* a16, const int32_t* sorted_rows, const int32_t* offsets,
                                  int64_t topk, const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                                  int64_t E, int64_t H, int64_t I, int act, void* out2, void* stream) {
    return ksl::launch_gateup(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, E, H, I, act, out2,
                              static_cast<hipStream_t>(stream));
}

extern "C" int ksl_moe_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q,
                            const void* dn_s, const void* dn_z, int64_t E, int64_t H, int64_t I,
                            void* out3, void* stream) {
    return ksl::launch_down(out2, offsets, dn_q, dn_s, dn_z, E, H, I, out3,
                            static_cast<hipStream_t>(stream));
}
