// RMSNorm, one launch per call, rows split across wavefront sub-groups.
//
// Semantics (kernels/fused_rmsnorm.py:10-21): fp32 sum of x^2 over the row,
// ms = sum / cols + eps, y = x * (1 / sqrt(ms)), y *= w, store bf16, then the
// wrapper casts to x.dtype (:32). Here the bf16-rounded value is converted to
// the output dtype in-register, so one launch covers the cast too.
//
// Layout: a row is split over LPR lanes (LPR = 64, 32, 16 or 8), each lane owns
// 8 consecutive columns per step (one 128-bit load for bf16/fp16), NSTEP steps
// cover the row, so the whole row stays in registers between the reduction and
// the scaled store (x is read once). The sum is a fixed xor-shuffle tree, so
// results are identical run to run. Rows longer than NSTEP_MAX*8*64 use a
// two-pass loop that re-reads x.
#include "ksl_common.h"

namespace ksl {
namespace {

constexpr int kRmsThreads = 256;
constexpr int kRmsRpw = 1;            // rows per wave of rmsnorm_rows_kernel
constexpr int64_t kRmsRowsFrom = 4096;  // from this many rows: the streaming kernel (small outputs stay cached)

template <int XD, int WD, int YD, int NSTEP, bool HAS_W>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_vec_kernel(
    const void* __restrict__ xv, const void* __restrict__ wv, void* __restrict__ yv, int64_t rows,
    int cols, int64_t xs, int64_t ys, float eps, int lpr_log2) {
    typedef typename Elem<XD>::T XT;
    typedef typename Elem<WD>::T WT;
    typedef typename Elem<YD>::T YT;
    const XT* x = static_cast<const XT*>(xv);
    const WT* w = static_cast<const WT*>(wv);
    YT* y = static_cast<YT*>(yv);

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int lpr = 1 << lpr_log2;
    const int sub = lane >> lpr_log2;
    const int sl = lane & (lpr - 1);
    const int rows_per_wave = kWave >> lpr_log2;
    const int64_t row =
        (static_cast<int64_t>(blockIdx.x) * (kRmsThreads / kWave) + wave) * rows_per_wave + sub;
    const bool row_ok = row < rows;
    const int stride_cols = 8 * lpr;

    constexpr int NS1 = NSTEP > 0 ? NSTEP : 1;
    if (NSTEP > 0) {
        YT* yr = y + (row_ok ? row : 0) * ys;
        rms_row<XD, WD, NS1, HAS_W>(x + (row_ok ? row : 0) * xs, w, cols, eps, sl, lpr_log2, row_ok,
                                    [&](int, int c0, const float (&o)[8]) {
                                        if (row_ok) store8<YD>(yr + c0, o);
                                    });
        return;
    }
    // long rows: two passes over x
    const XT* xr = x + (row_ok ? row : 0) * xs;
    float ss = 0.0f;
    for (int c0 = sl * 8; c0 < cols; c0 += stride_cols) {
        if (!row_ok) break;
        float t[8];
        load8<XD>(xr + c0, t);
#pragma unroll
        for (int j = 0; j < 8; ++j) ss = __builtin_fmaf(t[j], t[j], ss);
    }
    ss = xor_tree_sum(ss, lpr_log2);
    const float ms = ss / static_cast<float>(cols) + eps;
    const float r = 1.0f / __builtin_sqrtf(ms);
    if (!row_ok) return;
    YT* yr = y + row * ys;
    for (int c0 = sl * 8; c0 < cols; c0 += stride_cols) {
        float t[8], o[8], wf[8];
        load8<XD>(xr + c0, t);
        if (HAS_W) load8<WD>(w + c0, wf);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            o[j] = t[j] * r;
            if (HAS_W) o[j] = o[j] * wf[j];
            o[j] = bf16_bits_to_f32(f32_to_bf16_bits(o[j]));
        }
        store8<YD>(yr + c0, o);
    }
}

// Many rows of 512 to 4096 columns (one wave per row, NSTEP steps of 8
// columns per lane): a wave issues the weight's loads and then all of its
// rows' loads (RPW rows) before the first reduction; x is loaded and y stored
// non-temporal (each streamed once). Per row the arithmetic is rms_row's, so
// the bits are the same. At [32768, 2816] bf16 one row per wave with both
// hints is fastest (62-64 us against 71-77 us for rmsnorm_vec_kernel; two
// rows per wave 69 us, four 78 us: fewer waves in flight).
template <int XD, int WD, int YD, int NSTEP, bool HAS_W, int RPW>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_rows_kernel(
    const void* __restrict__ xv, const void* __restrict__ wv, void* __restrict__ yv, int64_t rows,
    int cols, int64_t xs, int64_t ys, float eps) {
    typedef typename Elem<XD>::T XT;
    typedef typename Elem<WD>::T WT;
    typedef typename Elem<YD>::T YT;
    const XT* x = static_cast<const XT*>(xv);
    const WT* w = static_cast<const WT*>(wv);
    YT* y = static_cast<YT*>(yv);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * (kRmsThreads / kWave) + threadIdx.x / kWave) * RPW;
    Raw8<WD> wr[HAS_W ? NSTEP : 1];
    Raw8<XD> xr[RPW][NSTEP];
    if constexpr (HAS_W) {
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) {
            const int c0 = s * 8 * kWave + lane * 8;
            wr[s] = c0 < cols ? raw_load8<WD>(w + c0) : Raw8<WD>{};
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t row = row0 + r;
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) {
            const int c0 = s * 8 * kWave + lane * 8;
            xr[r][s] = (row < rows && c0 < cols) ? raw_load8_nt<XD>(x + row * xs + c0) : Raw8<XD>{};
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int64_t row = row0 + r;
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) ss = rms_sumsq8<XD>(xr[r][s], ss);
        const float rs = rms_scale(ss, 6, cols, eps);
        if (row >= rows) continue;  // uniform over the wave
        YT* yr = y + row * ys;
#pragma unroll
        for (int s = 0; s < NSTEP; ++s) {
            const int c0 = s * 8 * kWave + lane * 8;
            if (c0 >= cols) continue;
            float xf[8], wf[8], o[8];
            raw_unpack8<XD>(xr[r][s], xf);
            if constexpr (HAS_W) raw_unpack8<WD>(wr[s], wf);
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = rms_apply<HAS_W>(xf[j], rs, HAS_W ? wf[j] : 1.0f);
            store8_nt<YD>(yr + c0, o);
        }
    }
}

// Any alignment / any cols: one wave per row, scalar element loop, two passes.
template <int XD, int WD, int YD, bool HAS_W>
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_scalar_kernel(
    const void* __restrict__ xv, const void* __restrict__ wv, void* __restrict__ yv, int64_t rows,
    int cols, int64_t xs, int64_t ys, float eps) {
    typedef typename Elem<XD>::T XT;
    typedef typename Elem<WD>::T WT;
    typedef typename Elem<YD>::T YT;
    const XT* x = static_cast<const XT*>(xv);
    const WT* w = static_cast<const WT*>(wv);
    YT* y = static_cast<YT*>(yv);
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t row = static_cast<int64_t>(blockIdx.x) * (kRmsThreads / kWave) + threadIdx.x / kWave;
    if (row >= rows) return;  // whole wave leaves together
    const XT* xr = x + row * xs;
    float ss = 0.0f;
    for (int c = lane; c < cols; c += kWave) {
        const float t = Elem<XD>::load(xr + c);
        ss = __builtin_fmaf(t, t, ss);
    }
    ss = xor_tree_sum(ss, 6);
    const float r = 1.0f / __builtin_sqrtf(ss / static_cast<float>(cols) + eps);
    YT* yr = y + row * ys;
    for (int c = lane; c < cols; c += kWave) {
        float o = Elem<XD>::load(xr + c) * r;
        if (HAS_W) o = o * Elem<WD>::load(w + c);
        Elem<YD>::store(yr + c, bf16_bits_to_f32(f32_to_bf16_bits(o)));
    }
}

template <int XD, int WD, int YD, bool HAS_W>
int launch_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int64_t cols, int64_t xs,
                   int64_t ys, float eps, hipStream_t st) {
    // 8-element vectors: 16 bytes for 2-byte types, two 16-byte halves for fp32;
    // rows stay 16-byte aligned when strides are multiples of 8 elements.
    const bool vec = (cols % 8 == 0) && (xs % 8 == 0) && (ys % 8 == 0) &&
                     (reinterpret_cast<uintptr_t>(x) % 16 == 0) &&
                     (reinterpret_cast<uintptr_t>(y) % 16 == 0) &&
                     (!HAS_W || reinterpret_cast<uintptr_t>(w) % 16 == 0);
    if (!vec) {
        const unsigned grid = static_cast<unsigned>((rows + 3) / 4);
        hipLaunchKernelGGL((rmsnorm_scalar_kernel<XD, WD, YD, HAS_W>), dim3(grid), dim3(kRmsThreads), 0,
                           st, x, w, y, rows, static_cast<int>(cols), xs, ys, eps);
        KSL_LAUNCH_CHECK();
        return KSL_OK;
    }
    const int64_t vecs = cols / 8;
    if (vecs >= kWave && vecs <= 8 * kWave && rows >= kRmsRowsFrom) {
        // one wave per row, kRmsRpw rows per wave
        const int nstep = static_cast<int>((vecs + kWave - 1) / kWave);
        const int64_t rows_per_block = (kRmsThreads / kWave) * kRmsRpw;
        const unsigned grid = static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block);
#define KSL_RMS_ROWS(NS)                                                                                    \
    hipLaunchKernelGGL((rmsnorm_rows_kernel<XD, WD, YD, NS, HAS_W, kRmsRpw>), dim3(grid), dim3(kRmsThreads), \
                       0, st, x, w, y, rows, static_cast<int>(cols), xs, ys, eps)
        if (nstep <= 2) KSL_RMS_ROWS(2);
        else if (nstep <= 4) KSL_RMS_ROWS(4);
        else if (nstep <= 6) KSL_RMS_ROWS(6);
        else KSL_RMS_ROWS(8);
#undef KSL_RMS_ROWS
        KSL_LAUNCH_CHECK();
        return KSL_OK;
    }
    int lpr_log2 = 3;  // 8 lanes minimum
    while ((1 << lpr_log2) < 64 && (1 << lpr_log2) < vecs) ++lpr_log2;
    const int lpr = 1 << lpr_log2;
    const int64_t nstep = (vecs + lpr - 1) / lpr;
    const int rows_per_block = (kRmsThreads / kWave) * (kWave / lpr);
    const unsigned grid = static_cast<unsigned>((rows + rows_per_block - 1) / rows_per_block);
#define KSL_RMS_CASE(NS)                                                                          \
    hipLaunchKernelGGL((rmsnorm_vec_kernel<XD, WD, YD, NS, HAS_W>), dim3(grid), dim3(kRmsThreads), \
                       0, st, x, w, y, rows, static_cast<int>(cols), xs, ys, eps, lpr_log2)
    if (nstep <= 1) KSL_RMS_CASE(1);
    else if (nstep <= 2) KSL_RMS_CASE(2);
    else if (nstep <= 4) KSL_RMS_CASE(4);
    else if (nstep <= 6) KSL_RMS_CASE(6);
    else if (nstep <= 8) KSL_RMS_CASE(8);
    else KSL_RMS_CASE(0);
#undef KSL_RMS_CASE
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

template <int XD, int WD, int YD>
int dispatch_w(const void* x, const void* w, void* y, int64_t rows, int64_t cols, int64_t xs,
               int64_t ys, float eps, hipStream_t st) {
    if (w) return launch_rmsnorm<XD, WD, YD, true>(x, w, y, rows, cols, xs, ys, eps, st);
    return launch_rmsnorm<XD, WD, YD, false>(x, w, y, rows, cols, xs, ys, eps, st);
}

template <int XD, int YD>
int dispatch_wd(int wd, const void* x, const void* w, void* y, int64_t rows, int64_t cols,
                int64_t xs, int64_t ys, float eps, hipStream_t st) {
    switch (wd) {
        case KSL_DTYPE_BF16: return dispatch_w<XD, KSL_DTYPE_BF16, YD>(x, w, y, rows, cols, xs, ys, eps, st);
        case KSL_DTYPE_F16: return dispatch_w<XD, KSL_DTYPE_F16, YD>(x, w, y, rows, cols, xs, ys, eps, st);
        case KSL_DTYPE_F32: return dispatch_w<XD, KSL_DTYPE_F32, YD>(x, w, y, rows, cols, xs, ys, eps, st);
    }
    return KSL_ERR_ARG;
}

template <int XD>
int dispatch_yd(int wd, int yd, const void* x, const void* w, void* y, int64_t rows, int64_t cols,
                int64_t xs, int64_t ys, float eps, hipStream_t st) {
    switch (yd) {
        case KSL_DTYPE_BF16: return dispatch_wd<XD, KSL_DTYPE_BF16>(wd, x, w, y, rows, cols, xs, ys, eps, st);
        case KSL_DTYPE_F16: return dispatch_wd<XD, KSL_DTYPE_F16>(wd, x, w, y, rows, cols, xs, ys, eps, st);
        case KSL_DTYPE_F32: return dispatch_wd<XD, KSL_DTYPE_F32>(wd, x, w, y, rows, cols, xs, ys, eps, st);
    }
    return KSL_ERR_ARG;
}

}  // namespace
}  // namespace ksl

extern "C" int ksl_rmsnorm(const void* x, int x_dtype, const void* w, int w_dtype, void* y,
                           int y_dtype, int64_t rows, int64_t cols, int64_t x_stride,
                           int64_t y_stride, float eps, void* stream) {
    using namespace ksl;
    if (rows < 0 || cols <= 0 || x_stride < cols || y_stride < cols) return KSL_ERR_SHAPE;
    if (cols > (1 << 30) || rows > (int64_t(1) << 40)) return KSL_ERR_SHAPE;
    if (rows == 0) return KSL_OK;
    if (!x || !y) return KSL_ERR_ARG;
    if (!w) w_dtype = KSL_DTYPE_BF16;
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (x_dtype) {
        case KSL_DTYPE_BF16: return dispatch_yd<KSL_DTYPE_BF16>(w_dtype, y_dtype, x, w, y, rows, cols, x_stride, y_stride, eps, st);
        case KSL_DTYPE_F16: return dispatch_yd<KSL_DTYPE_F16>(w_dtype, y_dtype, x, w, y, rows, cols, x_stride, y_stride, eps, st);
        case KSL_DTYPE_F32: return dispatch_yd<KSL_DTYPE_F32>(w_dtype, y_dtype, x, w, y, rows, cols, x_stride, y_stride, eps, st);
    }
    return KSL_ERR_ARG;
}
