// Fixed-order top-k combine and the fused forward's orchestration.
//
// Combine (kernels/fused_moe_w4_v2.py:248-263): for each token t and column,
// acc = 0; for k = 0..topk-1: acc = fma(fp32(w[t,k]), fp32(out3[inv[t*topk+k]]), acc);
// y = round(acc). No atomics; the order is the top-k slot order, so the output
// is bit-identical run to run. Each thread owns 8 consecutive columns of one
// token (128-bit loads of out3, 128-bit stores of y).
#include "ksl_common.h"

#include <atomic>
#include <mutex>

namespace ksl {

// bcnt: workspace for the per-block counts of the multi-block routing
// (ceil(T*topk / 1024) * E int32), or null for the single-workgroup routing.
// zero: nzero int32 words the routing launch clears (the expert FFN's
// counters), or null.
int route_compact(const int64_t* ids, int64_t T, int64_t topk, int64_t E, int32_t* sorted_rows,
                  int32_t* offsets, int32_t* inv, const void* hidden, int hd, int64_t hstride,
                  int64_t H, void* a16, int32_t* bcnt, hipStream_t st, int32_t* zero, int nzero);
int route_norm(const int64_t* ids, int64_t T, int64_t topk, int64_t E, int32_t* sorted_rows,
               int32_t* offsets, int32_t* inv, const void* x, int xd, int64_t xs, const void* w,
               int wd, float eps, int64_t H, void* a16, int32_t* bcnt, hipStream_t st, int32_t* zero, int nzero);
// the fused expert FFN (moe_ffn.hip)
size_t ffn_ctl_words(int64_t E);
bool ffn_supported(int64_t E, int64_t H, int64_t I, int64_t nrows);
int launch_ffn(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
               const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t E, int64_t H, int64_t I, int act,
               void* out2, void* out3, int32_t* ctl, int64_t nrows, hipStream_t st);
int launch_gateup(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                  const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H,
                  int64_t I, int act, void* out2, hipStream_t st, int64_t nrows_hint);
int launch_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                const void* dn_z, int64_t E, int64_t H, int64_t I, void* out3, hipStream_t st, int layout,
                int64_t nrows);
const int32_t* ffn_error_word(const int32_t* ctl);

namespace {

// Output of a call whose expert FFN reported a failed wait (its error word,
// read by the combine of the same call, is nonzero): every element NaN, so
// that the result cannot pass for a normal one.
__device__ __forceinline__ bool poisoned(const int32_t* __restrict__ err) { return err && *err != 0; }

constexpr int kCombThreads = 256;

// acc[j] = sum over slots k in order of fp32(w[t,k]) * fp32(out3[inv[t*topk+k], c0+j]).
// 8 slots at a time: all index/weight loads (uniform per token), then all row
// loads (clamped slot index: one round trip each), then the FMA chain in slot order.
// F16P (the v1 combine, kernels/fused_moe_w4.py:125-127): the weight is
// rounded to fp16 first and each product w * x to fp16 (torch's fp16 multiply),
// the products are summed in fp32 in slot order.
// WIDE (topk % 8 == 0, inv and w 16-byte aligned: the layer's case): the 8
// indices and 8 weights of a block in 16-byte loads (4 or 3 instructions
// instead of 16; every lane of a token loads the same ones), same values.
template <int WD, bool F16P = false, bool WIDE = false>
__device__ __forceinline__ void combine_acc(const f16* __restrict__ out3, const int32_t* __restrict__ inv,
                                            const typename Elem<WD>::T* __restrict__ w, int64_t t, int topk,
                                            int64_t H, int64_t c0, float (&acc)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int k0 = 0; k0 < topk; k0 += 8) {
        int32_t r[8];
        float wk[8];
        if constexpr (WIDE) {
            const u32x4* ip = reinterpret_cast<const u32x4*>(inv + t * topk + k0);
            const u32x4 i0 = ip[0], i1 = ip[1];
            float wr[8];
            if constexpr (WD == KSL_DTYPE_F32) {
                const f32x4* wp = reinterpret_cast<const f32x4*>(w + t * topk + k0);
                const f32x4 w0 = wp[0], w1 = wp[1];
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    wr[k] = w0[k];
                    wr[4 + k] = w1[k];
                }
            } else {
                raw_unpack8<WD>(raw_load8<WD>(w + t * topk + k0), wr);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                r[k] = static_cast<int32_t>(i0[k]);
                r[4 + k] = static_cast<int32_t>(i1[k]);
            }
#pragma unroll
            for (int k = 0; k < 8; ++k) wk[k] = F16P ? static_cast<float>(static_cast<f16>(wr[k])) : wr[k];
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int kk = k0 + k < topk ? k0 + k : topk - 1;
                r[k] = inv[t * topk + kk];
                wk[k] = Elem<WD>::load(w + t * topk + kk);
                if (F16P) wk[k] = static_cast<float>(static_cast<f16>(wk[k]));
            }
        }
        f16x8 x[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] = *reinterpret_cast<const f16x8*>(out3 + static_cast<int64_t>(r[k]) * H + c0);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            // WIDE: every slot of the block is real, so no branch (a branch per
            // slot let the compiler reload a row inside it, one round trip late)
            if (WIDE || k0 + k < topk) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    if (F16P)
                        acc[j] += static_cast<float>(static_cast<f16>(wk[k] * static_cast<float>(x[k][j])));
                    else
                        acc[j] = __builtin_fmaf(wk[k], static_cast<float>(x[k][j]), acc[j]);
                }
            }
        }
    }
}

template <int WD, int YD, bool F16P, bool WIDE>
__global__ __launch_bounds__(kCombThreads) void combine_kernel(const f16* __restrict__ out3,
                                                              const int32_t* __restrict__ inv,
                                                              const void* __restrict__ wv, int64_t T,
                                                              int topk, int64_t H, void* __restrict__ yv,
                                                              int64_t ys, const int32_t* __restrict__ err) {
    typedef typename Elem<YD>::T YT;
    YT* y = static_cast<YT*>(yv);
    const int64_t hv = H / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kCombThreads + threadIdx.x;
    const int64_t t = idx / hv;
    if (t >= T) return;
    const int64_t c0 = (idx - t * hv) * 8;
    float acc[8];
    combine_acc<WD, F16P, WIDE>(out3, inv, static_cast<const typename Elem<WD>::T*>(wv), t, topk, H, c0, acc);
    if (F16P) {  // the fp16 sum, then .to(y dtype)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = static_cast<float>(static_cast<f16>(acc[j]));
    }
    if (poisoned(err)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = __builtin_nanf("");
    }
    store8<YD>(y + t * ys + c0, acc);
}

template <int WD, bool F16P>
int launch_combine_y(int yd, const void* out3, const int32_t* inv, const void* w, int64_t T,
                     int64_t topk, int64_t H, void* y, int64_t ys, hipStream_t st, const int32_t* err) {
    const int64_t n = T * (H / 8);
    const unsigned grid = static_cast<unsigned>((n + kCombThreads - 1) / kCombThreads);
    const f16* o3 = static_cast<const f16*>(out3);
    const bool wide = topk % 8 == 0 && reinterpret_cast<uintptr_t>(inv) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(w) % 16 == 0;
    auto go = [&](auto yd_c, auto wide_c) {
        constexpr int YDC = decltype(yd_c)::value;
        constexpr bool WC = decltype(wide_c)::value;
        hipLaunchKernelGGL((combine_kernel<WD, YDC, F16P, WC>), dim3(grid), dim3(kCombThreads), 0, st, o3, inv, w,
                           T, static_cast<int>(topk), H, y, ys, err);
    };
    auto go_y = [&](auto yd_c) {
        if (wide)
            go(yd_c, std::true_type{});
        else
            go(yd_c, std::false_type{});
    };
    switch (yd) {
        case KSL_DTYPE_BF16: go_y(std::integral_constant<int, KSL_DTYPE_BF16>{}); break;
        case KSL_DTYPE_F16: go_y(std::integral_constant<int, KSL_DTYPE_F16>{}); break;
        case KSL_DTYPE_F32: go_y(std::integral_constant<int, KSL_DTYPE_F32>{}); break;
        default:
            return KSL_ERR_ARG;
    }
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

// ---- the stock experts loop's combine -----------------------------------------
// DiffusionGemmaTextExperts.forward (TF modeling_diffusion_gemma.py:578-588),
// as kernels/pack_experts.py:44-62 runs it over the W4 linears: y starts at
// zero in the hidden dtype; expert by expert in ascending id, each of its rows
// adds term = YD(h * w[t, k]) to y[t] with one rounding to YD per add
// (index_add_). h * w is the torch product of fp16 h and the routing weight:
// in fp32 for fp32 or bf16 weights (type promotion), in fp16 for fp16 ones.
// Per token the slots are taken in (expert id, slot) order; ids outside
// [0, E) contribute nothing. One thread per 8 columns of one token.
constexpr int kStockMaxTopk = 32;

template <int WD, int YD>
__global__ __launch_bounds__(kCombThreads) void combine_stock_kernel(const f16* __restrict__ out3,
                                                                    const int32_t* __restrict__ inv,
                                                                    const int64_t* __restrict__ ids, int64_t E,
                                                                    const void* __restrict__ wv, int64_t T, int topk,
                                                                    int64_t H, void* __restrict__ yv, int64_t ys) {
    typedef typename Elem<YD>::T YT;
    typedef typename Elem<WD>::T WT;
    const WT* w = static_cast<const WT*>(wv);
    const int64_t hv = H / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kCombThreads + threadIdx.x;
    const int64_t t = idx / hv;
    if (t >= T) return;
    const int64_t c0 = (idx - t * hv) * 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    int64_t prev_id = -1;
    int prev_k = -1;
    for (int r = 0; r < topk; ++r) {
        // the next slot in (id, slot) order
        int64_t best_id = INT64_MAX;
        int best_k = -1;
        for (int k = 0; k < topk; ++k) {
            const int64_t id = ids[t * topk + k];
            const bool after = id > prev_id || (id == prev_id && k > prev_k);
            if (after && (id < best_id || (id == best_id && k < best_k))) {
                best_id = id;
                best_k = k;
            }
        }
        prev_id = best_id;
        prev_k = best_k;
        if (best_id < 0 || best_id >= E) continue;
        const int64_t row = inv[t * topk + best_k];
        const f16x8 h = *reinterpret_cast<const f16x8*>(out3 + row * H + c0);
        const float wk = Elem<WD>::load(w + t * topk + best_k);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            // separately rounded product and sum, never contracted to an FMA
            // (the reference multiplies, then index_add_ adds)
#pragma clang fp contract(off)
            float term = static_cast<float>(h[j]) * wk;
            if (WD == KSL_DTYPE_F16) term = static_cast<float>(static_cast<f16>(term));
            if (YD == KSL_DTYPE_BF16) {
                acc[j] = bf16r(acc[j] + bf16r(term));
            } else if (YD == KSL_DTYPE_F16) {
                acc[j] = static_cast<float>(static_cast<f16>(acc[j] + static_cast<float>(static_cast<f16>(term))));
            } else {
                acc[j] = acc[j] + term;
            }
        }
    }
    store8<YD>(static_cast<YT*>(yv) + t * ys + c0, acc);
}

template <int WD>
int launch_combine_stock_y(int yd, const f16* out3, const int32_t* inv, const int64_t* ids, int64_t E, const void* w,
                           int64_t T, int64_t topk, int64_t H, void* y, int64_t ys, hipStream_t st) {
    const int64_t n = T * (H / 8);
    const unsigned grid = static_cast<unsigned>((n + kCombThreads - 1) / kCombThreads);
    const int k = static_cast<int>(topk);
    switch (yd) {
        case KSL_DTYPE_BF16:
            hipLaunchKernelGGL((combine_stock_kernel<WD, KSL_DTYPE_BF16>), dim3(grid), dim3(kCombThreads), 0, st, out3,
                               inv, ids, E, w, T, k, H, y, ys);
            break;
        case KSL_DTYPE_F16:
            hipLaunchKernelGGL((combine_stock_kernel<WD, KSL_DTYPE_F16>), dim3(grid), dim3(kCombThreads), 0, st, out3,
                               inv, ids, E, w, T, k, H, y, ys);
            break;
        case KSL_DTYPE_F32:
            hipLaunchKernelGGL((combine_stock_kernel<WD, KSL_DTYPE_F32>), dim3(grid), dim3(kCombThreads), 0, st, out3,
                               inv, ids, E, w, T, k, H, y, ys);
            break;
        default:
            return KSL_ERR_ARG;
    }
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

// ---- combine + the feed-forward block's tail --------------------------------
// After the experts the decoder layer computes (TF modeling_diffusion_gemma.py:734-744,
// every RMSNorm being the fused RMSNorm of kernels/fused_rmsnorm.py:10-21):
//   m  = bf16(combine)                    experts' output, hidden dtype bf16
//   n2 = bf16(m * r(m) * w2)              post_feedforward_layernorm_2
//   s  = bf16(h1 + n2)                    hidden_states_1 + hidden_states_2
//   n  = bf16(s * r(s) * w)               post_feedforward_layernorm
//   o  = bf16(res + n)                    residual + hidden_states
//   y  = bf16(o * layer_scalar)           hidden_states *= layer_scalar
// with r(v) = 1 / sqrt(sum(v^2) / H + eps). One workgroup per token, thread i
// owning columns 8i..8i+7 (threads past the row end hold zeros). A row sum is
// a per-thread FMA chain, a DPP wave reduction and the wave partials added in
// wave order: the same bits every run.
constexpr int kPostMaxWaves = 16;
constexpr int kPostMaxH = kPostMaxWaves * kWave * 8;

struct PostArgs {
    const f16* out3;
    const int32_t* inv;
    const void* w;          // top-k weights, dtype WD
    const uint16_t* h1;     // bf16 [T, h1s]
    const uint16_t* res;    // bf16 [T, rs]
    const uint16_t* w2;     // bf16 [H]: post_feedforward_layernorm_2 weight
    const uint16_t* wp;     // bf16 [H]: post_feedforward_layernorm weight
    const void* ls;         // layer scalar (one element) or null for 1
    uint16_t* y;            // bf16 [T, ys]
    const int32_t* err;     // the expert FFN's error word, or null
    int64_t h1s, rs, ys;
    float eps2, eps;
    int topk, H, ls_dt;
};

__device__ __forceinline__ float block_row_sum(float v, float* part, int nwaves) {
    v = __ockl_wfred_add_f32(v);
    if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nwaves; ++i) s += part[i];
    return s;
}

template <int WD, bool WIDE>
__global__ __launch_bounds__(kPostMaxWaves * kWave) void combine_post_kernel(PostArgs A) {
    constexpr int BF = KSL_DTYPE_BF16;
    __shared__ float part[2][kPostMaxWaves];
    const int64_t t = blockIdx.x;
    const int nw = static_cast<int>(blockDim.x) / kWave;
    const int64_t c0 = static_cast<int64_t>(threadIdx.x) * 8;
    const bool ok = c0 < A.H;
    // the token's other operands are independent of the gather: issue them first
    Raw8<BF> hv{}, rv{}, w2v{}, wpv{};
    if (ok) {
        hv = raw_load8<BF>(A.h1 + t * A.h1s + c0);
        rv = raw_load8<BF>(A.res + t * A.rs + c0);
        w2v = raw_load8<BF>(A.w2 + c0);
        wpv = raw_load8<BF>(A.wp + c0);
    }
    float ls = 1.0f;
    if (A.ls)
        ls = A.ls_dt == KSL_DTYPE_F32 ? *static_cast<const float*>(A.ls)
                                      : bf16_bits_to_f32(*static_cast<const uint16_t*>(A.ls));
    float m[8];
    if (ok) {
        combine_acc<WD, false, WIDE>(A.out3, A.inv, static_cast<const typename Elem<WD>::T*>(A.w), t, A.topk, A.H,
                                     c0, m);
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] = 0.0f;
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        m[j] = bf16r(m[j]);
        ss = __builtin_fmaf(m[j], m[j], ss);
    }
    const float r2 = rms_inv(block_row_sum(ss, part[0], nw), A.H, A.eps2);
    float hf[8], w2f[8], s[8];
    raw_unpack8<BF>(hv, hf);
    raw_unpack8<BF>(w2v, w2f);
    ss = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        s[j] = bf16r(hf[j] + rms_apply<true>(m[j], r2, w2f[j]));
        ss = __builtin_fmaf(s[j], s[j], ss);
    }
    const float r = rms_inv(block_row_sum(ss, part[1], nw), A.H, A.eps);
    float rf[8], wpf[8], o[8];
    raw_unpack8<BF>(rv, rf);
    raw_unpack8<BF>(wpv, wpf);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = bf16r(bf16r(rf[j] + rms_apply<true>(s[j], r, wpf[j])) * ls);
    if (poisoned(A.err)) {
#pragma unroll
        for (int j = 0; j < 8; ++j) o[j] = __builtin_nanf("");
    }
    if (ok) store8<BF>(A.y + t * A.ys + c0, o);
}

}  // namespace

// err: the expert FFN's error word of the same call (null: none).
int launch_combine(const void* out3, const int32_t* inv, const void* w, int wd, int64_t T,
                   int64_t topk, int64_t H, void* y, int yd, int64_t ys, hipStream_t st, bool f16p = false,
                   const int32_t* err = nullptr) {
    if (!out3 || !inv || !w || !y) return T == 0 ? KSL_OK : KSL_ERR_ARG;
    if (T < 0 || topk <= 0 || H <= 0 || H % 8 != 0 || ys < H) return KSL_ERR_SHAPE;
    if (ys % 8 != 0 || reinterpret_cast<uintptr_t>(out3) % 16 || reinterpret_cast<uintptr_t>(y) % 16)
        return KSL_ERR_ALIGN;
    if (T == 0) return KSL_OK;
    if (f16p) {
        switch (wd) {
            case KSL_DTYPE_F32: return launch_combine_y<KSL_DTYPE_F32, true>(yd, out3, inv, w, T, topk, H, y, ys, st, err);
            case KSL_DTYPE_F16: return launch_combine_y<KSL_DTYPE_F16, true>(yd, out3, inv, w, T, topk, H, y, ys, st, err);
            case KSL_DTYPE_BF16: return launch_combine_y<KSL_DTYPE_BF16, true>(yd, out3, inv, w, T, topk, H, y, ys, st, err);
        }
        return KSL_ERR_ARG;
    }
    switch (wd) {
        case KSL_DTYPE_F32: return launch_combine_y<KSL_DTYPE_F32, false>(yd, out3, inv, w, T, topk, H, y, ys, st, err);
        case KSL_DTYPE_F16: return launch_combine_y<KSL_DTYPE_F16, false>(yd, out3, inv, w, T, topk, H, y, ys, st, err);
        case KSL_DTYPE_BF16: return launch_combine_y<KSL_DTYPE_BF16, false>(yd, out3, inv, w, T, topk, H, y, ys, st, err);
    }
    return KSL_ERR_ARG;
}

// Argument checks of the tail (everything but the experts' rows), made before
// any launch of a fused forward.
static int check_post(int64_t T, int64_t topk, int64_t H, int wd, const void* h1, int64_t h1s,
                      const void* res, int64_t rs, const void* w2, const void* wp, const void* ls, int ls_dt,
                      const void* y, int64_t ys) {
    if (T < 0 || topk <= 0 || H <= 0 || H % 8 != 0 || H > kPostMaxH) return KSL_ERR_SHAPE;
    if (T == 0) return KSL_OK;
    if (!h1 || !res || !w2 || !wp || !y) return KSL_ERR_ARG;
    if (ls && ls_dt != KSL_DTYPE_F32 && ls_dt != KSL_DTYPE_BF16) return KSL_ERR_ARG;
    if (wd != KSL_DTYPE_F32 && wd != KSL_DTYPE_F16 && wd != KSL_DTYPE_BF16) return KSL_ERR_ARG;
    if (h1s < H || rs < H || ys < H) return KSL_ERR_SHAPE;
    if (h1s % 8 || rs % 8 || ys % 8) return KSL_ERR_ALIGN;
    for (const void* p : {h1, res, w2, wp, y})
        if (reinterpret_cast<uintptr_t>(p) % 16) return KSL_ERR_ALIGN;
    return KSL_OK;
}

int launch_combine_post(const void* out3, const int32_t* inv, const void* w, int wd, int64_t T,
                        int64_t topk, int64_t H, const void* h1, int64_t h1s, const void* res, int64_t rs,
                        const void* w2, float eps2, const void* wp, float eps, const void* ls, int ls_dt,
                        void* y, int64_t ys, hipStream_t st, const int32_t* err = nullptr) {
    const int rc = check_post(T, topk, H, wd, h1, h1s, res, rs, w2, wp, ls, ls_dt, y, ys);
    if (rc || T == 0) return rc;
    if (!out3 || !inv || !w) return KSL_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(out3) % 16) return KSL_ERR_ALIGN;
    PostArgs A;
    A.out3 = static_cast<const f16*>(out3);
    A.inv = inv;
    A.w = w;
    A.h1 = static_cast<const uint16_t*>(h1);
    A.res = static_cast<const uint16_t*>(res);
    A.w2 = static_cast<const uint16_t*>(w2);
    A.wp = static_cast<const uint16_t*>(wp);
    A.ls = ls;
    A.y = static_cast<uint16_t*>(y);
    A.err = err;
    A.h1s = h1s;
    A.rs = rs;
    A.ys = ys;
    A.eps2 = eps2;
    A.eps = eps;
    A.topk = static_cast<int>(topk);
    A.H = static_cast<int>(H);
    A.ls_dt = ls_dt;
    const int threads = static_cast<int>((H / 8 + kWave - 1) / kWave) * kWave;
    const dim3 grid(static_cast<unsigned>(T)), block(threads);
    const bool wide = topk % 8 == 0 && reinterpret_cast<uintptr_t>(inv) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(w) % 16 == 0;
    auto go = [&](auto wd_c) {
        constexpr int WDC = decltype(wd_c)::value;
        if (wide)
            hipLaunchKernelGGL((combine_post_kernel<WDC, true>), grid, block, 0, st, A);
        else
            hipLaunchKernelGGL((combine_post_kernel<WDC, false>), grid, block, 0, st, A);
    };
    switch (wd) {
        case KSL_DTYPE_F32: go(std::integral_constant<int, KSL_DTYPE_F32>{}); break;
        case KSL_DTYPE_F16: go(std::integral_constant<int, KSL_DTYPE_F16>{}); break;
        default: go(std::integral_constant<int, KSL_DTYPE_BF16>{}); break;
    }
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

// Workspace layout of the fused forward (each region 256-byte aligned):
//   sorted_rows i32[Nexp] | offsets i32[E+1] | inv i32[Nexp] |
//   a16 f16[T*H] | out2 f16[Nexp*I] | out3 f16[Nexp*H] |
//   bcnt i32[ceil(Nexp/1024) * E] (per-block expert counts of the multi-block routing) |
//   ctl i32[E+2] (the one-launch expert FFN's completion counters, unit queue and error word)
struct MoeWorkspace {
    size_t sorted_rows, offsets, inv, a16, out2, out3, bcnt, ctl, total;
};

static size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

static MoeWorkspace moe_workspace_layout(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I) {
    MoeWorkspace w;
    const size_t nexp = static_cast<size_t>(T * topk);
    size_t off = 0;
    w.sorted_rows = off; off += align256(nexp * 4);
    w.offsets = off;     off += align256(static_cast<size_t>(E + 1) * 4);
    w.inv = off;         off += align256(nexp * 4);
    w.a16 = off;         off += align256(static_cast<size_t>(T * H) * 2);
    w.out2 = off;        off += align256(nexp * static_cast<size_t>(I) * 2);
    w.out3 = off;        off += align256(nexp * static_cast<size_t>(H) * 2);
    w.bcnt = off;        off += align256((nexp + 1023) / 1024 * static_cast<size_t>(E) * 4);
    w.ctl = off;         off += align256(ffn_ctl_words(E) * 4);
    w.total = off;
    return w;
}

// The experts between routing and combine: the one-launch FFN over the pack
// layout when the pack buffers are given and the routing is small, else the
// gate/up and down launches over the reference (or tiled) layout.
static int run_experts(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                       const uint8_t* gu_q, const void* gu_s, const void* gu_z, const uint8_t* dn_q,
                       const void* dn_s, const void* dn_z, int dn_layout, const uint8_t* gu_pack,
                       const uint8_t* dn_pack, int64_t E, int64_t H, int64_t I, int act, void* out2, void* out3,
                       int32_t* ctl, int64_t nrows, hipStream_t st) {
    if (gu_pack && dn_pack && ffn_supported(E, H, I, nrows))
        return launch_ffn(a16, sorted_rows, offsets, topk, gu_pack, dn_pack, E, H, I, act, out2, out3, ctl, nrows,
                          st);
    int rc = launch_gateup(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, E, H, I, act, out2, st, nrows);
    if (rc) return rc;
    return launch_down(out2, offsets, dn_q, dn_s, dn_z, E, H, I, out3, st, dn_layout, nrows);
}

static bool use_ffn(const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t E, int64_t H, int64_t I, int64_t nrows) {
    return gu_pack && dn_pack && ffn_supported(E, H, I, nrows);
}

}  // namespace ksl

extern "C" int ksl_moe_combine(const void* out3, const int32_t* inv, const void* topk_w, int w_dtype,
                               int64_t T, int64_t topk, int64_t H, void* y, int y_dtype,
                               int64_t y_stride, void* stream) {
    return ksl::launch_combine(out3, inv, topk_w, w_dtype, T, topk, H, y, y_dtype, y_stride,
                               static_cast<hipStream_t>(stream));
}

extern "C" int ksl_moe_combine_v1(const void* out3, const int32_t* inv, const void* topk_w, int w_dtype,
                                  int64_t T, int64_t topk, int64_t H, void* y, int y_dtype, int64_t y_stride,
                                  void* stream) {
    return ksl::launch_combine(out3, inv, topk_w, w_dtype, T, topk, H, y, y_dtype, y_stride,
                               static_cast<hipStream_t>(stream), true);
}

extern "C" int ksl_moe_combine_stock(const void* out3, const int32_t* inv, const int64_t* topk_ids, int64_t E,
                                     const void* topk_w, int w_dtype, int64_t T, int64_t topk, int64_t H, void* y,
                                     int y_dtype, int64_t y_stride, void* stream) {
    using namespace ksl;
    if (T < 0 || topk <= 0 || topk > kStockMaxTopk || E <= 0 || H <= 0 || H % 8 != 0 || y_stride < H)
        return KSL_ERR_SHAPE;
    if (T == 0) return KSL_OK;
    if (!out3 || !inv || !topk_ids || !topk_w || !y) return KSL_ERR_ARG;
    if (y_stride % 8 != 0 || reinterpret_cast<uintptr_t>(out3) % 16 || reinterpret_cast<uintptr_t>(y) % 16 ||
        reinterpret_cast<uintptr_t>(topk_ids) % 8)
        return KSL_ERR_ALIGN;
    if (T * (H / 8) / kCombThreads >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    const f16* o3 = static_cast<const f16*>(out3);
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (w_dtype) {
        case KSL_DTYPE_F32:
            return launch_combine_stock_y<KSL_DTYPE_F32>(y_dtype, o3, inv, topk_ids, E, topk_w, T, topk, H, y,
                                                         y_stride, st);
        case KSL_DTYPE_F16:
            return launch_combine_stock_y<KSL_DTYPE_F16>(y_dtype, o3, inv, topk_ids, E, topk_w, T, topk, H, y,
                                                         y_stride, st);
        case KSL_DTYPE_BF16:
            return launch_combine_stock_y<KSL_DTYPE_BF16>(y_dtype, o3, inv, topk_ids, E, topk_w, T, topk, H, y,
                                                          y_stride, st);
    }
    return KSL_ERR_ARG;
}

extern "C" int ksl_moe_combine_post(const void* out3, const int32_t* inv, const void* topk_w, int w_dtype,
                                    int64_t T, int64_t topk, int64_t H, const void* h1, int64_t h1_stride,
                                    const void* residual, int64_t residual_stride, const void* post2_w,
                                    float post2_eps, const void* post_w, float post_eps,
                                    const void* layer_scalar, int ls_dtype, void* y, int64_t y_stride,
                                    void* stream) {
    return ksl::launch_combine_post(out3, inv, topk_w, w_dtype, T, topk, H, h1, h1_stride, residual,
                                    residual_stride, post2_w, post2_eps, post_w, post_eps, layer_scalar,
                                    ls_dtype, y, y_stride, static_cast<hipStream_t>(stream));
}

extern "C" size_t ksl_moe_workspace_bytes(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I) {
    if (T < 0 || topk <= 0 || E <= 0 || H <= 0 || I <= 0) return 0;
    return ksl::moe_workspace_layout(T, topk, E, H, I).total;
}

extern "C" int ksl_moe_w4a16_forward(const void* hidden, int hidden_dtype, int64_t hidden_stride,
                                     const int64_t* topk_ids, const void* topk_w, int w_dtype,
                                     const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                                     const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout,
                                     const uint8_t* gu_pack, const uint8_t* dn_pack,
                                     int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I, int act,
                                     void* y, int y_dtype, int64_t y_stride, void* workspace,
                                     size_t workspace_bytes, void* stream) {
    using namespace ksl;
    if (T < 0 || topk <= 0 || E <= 0 || H <= 0 || I <= 0) return KSL_ERR_SHAPE;
    if (H % 128 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (act != KSL_ACT_GELU_TANH && act != KSL_ACT_SILU) return KSL_ERR_ARG;
    if (dn_layout != KSL_DN_LAYOUT_REF && dn_layout != KSL_DN_LAYOUT_TILED) return KSL_ERR_ARG;
    if (T == 0) return KSL_OK;
    const MoeWorkspace L = moe_workspace_layout(T, topk, E, H, I);
    if (!workspace || workspace_bytes < L.total) return KSL_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return KSL_ERR_ALIGN;
    char* ws = static_cast<char*>(workspace);
    int32_t* sorted_rows = reinterpret_cast<int32_t*>(ws + L.sorted_rows);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
    int32_t* inv = reinterpret_cast<int32_t*>(ws + L.inv);
    void* a16 = ws + L.a16;
    void* out2 = ws + L.out2;
    void* out3 = ws + L.out3;
    int32_t* bcnt = reinterpret_cast<int32_t*>(ws + L.bcnt);
    int32_t* ctl = reinterpret_cast<int32_t*>(ws + L.ctl);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool ffn = use_ffn(gu_pack, dn_pack, E, H, I, T * topk);
    int rc = route_compact(topk_ids, T, topk, E, sorted_rows, offsets, inv, hidden, hidden_dtype,
                           hidden_stride, H, a16, bcnt, st, ffn ? ctl : nullptr, static_cast<int>(ffn_ctl_words(E) / kCtlStride));
    if (rc) return rc;
    rc = run_experts(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, dn_layout, gu_pack, dn_pack,
                     E, H, I, act, out2, out3, ctl, T * topk, st);
    if (rc) return rc;
    return launch_combine(out3, inv, topk_w, w_dtype, T, topk, H, y, y_dtype, y_stride, st, false,
                          ffn ? ffn_error_word(ctl) : nullptr);
}

namespace ksl {

// The body of ksl_moe_layer_forward after its argument checks, on the
// workspace `ws` (laid out by moe_workspace_layout, 256-byte aligned).
static int layer_forward_on(char* ws, const void* x, int x_dtype, int64_t x_stride, const void* norm_w,
                            int norm_w_dtype, float eps, const int64_t* topk_ids, const void* topk_w, int w_dtype,
                            const uint8_t* gu_q, const void* gu_s, const void* gu_z, const uint8_t* dn_q,
                            const void* dn_s, const void* dn_z, int dn_layout, const uint8_t* gu_pack,
                            const uint8_t* dn_pack, int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I,
                            int act, void* y, int y_dtype, int64_t y_stride, hipStream_t st) {
    const MoeWorkspace L = moe_workspace_layout(T, topk, E, H, I);
    int32_t* sorted_rows = reinterpret_cast<int32_t*>(ws + L.sorted_rows);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
    int32_t* inv = reinterpret_cast<int32_t*>(ws + L.inv);
    void* a16 = ws + L.a16;
    void* out2 = ws + L.out2;
    void* out3 = ws + L.out3;
    int32_t* bcnt = reinterpret_cast<int32_t*>(ws + L.bcnt);
    int32_t* ctl = reinterpret_cast<int32_t*>(ws + L.ctl);
    const bool ffn = use_ffn(gu_pack, dn_pack, E, H, I, T * topk);
    int rc = route_norm(topk_ids, T, topk, E, sorted_rows, offsets, inv, x, x_dtype, x_stride, norm_w,
                        norm_w_dtype, eps, H, a16, bcnt, st, ffn ? ctl : nullptr, static_cast<int>(ffn_ctl_words(E) / kCtlStride));
    if (rc) return rc;
    rc = run_experts(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, dn_layout, gu_pack, dn_pack,
                     E, H, I, act, out2, out3, ctl, T * topk, st);
    if (rc) return rc;
    return launch_combine(out3, inv, topk_w, w_dtype, T, topk, H, y, y_dtype, y_stride, st, false,
                          ffn ? ffn_error_word(ctl) : nullptr);
}

static int layer_forward_check(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I, int act, int dn_layout) {
    if (T < 0 || topk <= 0 || E <= 0 || H <= 0 || I <= 0) return KSL_ERR_SHAPE;
    if (H % 128 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (act != KSL_ACT_GELU_TANH && act != KSL_ACT_SILU) return KSL_ERR_ARG;
    if (dn_layout != KSL_DN_LAYOUT_REF && dn_layout != KSL_DN_LAYOUT_TILED) return KSL_ERR_ARG;
    return KSL_OK;
}

// The library's own workspace for ksl_moe_layer_forward_noalloc: one array per
// GPU, held from the library's load until the process ends. Host code never
// uses the array's name as an address (on the host it is only a stand-in for
// the symbol): scratch_on() returns the device address, looked up once per
// device with that device current.
static __device__ __align__(256) unsigned char scratch[KSL_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::atomic<char*> g_scratch_ptr[kMaxDevices];
static std::mutex g_scratch_mu;

// Device address of the current device's scratch array, or null on a failed lookup.
static char* scratch_on(int dev) {
    char* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p) return p;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p) return p;
    void* addr = nullptr;
    if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) {
        (void)hipGetLastError();
        return nullptr;
    }
    p = static_cast<char*>(addr);
    g_scratch_ptr[dev].store(p, std::memory_order_release);
    return p;
}

}  // namespace ksl

extern "C" int ksl_moe_layer_forward(const void* x, int x_dtype, int64_t x_stride, const void* norm_w,
                                     int norm_w_dtype, float eps, const int64_t* topk_ids,
                                     const void* topk_w, int w_dtype, const uint8_t* gu_q,
                                     const void* gu_s, const void* gu_z, const uint8_t* dn_q,
                                     const void* dn_s, const void* dn_z, int dn_layout, const uint8_t* gu_pack,
                                     const uint8_t* dn_pack, int64_t T, int64_t topk,
                                     int64_t E, int64_t H, int64_t I, int act, void* y, int y_dtype,
                                     int64_t y_stride, void* workspace, size_t workspace_bytes,
                                     void* stream) {
    using namespace ksl;
    int rc = layer_forward_check(T, topk, E, H, I, act, dn_layout);
    if (rc || T == 0) return rc;
    if (!workspace || workspace_bytes < moe_workspace_layout(T, topk, E, H, I).total) return KSL_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return KSL_ERR_ALIGN;
    return layer_forward_on(static_cast<char*>(workspace), x, x_dtype, x_stride, norm_w, norm_w_dtype, eps, topk_ids,
                            topk_w, w_dtype, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, dn_layout, gu_pack, dn_pack, T, topk,
                            E, H, I, act, y, y_dtype, y_stride, static_cast<hipStream_t>(stream));
}

extern "C" int ksl_moe_layer_forward_noalloc(const void* x, int x_dtype, int64_t x_stride, const void* norm_w,
                                             int norm_w_dtype, float eps, const int64_t* topk_ids,
                                             const void* topk_w, int w_dtype, const uint8_t* gu_q,
                                             const void* gu_s, const void* gu_z, const uint8_t* dn_q,
                                             const void* dn_s, const void* dn_z, int dn_layout,
                                             const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t T,
                                             int64_t topk, int64_t E, int64_t H, int64_t I, int act, void* y,
                                             int y_dtype, int64_t y_stride, void* stream) {
    using namespace ksl;
    int rc = layer_forward_check(T, topk, E, H, I, act, dn_layout);
    if (rc || T == 0) return rc;
    if (moe_workspace_layout(T, topk, E, H, I).total > static_cast<size_t>(KSL_NOALLOC_SCRATCH_BYTES))
        return KSL_ERR_SCRATCH;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return KSL_ERR_RUNTIME;
    char* ws = scratch_on(dev);
    if (!ws) return KSL_ERR_RUNTIME;
    return layer_forward_on(ws, x, x_dtype, x_stride, norm_w, norm_w_dtype, eps, topk_ids, topk_w, w_dtype, gu_q,
                            gu_s, gu_z, dn_q, dn_s, dn_z, dn_layout, gu_pack, dn_pack, T, topk, E, H, I, act, y,
                            y_dtype, y_stride, static_cast<hipStream_t>(stream));
}

extern "C" int ksl_moe_block_forward(const void* x, int64_t x_stride, const void* pre_norm_w, float pre_eps,
                                     const int64_t* topk_ids, const void* topk_w, int w_dtype,
                                     const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                                     const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout,
                                     const uint8_t* gu_pack, const uint8_t* dn_pack,
                                     int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I, int act,
                                     const void* h1,
                                     int64_t h1_stride, const void* post2_w, float post2_eps,
                                     const void* post_w, float post_eps, const void* layer_scalar,
                                     int ls_dtype, void* y, int64_t y_stride, void* workspace,
                                     size_t workspace_bytes, void* stream) {
    using namespace ksl;
    if (T < 0 || topk <= 0 || E <= 0 || H <= 0 || I <= 0) return KSL_ERR_SHAPE;
    if (H % 128 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (act != KSL_ACT_GELU_TANH && act != KSL_ACT_SILU) return KSL_ERR_ARG;
    if (dn_layout != KSL_DN_LAYOUT_REF && dn_layout != KSL_DN_LAYOUT_TILED) return KSL_ERR_ARG;
    int rc = check_post(T, topk, H, w_dtype, h1, h1_stride, x, x_stride, post2_w, post_w, layer_scalar,
                        ls_dtype, y, y_stride);
    if (rc || T == 0) return rc;
    const MoeWorkspace L = moe_workspace_layout(T, topk, E, H, I);
    if (!workspace || workspace_bytes < L.total) return KSL_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(workspace) % 256) return KSL_ERR_ALIGN;
    char* ws = static_cast<char*>(workspace);
    int32_t* sorted_rows = reinterpret_cast<int32_t*>(ws + L.sorted_rows);
    int32_t* offsets = reinterpret_cast<int32_t*>(ws + L.offsets);
    int32_t* inv = reinterpret_cast<int32_t*>(ws + L.inv);
    void* a16 = ws + L.a16;
    void* out2 = ws + L.out2;
    void* out3 = ws + L.out3;
    int32_t* bcnt = reinterpret_cast<int32_t*>(ws + L.bcnt);
    int32_t* ctl = reinterpret_cast<int32_t*>(ws + L.ctl);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool ffn = use_ffn(gu_pack, dn_pack, E, H, I, T * topk);
    rc = route_norm(topk_ids, T, topk, E, sorted_rows, offsets, inv, x, KSL_DTYPE_BF16, x_stride, pre_norm_w,
                    KSL_DTYPE_BF16, pre_eps, H, a16, bcnt, st, ffn ? ctl : nullptr, static_cast<int>(ffn_ctl_words(E) / kCtlStride));
    if (rc) return rc;
    rc = run_experts(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, dn_q, dn_s, dn_z, dn_layout, gu_pack, dn_pack,
                     E, H, I, act, out2, out3, ctl, T * topk, st);
    if (rc) return rc;
    return launch_combine_post(out3, inv, topk_w, w_dtype, T, topk, H, h1, h1_stride, x, x_stride, post2_w,
                               post2_eps, post_w, post_eps, layer_scalar, ls_dtype, y, y_stride, st,
                               ffn ? ffn_error_word(ctl) : nullptr);
}

extern "C" size_t ksl_moe_route_scratch_bytes(int64_t T, int64_t topk, int64_t E) {
    if (T < 0 || topk <= 0 || E <= 0) return 0;
    const int64_t nexp = T * topk;
    return nexp > 4096 ? static_cast<size_t>((nexp + 1023) / 1024 * E * 4) : 0;
}

extern "C" int ksl_moe_layer_route(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                                   int32_t* sorted_rows, int32_t* offsets, int32_t* inv, const void* x,
                                   int x_dtype, int64_t x_stride, const void* norm_w, int norm_w_dtype,
                                   float eps, int64_t H, void* a16, void* scratch, size_t scratch_bytes,
                                   void* stream) {
    const size_t need = ksl_moe_route_scratch_bytes(T, topk, E);
    int32_t* bcnt = need > 0 && scratch && scratch_bytes >= need && reinterpret_cast<uintptr_t>(scratch) % 4 == 0
                        ? static_cast<int32_t*>(scratch)
                        : nullptr;
    return ksl::route_norm(topk_ids, T, topk, E, sorted_rows, offsets, inv, x, x_dtype, x_stride, norm_w,
                           norm_w_dtype, eps, H, a16, bcnt, static_cast<hipStream_t>(stream), nullptr, 0);
}

extern "C" int ksl_version(void) { return 6; }

extern "C" const char* ksl_status_string(int status) {
    switch (status) {
        case KSL_OK: return "ok";
        case KSL_ERR_ARG: return "invalid argument (null pointer or unknown enum)";
        case KSL_ERR_SHAPE: return "shape or divisibility contract violated";
        case KSL_ERR_ALIGN: return "pointer or stride alignment contract violated";
        case KSL_ERR_LAUNCH: return "kernel launch failed";
        case KSL_ERR_WORKSPACE: return "workspace too small";
        case KSL_ERR_SCRATCH: return "input needs more than the no-allocation entry point's scratch (KSL_NOALLOC_SCRATCH_BYTES)";
        case KSL_ERR_RUNTIME: return "HIP runtime call failed";
    }
    return "unknown status";
}
