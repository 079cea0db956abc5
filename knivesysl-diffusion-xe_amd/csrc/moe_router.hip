// Expert router on the GPU: the step before the MoE (TF
// modeling_diffusion_gemma.py:529-548, DiffusionGemmaTextRouter.forward, its
// scale-free norm being the fused RMSNorm as the reference patches it,
// kernels/load_w4_checkpoint.py:126-127):
//   y      = bf16(x * r)                 r = 1/sqrt(mean(x^2) + eps)
//   h      = bf16(bf16(y * scale) * H^-1/2)
//   scores = bf16(h @ proj^T)            fp32 accumulate
//   probs  = softmax(fp32(scores))
//   w, idx = top-k of probs (descending, equal values: lower index first)
//   w      = w / sum(w) * per_expert_scale[idx]
// Two launches. Scores: one workgroup of 4 waves per 16 tokens x 16 experts
// (so the projection, 2*E*H bytes, is spread over E/16 workgroups per token
// block instead of streaming through one CU): the rows are normalised into LDS
// (bf16, padded rows: conflict-free MFMA operand reads) and multiplied with
// v_mfma_f32_16x16x32_bf16, the K steps split over the waves; the scores go to
// the probabilities buffer. Then one wave per token does softmax (in place),
// top-k and the renormalisation in registers.
#include "ksl_common.h"

namespace ksl {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kRtWaves = 16;           // one token row per wave in the scores launch
constexpr int kRtThreads = kRtWaves * kWave;
constexpr int kRtRows = 16;           // tokens per workgroup (one MFMA M tile)
constexpr int kRtMaxH = 4096;
constexpr int kRtMaxE = 256;
constexpr int kRtMaxK = 16;
constexpr int kRtRowPad = 16;         // bytes of padding per LDS row
constexpr int kRtKPer = (kRtMaxH / 32 + kRtWaves - 1) / kRtWaves;  // K steps per wave at most
constexpr int kRtKEarly = 4;                                        // of them loaded before the row

struct RouterArgs {
    const char* x;         // [T, H] bf16 / fp16, row stride xs elements
    const uint16_t* scale; // [H] bf16
    const uint16_t* proj;  // [E, H] bf16
    const uint16_t* pes;   // [E] bf16
    float* probs;          // [T, E]: the scores, then the probabilities
    float* topk_w;         // [T, k]
    int64_t* topk_ids;     // [T, k]
    int64_t xs;
    float eps;
    int T, H, E, k;
};

// bf16 rounding (round to nearest even) by the gfx950 conversion instruction:
// the same value as bf16r for every non-NaN input (fp32 denormals are kept,
// .amdhsa_float_denorm_mode_32 = 3); a NaN stays a NaN. Used for the router's
// intermediate activations, where only finite values are observable.
__device__ __forceinline__ float bf16r_hw(float v) {
    return __uint_as_float(static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(v))) << 16);
}

// Scores of 16 tokens x 16 experts per workgroup (grid: token blocks x expert
// tiles), 16 waves: each wave first issues its share of the projection tile
// (K steps w, w+16, ...: at most kRtKPer per wave, all in flight at once), then
// normalises one token row into LDS; after a barrier it multiplies its K steps
// with v_mfma_f32_16x16x32_bf16, and wave 0 sums the 16 partial tiles in a
// fixed order and stores the bf16-rounded scores as fp32 into probs.
template <int XD>
__global__ __launch_bounds__(kRtThreads) void router_scores_kernel(RouterArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int H = A.H, E = A.E;
    const int row_bytes = H * 2 + kRtRowPad;
    char* hrows = lds;                                                   // [16][row_bytes] bf16
    f32x4* part = reinterpret_cast<f32x4*>(lds + kRtRows * row_bytes);  // [kRtWaves][64]
    uint16_t* scl = reinterpret_cast<uint16_t*>(part + kRtWaves * kWave);  // [H] router scale
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int t0 = blockIdx.x * kRtRows;
    const int tile = blockIdx.y;
    const float root_py = static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(H)));  // fp32(H ** -0.5)
    const int col = lane & 15, c = lane >> 4;
    const int ksteps = H / 32;

    // 1. the projection fragments of this wave's K steps (independent of the
    //    rows): the first kRtKEarly now (all of them up to H = 2048), the rest
    //    once the row's registers are free
    const uint16_t* prow = A.proj + static_cast<int64_t>(tile * 16 + col) * H + c * 8;
    u32x4 b[kRtKPer];
    auto load_b = [&](int u) {
        int i = wave + u * kRtWaves;
        if (i >= ksteps) i = wave;  // clamped, never used
        b[u] = *reinterpret_cast<const u32x4*>(prow + i * 32);
    };
#pragma unroll
    for (int u = 0; u < kRtKEarly; ++u) load_b(u);

    // 2. token row t0 + wave: lane owns columns s*512 + lane*8 .. +8; the
    //    router scale goes to LDS once per workgroup
    {
        const int rr = wave;
        const int t = t0 + rr < A.T ? t0 + rr : A.T - 1;  // rows past T: computed, never stored
        const char* xr = A.x + static_cast<int64_t>(t) * A.xs * 2;
        Raw8<XD> xv[8];
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int c0 = s * 8 * kWave + lane * 8;
            xv[s] = c0 < H ? raw_load8<XD>(xr + c0 * 2) : Raw8<XD>{};
        }
        if (static_cast<int>(threadIdx.x) * 8 < H)
            *reinterpret_cast<u32x4*>(scl + threadIdx.x * 8) = *reinterpret_cast<const u32x4*>(A.scale + threadIdx.x * 8);
        __syncthreads();
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < 8; ++s) ss = rms_sumsq8<XD>(xv[s], ss);
        const float r = rms_scale(ss, 6, H, A.eps);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            const int c0 = s * 8 * kWave + lane * 8;
            if (c0 >= H) continue;
            float xf[8], sc[8];
            raw_unpack8<XD>(xv[s], xf);
            raw_unpack8<KSL_DTYPE_BF16>(Raw8<KSL_DTYPE_BF16>{{*reinterpret_cast<const u32x4*>(scl + c0)}}, sc);
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float h0 = bf16r_hw(bf16r_hw(bf16r_hw(xf[2 * j] * r) * sc[2 * j]) * root_py);
                const float h1 = bf16r_hw(bf16r_hw(bf16r_hw(xf[2 * j + 1] * r) * sc[2 * j + 1]) * root_py);
                o[j] = (__float_as_uint(h0) >> 16) | (__float_as_uint(h1) & 0xFFFF0000u);
            }
            *reinterpret_cast<u32x4*>(hrows + rr * row_bytes + c0 * 2) = o;
        }
    }
    if (ksteps > kRtKEarly * kRtWaves) {
#pragma unroll
        for (int u = kRtKEarly; u < kRtKPer; ++u) load_b(u);
    }
    __syncthreads();

    // 3. this wave's K steps, then the fixed-order sum of the 16 partial tiles
    const char* arow = hrows + col * row_bytes + c * 16;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < kRtKPer; ++u) {
        const int i = wave + u * kRtWaves;
        if (i < ksteps) {
            const u32x4 a = *reinterpret_cast<const u32x4*>(arow + i * 64);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                           __builtin_bit_cast(bf16x8, b[u]), acc, 0, 0, 0);
        }
    }
    part[wave * kWave + lane] = acc;
    __syncthreads();
    // thread u < 256 sums element (lane u/4, register u%4) over the waves in order;
    // D: lane l holds expert tile*16 + l%16, rows 4*(l/16) .. +3; scores rounded to bf16
    if (threadIdx.x < 4 * kWave) {
        const int l = threadIdx.x >> 2, q = threadIdx.x & 3;
        const float* pf = reinterpret_cast<const float*>(part);
        float sum = pf[l * 4 + q];
        for (int w = 1; w < kRtWaves; ++w) sum += pf[(w * kWave + l) * 4 + q];
        const int t = t0 + 4 * (l >> 4) + q;
        if (t < A.T) A.probs[static_cast<int64_t>(t) * E + tile * 16 + (l & 15)] = bf16r(sum);
    }
}

// One wave per token: softmax over the scores in probs (in place), then k
// rounds of a wave arg-max on 64-bit keys (probability bits, then the inverted
// id: the larger probability wins, equal probabilities go to the lower id),
// renormalisation and the per-expert scale. Lane l owns entries n = j*64 + l.
constexpr int kTkWaves = 4;
__global__ __launch_bounds__(kTkWaves * kWave) void router_topk_kernel(RouterArgs A) {
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * kTkWaves + wave;
    if (t >= A.T) return;
    const int E = A.E;
    float* row = A.probs + static_cast<int64_t>(t) * E;
    constexpr int J = kRtMaxE / kWave;
    float s[J];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int n = j * kWave + lane;
        s[j] = n < E ? row[n] : -INFINITY;
        mx = fmaxf(mx, s[j]);
    }
    mx = __ockl_wfred_max_f32(mx);
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int n = j * kWave + lane;
        s[j] = n < E ? expf(s[j] - mx) : 0.0f;
        part += s[j];
    }
    const float sum = __ockl_wfred_add_f32(part);
    unsigned long long key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int n = j * kWave + lane;
        s[j] = s[j] / sum;  // probabilities (>= 0)
        if (n < E) row[n] = s[j];
        key[j] = n < E ? (static_cast<unsigned long long>(__float_as_uint(s[j])) << 32) | (0xFFFFFFFFu - n) : 0ull;
    }
    float my_v = 0.0f, wsum = 0.0f;
    int my_i = 0;
    for (int r = 0; r < A.k; ++r) {
        unsigned long long best = 0ull;
#pragma unroll
        for (int j = 0; j < J; ++j) best = key[j] > best ? key[j] : best;
        best = __ockl_wfred_max_u64(best);
        const float v = __uint_as_float(static_cast<uint32_t>(best >> 32));
        const int n = static_cast<int>(0xFFFFFFFFu - static_cast<uint32_t>(best));
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (key[j] == best) key[j] = 0ull;  // taken
        if (lane == r) {
            my_v = v;
            my_i = n;
        }
        wsum += v;
    }
    if (lane < A.k) {
        A.topk_w[static_cast<int64_t>(t) * A.k + lane] = my_v / wsum * bf16_bits_to_f32(A.pes[my_i]);
        A.topk_ids[static_cast<int64_t>(t) * A.k + lane] = my_i;
    }
}

size_t router_lds_bytes(int H) {
    return static_cast<size_t>(kRtRows) * (H * 2 + kRtRowPad) + static_cast<size_t>(kRtWaves) * kWave * 16 +
           static_cast<size_t>(H) * 2;
}

}  // namespace

int launch_router(const void* x, int xd, int64_t xs, const void* scale, const void* proj, const void* pes,
                  int wd, float eps, int64_t T, int64_t H, int64_t E, int64_t k, float* probs, float* topk_w,
                  int64_t* topk_ids, hipStream_t st) {
    if (T < 0 || H <= 0 || E <= 0 || k <= 0) return KSL_ERR_SHAPE;
    if (T == 0) return KSL_OK;
    if (!x || !scale || !proj || !pes || !probs || !topk_w || !topk_ids) return KSL_ERR_ARG;
    if (H % 32 != 0 || H > kRtMaxH || E % 16 != 0 || E > kRtMaxE || k > E || k > kRtMaxK || xs < H)
        return KSL_ERR_SHAPE;
    if (wd != KSL_DTYPE_BF16 || (xd != KSL_DTYPE_BF16 && xd != KSL_DTYPE_F16)) return KSL_ERR_ARG;
    if (xs % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(scale) % 16 ||
        reinterpret_cast<uintptr_t>(proj) % 16)
        return KSL_ERR_ALIGN;
    RouterArgs A;
    A.x = static_cast<const char*>(x);
    A.scale = static_cast<const uint16_t*>(scale);
    A.proj = static_cast<const uint16_t*>(proj);
    A.pes = static_cast<const uint16_t*>(pes);
    A.probs = probs;
    A.topk_w = topk_w;
    A.topk_ids = topk_ids;
    A.xs = xs;
    A.eps = eps;
    A.T = static_cast<int>(T);
    A.H = static_cast<int>(H);
    A.E = static_cast<int>(E);
    A.k = static_cast<int>(k);
    const size_t lds = router_lds_bytes(A.H);
    const dim3 grid1(static_cast<unsigned>((T + kRtRows - 1) / kRtRows), static_cast<unsigned>(E / 16));
    static const bool attr = [] {
        const bool a = hipFuncSetAttribute(reinterpret_cast<const void*>(&router_scores_kernel<KSL_DTYPE_BF16>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        const bool b = hipFuncSetAttribute(reinterpret_cast<const void*>(&router_scores_kernel<KSL_DTYPE_F16>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
        (void)hipGetLastError();
        return a && b;
    }();
    (void)attr;
    if (xd == KSL_DTYPE_BF16)
        hipLaunchKernelGGL((router_scores_kernel<KSL_DTYPE_BF16>), grid1, dim3(kRtThreads), lds, st, A);
    else
        hipLaunchKernelGGL((router_scores_kernel<KSL_DTYPE_F16>), grid1, dim3(kRtThreads), lds, st, A);
    KSL_LAUNCH_CHECK();
    const unsigned grid2 = static_cast<unsigned>((T + kTkWaves - 1) / kTkWaves);
    hipLaunchKernelGGL(router_topk_kernel, dim3(grid2), dim3(kTkWaves * kWave), 0, st, A);
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

}  // namespace ksl

extern "C" int ksl_moe_router(const void* x, int x_dtype, int64_t x_stride, const void* scale, const void* proj_w,
                              const void* per_expert_scale, int w_dtype, float eps, int64_t T, int64_t H, int64_t E,
                              int64_t topk, float* probs, float* topk_w, int64_t* topk_ids, void* stream) {
    return ksl::launch_router(x, x_dtype, x_stride, scale, proj_w, per_expert_scale, w_dtype, eps, T, H, E, topk,
                              probs, topk_w, topk_ids, static_cast<hipStream_t>(stream));
}
