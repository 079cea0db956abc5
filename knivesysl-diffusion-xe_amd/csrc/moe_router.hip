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
// Two launches. Scores: one workgroup of 16 waves per 8 tokens x 16 experts
// (so the projection, 2*E*H bytes, is spread over E/16 workgroups per token
// block, and a CU reads 16 projection rows and 8 token rows): 8 waves
// normalise the rows into LDS (bf16, padded rows: conflict-free MFMA operand
// reads), 8 waves stream the projection and multiply with
// v_mfma_f32_16x16x32_bf16, the K steps split over them; the scores go to the
// probabilities buffer. Then one wave per token does softmax (in place),
// top-k and the renormalisation in registers.
#include <cmath>
#include <utility>

#include "ksl_common.h"

namespace ksl {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kRtWaves = 16;
constexpr int kRtThreads = kRtWaves * kWave;
constexpr int kRtRows = 8;                         // tokens per workgroup: one per normalising wave
constexpr int kRtLoad = kRtWaves - kRtRows;        // waves 0..7 load the projection and multiply
constexpr int kRtMaxH = 4096;
constexpr int kRtMaxE = 256;
constexpr int kRtMaxK = 16;
constexpr int kRtRowPad = 16;                      // bytes of padding per LDS row
constexpr int kRtKPer = kRtMaxH / 32 / kRtLoad;    // K steps per loading wave at most

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
    float root;            // fp32(H ** -0.5)
    int T, H, E, k;
};

// Two floats to two bf16 (round to nearest even) in one v_cvt_pk_bf16_f32,
// packed, a in the low half: the same values as bf16r for every non-NaN input
// (fp32 denormals are kept, .amdhsa_float_denorm_mode_32 = 3); a NaN stays a
// NaN. Used for the router's intermediate activations, where only finite
// values are observable.
__device__ __forceinline__ uint32_t bf16x2_rne(float a, float b) {
    const f32x2 v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Scores of 8 tokens x 16 experts per workgroup (grid: token blocks x expert
// tiles), 16 waves in two roles, so that the waves that stream the projection
// (2*16*H bytes per workgroup, the bulk of its reads) never hold up the
// normalisation:
//  - waves 0..7 normalise token rows 0..7, one each, in the RMSNorm kernels'
//    layout and order (8 columns per lane and step, an fma chain over the
//    steps, a fixed xor tree over the lanes: r has the bits of the fused
//    RMSNorm's), apply the router scale and H^-1/2 and write the bf16 rows to
//    LDS (padded: the MFMA operand reads are conflict-free), the first half of
//    the column steps, a barrier, then the rest;
//  - waves 8..15 load the projection fragments of K steps g, g + 8, ... for
//    g = wave - 8 (KPER = ceil(H/256) of them, a template parameter so that
//    the registers held are those the row needs, all in flight at once; no
//    load predicated, so the compiler waits for each by count), multiply the
//    first half of the rows with v_mfma_f32_16x16x32_bf16 (tokens in MFMA rows
//    0..7) while the second half is normalised, then the rest.
// The row loads are issued before a first barrier and the projection loads
// after it, so the rows are not queued behind the projection (a CU serves its
// loads in issue order); no barrier waits for global loads. 128 threads then add
// the 8 partial tiles of their (token, expert) in order and store the
// bf16-rounded score as fp32 into probs.
template <int XD, int KPER>
__global__ __launch_bounds__(kRtThreads) void router_scores_kernel(RouterArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    constexpr int NS = (KPER + 1) / 2;  // 512-column steps covering the row
    constexpr int NS1 = NS / 2;         // of them normalised before the first MFMAs
    const int H = A.H, E = A.E;
    const int row_bytes = H * 2 + kRtRowPad;
    char* hrows = lds;                                                  // [8][row_bytes] bf16
    f32x4* part = reinterpret_cast<f32x4*>(lds + kRtRows * row_bytes);  // [kRtLoad][32]
    const int wave = wave_id();
    const int lane = threadIdx.x & (kWave - 1);
    const int t0 = blockIdx.x * kRtRows;
    const int e0 = blockIdx.y * 16;
    const int ksteps = H / 32;
    const int col = lane & 15, c = lane >> 4;

    if (wave < kRtRows) {
        // normalising wave: token row t0 + wave, lane owns columns s*512 + lane*8 .. +8
        const int t = t0 + wave < A.T ? t0 + wave : A.T - 1;  // rows past T: computed, never stored
        const char* xr = A.x + static_cast<int64_t>(t) * A.xs * 2;
        Raw8<XD> xv[NS];
        u32x4 sv[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {  // not predicated: past the row end column 0, dropped
            const int c0 = s * 8 * kWave + lane * 8;
            const int cc = c0 < H ? c0 : 0;
            xv[s] = raw_load8<XD>(xr + cc * 2);
            sv[s] = *reinterpret_cast<const u32x4*>(A.scale + cc);
        }
        dma_barrier();  // every row load is queued before the first projection load
        float ss = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if (s * 8 * kWave + lane * 8 >= H) xv[s] = Raw8<XD>{};  // past the row end: exact zeros
            ss = rms_sumsq8<XD>(xv[s], ss);
        }
        const float r = rms_scale(ss, 6, H, A.eps);
        const float root_py = A.root;
        char* hr = hrows + wave * row_bytes;
        auto norm_step = [&](int s) {
            const int c0 = s * 8 * kWave + lane * 8;
            if (c0 >= H) return;
            float xf[8], sc[8];
            raw_unpack8<XD>(xv[s], xf);
            raw_unpack8<KSL_DTYPE_BF16>(Raw8<KSL_DTYPE_BF16>{{sv[s]}}, sc);
            u32x4 o;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t y = bf16x2_rne(xf[2 * j] * r, xf[2 * j + 1] * r);
                const uint32_t z = bf16x2_rne(__uint_as_float(y << 16) * sc[2 * j],
                                              __uint_as_float(y & 0xFFFF0000u) * sc[2 * j + 1]);
                o[j] = bf16x2_rne(__uint_as_float(z << 16) * root_py, __uint_as_float(z & 0xFFFF0000u) * root_py);
            }
            *reinterpret_cast<u32x4*>(hr + c0 * 2) = o;
        };
#pragma unroll
        for (int s = 0; s < NS1; ++s) norm_step(s);
        lds_sync();
#pragma unroll
        for (int s = NS1; s < NS; ++s) norm_step(s);
        lds_sync();
    } else {
        // loading wave g: K steps g, g + 8, ... (a step past the end reloads the
        // last one, unused); A fragment: lane holds token row col % 8, K columns
        // c*8 .. +8 (MFMA rows 8..15 repeat rows 0..7; their outputs are not
        // used). Steps u < 2*NS1 lie in the rows' first NS1 column steps and are
        // multiplied while the rest is normalised; steps u < KPER - 1 exist for
        // every wave, the last one for waves g < ksteps % 8.
        const int g = wave - kRtRows;
        const uint16_t* prow = A.proj + static_cast<int64_t>(e0 + col) * H + c * 8;
        u32x4 b[KPER];
        dma_barrier();
#pragma unroll
        for (int u = 0; u < KPER; ++u) {
            const int i = g + u * kRtLoad;
            b[u] = *reinterpret_cast<const u32x4*>(prow + (i < ksteps ? i : ksteps - 1) * 32);
        }
        const char* arow = hrows + (col & (kRtRows - 1)) * row_bytes + c * 16;
        u32x4 a[KPER];
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        lds_sync();
#pragma unroll
        for (int u = 0; u < 2 * NS1; ++u) a[u] = *reinterpret_cast<const u32x4*>(arow + (g + u * kRtLoad) * 64);
#pragma unroll
        for (int u = 0; u < 2 * NS1; ++u)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[u]),
                                                           __builtin_bit_cast(bf16x8, b[u]), acc, 0, 0, 0);
        asm volatile("" : "+v"(acc));  // these MFMAs before the barrier, not after it
        lds_sync();
#pragma unroll
        for (int u = 2 * NS1; u < KPER; ++u) {
            const int i = g + u * kRtLoad;
            a[u] = *reinterpret_cast<const u32x4*>(arow + (i < ksteps ? i : 0) * 64);
        }
#pragma unroll
        for (int u = 2 * NS1; u < KPER - 1; ++u)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[u]),
                                                           __builtin_bit_cast(bf16x8, b[u]), acc, 0, 0, 0);
        if (g + (KPER - 1) * kRtLoad < ksteps)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a[KPER - 1]),
                                                           __builtin_bit_cast(bf16x8, b[KPER - 1]), acc, 0, 0, 0);
        // D: lane l < 32 holds tokens 4*(l/16) .. +3 of expert column l % 16
        if (lane < 32) part[g * 32 + lane] = acc;
    }
    lds_sync();
    if (threadIdx.x < kRtRows * 16) {
        const int tt = threadIdx.x >> 4, e = threadIdx.x & 15;
        const float* pf = reinterpret_cast<const float*>(part) + ((tt >> 2) * 16 + e) * 4 + (tt & 3);
        float sum = pf[0];
#pragma unroll
        for (int g = 1; g < kRtLoad; ++g) sum += pf[g * 32 * 4];
        if (t0 + tt < A.T) A.probs[static_cast<int64_t>(t0 + tt) * E + e0 + e] = bf16r(sum);
    }
}

size_t router_lds_bytes(int H) {
    return static_cast<size_t>(kRtRows) * (H * 2 + kRtRowPad) + static_cast<size_t>(kRtLoad) * 32 * 16;
}

// One wave per token: softmax over the scores in probs (in place), then k
// rounds of selection: the wave max of the probability bits (as int: the
// probabilities are >= 0, taken entries -1, entries past E -2), then the
// lowest id holding it (one ballot per lane slot: ids n = j*64 + lane rise
// with j, then with the lane) — the larger probability first, equal
// probabilities to the lower id. Renormalisation in rank order, each rank's
// lane reading its expert's scale from the lane that loaded it.
constexpr int kTkWaves = 4;

// Wave max of an int or a float, left in every lane, by a butterfly of cross-lane moves
// (DPP quad_perm for partners l ^ 1 and l ^ 2, quad_perm then row_half_mirror
// for l ^ 4, row_ror:8 for l ^ 8, v_permlane16_swap / v_permlane32_swap for
// l ^ 16 and l ^ 32, where each lane ends up with its own value and the
// partner's): no round trip through scalar registers. A max is exact in any
// order.
template <int CTRL>
__device__ __forceinline__ int dpp_mov_i32(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}
__device__ __forceinline__ int wave_max_bfly(int v) {
    v = max(v, dpp_mov_i32<0xB1>(v));
    v = max(v, dpp_mov_i32<0x4E>(v));
    v = max(v, dpp_mov_i32<0x141>(dpp_mov_i32<0x1B>(v)));
    v = max(v, dpp_mov_i32<0x128>(v));
    const auto p16 = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
    v = max(static_cast<int>(p16[0]), static_cast<int>(p16[1]));
    const auto p32 = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
    return max(static_cast<int>(p32[0]), static_cast<int>(p32[1]));
}

__device__ __forceinline__ float wave_max_bfly(float v) {
    v = fmaxf(v, __int_as_float(dpp_mov_i32<0xB1>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov_i32<0x4E>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(dpp_mov_i32<0x141>(dpp_mov_i32<0x1B>(__float_as_int(v)))));
    v = fmaxf(v, __int_as_float(dpp_mov_i32<0x128>(__float_as_int(v))));
    const auto p16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(p16[0]), __uint_as_float(p16[1]));
    const auto p32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p32[0]), __uint_as_float(p32[1]));
}

template <int J>
__global__ __launch_bounds__(kTkWaves * kWave) void router_topk_kernel(RouterArgs A) {
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    const int t = blockIdx.x * kTkWaves + wave;
    if (t >= A.T) return;
    const int E = A.E;
    float* row = A.probs + static_cast<int64_t>(t) * E;
    float s[J], pe[J];
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < J; ++j) {  // loads not predicated: past E the last entry, dropped
        const int n = j * kWave + lane;
        const int nc = n < E ? n : E - 1;
        s[j] = row[nc];
        pe[j] = bf16_bits_to_f32(A.pes[nc]);
        if (n >= E) s[j] = -INFINITY;
        mx = fmaxf(mx, s[j]);
    }
    mx = wave_max_bfly(mx);
    float psum = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int n = j * kWave + lane;
        s[j] = n < E ? expf(s[j] - mx) : 0.0f;
        psum += s[j];
    }
    const float sum = __ockl_wfred_add_f32(psum);
    int key[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int n = j * kWave + lane;
        s[j] = s[j] / sum;  // probabilities (>= 0)
        if (n < E) row[n] = s[j];
        key[j] = n < E ? __float_as_int(s[j]) : -2;
    }
    // rounds without branches: the id is picked with scalar selects, and the
    // per-expert scale is fetched once at the end by the lane of each rank
    float my_v = 0.0f, wsum = 0.0f;
    int my_i = 0;
    for (int r = 0; r < A.k; ++r) {
        int m = key[0];
#pragma unroll
        for (int j = 1; j < J; ++j) m = key[j] > m ? key[j] : m;
        const int best = wave_max_bfly(m);
        int id = 0;
#pragma unroll
        for (int j = J - 1; j >= 0; --j) {  // the lowest slot with a hit wins
            const unsigned long long hit = __ballot(key[j] == best);
            const int cand = j * kWave + __ffsll(static_cast<long long>(hit)) - 1;
            id = hit != 0ull ? cand : id;
        }
#pragma unroll
        for (int j = 0; j < J; ++j)
            if (j * kWave + lane == id) key[j] = -1;  // taken
        const float v = __int_as_float(best);
        if (lane == r) {
            my_v = v;
            my_i = id;
        }
        wsum += v;
    }
    float my_sc = 0.0f;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const float pj = __shfl(pe[j], my_i & (kWave - 1), kWave);
        if ((my_i >> 6) == j) my_sc = pj;
    }
    if (lane < A.k) {
        A.topk_w[static_cast<int64_t>(t) * A.k + lane] = my_v / wsum * my_sc;
        A.topk_ids[static_cast<int64_t>(t) * A.k + lane] = my_i;
    }
}

template <int... I>
void set_scores_attr(bool& ok, std::integer_sequence<int, I...>) {
    auto one = [&](auto kernel) {
        ok = ok && hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    };
    (one(&router_scores_kernel<KSL_DTYPE_BF16, I + 1>), ...);
    (one(&router_scores_kernel<KSL_DTYPE_F16, I + 1>), ...);
}

template <int... I>
void launch_scores(int xd, int kper, dim3 grid, size_t lds, const RouterArgs& A, hipStream_t st,
                   std::integer_sequence<int, I...>) {
    auto one = [&](auto kp) {
        constexpr int KP = decltype(kp)::value;
        if (kper != KP) return;
        if (xd == KSL_DTYPE_BF16)
            hipLaunchKernelGGL((router_scores_kernel<KSL_DTYPE_BF16, KP>), grid, dim3(kRtThreads), lds, st, A);
        else
            hipLaunchKernelGGL((router_scores_kernel<KSL_DTYPE_F16, KP>), grid, dim3(kRtThreads), lds, st, A);
    };
    (one(std::integral_constant<int, I + 1>{}), ...);
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
    A.root = static_cast<float>(1.0 / std::sqrt(static_cast<double>(H)));  // correctly rounded, as in the module
    A.T = static_cast<int>(T);
    A.H = static_cast<int>(H);
    A.E = static_cast<int>(E);
    A.k = static_cast<int>(k);
    const dim3 grid1(static_cast<unsigned>((T + kRtRows - 1) / kRtRows), static_cast<unsigned>(E / 16));
    static const bool attr = [] {
        bool ok = true;
        set_scores_attr(ok, std::make_integer_sequence<int, kRtKPer>{});
        (void)hipGetLastError();
        return ok;
    }();
    (void)attr;
    const int kper = (A.H / 32 + kRtLoad - 1) / kRtLoad;  // K steps per loading wave, 1..16
    launch_scores(xd, kper, grid1, router_lds_bytes(A.H), A, st, std::make_integer_sequence<int, kRtKPer>{});
    KSL_LAUNCH_CHECK();
    const unsigned grid2 = static_cast<unsigned>((T + kTkWaves - 1) / kTkWaves);
    if (E <= 2 * kWave)
        hipLaunchKernelGGL((router_topk_kernel<2>), dim3(grid2), dim3(kTkWaves * kWave), 0, st, A);
    else
        hipLaunchKernelGGL((router_topk_kernel<kRtMaxE / kWave>), dim3(grid2), dim3(kTkWaves * kWave), 0, st, A);
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
