// Per-denoising-step sampler pass over [rows, V] logits: entropy, Gumbel-max
// sample and argmax (kernels/fused_sampler_ops.py:22-93), one workgroup per
// row, one read of the row.
//
//   entropy: H = logsumexp(x) - sum(softmax(x) * x), online over the row
//            (running max m, s = sum e^(x-m), t = sum x e^(x-m)); entries equal
//            to -inf contribute nothing (torch's Categorical.entropy).
//   sample : first index of the max of fp32(x + g), g = -log(-log(u)),
//            u = tl.rand(seed + row, col) clamped to [1e-10, 1 - 1e-7]: Triton's
//            generator, Philox4x32-10 on the counter (col, 0, 0, 0) with the
//            row's key, first output word to float (triton/language/random.py).
//   argmax : first index of the max of x.
// Each thread walks its own columns in increasing order; the per-thread
// states merge by a fixed xor tree per wave and then in wave order, so results
// do not depend on timing. A column whose x + 16 (above the largest possible
// g, 15.94) is below the thread's best noisy score cannot be sampled and skips
// the generator: the result is the same, and most columns of a peaked row skip.
#include "ksl_common.h"

namespace ksl {
namespace {

constexpr int kSmpWaves = 16;
constexpr int kSmpThreads = kSmpWaves * kWave;
constexpr float kGumbelBound = 16.0f;  // > -log(-log(1 - 1e-7)) = 15.94

struct SmpArgs {
    const void* x;
    int64_t stride;  // elements between rows
    int V;
    int64_t seed;
    float* ent;      // [rows] or null
    int64_t* samp;   // [rows] or null (with amax)
    int64_t* amax;   // [rows] or null
};

// First output word of Philox4x32-10 for the counter (c0, 0, 0, 0) and key (k0, k1).
__device__ __forceinline__ uint32_t philox_first(uint32_t c0, uint32_t k0, uint32_t k1) {
    uint32_t c1 = 0, c2 = 0, c3 = 0;
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint64_t p0 = static_cast<uint64_t>(0xD2511F53u) * c0;
        const uint64_t p2 = static_cast<uint64_t>(0xCD9E8D57u) * c2;
        const uint32_t n0 = static_cast<uint32_t>(p2 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        c1 = static_cast<uint32_t>(p2);
        c3 = static_cast<uint32_t>(p0);
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

// Triton's uint32 -> [0, 1): int32 bits, negative i mapped to -i - 1 (= ~i),
// times 4.6566127342e-10 (fp32 0x2fffffff).
__device__ __forceinline__ float uniform_from(uint32_t r) {
    int32_t i = static_cast<int32_t>(r);
    i = i < 0 ? ~i : i;
    return static_cast<float>(i) * __uint_as_float(0x2fffffffu);
}

__device__ __forceinline__ float gumbel(uint32_t col, uint32_t k0, uint32_t k1) {
    float u = uniform_from(philox_first(col, k0, k1));
    u = fminf(fmaxf(u, __uint_as_float(0x2edbe6ffu)), __uint_as_float(0x3f7ffffeu));  // [1e-10, 1 - 1e-7]
    return -logf(-logf(u));
}

struct SmpState {
    float m, s, t;     // entropy: running max, sum e^(x-m), sum x e^(x-m)
    float ab;          // argmax value
    int ai;
    float gb;          // best noisy score
    int gi;
};

__device__ __forceinline__ void ent_merge(float& m, float& s, float& t, float m2, float s2, float t2) {
    const float mn = fmaxf(m, m2);
    if (mn == -INFINITY) return;  // both empty
    const float a1 = m == -INFINITY ? 0.0f : __expf(m - mn);
    const float a2 = m2 == -INFINITY ? 0.0f : __expf(m2 - mn);
    s = s * a1 + s2 * a2;
    t = t * a1 + t2 * a2;
    m = mn;
}

// (value, index) maximum, equal values to the lower index.
__device__ __forceinline__ void arg_merge(float& b, int& i, float b2, int i2) {
    if (b2 > b || (b2 == b && i2 < i)) {
        b = b2;
        i = i2;
    }
}

template <bool ENT, bool SAMP>
__device__ __forceinline__ void take4(SmpState& st, const float (&x)[4], int v0, uint32_t k0, uint32_t k1, int n) {
    if constexpr (ENT) {
        float gm = -INFINITY;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (q < n) gm = fmaxf(gm, x[q]);
        if (gm > st.m) {
            const float a = st.m == -INFINITY ? 0.0f : __expf(st.m - gm);
            st.s *= a;
            st.t *= a;
            st.m = gm;
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (q < n && x[q] > -INFINITY) {
                const float e = __expf(x[q] - st.m);
                st.s += e;
                st.t = __builtin_fmaf(x[q], e, st.t);
            }
        }
    }
    if constexpr (SAMP) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (q >= n) continue;
            if (x[q] > st.ab) {
                st.ab = x[q];
                st.ai = v0 + q;
            }
            if (!(x[q] + kGumbelBound < st.gb)) {
                const float xg = x[q] + gumbel(static_cast<uint32_t>(v0 + q), k0, k1);
                if (xg > st.gb) {
                    st.gb = xg;
                    st.gi = v0 + q;
                }
            }
        }
    }
}

template <int XD, bool ENT, bool SAMP, bool VEC>
__global__ __launch_bounds__(kSmpThreads) void sampler_kernel(SmpArgs A) {
    typedef typename Elem<XD>::T XT;
    const int row = blockIdx.x;
    const XT* x = static_cast<const XT*>(A.x) + static_cast<int64_t>(row) * A.stride;
    const int tid = threadIdx.x;
    // the row's key: seed + row in int32 when the seed fits int32 (wrapping),
    // else in int64; sign-extended to 64 bits (k0 low, k1 high)
    uint64_t key;
    if (A.seed >= INT32_MIN && A.seed <= INT32_MAX)
        key = static_cast<uint64_t>(static_cast<int64_t>(
            static_cast<int32_t>(static_cast<uint32_t>(A.seed) + static_cast<uint32_t>(row))));
    else
        key = static_cast<uint64_t>(A.seed + row);
    const uint32_t k0 = static_cast<uint32_t>(key), k1 = static_cast<uint32_t>(key >> 32);
    SmpState st{-INFINITY, 0.0f, 0.0f, -INFINITY, 0, -INFINITY, 0};
    if constexpr (VEC) {
        // fp32, V % 4 == 0, 16-byte aligned rows: columns 4i .. 4i+3, i = tid + k*threads
        const int nv = A.V >> 2;
        const f32x4* xv = reinterpret_cast<const f32x4*>(x);
        for (int i0 = tid; i0 < nv; i0 += 4 * kSmpThreads) {
            f32x4 q[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * kSmpThreads;
                q[u] = xv[i < nv ? i : i0];
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const int i = i0 + u * kSmpThreads;
                if (i < nv) {
                    const float f[4] = {q[u][0], q[u][1], q[u][2], q[u][3]};
                    take4<ENT, SAMP>(st, f, 4 * i, k0, k1, 4);
                }
            }
        }
    } else {
        // any dtype and alignment: column c = tid + k*threads, one at a time
        for (int c = tid; c < A.V; c += kSmpThreads) {
            const float f[4] = {Elem<XD>::load(x + c), 0.0f, 0.0f, 0.0f};
            take4<ENT, SAMP>(st, f, c, k0, k1, 1);
        }
    }
    // merge: xor tree within the wave, then the waves in order
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        if constexpr (ENT)
            ent_merge(st.m, st.s, st.t, __shfl_xor(st.m, off, kWave), __shfl_xor(st.s, off, kWave),
                      __shfl_xor(st.t, off, kWave));
        if constexpr (SAMP) {
            arg_merge(st.ab, st.ai, __shfl_xor(st.ab, off, kWave), __shfl_xor(st.ai, off, kWave));
            arg_merge(st.gb, st.gi, __shfl_xor(st.gb, off, kWave), __shfl_xor(st.gi, off, kWave));
        }
    }
    __shared__ SmpState part[kSmpWaves];
    if ((tid & (kWave - 1)) == 0) part[tid / kWave] = st;
    __syncthreads();
    if (tid == 0) {
        SmpState r = part[0];
        for (int w = 1; w < kSmpWaves; ++w) {
            const SmpState& p = part[w];
            if constexpr (ENT) ent_merge(r.m, r.s, r.t, p.m, p.s, p.t);
            if constexpr (SAMP) {
                arg_merge(r.ab, r.ai, p.ab, p.ai);
                arg_merge(r.gb, r.gi, p.gb, p.gi);
            }
        }
        if constexpr (ENT) A.ent[row] = r.m + logf(r.s) - r.t / r.s;
        if constexpr (SAMP) {
            A.samp[row] = r.gi;
            A.amax[row] = r.ai;
        }
    }
}

template <int XD, bool ENT, bool SAMP>
void launch_smp_x(const SmpArgs& A, int64_t rows, bool vec, hipStream_t st) {
    if (XD == KSL_DTYPE_F32 && vec)
        hipLaunchKernelGGL((sampler_kernel<XD, ENT, SAMP, true>), dim3(static_cast<unsigned>(rows)),
                           dim3(kSmpThreads), 0, st, A);
    else
        hipLaunchKernelGGL((sampler_kernel<XD, ENT, SAMP, false>), dim3(static_cast<unsigned>(rows)),
                           dim3(kSmpThreads), 0, st, A);
}

template <bool ENT, bool SAMP>
int launch_smp(const void* x, int dtype, int64_t rows, int64_t V, int64_t stride, int64_t seed, float* ent,
               int64_t* samp, int64_t* amax, hipStream_t st) {
    if (rows < 0 || V < 1 || V >= (int64_t(1) << 31) || rows >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    if (rows > 0 && stride < V) return KSL_ERR_SHAPE;
    if (rows == 0) return KSL_OK;
    if (!x || (ENT && !ent) || (SAMP && (!samp || !amax))) return KSL_ERR_ARG;
    SmpArgs A{x, stride, static_cast<int>(V), seed, ent, samp, amax};
    const bool vec = V % 4 == 0 && stride % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0;
    switch (dtype) {
        case KSL_DTYPE_F32: launch_smp_x<KSL_DTYPE_F32, ENT, SAMP>(A, rows, vec, st); break;
        case KSL_DTYPE_BF16: launch_smp_x<KSL_DTYPE_BF16, ENT, SAMP>(A, rows, false, st); break;
        case KSL_DTYPE_F16: launch_smp_x<KSL_DTYPE_F16, ENT, SAMP>(A, rows, false, st); break;
        default: return KSL_ERR_ARG;
    }
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

}  // namespace
}  // namespace ksl

extern "C" int ksl_entropy(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                           float* entropy, void* stream) {
    return ksl::launch_smp<true, false>(logits, dtype, rows, V, row_stride, 0, entropy, nullptr, nullptr,
                                        static_cast<hipStream_t>(stream));
}

extern "C" int ksl_gumbel_argmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                                 int64_t seed, int64_t* sampled, int64_t* argmax, void* stream) {
    return ksl::launch_smp<false, true>(logits, dtype, rows, V, row_stride, seed, nullptr, sampled, argmax,
                                        static_cast<hipStream_t>(stream));
}

extern "C" int ksl_sample_step(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                               int64_t seed, int64_t* sampled, int64_t* argmax, float* entropy, void* stream) {
    return ksl::launch_smp<true, true>(logits, dtype, rows, V, row_stride, seed, entropy, sampled, argmax,
                                       static_cast<hipStream_t>(stream));
}
