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
// acc += scale[n, g] * partial. (Reference: fp16((q - z) * s) per weight then
// tl.dot, kernels/fused_moe_w4_v2.py:125-128, :172-175; the values agree within
// the fp16 rounding of the dequantised weight.)
//
// Memory pipeline. Loads retire in issue order (one vmcnt counter per wave),
// so a load consumed soon after issue would drain every weight prefetch behind
// it. Only weight loads therefore go through registers in the steady state:
//   - scales and zero-points of the workgroup's rows are copied to LDS once;
//   - activations are copied to LDS in MFMA fragment order (each lane's 16
//     bytes contiguous across the wave: conflict-free ds_read_b128);
//   - gate/up streams K in slabs of two groups through a double-buffered LDS
//     slab; the loads of slab s+1 are issued before the weight prefetches of
//     slab s, so waiting for them never waits for those prefetches;
//   - down holds all of its weights in registers (K = I is short) and reuses
//     them for every 32-row chunk of its expert.
//
// Work split: one workgroup per (expert, column block) walks all rows routed
// to its expert (sorted slots offsets[e] .. offsets[e+1]) in chunks of up to 32
// rows (one or two 16-row M tiles). Workgroups are remapped so that all column
// blocks of an expert run on the same XCD (shared L2 for its activations).
#include <type_traits>

#include "ksl_common.h"

namespace ksl {
namespace {

constexpr int kXcds = 8;

// blockIdx.x -> logical tile, placing consecutive logical tiles on one XCD
// (workgroups are dispatched round-robin over the XCDs).
__device__ __forceinline__ int xcd_remap(int bid, int nblocks) {
    if (nblocks % kXcds != 0) return bid;
    return (bid % kXcds) * (nblocks / kXcds) + bid / kXcds;
}


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

// ---------------------------------------------------------------- gate / up
constexpr int kGuWaves = 4;                   // each wave: one gate tile + one up tile
constexpr int kGuWgCols = 16 * kGuWaves;      // 64 columns of I per workgroup
constexpr int kGuThreads = kGuWaves * kWave;  // 256
constexpr int kGuSlab = 2;                    // quantisation groups (2 x 128 K) per A slab
constexpr int kGuPD = 2 * kGuSlab;            // weight groups in flight per wave
constexpr int kMaxMt = 2;                     // 16-row M tiles per row chunk
constexpr int kGuSlabBytes = kMaxMt * kGuSlab * 4 * kWave * 16;  // 16 KB per slab buffer
constexpr int kGuMaxG = 32;                   // H <= 4096
constexpr int kGuSzPer = 4 * 32 * kGuMaxG / kGuThreads;  // scale/zero dwords per thread (max)

struct GuArgs {
    const f16* a16;
    const int32_t* sorted_rows;
    const int32_t* offsets;
    const uint8_t* gu_q;
    const f16* gu_s;
    const f16* gu_z;
    f16* out2;
    int topk, I, H;
};

// Per-wave state for one (expert, column block) tile.
struct GuWave {
    const uint8_t* wq0;  // gate row of this lane, + c*16 bytes
    const uint8_t* wq1;  // up row
    int n0;              // first column of I of this wave
};

// Scale/zero dwords of the workgroup's 64 gate and 64 up rows, four [64 x G]
// fp16 blocks (s_gate, z_gate, s_up, z_up), loaded into registers first and
// written to LDS with the first activation slab.
struct GuSz {
    uint32_t v[kGuSzPer];
};

template <int ACT, int MT>
__device__ __forceinline__ void gateup_chunk(const GuArgs& A, const GuWave& W, char* __restrict__ lds_a,
                                             f16* __restrict__ lds_sz, const GuSz& sz, bool store_sz,
                                             int start, int m0, int mrows) {
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int G = A.H >> 7;
    const int NS = (G + kGuSlab - 1) / kGuSlab;
    const f16* sg = lds_sz;
    const f16* zg = lds_sz + 64 * G;
    const f16* su = lds_sz + 2 * 64 * G;
    const f16* zu = lds_sz + 3 * 64 * G;
    const int wcol = (tid / kWave) * 16 + col;  // row of this lane within the workgroup's 64

    // Staging of A slabs: chunk ch = tid + 256*j (j < 2*MT) covers row r = ch/32 and
    // the 16-byte K chunk kc = ch%32 of the slab (K offset kc*8 within 256).
    constexpr int NCH = 2 * MT;
    const f16* src[NCH];
    int dst[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
        const int ch = tid + kGuThreads * j;
        int r = ch >> 5;
        const int kc = ch & 31;
        const int rr = r & 15, t = r >> 4;
        const int gs = kc >> 4, cc = (kc >> 2) & 3, i = kc & 3;
        dst[j] = (((t * kGuSlab + gs) * 4 + i) * kWave + cc * 16 + rr) * 16;
        if (r >= mrows) r = mrows - 1;  // rows past the expert's last: loaded, never stored
        const int tok = A.sorted_rows[start + m0 + r] / A.topk;
        src[j] = A.a16 + static_cast<int64_t>(tok) * A.H + kc * 8;
    }
    // Every global load below is unconditional (addresses clamped instead):
    // a load under a branch makes the wait-count pass drain all loads in flight.
    auto stage_load = [&](int s, u32x4 (&stg)[NCH]) {
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
            const int kc8 = ((tid + kGuThreads * j) & 31) * 8;
            // past H (odd G, last slab): reload the slab start; feeds only groups >= G
            const int soff = s * 256 + kc8 < A.H ? s * 256 : -kc8;
            stg[j] = *reinterpret_cast<const u32x4*>(src[j] + soff);
        }
    };
    auto stage_store = [&](int buf, const u32x4 (&stg)[NCH]) {
#pragma unroll
        for (int j = 0; j < NCH; ++j)
            *reinterpret_cast<u32x4*>(lds_a + buf * kGuSlabBytes + dst[j]) = stg[j];
    };

    f32x4 acc[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    u32x4 wb[kGuPD][2];
    u32x4 stg[NCH];
    stage_load(0, stg);  // before the weight prefetch: waiting for it waits for nothing else
#pragma unroll
    for (int p = 0; p < kGuPD; ++p) {
        const int gp = p < G ? p : G - 1;
        wb[p][0] = *reinterpret_cast<const u32x4*>(W.wq0 + gp * 64);
        wb[p][1] = *reinterpret_cast<const u32x4*>(W.wq1 + gp * 64);
    }
    if (store_sz) {
        const int nd = 4 * 32 * G;
        uint32_t* d = reinterpret_cast<uint32_t*>(lds_sz);
#pragma unroll
        for (int k = 0; k < kGuSzPer; ++k) {
            const int i = tid + k * kGuThreads;
            if (i < nd) d[i] = sz.v[k];
        }
    }
    stage_store(0, stg);
    __syncthreads();

    // One quantisation group g, activations from LDS buffer P, weights from
    // prefetch slot SLOT (both compile-time); afterwards the slot is refilled
    // with group g + kGuPD (clamped: a redundant cached load, never a branch).
    auto group = [&](int g, auto GSc, auto Pc, auto SLOTc) {
        constexpr int gs = decltype(GSc)::value;
        constexpr int P = decltype(Pc)::value;
        constexpr int SLOT = decltype(SLOTc)::value;
        const u32x4 w0 = wb[SLOT][0], w1 = wb[SLOT][1];
        const float s0 = static_cast<float>(sg[wcol * G + g]);
        const float s1 = static_cast<float>(su[wcol * G + g]);
        const f16 z0 = zg[wcol * G + g] + static_cast<f16>(1024.0f);
        const f16 z1 = zu[wcol * G + g] + static_cast<f16>(1024.0f);
        const f16x2 zc0{z0, z0}, zc1{z1, z1};
        f32x4 part[2][MT];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16x8 b0 = nib8_minus_zero(w0[i], zc0);
            const f16x8 b1 = nib8_minus_zero(w1[i], zc1);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(
                    lds_a + P * kGuSlabBytes + (((t * kGuSlab + gs) * 4 + i) * kWave + lane) * 16);
                part[0][t] = mfma16x16x32(a, b0, part[0][t]);
                part[1][t] = mfma16x16x32(a, b1, part[1][t]);
            }
        }
        {
            const int gn = g + kGuPD < G ? g + kGuPD : G - 1;
            wb[SLOT][0] = *reinterpret_cast<const u32x4*>(W.wq0 + gn * 64);
            wb[SLOT][1] = *reinterpret_cast<const u32x4*>(W.wq1 + gn * 64);
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                acc[0][t][r] = __builtin_fmaf(s0, part[0][t][r], acc[0][t][r]);
                acc[1][t][r] = __builtin_fmaf(s1, part[1][t][r], acc[1][t][r]);
            }
        __builtin_amdgcn_sched_barrier(0);  // bound live ranges to one group
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    // The next slab's activation loads go out before the slab's weight prefetches.
    auto next_slab_load = [&](int s) {
        stage_load(s < NS ? s : NS - 1, stg);
        __builtin_amdgcn_sched_barrier(0);  // keep these loads ahead of the slab's weight prefetches
    };

    // Steady state: two slabs (four groups) per iteration, no branches inside.
    int g = 0;
    for (; g + 4 <= G; g += 4) {
        const int s = g / kGuSlab;
        next_slab_load(s + 1);
        group(g, I0{}, I0{}, I0{});
        group(g + 1, I1{}, I0{}, I1{});
        stage_store(1, stg);
        __syncthreads();
        next_slab_load(s + 2);
        group(g + 2, I0{}, I1{}, I2{});
        group(g + 3, I1{}, I1{}, I3{});
        stage_store(0, stg);
        __syncthreads();
    }
    // Tail of G % 4 groups (buffer 0 holds slab g/2, prefetch slots 0.. hold them).
    const int rem = G - g;
    if (rem == 1) {
        group(g, I0{}, I0{}, I0{});
    } else if (rem == 2) {
        group(g, I0{}, I0{}, I0{});
        group(g + 1, I1{}, I0{}, I1{});
    } else if (rem == 3) {
        next_slab_load(g / kGuSlab + 1);
        group(g, I0{}, I0{}, I0{});
        group(g + 1, I1{}, I0{}, I1{});
        stage_store(1, stg);
        __syncthreads();
        group(g + 2, I0{}, I1{}, I2{});
    }
    __syncthreads();  // LDS slab buffers free for the next chunk

    const int sc = perm8_store_index(W.n0 + col);
    f16* o = A.out2 + static_cast<int64_t>(start + m0) * A.I + sc;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = t * 16 + 4 * c + r;
            if (row < mrows)
                o[static_cast<int64_t>(row) * A.I] = static_cast<f16>(act_times_up<ACT>(acc[0][t][r], acc[1][t][r]));
        }
}

template <int ACT>
__global__ __launch_bounds__(kGuThreads) __attribute__((amdgpu_waves_per_eu(2))) void gateup_act_kernel(GuArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int nb_per_e = A.I / kGuWgCols;
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int e = tile / nb_per_e;
    const int nb = tile - e * nb_per_e;
    const int start = A.offsets[e];
    const int M = A.offsets[e + 1] - start;
    if (M <= 0) return;
    const int G = A.H >> 7;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;

    char* lds_a = lds;
    f16* lds_sz = reinterpret_cast<f16*>(lds + 2 * kGuSlabBytes);
    // scales / zeros: loads issued first, stored to LDS by the first chunk
    GuSz sz;
    {
        const int64_t gate0 = static_cast<int64_t>(e) * 2 * A.I + nb * kGuWgCols;
        const int64_t up0 = gate0 + A.I;
        const int nd = 32 * G;  // dwords per [64 x G] block (block starts are 4-byte aligned)
#pragma unroll
        for (int k = 0; k < kGuSzPer; ++k) {
            int i = tid + k * kGuThreads;
            if (i >= 4 * nd) i = 0;  // clamped, never stored
            const int b = i / nd, o = i - b * nd;
            const f16* base = ((b & 1) ? A.gu_z : A.gu_s) + ((b & 2) ? up0 : gate0) * G;
            sz.v[k] = reinterpret_cast<const uint32_t*>(base)[o];
        }
    }
    GuWave W;
    W.n0 = nb * kGuWgCols + wave * 16;
    const int64_t rg = static_cast<int64_t>(e) * 2 * A.I + W.n0 + col;
    W.wq0 = A.gu_q + rg * (A.H >> 1) + c * 16;
    W.wq1 = A.gu_q + (rg + A.I) * (A.H >> 1) + c * 16;
    // the first chunk's barrier (after its slab 0 staging) also publishes lds_sz
    for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
        const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
        if (mrows <= 16)
            gateup_chunk<ACT, 1>(A, W, lds_a, lds_sz, sz, m0 == 0, start, m0, mrows);
        else
            gateup_chunk<ACT, 2>(A, W, lds_a, lds_sz, sz, m0 == 0, start, m0, mrows);
    }
}

// --------------------------------------------------------------------- down
constexpr int kDnWaves = 4;
constexpr int kDnTiles = 2;                          // 16-column tiles of H per wave
constexpr int kDnWgCols = 16 * kDnTiles * kDnWaves;  // 128 columns of H per workgroup
constexpr int kDnThreads = kDnWaves * kWave;         // 256
constexpr int kDnBlock = kWave * 16;                 // one LDS fragment block: 64 lanes x 16 B
constexpr int kDnSzPer = (2 * kDnWgCols * 16 / 2 + kDnThreads - 1) / kDnThreads;  // I <= 1024

struct DnArgs {
    const f16* out2;
    const int32_t* offsets;
    const uint8_t* dn_q;
    const f16* dn_s;
    const f16* dn_z;
    f16* out3;
    int H, I;
};

typedef __attribute__((address_space(3))) void* lds_vptr;
typedef __attribute__((address_space(1))) void* gbl_vptr;

// Direct global -> LDS copy of one fragment block: lane L's 16 bytes land at
// lds_block + 16*L. lds_block must be wave-uniform.
__device__ __forceinline__ void dma16(const void* src, char* lds_block) {
    __builtin_amdgcn_global_load_lds((gbl_vptr)(const_cast<void*>(src)), (lds_vptr)lds_block, 16, 0, 0);
}

// The activation rows of one chunk, A[g][t][i] blocks: block (g, t, i) holds,
// for lane L = c*16 + rr, out2[row t*16 + rr][g*64 + c*16 + i*8 .. +8].
template <int G>
__device__ __forceinline__ void down_stage_a(const DnArgs& A, char* lds_a, int start, int m0, int mrows,
                                             int mt) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int rr = lane & 15, c = lane >> 4;
    const int nblk = G * mt * 2;
    for (int b = wave; b < nblk; b += kDnWaves) {
        const int i = b & 1;
        const int t = (b >> 1) % mt;
        const int g = (b >> 1) / mt;
        int r = t * 16 + rr;
        if (r >= mrows) r = mrows - 1;
        const f16* src = A.out2 + static_cast<int64_t>(start + m0 + r) * A.I + g * 64 + c * 16 + i * 8;
        dma16(src, lds_a + ((g * kMaxMt + t) * 2 + i) * kDnBlock);
    }
}

template <int G, int MT>
__device__ __forceinline__ void down_chunk(const DnArgs& A, const u32x2 (&w)[kDnTiles][G],
                                           const char* __restrict__ lds_a, const f16* __restrict__ lds_s,
                                           const f16* __restrict__ lds_z, int n0w, int wrow0, int start,
                                           int m0, int mrows) {
    // Down keeps one accumulator chain per tile: the scale is folded into the
    // B operand, b = fp16((q - z) * s), the reference's own dequantised weight.
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    f32x4 acc[kDnTiles][MT];
#pragma unroll
    for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < G; ++g) {
        f16x2 sc[kDnTiles], zc[kDnTiles];
#pragma unroll
        for (int j = 0; j < kDnTiles; ++j) {
            const int r = wrow0 + j * 16 + col;
            const f16 sv = lds_s[r * G + g];
            const f16 z = lds_z[r * G + g] + static_cast<f16>(1024.0f);
            sc[j] = f16x2{sv, sv};
            zc[j] = f16x2{z, z};
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            f16x8 a[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                a[t] = *reinterpret_cast<const f16x8*>(lds_a + ((g * kMaxMt + t) * 2 + i) * kDnBlock + lane * 16);
#pragma unroll
            for (int j = 0; j < kDnTiles; ++j) {
                const f16x8 b = nib8_dequant(w[j][g][i], zc[j], sc[j]);
#pragma unroll
                for (int t = 0; t < MT; ++t) acc[j][t] = mfma16x16x32(a[t], b, acc[j][t]);
            }
        }
    }
    f16* o = A.out3 + static_cast<int64_t>(start + m0) * A.H + n0w + col;
#pragma unroll
    for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = t * 16 + 4 * c + r;
                if (row < mrows) o[static_cast<int64_t>(row) * A.H + j * 16] = static_cast<f16>(acc[j][t][r]);
            }
}

// One workgroup: expert e, 128 columns of H. All of a wave's weights (2 tiles x
// G groups x 8 bytes per lane) are loaded once into registers and reused for
// every 32-row chunk of the expert; the chunk's activations go to LDS by
// direct global->LDS loads.
template <int G>
__global__ __launch_bounds__(kDnThreads) __attribute__((amdgpu_waves_per_eu(3))) void down_kernel(DnArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int nb_per_e = (A.H + kDnWgCols - 1) / kDnWgCols;
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int e = tile / nb_per_e;
    const int nb = tile - e * nb_per_e;
    const int start = A.offsets[e];
    const int M = A.offsets[e + 1] - start;
    if (M <= 0) return;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int nbase = nb * kDnWgCols;                                     // first column of the workgroup
    const int nrows = A.H - nbase < kDnWgCols ? A.H - nbase : kDnWgCols;  // multiple of 64
    const int n0w = nbase + wave * 16 * kDnTiles;                         // first column of this wave
    const bool wave_active = n0w < A.H;

    char* lds_a = lds;                                                      // [G][kMaxMt][2] blocks
    f16* lds_s = reinterpret_cast<f16*>(lds + G * kMaxMt * 2 * kDnBlock);  // [128][G]
    f16* lds_z = lds_s + kDnWgCols * G;

    // 1. scales / zeros of the workgroup's rows into registers
    const int64_t row0 = static_cast<int64_t>(e) * A.H + nbase;
    const int nd = nrows * G / 2;  // dwords per block; row0 even, so 4-byte aligned
    uint32_t szs[kDnSzPer], szz[kDnSzPer];
#pragma unroll
    for (int k = 0; k < kDnSzPer; ++k) {
        const int i = tid + k * kDnThreads < nd ? tid + k * kDnThreads : 0;  // clamped, never stored
        szs[k] = reinterpret_cast<const uint32_t*>(A.dn_s + row0 * G)[i];
        szz[k] = reinterpret_cast<const uint32_t*>(A.dn_z + row0 * G)[i];
    }
    // 2. all weights of this wave
    u32x2 w[kDnTiles][G];
    {
        // an inactive wave (H % 128 == 64, last block) loads the block's first rows instead
        const int wr = wave_active ? wave * 16 * kDnTiles : 0;
#pragma unroll
        for (int j = 0; j < kDnTiles; ++j) {
            const uint8_t* wp = A.dn_q + (row0 + wr + j * 16 + col) * (A.I >> 1) + c * 8;
#pragma unroll
            for (int g = 0; g < G; ++g) w[j][g] = *reinterpret_cast<const u32x2*>(wp + g * 32);
        }
    }
    // 3. activations of the first chunk, straight into LDS
    {
        const int mrows = M < 16 * kMaxMt ? M : 16 * kMaxMt;
        down_stage_a<G>(A, lds_a, start, 0, mrows, mrows <= 16 ? 1 : 2);
    }
#pragma unroll
    for (int k = 0; k < kDnSzPer; ++k) {
        const int i = tid + k * kDnThreads;
        if (i < nd) {
            reinterpret_cast<uint32_t*>(lds_s)[i] = szs[k];
            reinterpret_cast<uint32_t*>(lds_z)[i] = szz[k];
        }
    }
    // every wave's direct-to-LDS loads must have landed before any wave reads
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
        const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
        if (m0 > 0) {
            __syncthreads();  // previous chunk's LDS reads done
            down_stage_a<G>(A, lds_a, start, m0, mrows, mrows <= 16 ? 1 : 2);
            __builtin_amdgcn_s_waitcnt(0);
            __syncthreads();
        }
        if (wave_active) {
            // The nibble decode of w does not depend on the chunk: without this
            // (empty) redefinition it is hoisted out of the loop for all G
            // groups and keeps ~4x the weight registers live.
#pragma unroll
            for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
                for (int g = 0; g < G; ++g) asm volatile("" : "+v"(w[j][g]));
            if (mrows <= 16)
                down_chunk<G, 1>(A, w, lds_a, lds_s, lds_z, n0w, wave * 16 * kDnTiles, start, m0, mrows);
            else
                down_chunk<G, 2>(A, w, lds_a, lds_s, lds_z, n0w, wave * 16 * kDnTiles, start, m0, mrows);
        }
    }
}

}  // namespace

int launch_gateup(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                  const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H,
                  int64_t I, int act, void* out2, hipStream_t st) {
    if (!a16 || !sorted_rows || !offsets || !gu_q || !gu_s || !gu_z || !out2) return KSL_ERR_ARG;
    if (E <= 0 || H <= 0 || I <= 0 || topk <= 0) return KSL_ERR_SHAPE;
    if (H % 128 != 0 || I % kGuWgCols != 0 || H > 128 * kGuMaxG) return KSL_ERR_SHAPE;
    if (E * 2 * I * (H / 2) >= (int64_t(1) << 40)) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(gu_q) % 16 || reinterpret_cast<uintptr_t>(a16) % 16 ||
        reinterpret_cast<uintptr_t>(gu_s) % 4 || reinterpret_cast<uintptr_t>(gu_z) % 4 ||
        reinterpret_cast<uintptr_t>(out2) % 2)
        return KSL_ERR_ALIGN;
    GuArgs A;
    A.a16 = static_cast<const f16*>(a16);
    A.sorted_rows = sorted_rows;
    A.offsets = offsets;
    A.gu_q = gu_q;
    A.gu_s = static_cast<const f16*>(gu_s);
    A.gu_z = static_cast<const f16*>(gu_z);
    A.out2 = static_cast<f16*>(out2);
    A.topk = static_cast<int>(topk);
    A.I = static_cast<int>(I);
    A.H = static_cast<int>(H);
    const unsigned grid = static_cast<unsigned>(E * (I / kGuWgCols));
    const size_t lds = 2 * kGuSlabBytes + 4 * 64 * (H / 128) * sizeof(f16);
    if (act == KSL_ACT_GELU_TANH)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_GELU_TANH>), dim3(grid), dim3(kGuThreads), lds, st, A);
    else if (act == KSL_ACT_SILU)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_SILU>), dim3(grid), dim3(kGuThreads), lds, st, A);
    else
        return KSL_ERR_ARG;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

int launch_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                const void* dn_z, int64_t E, int64_t H, int64_t I, void* out3, hipStream_t st) {
    if (!out2 || !offsets || !dn_q || !dn_s || !dn_z || !out3) return KSL_ERR_ARG;
    if (E <= 0 || H <= 0 || I <= 0) return KSL_ERR_SHAPE;
    if (H % 64 != 0 || I % 64 != 0 || I > 1024) return KSL_ERR_SHAPE;
    if (E * H * (I / 2) >= (int64_t(1) << 40)) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(dn_q) % 8 || reinterpret_cast<uintptr_t>(out2) % 16 ||
        reinterpret_cast<uintptr_t>(dn_s) % 4 || reinterpret_cast<uintptr_t>(dn_z) % 4 ||
        reinterpret_cast<uintptr_t>(out3) % 2)
        return KSL_ERR_ALIGN;
    DnArgs A;
    A.out2 = static_cast<const f16*>(out2);
    A.offsets = offsets;
    A.dn_q = dn_q;
    A.dn_s = static_cast<const f16*>(dn_s);
    A.dn_z = static_cast<const f16*>(dn_z);
    A.out3 = static_cast<f16*>(out3);
    A.H = static_cast<int>(H);
    A.I = static_cast<int>(I);
    const int G = static_cast<int>(I / 64);
    const unsigned grid = static_cast<unsigned>(E * ((H + kDnWgCols - 1) / kDnWgCols));
    const size_t lds = static_cast<size_t>(G) * kMaxMt * 2 * kDnBlock + 2 * kDnWgCols * G * sizeof(f16);
    switch (G) {
#define KSL_DN_CASE(GG) \
    case GG: hipLaunchKernelGGL(down_kernel<GG>, dim3(grid), dim3(kDnThreads), lds, st, A); break;
        KSL_DN_CASE(1) KSL_DN_CASE(2) KSL_DN_CASE(3) KSL_DN_CASE(4) KSL_DN_CASE(5) KSL_DN_CASE(6)
        KSL_DN_CASE(7) KSL_DN_CASE(8) KSL_DN_CASE(9) KSL_DN_CASE(10) KSL_DN_CASE(11) KSL_DN_CASE(12)
        KSL_DN_CASE(13) KSL_DN_CASE(14) KSL_DN_CASE(15) KSL_DN_CASE(16)
#undef KSL_DN_CASE
        default: return KSL_ERR_SHAPE;
    }
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
