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
// One workgroup covers NC*16 columns of I of one expert (NC = 11: 176 columns,
// a quarter of DiffusionGemma's I = 704) with NC consumer waves and NP
// producer waves:
//   - consumer w owns columns w*16 .. w*16+15: one gate tile and one up tile
//     of 16 weight rows; it only reads LDS, decodes nibbles and runs MFMA;
//   - producers only issue global loads: per quantisation group (128 K) all
//     2*NC weight fragment blocks (16 rows x 64 B) and the 4*MT activation
//     fragment blocks, two groups in flight, and write them into a ring of two
//     half-group slots (64 K each) in LDS.
// One barrier per half group hands a slot from producers to consumers. Wide
// workgroups keep the activation re-reads small (every requested byte costs
// load bandwidth, L2 hit or not): the gathered rows of an expert are read
// I/(16*NC) times per layer instead of once per 64-column block.
constexpr int kMaxMt = 2;                        // 16-row M tiles per row chunk
constexpr int kBlk = kWave * 16;                 // one full-group fragment block: 64 lanes x 16 B
constexpr int kHalfBlk = kWave * 8;              // one half-group weight block: 64 lanes x 8 B
constexpr int kGuMaxG = 32;                      // H <= 4096

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

template <int NC, int NP>
struct GuShape {
    static constexpr int kCols = 16 * NC;                      // columns of I per workgroup
    static constexpr int kThreads = (NC + NP) * kWave;
    static constexpr int kSlotW = 2 * NC * kHalfBlk;           // weight bytes per half slot
    static constexpr int kSlot = kSlotW + kMaxMt * 2 * kBlk;   // + activation bytes per half slot
    static constexpr int kSzBytesMaxG = 4 * kCols * kGuMaxG * 2;
    static constexpr int kSzPer = (kSzBytesMaxG / 16 + kThreads - 1) / kThreads;  // 16-B scale chunks per thread
    static size_t lds_bytes(int G) { return 2 * kSlot + static_cast<size_t>(4) * kCols * G * 2; }
};

// Producer side of one row chunk: 1 + 2*Gp barriers (Gp = G rounded up to even).
template <int NC, int NP, int MT>
__device__ __forceinline__ void gateup_produce(const GuArgs& A, int e, int c0, char* __restrict__ lds, int start,
                                               int m0, int mrows) {
    using S = GuShape<NC, NP>;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int G = A.H >> 7;
    {
        // blocks b = p + NP*k: b < 2*NC -> weight block (w = b/2, tile j = b%2:
        // gate, up), else activation block (t, i) = ((b - 2*NC)/4, (b - 2*NC)%4).
        // Past the last block: clamped (a duplicate load and an identical LDS write).
        constexpr int NB = 2 * NC + 4 * MT;
        constexpr int KP = (NB + NP - 1) / NP;
        const int p = wave - NC;
        uint32_t off[KP];    // offset of group 0 from gu_q / a16, in 16-byte units (all terms are)
        int dst[KP];         // LDS byte offset of the block within a half slot (lane included)
        bool isw[KP];
#pragma unroll
        for (int k = 0; k < KP; ++k) {
            int b = p + NP * k;
            if (b >= NB) b = NB - 1;
            isw[k] = b < 2 * NC;
            if (isw[k]) {
                const int w = b >> 1, j = b & 1;
                const int64_t row = static_cast<int64_t>(e) * 2 * A.I + (j ? A.I : 0) + c0 + w * 16 + col;
                off[k] = static_cast<uint32_t>((row * (A.H >> 1) + c * 16) >> 4);
                dst[k] = (b * kWave + lane) * 8;
            } else {
                const int a = b - 2 * NC, t = a >> 2, i = a & 3;
                int r = t * 16 + col;
                if (r >= mrows) r = mrows - 1;  // rows past the expert's last: loaded, never stored
                const int tok = A.sorted_rows[start + m0 + r] / A.topk;
                off[k] = static_cast<uint32_t>((static_cast<int64_t>(tok) * A.H + i * 32 + c * 8) >> 3);
                dst[k] = S::kSlotW + ((t * 2 + (i & 1)) * kWave + lane) * 16 + (i >> 1) * (1 << 30);
            }
        }
        const char* wbase = reinterpret_cast<const char*>(A.gu_q);
        const char* abase = reinterpret_cast<const char*>(A.a16);
        u32x4 v[2][KP];
        auto load_group = [&](int g, u32x4 (&dstv)[KP]) {
            const int gc = g < G ? g : G - 1;
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                const char* src = isw[k] ? wbase + static_cast<uint64_t>(off[k]) * 16 + gc * 64
                                         : abase + static_cast<uint64_t>(off[k]) * 16 + gc * 256;
                dstv[k] = *reinterpret_cast<const u32x4*>(src);
            }
        };
        // half hh of a group into slot `slot`: weight blocks give 8 bytes per half,
        // activation blocks belong to half i/2 (encoded in bit 30 of dst)
        auto store_half = [&](int hh, const u32x4 (&srcv)[KP]) {
            char* base = lds + hh * S::kSlot;
#pragma unroll
            for (int k = 0; k < KP; ++k) {
                if (isw[k]) {
                    const u32x2 h = hh ? u32x2{srcv[k][2], srcv[k][3]} : u32x2{srcv[k][0], srcv[k][1]};
                    *reinterpret_cast<u32x2*>(base + dst[k]) = h;
                } else if ((dst[k] >> 30) == hh) {
                    *reinterpret_cast<u32x4*>(base + (dst[k] & ((1 << 30) - 1))) = srcv[k];
                }
            }
        };
        load_group(0, v[0]);
        load_group(1, v[1]);
        store_half(0, v[0]);
        __syncthreads();
        // half step s: consumers read slot s%2; producers fill slot (s+1)%2 with
        // half step s+1: (s even) half 1 of group s/2, (s odd) half 0 of group s/2+1.
        for (int g = 0; g < G; g += 2) {
            // s = 2g
            store_half(1, v[0]);
            load_group(g + 2, v[0]);
            __syncthreads();
            // s = 2g + 1
            store_half(0, v[1]);
            __syncthreads();
            // s = 2g + 2
            store_half(1, v[1]);
            load_group(g + 3, v[1]);
            __syncthreads();
            // s = 2g + 3
            store_half(0, v[0]);
            __syncthreads();
        }
    }
}

// Consumer side of one row chunk: 1 + 2*Gp barriers, matching gateup_produce.
template <int ACT, int NC, int NP, int MT>
__device__ __forceinline__ void gateup_consume(const GuArgs& A, int c0, const char* __restrict__ lds,
                                               const f16* __restrict__ lds_sz, int start, int m0, int mrows) {
    using S = GuShape<NC, NP>;
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int G = A.H >> 7;
    const NibConsts kn = nib_consts();
    const int kc = S::kCols;
    const f16* s_g = lds_sz;
    const f16* z_g = lds_sz + kc * G;
    const f16* s_u = lds_sz + 2 * kc * G;
    const f16* z_u = lds_sz + 3 * kc * G;
    f32x4 acc[2][MT], part[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();  // slot 0 and the scale table are ready
    const int Gp = (G + 1) & ~1;  // producers run whole pairs of groups
    for (int s = 0; s < 2 * Gp; ++s) {
        const int g = s >> 1, hh = s & 1;
        if (g < G) {
            const char* slot = lds + hh * S::kSlot;
            if (hh == 0) {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            const int r = wave * 16 + col;  // row of the tile within the workgroup
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const ZeroPair zc = zero_pair((j ? z_u : z_g)[r * G + g]);
                const u32x2 wv = *reinterpret_cast<const u32x2*>(slot + ((wave * 2 + j) * kWave + lane) * 8);
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) {
                    const f16x8 b = nib8_minus_zero(wv[ii], zc, kn);
#pragma unroll
                    for (int t = 0; t < MT; ++t) {
                        const f16x8 a = *reinterpret_cast<const f16x8*>(slot + S::kSlotW + ((t * 2 + ii) * kWave + lane) * 16);
                        part[j][t] = mfma16x16x32(a, b, part[j][t]);
                    }
                }
            }
            if (hh == 1) {
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const float sc = static_cast<float>((j ? s_u : s_g)[r * G + g]);
#pragma unroll
                    for (int t = 0; t < MT; ++t)
#pragma unroll
                        for (int q = 0; q < 4; ++q) acc[j][t][q] = __builtin_fmaf(sc, part[j][t][q], acc[j][t][q]);
                }
            }
        }
        __syncthreads();
    }
    // epilogue: column c0 + wave*16 + col, gate tile 0 with up tile 1
    {
        const int sc = act_store_index<64>(c0 + wave * 16 + col);  // out2 is the down GEMM's activation
        f16* o = A.out2 + static_cast<int64_t>(start + m0) * A.I + sc;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = t * 16 + 4 * c + q;
                if (row < mrows)
                    o[static_cast<int64_t>(row) * A.I] = static_cast<f16>(act_times_up<ACT>(acc[0][t][q], acc[1][t][q]));
            }
    }
}

template <int ACT, int NC, int NP>
__global__ __launch_bounds__((NC + NP) * kWave) void gateup_act_kernel(GuArgs A) {
    using S = GuShape<NC, NP>;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int nb_per_e = A.I / S::kCols;
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int e = tile / nb_per_e;
    const int c0 = (tile - e * nb_per_e) * S::kCols;
    const int start = A.offsets[e];
    const int M = A.offsets[e + 1] - start;
    if (M <= 0) return;
    const int G = A.H >> 7;
    const int tid = threadIdx.x;
    f16* lds_sz = reinterpret_cast<f16*>(lds + 2 * S::kSlot);
    // scale / zero table of the workgroup's rows: four [kCols x G] fp16 blocks
    // (s_gate, z_gate, s_up, z_up), each contiguous in global memory and
    // 16-byte aligned; copied by all waves, published by the first barrier.
    {
        const int64_t gate0 = static_cast<int64_t>(e) * 2 * A.I + c0;
        const int64_t up0 = gate0 + A.I;
        const int nq = S::kCols * G * 2 / 16;  // 16-byte chunks per block
        u32x4 v[S::kSzPer];
#pragma unroll
        for (int k = 0; k < S::kSzPer; ++k) {
            int i = tid + k * S::kThreads;
            if (i >= 4 * nq) i = 0;  // clamped, never stored
            const int b = i / nq, o = i - b * nq;
            const f16* base = ((b & 1) ? A.gu_z : A.gu_s) + ((b & 2) ? up0 : gate0) * G;
            v[k] = reinterpret_cast<const u32x4*>(base)[o];
        }
#pragma unroll
        for (int k = 0; k < S::kSzPer; ++k) {
            const int i = tid + k * S::kThreads;
            if (i < 4 * nq) reinterpret_cast<u32x4*>(lds_sz)[i] = v[k];
        }
    }
    // Roles split once; both loops run the same chunks with the same barrier count.
    if (tid / kWave >= NC) {
        for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
            const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
            if (mrows <= 16)
                gateup_produce<NC, NP, 1>(A, e, c0, lds, start, m0, mrows);
            else
                gateup_produce<NC, NP, 2>(A, e, c0, lds, start, m0, mrows);
            __syncthreads();  // ring free for the next chunk
        }
    } else {
        for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
            const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
            if (mrows <= 16)
                gateup_consume<ACT, NC, NP, 1>(A, c0, lds, lds_sz, start, m0, mrows);
            else
                gateup_consume<ACT, NC, NP, 2>(A, c0, lds, lds_sz, start, m0, mrows);
            __syncthreads();  // ring free for the next chunk
        }
    }
}

template <int NC, int NP>
int launch_gateup_nc(const GuArgs& A, int64_t E, int act, hipStream_t st) {
    using S = GuShape<NC, NP>;
    const unsigned grid = static_cast<unsigned>(E * (A.I / S::kCols));
    const size_t lds = S::lds_bytes(A.H / 128);
    if (act == KSL_ACT_GELU_TANH)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_GELU_TANH, NC, NP>), dim3(grid), dim3(S::kThreads), lds, st, A);
    else if (act == KSL_ACT_SILU)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_SILU, NC, NP>), dim3(grid), dim3(S::kThreads), lds, st, A);
    else
        return KSL_ERR_ARG;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
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
// for lane L = c*16 + rr, logical out2[row t*16 + rr][g*64 + c*16 + i*8 .. +8],
// stored at g*64 + i*32 + c*8 (act_store_index<64>).
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
        const f16* src = A.out2 + static_cast<int64_t>(start + m0 + r) * A.I + g * 64 + i * 32 + c * 8;
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
    const NibConsts kn = nib_consts();
    f32x4 acc[kDnTiles][MT];
#pragma unroll
    for (int j = 0; j < kDnTiles; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < G; ++g) {
        f16x2 sc[kDnTiles];
        ZeroPair zc[kDnTiles];
#pragma unroll
        for (int j = 0; j < kDnTiles; ++j) {
            const int r = wrow0 + j * 16 + col;
            const f16 sv = lds_s[r * G + g];
            sc[j] = f16x2{sv, sv};
            zc[j] = zero_pair(lds_z[r * G + g]);
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            f16x8 a[MT];
#pragma unroll
            for (int t = 0; t < MT; ++t)
                a[t] = *reinterpret_cast<const f16x8*>(lds_a + ((g * kMaxMt + t) * 2 + i) * kDnBlock + lane * 16);
#pragma unroll
            for (int j = 0; j < kDnTiles; ++j) {
                const f16x8 b = nib8_dequant(w[j][g][i], zc[j], sc[j], kn);
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
    if (H % 128 != 0 || I % 64 != 0 || H > 128 * kGuMaxG) return KSL_ERR_SHAPE;
    if (E * 2 * I * (H / 2) >= (int64_t(1) << 36)) return KSL_ERR_SHAPE;  // 32-bit offsets in 16-B units
    if (reinterpret_cast<uintptr_t>(gu_q) % 16 || reinterpret_cast<uintptr_t>(a16) % 16 ||
        reinterpret_cast<uintptr_t>(gu_s) % 16 || reinterpret_cast<uintptr_t>(gu_z) % 16 ||
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
    // widest column block that divides I: 176 (11 consumers), 128, or 64
    if (I % 176 == 0) return launch_gateup_nc<11, 5>(A, E, act, st);
    if (I % 128 == 0) return launch_gateup_nc<8, 4>(A, E, act, st);
    return launch_gateup_nc<4, 4>(A, E, act, st);
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
