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
// Producer / consumer workgroup: 4 consumer waves (each one gate tile and one
// up tile of 16 columns of I) and 4 producer waves. Producers only issue
// global loads - the workgroup's weights and gathered activations for one
// quantisation group (128 K) at a time - keep kGuLead groups in flight in
// their registers, and write each arrived group into a two-slot LDS ring.
// Consumers only read LDS, decode and run MFMA; they never wait on memory
// counters. One barrier per group hands a slot from producers to consumers.
constexpr int kGuCons = 4;                       // consumer waves
constexpr int kGuProd = 4;                       // producer waves
constexpr int kGuWgCols = 16 * kGuCons;          // 64 columns of I per workgroup
constexpr int kGuThreads = (kGuCons + kGuProd) * kWave;  // 512
constexpr int kGuLead = 4;                       // groups of loads in flight per producer
constexpr int kMaxMt = 2;                        // 16-row M tiles per row chunk
constexpr int kBlk = kWave * 16;                 // one fragment block: 64 lanes x 16 B
constexpr int kGuSlotW = 2 * kGuCons * kBlk;     // 8 KB of weights per group
constexpr int kGuSlot = kGuSlotW + kMaxMt * 4 * kBlk;  // + 8 KB of activations
constexpr int kGuMaxG = 32;                      // H <= 4096
constexpr int kGuSzPer = 4 * 32 * kGuMaxG / (kGuProd * kWave);  // scale/zero dwords per producer lane

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

// Producer wave p (0..3) loads, per group: the gate and up fragment blocks of
// consumer wave p (lane L = c*16 + col: row col of the tile, bytes c*16.. of
// the group's 64) and the activation blocks (t, i = p) for t < MT (lane L:
// row t*16 + L%16, stored chunk g*128 + p*32 + (L/16)*8: 64 contiguous bytes
// per row, see act_store_index).
template <int MT>
struct GuProducer {
    const uint8_t* wq0;   // gate row, + c*16
    const uint8_t* wq1;   // up row
    const f16* ar[MT];    // activation row (gathered token), + c*32 + p*8
    u32x4 v[kGuLead][2 + MT];

    __device__ __forceinline__ void load(int g, u32x4 (&dst)[2 + MT]) const {
        dst[0] = *reinterpret_cast<const u32x4*>(wq0 + g * 64);
        dst[1] = *reinterpret_cast<const u32x4*>(wq1 + g * 64);
#pragma unroll
        for (int t = 0; t < MT; ++t) dst[2 + t] = *reinterpret_cast<const u32x4*>(ar[t] + g * 128);
    }
    __device__ __forceinline__ void store(char* slot, int p, int lane, const u32x4 (&src)[2 + MT]) const {
        *reinterpret_cast<u32x4*>(slot + (p * 2 + 0) * kBlk + lane * 16) = src[0];
        *reinterpret_cast<u32x4*>(slot + (p * 2 + 1) * kBlk + lane * 16) = src[1];
#pragma unroll
        for (int t = 0; t < MT; ++t)
            *reinterpret_cast<u32x4*>(slot + kGuSlotW + (t * 4 + p) * kBlk + lane * 16) = src[2 + t];
    }
};

template <int ACT, int MT>
__device__ __forceinline__ void gateup_chunk(const GuArgs& A, int e, int nb, char* __restrict__ lds,
                                             const f16* __restrict__ lds_sz, int start, int m0, int mrows) {
    const int tid = threadIdx.x;
    const int wave = tid / kWave;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int G = A.H >> 7;
    const int Gp = (G + kGuLead - 1) / kGuLead * kGuLead;  // groups padded to whole load rounds
    char* slot0 = lds;

    if (wave >= kGuCons) {
        // ------------------------------------------------------------ producer
        const int p = wave - kGuCons;
        GuProducer<MT> P;
        const int64_t rg = static_cast<int64_t>(e) * 2 * A.I + nb * kGuWgCols + p * 16 + col;
        P.wq0 = A.gu_q + rg * (A.H >> 1) + c * 16;
        P.wq1 = A.gu_q + (rg + A.I) * (A.H >> 1) + c * 16;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            int r = t * 16 + col;
            if (r >= mrows) r = mrows - 1;  // rows past the expert's last: loaded, never stored
            const int tok = A.sorted_rows[start + m0 + r] / A.topk;
            P.ar[t] = A.a16 + static_cast<int64_t>(tok) * A.H + p * 32 + c * 8;
        }
        // prologue: groups 0..kGuLead-1 in flight, group 0 into slot 0
#pragma unroll
        for (int u = 0; u < kGuLead; ++u) P.load(u < G ? u : G - 1, P.v[u]);
        P.store(slot0, p, lane, P.v[0]);
        __syncthreads();
        // step i: group i+1 (set (i+1)%L) -> slot (i+1)%2; loads of group i+L -> set i%L
        for (int g0 = 0; g0 < Gp; g0 += kGuLead) {
#pragma unroll
            for (int u = 0; u < kGuLead; ++u) {
                const int i = g0 + u;
                P.store(slot0 + ((i + 1) & 1) * kGuSlot, p, lane, P.v[(u + 1) % kGuLead]);
                const int gl = i + kGuLead < G ? i + kGuLead : G - 1;
                P.load(gl, P.v[u]);
                __syncthreads();
            }
        }
        return;
    }

    // -------------------------------------------------------------- consumer
    const NibConsts kn = nib_consts();
    const f16* sg = lds_sz;
    const f16* zg = lds_sz + 64 * G;
    const f16* su = lds_sz + 2 * 64 * G;
    const f16* zu = lds_sz + 3 * 64 * G;
    const int wcol = wave * 16 + col;  // row of this lane within the workgroup's 64
    f32x4 acc[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();  // slot 0 and the scale table are ready
    for (int i = 0; i < Gp; ++i) {
        if (i < G) {
            const char* slot = slot0 + (i & 1) * kGuSlot;
            const u32x4 w0 = *reinterpret_cast<const u32x4*>(slot + (wave * 2 + 0) * kBlk + lane * 16);
            const u32x4 w1 = *reinterpret_cast<const u32x4*>(slot + (wave * 2 + 1) * kBlk + lane * 16);
            const float s0 = static_cast<float>(sg[wcol * G + i]);
            const float s1 = static_cast<float>(su[wcol * G + i]);
            const ZeroPair zc0 = zero_pair(zg[wcol * G + i]);
            const ZeroPair zc1 = zero_pair(zu[wcol * G + i]);
            f32x4 part[2][MT];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const f16x8 b0 = nib8_minus_zero(w0[k], zc0, kn);
                const f16x8 b1 = nib8_minus_zero(w1[k], zc1, kn);
#pragma unroll
                for (int t = 0; t < MT; ++t) {
                    const f16x8 a = *reinterpret_cast<const f16x8*>(slot + kGuSlotW + (t * 4 + k) * kBlk + lane * 16);
                    part[0][t] = mfma16x16x32(a, b0, part[0][t]);
                    part[1][t] = mfma16x16x32(a, b1, part[1][t]);
                }
            }
#pragma unroll
            for (int t = 0; t < MT; ++t)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    acc[0][t][r] = __builtin_fmaf(s0, part[0][t][r], acc[0][t][r]);
                    acc[1][t][r] = __builtin_fmaf(s1, part[1][t][r], acc[1][t][r]);
                }
        }
        __syncthreads();
    }
    const int n0 = nb * kGuWgCols + wave * 16;
    const int sc = act_store_index<64>(n0 + col);  // out2 is the down GEMM's activation
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
__global__ __launch_bounds__(kGuThreads) __attribute__((amdgpu_waves_per_eu(4))) void gateup_act_kernel(GuArgs A) {
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
    f16* lds_sz = reinterpret_cast<f16*>(lds + 2 * kGuSlot);
    // scales / zeros of the 64 gate and 64 up rows: four [64 x G] fp16 blocks
    // (s_gate, z_gate, s_up, z_up), copied by the producers; published by the
    // first barrier of the first chunk.
    if (wave >= kGuCons) {
        const int pt = tid - kGuCons * kWave;
        const int64_t gate0 = static_cast<int64_t>(e) * 2 * A.I + nb * kGuWgCols;
        const int64_t up0 = gate0 + A.I;
        const int nd = 32 * G;  // dwords per block (block starts are 4-byte aligned)
        uint32_t v[kGuSzPer];
#pragma unroll
        for (int k = 0; k < kGuSzPer; ++k) {
            int i = pt + k * kGuProd * kWave;
            if (i >= 4 * nd) i = 0;  // clamped, never stored
            const int b = i / nd, o = i - b * nd;
            const f16* base = ((b & 1) ? A.gu_z : A.gu_s) + ((b & 2) ? up0 : gate0) * G;
            v[k] = reinterpret_cast<const uint32_t*>(base)[o];
        }
        uint32_t* d = reinterpret_cast<uint32_t*>(lds_sz);
#pragma unroll
        for (int k = 0; k < kGuSzPer; ++k) {
            const int i = pt + k * kGuProd * kWave;
            if (i < 4 * nd) d[i] = v[k];
        }
    }
    for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
        const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
        if (mrows <= 16)
            gateup_chunk<ACT, 1>(A, e, nb, lds, lds_sz, start, m0, mrows);
        else
            gateup_chunk<ACT, 2>(A, e, nb, lds, lds_sz, start, m0, mrows);
        __syncthreads();  // ring free for the next chunk
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
    const size_t lds = 2 * kGuSlot + 4 * 64 * (H / 128) * sizeof(f16);
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
