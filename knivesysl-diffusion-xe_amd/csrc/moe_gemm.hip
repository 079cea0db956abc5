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
// so a load consumed soon after issue would drain every prefetch behind it:
//   - scales and zero-points of the workgroup's rows are copied to LDS once;
//   - activations are copied to LDS in MFMA fragment order (each lane's 16
//     bytes contiguous across the wave: conflict-free ds_read_b128);
//   - gate/up: producer waves stream weight and activation fragments of one
//     128-K group per slot into an LDS ring by direct global -> LDS loads,
//     consumer waves only read LDS (one barrier per group);
//   - down: each wave loads a pair of 16-column weight tiles (with their
//     scale / zero-point pair words) straight into registers by ordinary,
//     compiler-tracked loads, and other waves of the SIMD cover the latency.
//
// Work split: one workgroup per (expert, column block) walks all rows routed
// to its expert (sorted slots offsets[e] .. offsets[e+1]) in chunks of up to 32
// rows for gate/up (one or two 16-row M tiles) and 64 rows for down; with more
// gate/up items than CUs, one persistent gate/up workgroup per CU walks
// several of them through one LDS ring (gateup_flow_kernel). Above 8192
// routed rows both GEMMs run the GEMM-form row-block kernels of
// moe_rbgemm.hip instead. Workgroups are remapped so that all column blocks
// of an expert run on the same XCD (shared L2 for its activations).

#include <algorithm>
#include <atomic>
#include <type_traits>
#include <utility>

#include "ksl_common.h"

namespace ksl {

// Row-block GEMM kernels of large routings (moe_rbgemm.hip).
bool rb_gateup_fits(int64_t H, int64_t I);
bool rb_down_fits(int64_t H, int64_t I);
int launch_rb_gateup(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                     const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H, int64_t I,
                     int act, void* out2, hipStream_t st, int64_t nrows);
int launch_rb_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                   const void* dn_z, int64_t E, int64_t H, int64_t I, void* out3, hipStream_t st, int layout,
                   int64_t nrows);

namespace {

constexpr int kRowBlockFrom = 8192;  // routed rows above which the row-block kernels run

// Compile-time loop: f(integral_constant<int, 0>) .. f(integral_constant<int, N-1>).
template <int N, typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, Is>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

// ---------------------------------------------------------------- gate / up
// One workgroup covers NC*16 columns of I of one expert (NC = 11: 176 columns,
// a quarter of DiffusionGemma's I = 704) with NC consumer waves and NP
// producer waves:
//   - consumer w owns columns w*16 .. w*16+15: one gate tile and one up tile
//     of 16 weight rows; it only reads LDS, decodes nibbles and runs MFMA;
//   - producers only issue direct global->LDS loads: per quantisation group
//     (128 K) all 2*NC weight fragment blocks (16 rows x 64 B) and the 4*MT
//     activation fragment blocks go into one slot of an R-slot LDS ring, with
//     up to R-1 groups in flight and no register staging; each block is
//     fetched row-major and lands in the swizzled order of frag_pos.
// One barrier per group hands a slot from producers to consumers. Wide
// workgroups keep the activation re-reads small (every requested byte costs
// load bandwidth, L2 hit or not): the gathered rows of an expert are read
// I/(16*NC) times per layer instead of once per 64-column block.

constexpr int kMaxMt = 2;                        // 16-row M tiles per row chunk

constexpr size_t kLdsBytes = 160 * 1024;         // LDS per workgroup on gfx950
// Static LDS reserved beside the dynamic LDS of a launch (these kernels
// declare none today; the reserve keeps a helper with a small __shared__
// array from pushing a launch sized to the limit over it).
constexpr size_t kLdsStatic = 64;
constexpr size_t kLdsDynMax = kLdsBytes - kLdsStatic;
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
    int early;  // producers issue the first weight groups before reading the routing
};

template <int NC, int NP, int R>
struct GuShape {
    static constexpr int kCols = 16 * NC;                      // columns of I per workgroup
    static constexpr int kThreads = (NC + NP) * kWave;
    static constexpr int kSlotW = 2 * NC * kBlk;               // weight bytes per slot
    static constexpr int kSlot = kSlotW + 4 * kMaxMt * kBlk;   // + activation bytes per slot (two M tiles)
    static constexpr int kSzPer = (4 * kCols * kGuMaxG * 2 / 16 + NC * kWave - 1) / (NC * kWave);
    static constexpr size_t lds_bytes(int G) { return static_cast<size_t>(R) * kSlot + static_cast<size_t>(4) * kCols * G * 2; }
};

// Producer side of one row chunk: 1 + G barriers. Slot of group g: g % R.
// Wave p issues blocks b = p + NP*k (k < KP, b < NB): b < 2*NC is weight block
// (w, j) = (b/2, b%2) (j: gate, up), else activation block (t, i) =
// ((b - 2*NC)/4, (b - 2*NC)%4) of M tile t and 32-K step i.
// Weight blocks of the first groups 0 .. min(R-1, G)-1 of a producer wave (the
// blocks b = p + NP*k < 2*NC of gateup_produce), issued before the routing is
// read: they do not depend on it.
template <int NC, int NP, int R>
__device__ __forceinline__ void gateup_issue_first_weights(const GuArgs& A, int e, int c0, char* __restrict__ lds) {
    using S = GuShape<NC, NP, R>;
    const int lane = threadIdx.x & (kWave - 1);
    const int p = wave_id() - NC;
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int G = A.H >> 7;
    const int n0 = R - 1 < G ? R - 1 : G;
    for (int b = p; b < 2 * NC; b += NP) {
        const int w = b >> 1, j = b & 1;
        const int64_t row = static_cast<int64_t>(e) * 2 * A.I + (j ? A.I : 0) + c0 + w * 16 + rr;
        const char* src = reinterpret_cast<const char*>(A.gu_q) + row * (A.H >> 1) + ch * 16;
        for (int g = 0; g < n0; ++g) dma16(src + g * 64, lds + g * S::kSlot + b * kBlk);
    }
}

template <int NC, int NP, int R, int MT>
__device__ __forceinline__ void gateup_produce(const GuArgs& A, int e, int c0, char* __restrict__ lds, int start,
                                               int m0, int mrows, bool w_issued) {
    using S = GuShape<NC, NP, R>;
    constexpr int NB = 2 * NC + 4 * MT;
    constexpr int KP = (NB + NP - 1) / NP;
    const int lane = threadIdx.x & (kWave - 1);
    const int p = wave_id() - NC;
    // row-major fetch: lanes 4r .. 4r+3 cover the 64 bytes of block row r
    // (4 rows per 256 B), chunk order swizzled per row (frag_pos)
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int G = A.H >> 7;
    const bool full = p + NP * (KP - 1) < NB;  // this wave issues KP blocks per group, else KP - 1
    const char* src[KP];
    int dst[KP];   // LDS byte offset of the block within a slot
    int gstep[KP]; // global bytes per group
#pragma unroll
    for (int k = 0; k < KP; ++k) {
        int b = p + NP * k;
        if (b >= NB) b = NB - 1;  // never issued
        if (b < 2 * NC) {
            const int w = b >> 1, j = b & 1;
            const int64_t row = static_cast<int64_t>(e) * 2 * A.I + (j ? A.I : 0) + c0 + w * 16 + rr;
            src[k] = reinterpret_cast<const char*>(A.gu_q) + row * (A.H >> 1) + ch * 16;
            gstep[k] = 64;
        } else {
            const int a = b - 2 * NC, t = a >> 2, i = a & 3;
            int r = t * 16 + rr;
            if (r >= mrows) r = mrows - 1;  // rows past the expert's last: loaded, never stored
            const int tok = A.sorted_rows[start + m0 + r] / A.topk;
            src[k] = reinterpret_cast<const char*>(A.a16 + static_cast<int64_t>(tok) * A.H + i * 32 + ch * 8);
            gstep[k] = 256;
        }
        dst[k] = b * kBlk;
    }
    auto issue = [&](int g, int slot, bool wts = true) {
        char* base = lds + slot * S::kSlot;
#pragma unroll
        for (int k = 0; k < KP; ++k)
            if ((k < KP - 1 || full) && (wts || p + NP * k >= 2 * NC)) dma16(src[k] + g * gstep[k], base + dst[k]);
    };
    auto wait_groups = [&](int n) {
        if (full)
            vm_wait_groups<KP, R - 2>(n);
        else
            vm_wait_groups<KP - 1, R - 2>(n);
    };
    // prologue: groups 0 .. R-2 (their weights may be in flight already: then
    // the activations follow and everything lands before the first barrier)
    int issued = 0;
    for (; issued < R - 1 && issued < G; ++issued) issue(issued, issued, !w_issued);
    if (w_issued)
        vm_wait<0>();
    else
        wait_groups(issued - 1);  // group 0 landed
    dma_barrier();
    int slot_next = issued % R;  // slot of group `issued`
    for (int g = 0; g < G; ++g) {
        // consumers read slot g % R; slot (g - 1) % R was released by the last barrier
        if (issued < G) {
            issue(issued, slot_next);
            ++issued;
            slot_next = slot_next + 1 == R ? 0 : slot_next + 1;
        }
        // group g + 1 must have landed before the barrier (none left after G - 1)
        wait_groups(g + 1 < G ? issued - g - 2 : 0);
        dma_barrier();
    }
}

// Producer side with a single producer wave (NP = 1, the 12-wave
// configuration whose consumers hold eight M tiles): all 2*NC + 4*MT blocks of
// a group from one wave, each address computed from a per-lane base (a wave
// cannot keep one pointer per block in registers). Same slots, order and
// barriers as gateup_produce.
template <int NC, int R, int MT>
__device__ __forceinline__ void gateup_produce_1w(const GuArgs& A, int e, int c0, char* __restrict__ lds, int start,
                                                  int m0, int mrows, bool w_issued) {
    using S = GuShape<NC, 1, R>;
    constexpr int NB = 2 * NC + 4 * MT;
    const int lane = threadIdx.x & (kWave - 1);
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int G = A.H >> 7;
    const int rowbytes = A.H >> 1;
    // weights: the expert's first gate row of the column block, plus the lane's
    // row and 16-byte piece; block (w, j) adds (j*I + w*16) rows
    const char* wbase =
        reinterpret_cast<const char*>(A.gu_q) + (static_cast<int64_t>(e) * 2 * A.I + c0) * rowbytes;
    const int wlane = rr * rowbytes + ch * 16;
    // activations: the lane's token row of each M tile (rows past the chunk
    // repeat its last row: loaded, never stored)
    const char* abase = reinterpret_cast<const char*>(A.a16);
    int64_t aoff[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        int r = t * 16 + rr;
        if (r >= mrows) r = mrows - 1;
        const int tok = A.sorted_rows[start + m0 + r] / A.topk;
        aoff[t] = (static_cast<int64_t>(tok) * A.H + ch * 8) * 2;
    }
    auto issue = [&](int g, int slot, bool wts) {
        char* base = lds + slot * S::kSlot;
        if (wts) {
#pragma unroll
            for (int b = 0; b < 2 * NC; ++b) {
                const int w = b >> 1, j = b & 1;
                dma16(wbase + static_cast<int64_t>((j ? A.I : 0) + w * 16) * rowbytes + wlane + g * 64,
                      base + b * kBlk);
            }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dma16(abase + aoff[t] + (i * 32 + g * 128) * 2, base + (2 * NC + t * 4 + i) * kBlk);
    };
    int issued = 0;
    for (; issued < R - 1 && issued < G; ++issued) issue(issued, issued, !w_issued);
    if (w_issued)
        vm_wait<0>();
    else
        vm_wait_groups<NB, R - 2>(issued - 1);  // group 0 landed
    dma_barrier();
    int slot_next = issued % R;
    for (int g = 0; g < G; ++g) {
        if (issued < G) {
            issue(issued, slot_next, true);
            ++issued;
            slot_next = slot_next + 1 == R ? 0 : slot_next + 1;
        }
        vm_wait_groups<NB, R - 2>(g + 1 < G ? issued - g - 2 : 0);
        dma_barrier();
    }
}

// One quantisation group g of a consumer wave: its gate and up weight words in
// slot sp, decoded against their zero-points, times the MT activation tiles
// of the slot; the fp32 group partials are scaled into acc. sz: the
// [s_gate | z_gate | s_up | z_up] table of the workgroup's rows, kCols x G each.
template <int NC, int MT>
__device__ __forceinline__ void gateup_group(const char* __restrict__ sp, const f16* __restrict__ sz, int G, int g,
                                             const NibConsts& kn, f32x4 (&acc)[2][MT]) {
    constexpr int kSlotW = 2 * NC * kBlk;
    constexpr int kc = 16 * NC;
    const int wave = wave_id();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const f16* s_g = sz;
    const f16* z_g = sz + kc * G;
    const f16* s_u = sz + 2 * kc * G;
    const f16* z_u = sz + 3 * kc * G;
    const int r = wave * 16 + col;  // row of the tile within the workgroup
    const int fo = frag_pos(col, c) * 16;
    f32x4 part[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    u32x4 wv[2];
    ZeroPair zc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        wv[j] = *reinterpret_cast<const u32x4*>(sp + (wave * 2 + j) * kBlk + fo);
        zc[j] = zero_pair((j ? z_u : z_g)[r * G + g]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f16x8 a[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) a[t] = *reinterpret_cast<const f16x8*>(sp + kSlotW + (t * 4 + i) * kBlk + fo);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f16x8 b = nib8_minus_zero(wv[j][i], zc[j], kn);
#pragma unroll
            for (int t = 0; t < MT; ++t) part[j][t] = mfma16x16x32(a[t], b, part[j][t]);
        }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float sc = static_cast<float>((j ? s_u : s_g)[r * G + g]);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[j][t][q] = __builtin_fmaf(sc, part[j][t][q], acc[j][t][q]);
    }
}

// Epilogue of a consumer wave: column c0 + wave*16 + col of sorted slots
// row0 .. row0 + mrows - 1, gate tile 0 with up tile 1.
template <int ACT, int MT>
__device__ __forceinline__ void gateup_store(const GuArgs& A, const f32x4 (&acc)[2][MT], int c0, int row0, int mrows) {
    const int wave = wave_id();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    if (ACT == KSL_ACT_NONE) {
        // gate and up themselves, fp16, in plain column order: out1 [rows, 2I]
        const int64_t ld = 2 * static_cast<int64_t>(A.I);
        f16* o = A.out2 + (static_cast<int64_t>(row0) + 4 * c) * ld + c0 + wave * 16 + col;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = t * 16 + 4 * c + q;
                if (row < mrows) {
                    o[(t * 16 + q) * ld] = static_cast<f16>(acc[0][t][q]);
                    o[(t * 16 + q) * ld + A.I] = static_cast<f16>(acc[1][t][q]);
                }
            }
    } else {
        const int sc = out2_store_index(c0 + wave * 16 + col, A.I & ~127);  // out2 is the down GEMM's activation
        // the lane's part of the row offset (4c rows) in its pointer, the
        // uniform part ((16t + q) rows) as a scalar offset
        f16* o = A.out2 + (static_cast<int64_t>(row0) + 4 * c) * A.I + sc;
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int row = t * 16 + 4 * c + q;
                if (row < mrows)
                    o[(t * 16 + q) * A.I] = static_cast<f16>(act_times_up<ACT>(acc[0][t][q], acc[1][t][q]));
            }
    }
}

// Consumer side of one row chunk: 1 + G barriers, matching gateup_produce.
template <int ACT, int NC, int NP, int R, int MT>
__device__ __forceinline__ void gateup_consume(const GuArgs& A, int c0, const char* __restrict__ lds,
                                               const f16* __restrict__ lds_sz, int start, int m0, int mrows) {
    using S = GuShape<NC, NP, R>;
    const int G = A.H >> 7;
    const NibConsts kn = nib_consts();
    f32x4 acc[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();  // group 0 and the scale table are ready
    int slot = 0;
    for (int g = 0; g < G; ++g) {
        gateup_group<NC, MT>(lds + slot * S::kSlot, lds_sz, G, g, kn, acc);
        slot = slot + 1 == R ? 0 : slot + 1;
        __syncthreads();
    }
    gateup_store<ACT, MT>(A, acc, c0, start + m0, mrows);
}

template <int ACT, int NC, int NP, int R>
__global__ __launch_bounds__((NC + NP) * kWave) void gateup_act_kernel(GuArgs A) {
    using S = GuShape<NC, NP, R>;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    // Producer waves issue first on their SIMD after each barrier (the arbiter
    // otherwise favours the older consumer waves).
    if (wave_id() >= NC) __builtin_amdgcn_s_setprio(3);
    const int nb_per_e = A.I / S::kCols;
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int e = tile / nb_per_e;
    const int c0 = (tile - e * nb_per_e) * S::kCols;
    if (A.early && wave_id() >= NC) gateup_issue_first_weights<NC, NP, R>(A, e, c0, lds);
    const int start = A.offsets[e];
    const int M = A.offsets[e + 1] - start;
    if (M <= 0) {
        vm_wait<0>();  // early weight loads land before the workgroup's LDS is released
        return;
    }
    const int G = A.H >> 7;
    const int tid = threadIdx.x;
    f16* lds_sz = reinterpret_cast<f16*>(lds + R * S::kSlot);
    // Roles split once; both loops run the same chunks with the same barrier
    // count (1 + G per chunk), and the ring is free after a chunk's last barrier.
    if (wave_id() >= NC) {
        for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
            const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
            const bool w_issued = m0 == 0 && A.early;
            if constexpr (NP == 1) {
                if (mrows <= 16)
                    gateup_produce_1w<NC, R, 1>(A, e, c0, lds, start, m0, mrows, w_issued);
                else
                    gateup_produce_1w<NC, R, 2>(A, e, c0, lds, start, m0, mrows, w_issued);
            } else {
                if (mrows <= 16)
                    gateup_produce<NC, NP, R, 1>(A, e, c0, lds, start, m0, mrows, w_issued);
                else
                    gateup_produce<NC, NP, R, 2>(A, e, c0, lds, start, m0, mrows, w_issued);
            }
        }
    } else {
        // scale / zero table of the workgroup's rows: four [kCols x G] fp16
        // blocks (s_gate, z_gate, s_up, z_up), each contiguous in global memory
        // and 16-byte aligned; published by the first barrier.
        {
            const int64_t gate0 = static_cast<int64_t>(e) * 2 * A.I + c0;
            const int64_t up0 = gate0 + A.I;
            const int nq = S::kCols * G * 2 / 16;  // 16-byte chunks per block
            u32x4 v[S::kSzPer];
#pragma unroll
            for (int k = 0; k < S::kSzPer; ++k) {
                int i = tid + k * NC * kWave;
                if (i >= 4 * nq) i = 0;  // clamped, never stored
                const int b = i / nq, o = i - b * nq;
                const f16* base = ((b & 1) ? A.gu_z : A.gu_s) + ((b & 2) ? up0 : gate0) * G;
                v[k] = reinterpret_cast<const u32x4*>(base)[o];
            }
#pragma unroll
            for (int k = 0; k < S::kSzPer; ++k) {
                const int i = tid + k * NC * kWave;
                if (i < 4 * nq) reinterpret_cast<u32x4*>(lds_sz)[i] = v[k];
            }
        }
        for (int m0 = 0; m0 < M; m0 += 16 * kMaxMt) {
            const int mrows = M - m0 < 16 * kMaxMt ? M - m0 : 16 * kMaxMt;
            if (mrows <= 16)
                gateup_consume<ACT, NC, NP, R, 1>(A, c0, lds, lds_sz, start, m0, mrows);
            else
                gateup_consume<ACT, NC, NP, R, 2>(A, c0, lds, lds_sz, start, m0, mrows);
        }
    }
}

// ------------------------------------------------ gate/up, flowing ring
// Persistent form of the 11 + 1-wave kernel above (NC consumers, one producer,
// ring depth 3) for launches with more (expert, column block) items than CUs:
// W workgroups (one per CU), workgroup w owns the items w, w + W, w + 2W, ...
// of gateup_act_kernel's numbering (all column blocks of an expert on one XCD
// while W is a multiple of 8). Every item is cut into passes of up to 32 rows,
// and the producer streams the quantisation groups of all the workgroup's
// passes through one ring without draining it between them: the ring fills
// once per workgroup instead of once per item, and the first groups of the
// next pass land while the consumers finish the current one. While they
// compute, the consumers also fetch what the next pass needs into spare LDS:
// the token ids of its rows, and the scale / zero table when it starts a new
// item (two table buffers, alternating per item with rows).
// Balanced pairs: with exactly two items per workgroup and whole experts in
// each XCD's first-round items, the second item is not w + W: the first-round
// experts ranked by rows (most first) are matched with the second-round
// experts ranked the other way (fewest first), so a workgroup with a heavy
// first item gets a light second one. The column blocks of a matched expert
// follow those of its partner, so they stay together on one XCD.
// Arithmetic and outputs are those of gateup_act_kernel, bit for bit.
constexpr int kFlowMaxItems = 64;  // items per workgroup (table entries)
constexpr int kFlowR = 3;          // ring depth
constexpr int kFlowMinG = 8;       // groups per pass: the next pass's token ids go
                                   // to LDS at group G/2, its first issue is at G-2

// int32 read through the constant address space: uniform loads become scalar
// loads (counted by lgkmcnt, not by the vmcnt of the direct-to-LDS loads)
using ConstI32 = const int32_t __attribute__((address_space(4)));
__device__ __forceinline__ const ConstI32* as_scalar_i32(const int32_t* p) { return (const ConstI32*)p; }

template <int NC>
struct GuFlowShape {
    using B = GuShape<NC, 1, kFlowR>;
    static constexpr size_t sz_bytes(int G) { return static_cast<size_t>(4) * B::kCols * G * 2; }
    static constexpr size_t sz_off(int G, int buf) { return static_cast<size_t>(kFlowR) * B::kSlot + buf * sz_bytes(G); }
    static constexpr size_t tok_off(int G) { return sz_off(G, 2); }
    // item table: (first sorted slot, rows, expert, first column) per item
    static constexpr size_t info_off(int G) { return tok_off(G) + 2 * 16 * kMaxMt * 4; }
    static constexpr size_t lds_bytes(int G) { return info_off(G) + kFlowMaxItems * 16; }
};

// Item table of workgroup w, written by the calling wave (wave 0 of the
// consumers): (first sorted slot, rows, expert, first column) of items
// 0 .. K-1. Without pairs item k is w + k*W. With balanced pairs (K = 2,
// W = items / 2, n = W / nb <= 64 experts per round, one per lane): lane j
// holds the expert of the first-round workgroup 8*nb*(j/8) + j%8 (column
// block 0) and the expert of that workgroup's natural second item; the
// caller's first item is the expert of lane jm, column block b, and its rank r
// among the first-round experts (most rows first, ties: lower expert first)
// picks the second-round expert of rank r (fewest rows first, same ties),
// column block b. All loads go out before any is used.
__device__ __forceinline__ void gu_flow_fill_table(const GuArgs& A, int4* __restrict__ info, int w, int W, int items,
                                                   int K, int nb, int kCols, bool pair) {
    const int lane = threadIdx.x & (kWave - 1);
    if (!pair) {
        if (lane < K) {
            const int tile = xcd_remap(w + lane * W, items);
            const int e = tile / nb;
            const int start = A.offsets[e];
            info[lane] = int4{start, A.offsets[e + 1] - start, e, (tile - e * nb) * kCols};
        }
        return;
    }
    const int n = W / nb;
    const int wj = 8 * nb * (lane >> 3) + (lane & 7);
    int e1 = 0, e2 = 0, s1 = 0, s2 = 0, m1 = -1, m2 = 0x7fffffff;
    if (lane < n) {
        e1 = xcd_remap(wj, items) / nb;
        e2 = xcd_remap(wj + W, items) / nb;
        s1 = A.offsets[e1];
        s2 = A.offsets[e2];
        m1 = A.offsets[e1 + 1] - s1;
        m2 = A.offsets[e2 + 1] - s2;
    }
    const int q = w >> 3;
    const int b = q % nb;
    const int jm = (q / nb) * 8 + (w & 7);
    const int m1me = __builtin_amdgcn_readlane(m1, jm), e1me = __builtin_amdgcn_readlane(e1, jm);
    const int r = __popcll(__ballot(lane < n && (m1 > m1me || (m1 == m1me && e1 < e1me))));
    int rank2 = 0;
    for (int k = 0; k < n; ++k) {
        const int mk = __builtin_amdgcn_readlane(m2, k), ek = __builtin_amdgcn_readlane(e2, k);
        rank2 += (mk < m2 || (mk == m2 && ek < e2)) ? 1 : 0;
    }
    const int jl = __ffsll(static_cast<unsigned long long>(__ballot(lane < n && rank2 == r))) - 1;  // one lane
    const int4 first{__builtin_amdgcn_readlane(s1, jm), m1me, e1me, b * kCols};
    const int4 second{__builtin_amdgcn_readlane(s2, jl), __builtin_amdgcn_readlane(m2, jl),
                      __builtin_amdgcn_readlane(e2, jl), b * kCols};
    if (lane == 0) info[0] = first;
    if (lane == 1) info[1] = second;
}

// A pass: rows start + m0 .. start + min(M, m0 + 32) - 1 of item k (k == K: none left).
struct GuPass {
    int k, m0, start, M;
};

// The item table held in registers after the first barrier: lane k holds
// item k (one LDS read per wave); entries are then taken with v_readlane,
// without LDS round trips at the pass changes.
__device__ __forceinline__ int4 gu_flow_table(const int4* info, int K) {
    const int lane = threadIdx.x & (kWave - 1);
    return lane < K ? info[lane] : int4{0, 0, 0, 0};
}

// The first pass at or after (k, m0) with rows. All values wave-uniform.
__device__ __forceinline__ GuPass gu_flow_seek(int k, int m0, int K, const int4& tab) {
    while (k < K) {
        const int start = __builtin_amdgcn_readlane(tab.x, k), M = __builtin_amdgcn_readlane(tab.y, k);
        if (m0 < M) return GuPass{k, m0, start, M};
        ++k;
        m0 = 0;
    }
    return GuPass{K, 0, 0, 0};
}

__device__ __forceinline__ int gu_flow_npass(int K, const int4& tab) {
    int n = 0;
    for (int k = 0; k < K; ++k) n += (__builtin_amdgcn_readlane(tab.y, k) + 16 * kMaxMt - 1) / (16 * kMaxMt);
    return n;
}

__device__ __forceinline__ void gu_flow_item(const int4& tab, int k, int& e, int& c0) {
    e = __builtin_amdgcn_readlane(tab.z, k);
    c0 = __builtin_amdgcn_readlane(tab.w, k);
}

// The scale / zero table of an item's kCols rows: four [kCols x G] fp16 blocks
// (s_gate, z_gate, s_up, z_up), each contiguous in global memory, fetched by
// the consumer threads into registers (issue) and written to LDS (commit).
template <int NC>
struct GuSzFetch {
    using S = GuShape<NC, 1, kFlowR>;
    u32x4 v[S::kSzPer];
    // chunk k of this thread: 16 bytes of block b at o, or none
    __device__ __forceinline__ static const u32x4* src(const GuArgs& A, int e, int c0, int G, int k) {
        const int nq = S::kCols * G * 2 / 16;  // 16-byte chunks per block
        int i = threadIdx.x + k * NC * kWave;
        if (i >= 4 * nq) i = 0;  // clamped, never stored
        const int64_t gate0 = static_cast<int64_t>(e) * 2 * A.I + c0;
        const int b = i / nq, o = i - b * nq;
        const f16* base = ((b & 1) ? A.gu_z : A.gu_s) + ((b & 2) ? gate0 + A.I : gate0) * G;
        return reinterpret_cast<const u32x4*>(base) + o;
    }
    __device__ __forceinline__ void issue(const GuArgs& A, int e, int c0, int G) {
#pragma unroll
        for (int k = 0; k < S::kSzPer; ++k) v[k] = *src(A, e, c0, G, k);
    }
    __device__ __forceinline__ void commit(f16* __restrict__ dst, int G) const {
        const int nq = S::kCols * G * 2 / 16;
#pragma unroll
        for (int k = 0; k < S::kSzPer; ++k) {
            const int i = threadIdx.x + k * NC * kWave;
            if (i < 4 * nq) reinterpret_cast<u32x4*>(dst)[i] = v[k];
        }
    }
};

template <int NC>
__device__ __forceinline__ void gu_flow_produce(const GuArgs& A, char* __restrict__ lds, int w, int items, int K) {
    using S = GuShape<NC, 1, kFlowR>;
    using F = GuFlowShape<NC>;
    constexpr int R = kFlowR;
    const int lane = threadIdx.x & (kWave - 1);
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int G = A.H >> 7;
    const int nb = A.I / S::kCols;
    const int rowbytes = A.H >> 1;
    const int wlane = rr * rowbytes + ch * 16;
    const int* tok = reinterpret_cast<const int*>(lds + F::tok_off(G));
    const int4* info = reinterpret_cast<const int4*>(lds + F::info_off(G));
    const char* abase = reinterpret_cast<const char*>(A.a16);
    // the issue cursor's pass: weights of its item (first gate row + the lane's
    // piece), the lane's activation row of each M tile, its M tiles
    const char* wbase = nullptr;
    int64_t aoff[kMaxMt];
    int mt = 1;
    auto set_item = [&](int e, int c0) {
        wbase = reinterpret_cast<const char*>(A.gu_q) + (static_cast<int64_t>(e) * 2 * A.I + c0) * rowbytes + wlane;
    };
    // token row of M tile t of pass p for this lane (rows past the pass's last
    // repeat it: loaded, never stored): from the consumers' LDS copy (toks)
    // for all passes but a workgroup's first
    auto set_rows = [&](const GuPass& p, const int* toks) {
        const int mrows = min(p.M - p.m0, 16 * kMaxMt);
        mt = mrows > 16 ? 2 : 1;
#pragma unroll
        for (int t = 0; t < kMaxMt; ++t) aoff[t] = (static_cast<int64_t>(toks[t * 16 + rr]) * A.H + ch * 8) * 2;
    };
    // ... and for the first pass from the routing itself, by scalar loads: a
    // vector load here would wait (in-order vmcnt) for the weight groups
    // already in flight
    auto set_rows_first = [&](const GuPass& p) {
        const int mrows = min(p.M - p.m0, 16 * kMaxMt);
        mt = mrows > 16 ? 2 : 1;
        const ConstI32* rows = as_scalar_i32(A.sorted_rows) + p.start + p.m0;
        int v[16 * kMaxMt];  // all loads first (uniform, in flight together), then a per-lane pick
#pragma unroll
        for (int i = 0; i < 16 * kMaxMt; ++i) v[i] = rows[min(i, mrows - 1)];
#pragma unroll
        for (int i = 0; i < 16 * kMaxMt; ++i) asm volatile("" : "+s"(v[i]));  // not folded into a per-lane load
#pragma unroll
        for (int t = 0; t < kMaxMt; ++t) {
            int row = v[t * 16];
#pragma unroll
            for (int i = 1; i < 16; ++i) row = rr == i ? v[t * 16 + i] : row;
            aoff[t] = (static_cast<int64_t>(row / A.topk) * A.H + ch * 8) * 2;
        }
    };
    auto issue_w = [&](int g, int slot) {
        char* base = lds + slot * S::kSlot;
#pragma unroll
        for (int b = 0; b < 2 * NC; ++b) {
            const int wv = b >> 1, j = b & 1;
            dma16(wbase + static_cast<int64_t>((j ? A.I : 0) + wv * 16) * rowbytes + g * 64, base + b * kBlk);
        }
    };
    auto issue_a = [&](int g, int slot) {
        char* base = lds + slot * S::kSlot;
#pragma unroll
        for (int t = 0; t < kMaxMt; ++t)
            if (t < mt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    dma16(abase + aoff[t] + (i * 32 + g * 128) * 2, base + (2 * NC + t * 4 + i) * kBlk);
    };

    // prologue. The first item is known without the table (item w): its first
    // weight groups go out before the routing is read. When it has no rows,
    // the first pass is found in the table after the first barrier and one
    // more barrier publishes its first group (the consumers take it too).
    const int t0 = xcd_remap(w, items);
    const int e0 = t0 / nb;
    set_item(e0, (t0 - e0 * nb) * S::kCols);
    const bool early = A.early != 0;
    if (early)
        for (int g = 0; g < R - 1; ++g) issue_w(g, g);
    const ConstI32* offs = as_scalar_i32(A.offsets);  // scalar loads, as above
    const int start0 = offs[e0];
    GuPass p{0, 0, start0, offs[e0 + 1] - start0};
    const bool first_rows = p.M > 0;
    if (first_rows) {
        set_rows_first(p);
        for (int g = 0; g < R - 1; ++g) {
            if (!early) issue_w(g, g);
            issue_a(g, g);
        }
    }
    vm_wait<0>();
    dma_barrier();
    const int4 tab = gu_flow_table(info, K);
    const int S_total = gu_flow_npass(K, tab) * G;  // group steps of all passes
    if (!first_rows && S_total > 0) {
        p = gu_flow_seek(0, 0, K, tab);
        int e, c0;
        gu_flow_item(tab, p.k, e, c0);
        set_item(e, c0);
        set_rows_first(p);
        for (int g = 0; g < R - 1; ++g) {
            issue_w(g, g);
            issue_a(g, g);
        }
        vm_wait<0>();
        dma_barrier();
    }
    int ig = R - 1;      // group of the issue cursor's pass
    int ipass = 0;       // ordinal of the issue cursor's pass
    int slot_i = R - 1;  // slot of the next issue
    int issued = S_total > 0 ? R - 1 : 0;
    for (int s = 0; s < S_total; ++s) {
        // consumers read step s from slot s % R; the slot of step s - 1 is free
        int mt_issued = 0;
        if (issued < S_total) {
            if (ig == G) {  // the issue cursor enters the next pass
                const GuPass q = gu_flow_seek(p.k, p.m0 + 16 * kMaxMt, K, tab);
                if (q.k != p.k) {
                    int e, c0;
                    gu_flow_item(tab, q.k, e, c0);
                    set_item(e, c0);
                }
                p = q;
                ++ipass;
                ig = 0;
                set_rows(p, tok + (ipass & 1) * 16 * kMaxMt);
            }
            issue_w(ig, slot_i);
            issue_a(ig, slot_i);
            mt_issued = mt;
            ++ig;
            ++issued;
            slot_i = slot_i + 1 == R ? 0 : slot_i + 1;
        }
        // step s + 1 must have landed before the barrier: only the step just
        // issued (2*NC + 4*mt loads) may still be in flight
        if (mt_issued == 1)
            vm_wait<2 * NC + 4>();
        else if (mt_issued == 2)
            vm_wait<2 * NC + 8>();
        else
            vm_wait<0>();
        dma_barrier();
    }
    vm_wait<0>();
}

// Consumer side of one pass: G barriers. At group 1 the loads for the next pass
// go out (the expanded rows of its slots from wave 0; the scale / zero table
// of its item when it starts a new one), at group G/2 they go to LDS.
template <int ACT, int NC, int MT>
__device__ __forceinline__ void gu_flow_consume_pass(const GuArgs& A, char* __restrict__ lds, int& slot,
                                                     const f16* __restrict__ sz, int c0, int row0, int mrows,
                                                     int nrow0, int nmrows, int* __restrict__ ntok, int ne, int nc0,
                                                     f16* __restrict__ nsz) {
    using S = GuShape<NC, 1, kFlowR>;
    const int G = A.H >> 7;
    const int tid = threadIdx.x;
    const NibConsts kn = nib_consts();
    f32x4 acc[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    GuSzFetch<NC> nf;
    int row = 0;
    for (int g = 0; g < G; ++g) {
        gateup_group<NC, MT>(lds + slot * S::kSlot, sz, G, g, kn, acc);
        if (g == 1) {
            // the expanded row only: its token (row / topk) is taken at G/2, once it has landed
            if (ntok && tid < 16 * kMaxMt) row = A.sorted_rows[nrow0 + min(tid, nmrows - 1)];
            if (nsz) nf.issue(A, ne, nc0, G);
        } else if (g == G / 2) {
            if (ntok && tid < 16 * kMaxMt) ntok[tid] = row / A.topk;
            if (nsz) nf.commit(nsz, G);
        }
        slot = slot + 1 == kFlowR ? 0 : slot + 1;
        __syncthreads();
    }
    // the prefetch registers landed at G/2; an explicit wait tells the
    // compiler so (it cannot pair the two conditional blocks), else it waits
    // for this epilogue's stores before reusing those registers in the next pass
    vm_wait<0>();
    gateup_store<ACT, MT>(A, acc, c0, row0, mrows);
}

template <int ACT, int NC>
__device__ __forceinline__ void gu_flow_consume(const GuArgs& A, char* __restrict__ lds, int w, int W, int items,
                                                int K, bool pair) {
    using S = GuShape<NC, 1, kFlowR>;
    using F = GuFlowShape<NC>;
    const int G = A.H >> 7;
    const int nb = A.I / S::kCols;
    int* tok = reinterpret_cast<int*>(lds + F::tok_off(G));
    int4* info = reinterpret_cast<int4*>(lds + F::info_off(G));
    f16* sz0 = reinterpret_cast<f16*>(lds + F::sz_off(G, 0));
    // the first item's scale / zero table into buffer 0, issued first (item w,
    // known without the table; read in vain when it has no rows), then the
    // item table by wave 0, whose routing loads overlap the table's
    const int t0 = xcd_remap(w, items);
    const int e0 = t0 / nb;
    {
        GuSzFetch<NC> f;
        f.issue(A, e0, (t0 - e0 * nb) * S::kCols, G);
        if (wave_id() == 0) gu_flow_fill_table(A, info, w, W, items, K, nb, S::kCols, pair);
        f.commit(sz0, G);
    }
    __syncthreads();  // first barrier: the table, buffer 0 and the first pass's group 0 are ready
    const int4 tab = gu_flow_table(info, K);
    const int npass = gu_flow_npass(K, tab);
    GuPass p = gu_flow_seek(0, 0, K, tab);
    const bool first_rows = __builtin_amdgcn_readlane(tab.y, 0) > 0;
    if (!first_rows && npass > 0) {  // the first pass is a later item's (one more barrier, as the producer)
        int e, c0;
        gu_flow_item(tab, p.k, e, c0);
        GuSzFetch<NC> f;
        f.issue(A, e, c0, G);
        f.commit(sz0, G);
        __syncthreads();
    }
    int zb = 0;  // table buffer of the current item
    int slot = 0;
    for (int ip = 0; ip < npass; ++ip) {
        const GuPass q = gu_flow_seek(p.k, p.m0 + 16 * kMaxMt, K, tab);
        const bool more = q.k < K, fresh = more && q.k != p.k;
        int e, c0, ne = 0, nc0 = 0;
        gu_flow_item(tab, p.k, e, c0);
        if (fresh) gu_flow_item(tab, q.k, ne, nc0);
        const f16* sz = reinterpret_cast<const f16*>(lds + F::sz_off(G, zb));
        int* ntok = more ? tok + ((ip + 1) & 1) * 16 * kMaxMt : nullptr;
        f16* nsz = fresh ? reinterpret_cast<f16*>(lds + F::sz_off(G, zb ^ 1)) : nullptr;
        const int mrows = min(p.M - p.m0, 16 * kMaxMt);
        const int nrow0 = q.start + q.m0, nmrows = more ? min(q.M - q.m0, 16 * kMaxMt) : 1;
        if (mrows <= 16)
            gu_flow_consume_pass<ACT, NC, 1>(A, lds, slot, sz, c0, p.start + p.m0, mrows, nrow0, nmrows, ntok, ne, nc0,
                                             nsz);
        else
            gu_flow_consume_pass<ACT, NC, 2>(A, lds, slot, sz, c0, p.start + p.m0, mrows, nrow0, nmrows, ntok, ne, nc0,
                                             nsz);
        if (fresh) zb ^= 1;
        p = q;
    }
}

template <int ACT, int NC>
__global__ __launch_bounds__((NC + 1) * kWave) void gateup_flow_kernel(GuArgs A, int W, int items, int pair) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int w = blockIdx.x;
    const int K = (items - w + W - 1) / W;  // items of this workgroup (1 .. kFlowMaxItems)
    if (wave_id() >= NC) {
        // the producer issues first on its SIMD after each barrier
        __builtin_amdgcn_s_setprio(3);
        gu_flow_produce<NC>(A, lds, w, items, K);
    } else {
        gu_flow_consume<ACT, NC>(A, lds, w, W, items, K, pair != 0);
    }
}

// Dynamic LDS beyond 64 KB: raise a kernel's limit (called once per kernel).
bool set_max_lds(const void* fn) {
    const bool ok = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, kLdsDynMax) == hipSuccess;
    (void)hipGetLastError();
    return ok;
}

// Compute units of the current device (cached per device).
int device_cus() {
    constexpr int kMaxDev = 64;
    static std::atomic<int> cache[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
        (void)hipGetLastError();
        return 256;
    }
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

template <int NC, int NP, int R>
int launch_gateup_nc(const GuArgs& A, int64_t E, int64_t nrows, int act, hipStream_t st) {
    using S = GuShape<NC, NP, R>;
    (void)nrows;
    if (E * (A.I / S::kCols) >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    const unsigned grid = static_cast<unsigned>(E * (A.I / S::kCols));
    const size_t lds = S::lds_bytes(A.H / 128);
    if (lds > kLdsDynMax) return KSL_ERR_SHAPE;
    static const bool attr_set =
        set_max_lds(reinterpret_cast<const void*>(&gateup_act_kernel<KSL_ACT_GELU_TANH, NC, NP, R>)) &&
        set_max_lds(reinterpret_cast<const void*>(&gateup_act_kernel<KSL_ACT_SILU, NC, NP, R>)) &&
        set_max_lds(reinterpret_cast<const void*>(&gateup_act_kernel<KSL_ACT_NONE, NC, NP, R>));
    (void)attr_set;
    if (act == KSL_ACT_GELU_TANH)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_GELU_TANH, NC, NP, R>), dim3(grid), dim3(S::kThreads), lds, st, A);
    else if (act == KSL_ACT_SILU)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_SILU, NC, NP, R>), dim3(grid), dim3(S::kThreads), lds, st, A);
    else if (act == KSL_ACT_NONE)
        hipLaunchKernelGGL((gateup_act_kernel<KSL_ACT_NONE, NC, NP, R>), dim3(grid), dim3(S::kThreads), lds, st, A);
    else
        return KSL_ERR_ARG;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

template <int NC>
int launch_gateup_flow(const GuArgs& A, int act, int W, int items, hipStream_t st) {
    using F = GuFlowShape<NC>;
    constexpr int kThreads = (NC + 1) * kWave;
    const size_t lds = F::lds_bytes(A.H / 128);
    if (lds > kLdsDynMax) return KSL_ERR_SHAPE;
    // balanced pairs: two items per workgroup, whole experts in each XCD's
    // first-round items, at most one first-round expert per lane of a wave
    const int nb = A.I / GuShape<NC, 1, kFlowR>::kCols;
    const int pair = items == 2 * W && (W / kXcds) % nb == 0 && (items / kXcds) % nb == 0 && W / nb <= kWave;
    static const bool attr_set =
        set_max_lds(reinterpret_cast<const void*>(&gateup_flow_kernel<KSL_ACT_GELU_TANH, NC>)) &&
        set_max_lds(reinterpret_cast<const void*>(&gateup_flow_kernel<KSL_ACT_SILU, NC>)) &&
        set_max_lds(reinterpret_cast<const void*>(&gateup_flow_kernel<KSL_ACT_NONE, NC>));
    (void)attr_set;
    if (act == KSL_ACT_GELU_TANH)
        hipLaunchKernelGGL((gateup_flow_kernel<KSL_ACT_GELU_TANH, NC>), dim3(W), dim3(kThreads), lds, st, A, W, items,
                           pair);
    else if (act == KSL_ACT_SILU)
        hipLaunchKernelGGL((gateup_flow_kernel<KSL_ACT_SILU, NC>), dim3(W), dim3(kThreads), lds, st, A, W, items, pair);
    else if (act == KSL_ACT_NONE)
        hipLaunchKernelGGL((gateup_flow_kernel<KSL_ACT_NONE, NC>), dim3(W), dim3(kThreads), lds, st, A, W, items, pair);
    else
        return KSL_ERR_ARG;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

// Workgroups of the flowing gate/up launch for `items` (expert, column block)
// items, H/128 groups per pass: one per CU (a multiple of 8, so an expert's
// column blocks share an XCD), or 0 where the launch of one workgroup per item
// is used instead (no more items than CUs, short passes, more items per
// workgroup than the item table holds, or LDS).
int gateup_flow_workgroups(int64_t items, int64_t H, int cus) {
    constexpr int NC = 11;
    const int W = cus - cus % kXcds;
    const int G = static_cast<int>(H / 128);
    if (W < kXcds || items <= cus || items > static_cast<int64_t>(W) * kFlowMaxItems) return 0;
    if (G < kFlowMinG || GuFlowShape<NC>::lds_bytes(G) > kLdsDynMax) return 0;
    return W;
}

// --------------------------------------------------------------------- down
// Register-streamed kernel. A workgroup of kDnWaves waves owns one expert and
// a range of its output columns (the expert's H columns split over
// ceil(#CUs / E) workgroups). The expert's activation rows (out2, up to 64 per
// chunk) are copied into LDS once per chunk (direct global->LDS loads). Every
// wave then walks pairs of 16-column tiles (pairs w, w + kDnWaves, ...): each
// lane loads its weight words and the scale / zero-point of its groups for
// both tiles of the pair straight into registers, by ordinary loads that the
// compiler tracks and waits for, then decodes and multiplies them; while one
// wave waits for its pair the other wave of its SIMD computes (a second
// register buffer per wave, measured, was not faster). The two tiles of a
// pair share every activation fragment read from LDS (half the LDS reads of
// one tile at a time). Nothing is staged before a wave's first pair but the
// activations, and no load is issued past a wave's last pair (each weight
// byte is fetched once).
//
// K mapping: one 16-byte load per lane and 128-K block, lane (col, c) holding
// row col, nibbles 32c .. 32c+31 of the block: MFMA step i takes nibbles
// 32c + 8i .. +8, the 128-group order of the activations (out2_store_index);
// the lane's 32 nibbles of a block lie in one 64-K quantisation group,
// 2*g2 + c/2. A trailing 64-K group (I % 128 == 64) takes an 8-byte load per
// lane, the 64-group order. B = fp16((q - z) * s), the reference's own
// dequantised weight (kernels/fused_moe_w4_v2.py:172-175), accumulated in
// fp32 in K order, so each output element sees the same MFMA sequence as the
// row-block kernel of large routings (moe_rbgemm.hip).
constexpr int kDnWaves = 8;
constexpr int kDnMaxMt = 4;  // 16-row M tiles per row chunk of down (64 rows)
constexpr int kDnThreads = kDnWaves * kWave;
constexpr int kDnMaxG = 16;  // I <= 1024

// Down weight layouts (dn_layout of the C ABI):
//   reference: dn_q [E, H, I/2], one row per output column;
//   tiled    : the same bytes regrouped per 16-row tile (the tile's base
//              address unchanged) in the order lanes load them: unit u
//              (u < I/128) is 64 lanes x 16 B, lane l = c*16 + col holding
//              row col, bytes u*64 + c*16 .. +16; then, when I % 128 == 64, the
//              tail: 64 lanes x 8 B, lane l holding row col, bytes
//              (I/128)*64 + c*8 .. +8. Every load instruction then reads 1 KB
//              (512 B for the tail) of contiguous memory instead of 16 row
//              pieces of 64 B; the values, and so the results, are the same.
enum DnLayout { kDnRef = KSL_DN_LAYOUT_REF, kDnTiled = KSL_DN_LAYOUT_TILED };

struct DnArgs {
    const f16* out2;
    const int32_t* offsets;
    const uint8_t* dn_q;
    const f16* dn_s;
    const f16* dn_z;
    f16* out3;
    const uint32_t* sz;     // tiled layout: the (scale, zero) pair table after the tiled weights
    int H, I, nsplit, tpw;  // tpw: 16-column tiles per workgroup
    int early;              // weights of the first pair are requested before the routing is read
};

// LDS: activation blocks [kDnMaxMt][2G] (1 KB each, frag_pos order), then
// one output staging area per wave (two 16-row M tiles of a pair's 32
// columns, kDnOutRow bytes per row).
constexpr int kDnOutRow = 80;  // 64 bytes of a row + 16 of padding (2-way bank conflicts at most)
constexpr int kDnOutWave = 2 * 16 * kDnOutRow;
__host__ __device__ inline size_t dn_act_bytes(int G) { return static_cast<size_t>(kDnMaxMt) * 2 * G * kBlk; }
inline size_t dn_lds_bytes(int G) { return dn_act_bytes(G) + static_cast<size_t>(kDnWaves) * kDnOutWave; }

// One lane's part of one tile: G2 16-byte weight words, the 8-byte tail, and
// the (scale, zero-point) of the lane's group in each 128-K block and of the
// tail group: one (s | z << 16) word each in the tiled layout (the pair
// table), two 16-bit values (in 32-bit registers: as 16-bit array elements
// they were kept in scratch memory) in the reference layout.
template <int G2, bool TAIL, int LAYOUT>
struct DnTile {
    static constexpr int NG = G2 + (TAIL ? 1 : 0);
    // load instructions of one tile (dn_fetch)
    static constexpr int kLoads = G2 + (TAIL ? 1 : 0) + (LAYOUT == kDnTiled ? NG : 2 * NG);
    u32x4 q[G2];
    u32x2 t[TAIL ? 1 : 0];
    uint32_t sz[LAYOUT == kDnTiled ? NG : 0];
    uint32_t s[LAYOUT == kDnTiled ? 0 : NG], z[LAYOUT == kDnTiled ? 0 : NG];
    __device__ __forceinline__ f16 scale(int j) const {
        if constexpr (LAYOUT == kDnTiled) return __builtin_bit_cast(f16x2, sz[j])[0];
        else return __builtin_bit_cast(f16, static_cast<uint16_t>(s[j]));
    }
    __device__ __forceinline__ f16 zero(int j) const {
        if constexpr (LAYOUT == kDnTiled) return __builtin_bit_cast(f16x2, sz[j])[1];
        else return __builtin_bit_cast(f16, static_cast<uint16_t>(z[j]));
    }
};

// Per-lane byte offsets of a tile's loads, the same for every tile (kept in
// registers across the walk, so that a fetch only changes wave-uniform bases).
struct DnLane {
    int q;    // weight words (+ g2 * 1024 tiled, + g2 * 64 reference)
    int t;    // the tail word
    int sz;   // the lane's (scale, zero) of 128-K block g2 (+ g2 * 128 tiled, + g2 * 4 reference)
    int szt;  // the tail group's (scale, zero)
};

template <int G2, bool TAIL, int LAYOUT>
__device__ __forceinline__ DnLane dn_lane(int I, int col, int c) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    const int rb = I >> 1;
    if constexpr (LAYOUT == kDnTiled)
        return DnLane{(c * 16 + col) * 16, G2 * 1024 + (c * 16 + col) * 8, ((c >> 1) * 16 + col) * 4,
                      (2 * G2 * 16 + col) * 4};
    else
        return DnLane{col * rb + c * 16, col * rb + G2 * 64 + c * 8, (col * G + (c >> 1)) * 2, (col * G + 2 * G2) * 2};
}

template <typename T>
__device__ __forceinline__ T ld_nt(const uint8_t* base, int off) {
    return __builtin_nontemporal_load(reinterpret_cast<const T*>(base + off));
}

// Requests tile `row` (its first dn row: expert * H + column) into w:
// ordinary non-temporal loads, which the compiler waits for before the first
// use of each register.
template <int G2, bool TAIL, int LAYOUT>
__device__ __forceinline__ void dn_fetch(DnTile<G2, TAIL, LAYOUT>& w, const DnArgs& A, int64_t row,
                                         const DnLane& ln) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    // wave-uniform bases, lane offsets from ln
    const uint8_t* tb = A.dn_q + row * (A.I >> 1);
    if constexpr (LAYOUT == kDnTiled) {
        // pair table: tile (row / 16), group g, column col at ((tile * G + g) * 16 + col)
        const uint8_t* pb = reinterpret_cast<const uint8_t*>(A.sz + (row >> 4) * (G * 16));
        static_for<G2>([&](auto j) { w.q[j] = ld_nt<u32x4>(tb, ln.q + j * 1024); });
        if constexpr (TAIL) w.t[0] = ld_nt<u32x2>(tb, ln.t);
        static_for<G2>([&](auto j) { w.sz[j] = ld_nt<uint32_t>(pb, ln.sz + j * 128); });
        if constexpr (TAIL) w.sz[G2] = ld_nt<uint32_t>(pb, ln.szt);
    } else {
        const uint8_t* sb = reinterpret_cast<const uint8_t*>(A.dn_s + row * G);
        const uint8_t* zb = reinterpret_cast<const uint8_t*>(A.dn_z + row * G);
        static_for<G2>([&](auto j) { w.q[j] = ld_nt<u32x4>(tb, ln.q + j * 64); });
        if constexpr (TAIL) w.t[0] = ld_nt<u32x2>(tb, ln.t);
        static_for<G2>([&](auto j) {
            w.s[j] = ld_nt<uint16_t>(sb, ln.sz + j * 4);
            w.z[j] = ld_nt<uint16_t>(zb, ln.sz + j * 4);
        });
        if constexpr (TAIL) {
            w.s[G2] = ld_nt<uint16_t>(sb, ln.szt);
            w.z[G2] = ld_nt<uint16_t>(zb, ln.szt);
        }
    }
}

// Both tiles of a pair against two M tiles of activations: every activation
// fragment read from LDS feeds one MFMA of each tile. NT M tiles (1 or 2) per
// pass.
template <int G2, bool TAIL, int LAYOUT, int NT>
__device__ __forceinline__ void dn_pair_mma(const DnTile<G2, TAIL, LAYOUT>& w0, const DnTile<G2, TAIL, LAYOUT>& w1,
                                            f32x4 (&acc0)[NT], f32x4 (&acc1)[NT], const char* __restrict__ a_lds,
                                            int fo, const NibConsts& kn) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    auto step = [&](const f16x8& b0, const f16x8& b1, int blk) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const f16x8 a = *reinterpret_cast<const f16x8*>(a_lds + (t * 2 * G + blk) * kBlk + fo);
            acc0[t] = mfma16x16x32(b0, a, acc0[t]);
            acc1[t] = mfma16x16x32(b1, a, acc1[t]);
        }
    };
    // the weight words pass through an empty asm, so that the decode happens
    // here, in each pass, block by block: decoded weights (four times the
    // registers of the words) are neither hoisted nor kept for a later pass
    static_for<G2>([&](auto g2) {
        const f16 s0 = w0.scale(g2), s1 = w1.scale(g2);
        const ZeroPair z0 = zero_pair(w0.zero(g2)), z1 = zero_pair(w1.zero(g2));
        u32x4 q0 = w0.q[g2], q1 = w1.q[g2];
        asm volatile("" : "+v"(q0), "+v"(q1));
#pragma unroll
        for (int i = 0; i < 4; ++i)
            step(nib8_dequant(q0[i], z0, f16x2{s0, s0}, kn), nib8_dequant(q1[i], z1, f16x2{s1, s1}, kn), g2 * 4 + i);
        // one 128-K block at a time: hoisting every block's operands would
        // exceed the register budget
        __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (TAIL) {
        const f16 s0 = w0.scale(G2), s1 = w1.scale(G2);
        const ZeroPair z0 = zero_pair(w0.zero(G2)), z1 = zero_pair(w1.zero(G2));
        u32x2 q0 = w0.t[0], q1 = w1.t[0];
        asm volatile("" : "+v"(q0), "+v"(q1));
#pragma unroll
        for (int i = 0; i < 2; ++i)
            step(nib8_dequant(q0[i], z0, f16x2{s0, s0}, kn), nib8_dequant(q1[i], z1, f16x2{s1, s1}, kn), G2 * 4 + i);
    }
}

// A pair's outputs for NT M tiles. The weights are the MFMA's A operand and
// the activations its B operand, so each accumulator is its tile transposed:
// lane (col, c) holds row col of the M tile, the tile's output columns 4c ..
// 4c+3. They go through the wave's LDS staging area (row-major, the pair's 32
// columns per row) and out as 16 bytes per lane, four lanes per row: 64
// contiguous bytes per row and one store per M tile. Rows past the chunk, or
// a second tile past the workgroup's last, take an out-of-range offset
// (dropped by the buffer store).
template <int NT>
__device__ __forceinline__ void dn_store_pair(const f32x4 (&acc0)[NT], const f32x4 (&acc1)[NT], char* o_lds,
                                              __amdgpu_buffer_rsrc_t out, int H, int colw, bool second, int mrows,
                                              int lane, int row0) {
    const int col = lane & 15, c = lane >> 4;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const f16x4 v0{static_cast<f16>(acc0[t][0]), static_cast<f16>(acc0[t][1]), static_cast<f16>(acc0[t][2]),
                       static_cast<f16>(acc0[t][3])};
        const f16x4 v1{static_cast<f16>(acc1[t][0]), static_cast<f16>(acc1[t][1]), static_cast<f16>(acc1[t][2]),
                       static_cast<f16>(acc1[t][3])};
        char* rowp = o_lds + (t * 16 + col) * kDnOutRow;
        *reinterpret_cast<f16x4*>(rowp + c * 8) = v0;
        *reinterpret_cast<f16x4*>(rowp + 32 + c * 8) = v1;
    }
    // lane (r = lane / 4, part = lane % 4): 16 bytes of row r, columns 8 * part ..
    const int r = lane >> 2, part = lane & 3;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(o_lds + (t * 16 + r) * kDnOutRow + part * 16);
        const int row = t * 16 + r;  // row0 + row of the chunk; mrows counted from row0
        const bool ok = row < mrows && (second || part < 2);
        const uint32_t off = ok ? static_cast<uint32_t>(((row0 + row) * H + colw + 8 * part) * 2) : kDropOffset;
        __builtin_amdgcn_raw_buffer_store_b128(v, out, off, 0, 0);
    }
}

// Activation blocks of one chunk into LDS: block b = t*2G + bb, bb < 4*G2 the
// 128-K block bb/4, step bb%4; else tail step bb - 4*G2. Rows fetched
// row-major (frag_pos). Issued by every wave, round-robin.
template <int G2, bool TAIL>
__device__ __forceinline__ void dn_stage_a(const DnArgs& A, char* a_lds, int start, int m0, int mrows, int mt,
                                           int wave, int rr, int ch) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    for (int b = wave; b < mt * 2 * G; b += kDnWaves) {
        const int t = b / (2 * G), bb = b - t * 2 * G;
        const int off = bb < 4 * G2 ? (bb >> 2) * 128 + (bb & 3) * 32 : G2 * 128 + (bb - 4 * G2) * 32;
        int r = t * 16 + rr;
        if (r >= mrows) r = mrows - 1;  // rows past the expert's last: loaded, never stored
        dma16(A.out2 + static_cast<int64_t>(start + m0 + r) * A.I + off + ch * 8, a_lds + b * kBlk);
    }
}

// Each wave walks pairs of 16-column tiles of the workgroup (pair p = wave +
// k*kDnWaves: tiles 2p and 2p+1; an odd last tile pairs with itself, its
// second outputs dropped) for one chunk of mt M tiles: the pair's weights are
// requested, then decoded and multiplied as they arrive. Latency is hidden
// by the other waves of the SIMD rather than by a second register buffer (a
// second buffer, measured, was not faster: the decode, the MFMAs with their
// LDS reads and the stores already keep the SIMD busy while a wave waits).
// The M tiles go in passes of at most two over the same weight registers
// (accumulators for more would not fit), so a chunk of three or four M tiles
// decodes its weights twice but streams them once.
template <int G2, bool TAIL, int LAYOUT>
__global__ __launch_bounds__(kDnThreads) void down_kernel(DnArgs A) {
    constexpr int MTX = kDnMaxMt;
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int e = bid / A.nsplit;
    const int h = bid - e * A.nsplit;
    const int col0 = h * A.tpw * 16;
    const int ncols = A.H - col0 < A.tpw * 16 ? A.H - col0 : A.tpw * 16;
    if (ncols <= 0) return;
    const int ntiles = ncols >> 4;
    const int npairs = (ntiles + 1) >> 1;
    const int wave = wave_id();
    const int npw = wave < npairs ? (npairs - 1 - wave) / kDnWaves + 1 : 0;
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int fo = frag_pos(col, c) * 16;
    const NibConsts kn = nib_consts();
    const int64_t row0 = static_cast<int64_t>(e) * A.H + col0;  // first dn row of the workgroup
    char* o_lds = lds + dn_act_bytes(G) + wave * kDnOutWave;
    using Tile = DnTile<G2, TAIL, LAYOUT>;
    Tile x0, x1;
    const DnLane ln = dn_lane<G2, TAIL, LAYOUT>(A.I, col, c);
    auto fetch = [&](int k) {
        const int p = wave + k * kDnWaves;
        const int t1i = 2 * p + 1 < ntiles ? 2 * p + 1 : 2 * p;
        dn_fetch<G2, TAIL, LAYOUT>(x0, A, row0 + 32 * p, ln);
        dn_fetch<G2, TAIL, LAYOUT>(x1, A, row0 + 16 * t1i, ln);
    };
    const int start = A.offsets[e];
    const int M = A.offsets[e + 1] - start;
    if (M <= 0) return;
    for (int m0 = 0; m0 < M; m0 += 16 * MTX) {
        const int mrows = M - m0 < 16 * MTX ? M - m0 : 16 * MTX;
        const int mt = (mrows + 15) >> 4;
        if (m0 > 0) __syncthreads();  // every wave is done with the previous chunk's activations
        dn_stage_a<G2, TAIL>(A, lds, start, m0, mrows, mt, wave, rr, ch);
        // the first pair's weights go out behind the activations; the barrier
        // waits for the activations only (each wave's loads retire in order),
        // so a wave starts once its own pair has landed, not the slowest one's
        if (npw > 0) {
            fetch(0);
            vm_wait<2 * Tile::kLoads>();
        } else {
            vm_wait<0>();
        }
        dma_barrier();
        const __amdgpu_buffer_rsrc_t out =
            raw_rsrc(A.out3 + static_cast<int64_t>(start + m0) * A.H, static_cast<uint32_t>(mrows * A.H * 2));
        for (int k = 0; k < npw; ++k) {
            if (k > 0) fetch(k);
            const int p = wave + k * kDnWaves;
            // two straight-line passes, not a loop (a loop kept both tiles'
            // weights and every pass temporary live at once: spills)
            auto pass = [&](auto nt_c, int t0) {
                constexpr int NT = decltype(nt_c)::value;
                f32x4 acc0[NT], acc1[NT];
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    acc0[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                    acc1[t] = f32x4{0.f, 0.f, 0.f, 0.f};
                }
                dn_pair_mma<G2, TAIL, LAYOUT, NT>(x0, x1, acc0, acc1, lds + t0 * 2 * G * kBlk, fo, kn);
                dn_store_pair<NT>(acc0, acc1, o_lds, out, A.H, col0 + 32 * p, 2 * p + 1 < ntiles, mrows - 16 * t0,
                                  lane, t0 * 16);
            };
            // an odd last M tile goes in a one-tile pass (half the MFMAs and
            // LDS reads of a two-tile pass)
            if (mt == 1) {
                pass(std::integral_constant<int, 1>{}, 0);
            } else {
                pass(std::integral_constant<int, 2>{}, 0);
                if (mt == 3) pass(std::integral_constant<int, 1>{}, 2);
                if (mt == 4) pass(std::integral_constant<int, 2>{}, 2);
            }
        }
    }
}

template <int G2, bool TAIL>
int launch_down_g(const DnArgs& A, unsigned grid, size_t lds, int layout, hipStream_t st) {
    static const bool attr = set_max_lds(reinterpret_cast<const void*>(&down_kernel<G2, TAIL, kDnRef>)) &&
                             set_max_lds(reinterpret_cast<const void*>(&down_kernel<G2, TAIL, kDnTiled>));
    (void)attr;
    if (layout == kDnTiled)
        hipLaunchKernelGGL((down_kernel<G2, TAIL, kDnTiled>), dim3(grid), dim3(kDnThreads), lds, st, A);
    else
        hipLaunchKernelGGL((down_kernel<G2, TAIL, kDnRef>), dim3(grid), dim3(kDnThreads), lds, st, A);
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

// The (scale, zero) pair table of the tiled layout: per 16-row tile T and
// group g, the 16 rows' (scale | zero << 16) at ((T * G + g) * 16 + col).
__global__ __launch_bounds__(256) void pair_scales_kernel(const uint16_t* __restrict__ s,
                                                          const uint16_t* __restrict__ z, int64_t ntiles, int G,
                                                          uint32_t* __restrict__ out) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= ntiles * G * 16) return;
    const int64_t t = i / (G * 16);
    const int r = static_cast<int>(i - t * G * 16);
    const int g = r >> 4, col = r & 15;
    const int64_t src = (t * 16 + col) * G + g;
    out[i] = static_cast<uint32_t>(s[src]) | (static_cast<uint32_t>(z[src]) << 16);
}

// The tiled down layout from the reference one: one thread per 16-byte unit
// (8-byte tail unit) of the output.
__global__ __launch_bounds__(256) void repack_down_kernel(const uint8_t* __restrict__ src,
                                                           uint8_t* __restrict__ dst, int64_t ntiles, int rb,
                                                           int g2n, int tail) {
    const int per_tile = g2n * kWave + (tail ? kWave : 0);
    const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= ntiles * per_tile) return;
    const int64_t t = i / per_tile;
    const int k = static_cast<int>(i - t * per_tile);
    const uint8_t* tb = src + t * 16 * rb;
    uint8_t* ob = dst + t * 16 * rb;
    if (k < g2n * kWave) {
        const int u = k / kWave, l = k - u * kWave, c = l >> 4, col = l & 15;
        *reinterpret_cast<u32x4*>(ob + u * 1024 + l * 16) =
            *reinterpret_cast<const u32x4*>(tb + col * rb + u * 64 + c * 16);
    } else {
        const int l = k - g2n * kWave, c = l >> 4, col = l & 15;
        *reinterpret_cast<u32x2*>(ob + g2n * 1024 + l * 8) =
            *reinterpret_cast<const u32x2*>(tb + col * rb + g2n * 64 + c * 8);
    }
}

// The MOE_NS down pack back to the reference layout (load time). NS
// (kernels/fused_moe_w4_v2.py:187-197): per expert [I/2, H]; within each
// 64-K chunk kb, byte row kb*32 + j of column n holds q[kb*64 + j] (low
// nibble) and q[kb*64 + 32 + j] (high nibble). Reference: [H, I/2], byte b of
// row n = q[2b] | q[2b+1] << 4. One workgroup per (expert, chunk, 64 columns):
// the chunk's 32 x 64 NS bytes go through LDS; each thread then writes 8
// output bytes (k = 16m .. 16m+15 of one column).
__global__ __launch_bounds__(256) void unshuffle_ns_down_kernel(const uint8_t* __restrict__ ns,
                                                                uint8_t* __restrict__ out, int H, int I) {
    __shared__ uint8_t tile[32][64];
    const int nt = blockIdx.x, kb = blockIdx.y, e = blockIdx.z, t = threadIdx.x;
    const int ih = I / 2;
    const uint8_t* src = ns + (static_cast<int64_t>(e) * ih + kb * 32) * H + nt * 64;
    {
        const int r = t >> 3, c8 = (t & 7) * 8;
        *reinterpret_cast<uint64_t*>(&tile[r][c8]) =
            *reinterpret_cast<const uint64_t*>(src + static_cast<int64_t>(r) * H + c8);
    }
    __syncthreads();
    const int n = t >> 2, m = t & 3;  // column n, output bytes 8m .. 8m+7 of the chunk
    uint64_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int k0 = 2 * (8 * m + i);           // first K index of output byte 8m+i (within the chunk)
        const int hi = k0 >= 32, j = k0 & 31;     // NS row j (and j+1), high nibbles for the second half
        const uint32_t b0 = tile[j][n], b1 = tile[j + 1][n];
        const uint32_t q0 = hi ? b0 >> 4 : b0 & 15u, q1 = hi ? b1 >> 4 : b1 & 15u;
        v |= static_cast<uint64_t>(q0 | (q1 << 4)) << (8 * i);
    }
    *reinterpret_cast<uint64_t*>(out + (static_cast<int64_t>(e) * H + nt * 64 + n) * ih + kb * 32 + 8 * m) = v;
}

// The reference layout to the MOE_NS down pack, preshuffle_T_dn
// (kernels/fused_moe_w4_v2.py:186-197): per expert [I/2, H]; within 64-K
// chunk kb, NS byte row kb*32 + j of column n = q[kb*64 + j] | q[kb*64 + 32 + j] << 4.
// One workgroup per (expert, chunk, 64 columns): the 64 columns' 32-byte
// chunk pieces go through LDS; each thread then writes 8 columns of one NS row.
__global__ __launch_bounds__(256) void preshuffle_ns_down_kernel(const uint8_t* __restrict__ dn,
                                                                 uint8_t* __restrict__ ns, int H, int I) {
    __shared__ uint8_t tile[64][32];
    const int nt = blockIdx.x, kb = blockIdx.y, e = blockIdx.z, t = threadIdx.x;
    const int ih = I / 2;
    {
        const int n = t >> 2, m = t & 3;  // column n, chunk bytes 8m .. 8m+7
        *reinterpret_cast<uint64_t*>(&tile[n][8 * m]) = *reinterpret_cast<const uint64_t*>(
            dn + (static_cast<int64_t>(e) * H + nt * 64 + n) * ih + kb * 32 + 8 * m);
    }
    __syncthreads();
    const int j = t >> 3, n8 = (t & 7) * 8;  // NS row j of the chunk, columns n8 .. n8+7
    const int sh = 4 * (j & 1);
    uint64_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = (static_cast<uint32_t>(tile[n8 + i][j >> 1]) >> sh) & 15u;
        const uint32_t hi = (static_cast<uint32_t>(tile[n8 + i][16 + (j >> 1)]) >> sh) & 15u;
        v |= static_cast<uint64_t>(lo | (hi << 4)) << (8 * i);
    }
    *reinterpret_cast<uint64_t*>(ns + (static_cast<int64_t>(e) * ih + kb * 32 + j) * H + nt * 64 + n8) = v;
}

// Activation rows in plain column order -> the down kernel's activation
// order (out2_store_index): thread i moves 8 consecutive columns of one row.
__global__ __launch_bounds__(256) void act_to_down_order_kernel(const f16* __restrict__ src, int64_t rows, int I,
                                                                f16* __restrict__ dst) {
    const int64_t n8 = I / 8;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= rows * n8) return;
    const int64_t r = idx / n8;
    const int n0 = static_cast<int>(idx - r * n8) * 8;
    const f16x8 v = *reinterpret_cast<const f16x8*>(src + r * I + n0);
    f16* o = dst + r * I;
    const int i128 = I & ~127;
#pragma unroll
    for (int j = 0; j < 8; ++j) o[out2_store_index(n0 + j, i128)] = v[j];
}

}  // namespace

int launch_gateup(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                  const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H,
                  int64_t I, int act, void* out2, hipStream_t st, int64_t nrows_hint) {
    if (!a16 || !sorted_rows || !offsets || !gu_q || !gu_s || !gu_z || !out2) return KSL_ERR_ARG;
    if (E <= 0 || H <= 0 || I <= 0 || topk <= 0) return KSL_ERR_SHAPE;
    if (H % 128 != 0 || I % 64 != 0 || H > 128 * kGuMaxG) return KSL_ERR_SHAPE;
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
    // with at least as many routed rows as experts most experts have rows: the
    // first weight groups go out before the routing is read
    A.early = nrows_hint >= E ? 1 : 0;
    // large routings (a heavy expert gets thousands of rows at prefill): the
    // GEMM-form row-block kernel, 128-row blocks of each expert's rows
    if (act != KSL_ACT_GELU_TANH && act != KSL_ACT_SILU && act != KSL_ACT_NONE) return KSL_ERR_ARG;
    // (gate and up without the activation: the per-expert kernel at every size)
    if (nrows_hint > kRowBlockFrom && act != KSL_ACT_NONE) {
        if (!rb_gateup_fits(H, I)) return KSL_ERR_SHAPE;  // not reached within H <= 4096
        return launch_rb_gateup(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, E, H, I, act, out2, st,
                                nrows_hint);
    }
    // widest column block that divides I: 176 (11 consumers), 128, or 64.
    // One workgroup per expert with 176 columns: 11 consumers and one
    // producer wave (12 waves, 3 per SIMD), ring depth 3
    if (I % 176 == 0) {
        static_assert(GuShape<11, 1, 3>::lds_bytes(kGuMaxG) <= kLdsDynMax, "gate/up LDS");
        // more items than CUs: one persistent workgroup per CU, the ring
        // flowing across its items
        const int64_t items = E * (I / 176);
        const int W = gateup_flow_workgroups(items, H, device_cus());
        if (W > 0) return launch_gateup_flow<11>(A, act, W, static_cast<int>(items), st);
        return launch_gateup_nc<11, 1, 3>(A, E, nrows_hint, act, st);
    }
    if (I % 128 == 0) return launch_gateup_nc<8, 4, 4>(A, E, nrows_hint, act, st);
    return launch_gateup_nc<4, 4, 4>(A, E, nrows_hint, act, st);
}

// Column split of the down launch: each expert's H/16 column tiles go to
// nsplit workgroups of tpw tiles, enough workgroups to fill the CUs.
struct DnPlan {
    int64_t tpw, nsplit;
    size_t lds;
};
DnPlan plan_down(int64_t E, int64_t H, int64_t I, int cus) {
    const int G = static_cast<int>(I / 64);
    const int64_t te = H / 16;  // 16-column tiles per expert
    int64_t nsplit = (cus + E - 1) / E;
    nsplit = std::max<int64_t>(1, std::min<int64_t>(nsplit, te));
    const int64_t tpw = (te + nsplit - 1) / nsplit;
    nsplit = (te + tpw - 1) / tpw;
    return DnPlan{tpw, nsplit, dn_lds_bytes(G)};
}

int launch_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                const void* dn_z, int64_t E, int64_t H, int64_t I, void* out3, hipStream_t st, int layout,
                int64_t nrows) {
    if (!out2 || !offsets || !dn_q || !dn_s || !dn_z || !out3) return KSL_ERR_ARG;
    if (layout != kDnRef && layout != kDnTiled) return KSL_ERR_ARG;
    if (E <= 0 || H <= 0 || I <= 0) return KSL_ERR_SHAPE;
    if (H % 64 != 0 || I % 64 != 0 || I > 64 * kDnMaxG || H >= (1 << 24) || E >= (1 << 24)) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(dn_q) % 16 || reinterpret_cast<uintptr_t>(out2) % 16 ||
        reinterpret_cast<uintptr_t>(dn_s) % 16 || reinterpret_cast<uintptr_t>(dn_z) % 16 ||
        reinterpret_cast<uintptr_t>(out3) % 16)
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
    A.early = nrows >= E ? 1 : 0;
    A.sz = layout == kDnTiled ? reinterpret_cast<const uint32_t*>(dn_q + E * H * (I / 2)) : nullptr;
    // large routings: the GEMM-form row-block kernel (128-row blocks)
    if (nrows > kRowBlockFrom) {
        if (!rb_down_fits(H, I)) return KSL_ERR_SHAPE;  // not reached within the contract above
        return launch_rb_down(out2, offsets, dn_q, dn_s, dn_z, E, H, I, out3, st, layout, nrows);
    }
    const int G = static_cast<int>(I / 64);
    const DnPlan plan = plan_down(E, H, I, device_cus());
    A.tpw = static_cast<int>(plan.tpw);
    A.nsplit = static_cast<int>(plan.nsplit);
    const int64_t grid = E * plan.nsplit;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    const size_t lds = plan.lds;
    switch (G) {
#define KSL_DN_CASE(GG) \
    case GG: return launch_down_g<GG / 2, (GG % 2) != 0>(A, static_cast<unsigned>(grid), lds, layout, st);
        KSL_DN_CASE(1) KSL_DN_CASE(2) KSL_DN_CASE(3) KSL_DN_CASE(4) KSL_DN_CASE(5) KSL_DN_CASE(6)
        KSL_DN_CASE(7) KSL_DN_CASE(8) KSL_DN_CASE(9) KSL_DN_CASE(10) KSL_DN_CASE(11) KSL_DN_CASE(12)
        KSL_DN_CASE(13) KSL_DN_CASE(14) KSL_DN_CASE(15) KSL_DN_CASE(16)
#undef KSL_DN_CASE
        default: return KSL_ERR_SHAPE;
    }
}

}  // namespace ksl

extern "C" int ksl_moe_gateup_act(const void* a16, const int32_t* sorted_rows, const int32_t* offsets,
                                  int64_t T, int64_t topk, const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                                  int64_t E, int64_t H, int64_t I, int act, void* out2, void* stream) {
    return ksl::launch_gateup(a16, sorted_rows, offsets, topk, gu_q, gu_s, gu_z, E, H, I, act, out2,
                              static_cast<hipStream_t>(stream), T > 0 ? T * topk : 0);
}

extern "C" int ksl_moe_act_to_down_order(const void* src, int64_t rows, int64_t I, void* dst, void* stream) {
    using namespace ksl;
    if (rows < 0 || I <= 0 || I % 64 != 0 || I > (int64_t(1) << 20)) return KSL_ERR_SHAPE;
    if (rows == 0) return KSL_OK;
    if (!src || !dst || src == dst) return KSL_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(src) % 16 || reinterpret_cast<uintptr_t>(dst) % 16) return KSL_ERR_ALIGN;
    const int64_t n = rows * (I / 8);
    if ((n + 255) / 256 >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipLaunchKernelGGL(act_to_down_order_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), static_cast<const f16*>(src), rows, static_cast<int>(I),
                       static_cast<f16*>(dst));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

extern "C" int ksl_moe_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q,
                            const void* dn_s, const void* dn_z, int64_t E, int64_t H, int64_t I,
                            int64_t nrows, void* out3, int dn_layout, void* stream) {
    if (nrows < 0) return KSL_ERR_SHAPE;
    return ksl::launch_down(out2, offsets, dn_q, dn_s, dn_z, E, H, I, out3,
                            static_cast<hipStream_t>(stream), dn_layout, nrows);
}

extern "C" size_t ksl_moe_down_lds_bytes(int64_t E, int64_t H, int64_t I, int64_t cus) {
    if (E <= 0 || H <= 0 || I <= 0 || cus <= 0 || H % 16 != 0 || I % 64 != 0 || I > 1024) return 0;
    return ksl::plan_down(E, H, I, static_cast<int>(cus)).lds;
}

extern "C" int ksl_moe_unshuffle_ns_down(const uint8_t* ns_q, int64_t E, int64_t H, int64_t I, uint8_t* dn_q,
                                         void* stream) {
    using namespace ksl;
    if (E <= 0 || H <= 0 || I <= 0 || H % 64 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (E > 65535 || I / 64 > 65535 || H / 64 > (int64_t(1) << 31) - 1) return KSL_ERR_SHAPE;
    if (!ns_q || !dn_q) return KSL_ERR_ARG;
    if (ns_q == dn_q) return KSL_ERR_ARG;  // out of place
    if (reinterpret_cast<uintptr_t>(ns_q) % 8 || reinterpret_cast<uintptr_t>(dn_q) % 8) return KSL_ERR_ALIGN;
    hipLaunchKernelGGL(unshuffle_ns_down_kernel,
                       dim3(static_cast<unsigned>(H / 64), static_cast<unsigned>(I / 64), static_cast<unsigned>(E)),
                       dim3(256), 0, static_cast<hipStream_t>(stream), ns_q, dn_q, static_cast<int>(H),
                       static_cast<int>(I));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

extern "C" int ksl_moe_preshuffle_ns_down(const uint8_t* dn_q, int64_t E, int64_t H, int64_t I, uint8_t* ns_q,
                                          void* stream) {
    using namespace ksl;
    if (E <= 0 || H <= 0 || I <= 0 || H % 64 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (E > 65535 || I / 64 > 65535 || H / 64 > (int64_t(1) << 31) - 1) return KSL_ERR_SHAPE;
    if (!dn_q || !ns_q) return KSL_ERR_ARG;
    if (dn_q == ns_q) return KSL_ERR_ARG;  // out of place
    if (reinterpret_cast<uintptr_t>(dn_q) % 8 || reinterpret_cast<uintptr_t>(ns_q) % 8) return KSL_ERR_ALIGN;
    hipLaunchKernelGGL(preshuffle_ns_down_kernel,
                       dim3(static_cast<unsigned>(H / 64), static_cast<unsigned>(I / 64), static_cast<unsigned>(E)),
                       dim3(256), 0, static_cast<hipStream_t>(stream), dn_q, ns_q, static_cast<int>(H),
                       static_cast<int>(I));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

extern "C" size_t ksl_moe_repack_down_bytes(int64_t E, int64_t H, int64_t I) {
    if (E <= 0 || H <= 0 || I <= 0 || H % 16 != 0 || I % 64 != 0) return 0;
    return static_cast<size_t>(E * H * (I / 2) + E * H * (I / 64) * 4);
}

extern "C" int ksl_moe_repack_down(const uint8_t* dn_q, const void* dn_s, const void* dn_z, int64_t E, int64_t H,
                                   int64_t I, uint8_t* dn_q_tiled, void* stream) {
    using namespace ksl;
    if (E <= 0 || H <= 0 || I <= 0 || H % 16 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (!dn_q || !dn_s || !dn_z || !dn_q_tiled) return KSL_ERR_ARG;
    if (dn_q == dn_q_tiled) return KSL_ERR_ARG;  // out of place
    if (reinterpret_cast<uintptr_t>(dn_q) % 16 || reinterpret_cast<uintptr_t>(dn_q_tiled) % 16 ||
        reinterpret_cast<uintptr_t>(dn_s) % 2 || reinterpret_cast<uintptr_t>(dn_z) % 2)
        return KSL_ERR_ALIGN;
    const int64_t ntiles = E * (H / 16);
    const int g2n = static_cast<int>(I / 128), tail = (I % 128) != 0;
    const int64_t n = ntiles * (g2n * kWave + (tail ? kWave : 0));
    const int64_t grid = (n + 255) / 256;
    const int G = static_cast<int>(I / 64);
    const int64_t gridp = (ntiles * G * 16 + 255) / 256;
    if (grid >= (int64_t(1) << 31) || gridp >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(repack_down_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0, st, dn_q, dn_q_tiled,
                       ntiles, static_cast<int>(I / 2), g2n, tail);
    KSL_LAUNCH_CHECK();
    hipLaunchKernelGGL(pair_scales_kernel, dim3(static_cast<unsigned>(gridp)), dim3(256), 0, st,
                       static_cast<const uint16_t*>(dn_s), static_cast<const uint16_t*>(dn_z), ntiles, G,
                       reinterpret_cast<uint32_t*>(dn_q_tiled + E * H * (I / 2)));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}
