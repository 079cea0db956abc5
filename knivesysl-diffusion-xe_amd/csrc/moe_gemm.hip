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
//   - down: each wave streams its 16-column weight tiles through two register
//     buffers with explicit vmcnt waits.
//
// Work split: one workgroup per (expert, column block) walks all rows routed
// to its expert (sorted slots offsets[e] .. offsets[e+1]) in chunks of up to 32
// rows for gate/up (one or two 16-row M tiles) and 64 rows for down. Above
// 8192 routed rows both GEMMs run the GEMM-form row-block kernels of
// moe_rbgemm.hip instead. Workgroups are remapped so that all column blocks
// of an expert run on the same XCD (shared L2 for its activations).

#include <algorithm>
#include <atomic>
#include <type_traits>

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

// Consumer side of one row chunk: 1 + G barriers, matching gateup_produce.
template <int ACT, int NC, int NP, int R, int MT>
__device__ __forceinline__ void gateup_consume(const GuArgs& A, int c0, const char* __restrict__ lds,
                                               const f16* __restrict__ lds_sz, int start, int m0, int mrows) {
    using S = GuShape<NC, NP, R>;
    const int wave = wave_id();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int G = A.H >> 7;
    const NibConsts kn = nib_consts();
    const int kc = S::kCols;
    const f16* s_g = lds_sz;
    const f16* z_g = lds_sz + kc * G;
    const f16* s_u = lds_sz + 2 * kc * G;
    const f16* z_u = lds_sz + 3 * kc * G;
    const int r = wave * 16 + col;  // row of the tile within the workgroup
    const int fo = frag_pos(col, c) * 16;
    f32x4 acc[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();  // group 0 and the scale table are ready
    int slot = 0;
    for (int g = 0; g < G; ++g) {
        const char* sp = lds + slot * S::kSlot;
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
            for (int t = 0; t < MT; ++t)
                a[t] = *reinterpret_cast<const f16x8*>(sp + S::kSlotW + (t * 4 + i) * kBlk + fo);
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
        slot = slot + 1 == R ? 0 : slot + 1;
        __syncthreads();
    }
    // epilogue: column c0 + wave*16 + col, gate tile 0 with up tile 1
    if (ACT == KSL_ACT_NONE) {
        // gate and up themselves, fp16, in plain column order: out1 [rows, 2I]
        const int64_t ld = 2 * static_cast<int64_t>(A.I);
        f16* o = A.out2 + (static_cast<int64_t>(start + m0) + 4 * c) * ld + c0 + wave * 16 + col;
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
        f16* o = A.out2 + (static_cast<int64_t>(start + m0) + 4 * c) * A.I + sc;
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

// --------------------------------------------------------------------- down
// Register-streamed kernel. A workgroup of kDnWaves waves owns one expert and
// a range of its output columns (the expert's H columns split over
// ceil(#CUs / E) workgroups); the expert's activation rows (out2, up to 64 per
// chunk) and the scale / zero rows of the workgroup's columns are copied into
// LDS once (direct global->LDS loads), so each activation row is read once
// per workgroup. Every wave then walks its 16-column tiles (tiles w, w+12, ...)
// with the weights in registers, double buffered: the next tile's 16 rows x
// I/2 bytes are loaded while the current tile is decoded and multiplied, and
// all waves do MFMA and nibble decoding (down's decode, with the scale folded
// in, costs as much VALU time as the bytes take to stream).
//
// K mapping: one 16-byte load per lane and 128-K block, lane (col, c) holding
// row col, nibbles 32c .. 32c+31 of the block: MFMA step i takes nibbles
// 32c + 8i .. +8, the 128-group activation order (out2_store_index); the scale
// group of lane group c is 2*g2 + c/2. A trailing 64-K group (I % 128 == 64)
// takes an 8-byte load, the 64-group order. B = fp16((q - z) * s), the
// reference's own dequantised weight (kernels/fused_moe_w4_v2.py:172-175).
constexpr int kDnWaves = 12;
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
    int H, I, nsplit, tpw;  // tpw: 16-column tiles per workgroup
};

// LDS: activation blocks [kDnMaxMt][2G] (1 KB each, frag_pos order), then the
// s rows and the z rows ([nrows][G] fp16 each) of the workgroup's columns.
inline size_t dn_lds_bytes(int G, int nrows) {
    return static_cast<size_t>(kDnMaxMt) * 2 * G * kBlk + static_cast<size_t>(nrows) * G * 4;
}

template <int G2, bool TAIL>
struct DnW {
    u32x4 q[G2];
    u32x2 t[TAIL ? 1 : 0];
};

// A tile's weights: G2 16-byte loads and, with TAIL, one 8-byte load. Issued
// as asm so that the compiler's conservative wait at the tile loop's head
// (vmcnt(0), which would drain the next tile's prefetch) is not inserted; the
// waits are explicit (dn_wait_w), the compiler-placed ones can only wait more.
// The compiler takes the registers as written at the asm: nothing may copy
// them before dn_wait_w, so a buffer enters the tile loop only once complete
// and is otherwise loaded and used inside one loop iteration pair (checked in
// the generated code: no register copies of a loading buffer).
template <int G2, bool TAIL, int LAYOUT>
__device__ __forceinline__ void dn_load_w(DnW<G2, TAIL>& w, const uint8_t* tbase, int col, int c, int rb) {
    if constexpr (LAYOUT == kDnTiled) {
        // non-temporal: each weight byte is read once per launch (about 1 us
        // faster at the 256-token layer than the cached load; the same hint on
        // gate/up's direct-to-LDS loads costs 15 us there)
        const uint8_t* p = tbase + (c * 16 + col) * 16;
#pragma unroll
        for (int g2 = 0; g2 < G2; ++g2)
            asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(w.q[g2]) : "v"(p + g2 * 1024) : "memory");
        if constexpr (TAIL) {
            const uint8_t* pt = tbase + G2 * 1024 + (c * 16 + col) * 8;
            asm volatile("global_load_dwordx2 %0, %1, off nt" : "=v"(w.t[0]) : "v"(pt) : "memory");
        }
    } else {
        const uint8_t* p = tbase + col * rb + c * 16;
#pragma unroll
        for (int g2 = 0; g2 < G2; ++g2)
            asm volatile("global_load_dwordx4 %0, %1, off offset:%2" : "=v"(w.q[g2]) : "v"(p), "i"(g2 * 64) : "memory");
        if constexpr (TAIL) {
            const uint8_t* pt = tbase + col * rb + G2 * 64 + c * 8;
            asm volatile("global_load_dwordx2 %0, %1, off nt" : "=v"(w.t[0]) : "v"(pt) : "memory");
        }
    }
}

// Wait until the loads of w have landed, N memory operations issued after
// them allowed in flight; the empty asm orders every use of w after the wait.
template <int N, int G2, bool TAIL>
__device__ __forceinline__ void dn_wait_w(DnW<G2, TAIL>& w) {
    vm_wait<N>();
#pragma unroll
    for (int g2 = 0; g2 < G2; ++g2) asm volatile("" : "+v"(w.q[g2]));
    if constexpr (TAIL) asm volatile("" : "+v"(w.t[0]));
}

template <int G2, bool TAIL, int MT>
__device__ __forceinline__ void dn_tile(const DnW<G2, TAIL>& w, f32x4 (&acc)[MT], const char* __restrict__ a_lds,
                                        const f16* __restrict__ srow, const f16* __restrict__ zrow, int c, int fo,
                                        const NibConsts& kn) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
#pragma unroll
    for (int g2 = 0; g2 < G2; ++g2) {
        const int grp = 2 * g2 + (c >> 1);
        const f16 sv = srow[grp];
        const ZeroPair zc = zero_pair(zrow[grp]);
        // decode here, not where the load lands (decoded nibbles take 4x the registers)
        u32x4 wq = w.q[g2];
        asm volatile("" : "+v"(wq));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16x8 b = nib8_dequant(wq[i], zc, f16x2{sv, sv}, kn);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(a_lds + (t * 2 * G + g2 * 4 + i) * kBlk + fo);
                acc[t] = mfma16x16x32(b, a, acc[t]);
            }
        }
        // one 128-K block at a time: the other waves hide its LDS latency, and
        // hoisting every block's operands would exceed the register budget
        __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (TAIL) {
        const f16 sv = srow[2 * G2];
        const ZeroPair zc = zero_pair(zrow[2 * G2]);
        u32x2 wt = w.t[0];
        asm volatile("" : "+v"(wt));
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const f16x8 b = nib8_dequant(wt[i], zc, f16x2{sv, sv}, kn);
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                const f16x8 a = *reinterpret_cast<const f16x8*>(a_lds + (t * 2 * G + G2 * 4 + i) * kBlk + fo);
                acc[t] = mfma16x16x32(b, a, acc[t]);
            }
        }
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



// One tile: MT M tiles x 16 columns. The weights are the MFMA's A operand and
// the activations its B operand, so the accumulator is the tile transposed:
// lane (col, c) holds row col of the M tile, output columns 4c .. 4c+3, and
// writes them with one 8-byte store (out3 is 8-byte aligned, H % 64 == 0).
// The stores have no branches (rows past the chunk, or a
// repeated tile, take an out-of-range offset), so every wave issues the same
// number of memory operations per tile and the waits on the prefetched
// weights are exact.
template <int G2, bool TAIL, int MT>
__device__ __forceinline__ void dn_do_tile(const DnW<G2, TAIL>& w, const char* a_lds, const f16* s_lds,
                                           const f16* z_lds, __amdgpu_buffer_rsrc_t out, int H, int tile,
                                           int colw, bool valid, int mrows, int col, int c, int fo,
                                           const NibConsts& kn) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    f32x4 acc[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int rl = tile * 16 + col;  // row of dn within the workgroup's columns
    dn_tile<G2, TAIL, MT>(w, acc, a_lds, s_lds + rl * G, z_lds + rl * G, c, fo, kn);
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const int row = t * 16 + col;
        const uint32_t off = valid && row < mrows ? static_cast<uint32_t>((row * H + colw + tile * 16 + 4 * c) * 2)
                                                  : kDropOffset;
        const f16x4 v{static_cast<f16>(acc[t][0]), static_cast<f16>(acc[t][1]), static_cast<f16>(acc[t][2]),
                      static_cast<f16>(acc[t][3])};
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), out, off, 0, 0);
    }
}

// A wave's tiles of one chunk: tiles wave + k*kDnWaves, k < nmine, weights of
// tile k+1 loaded while tile k is computed. Loads are unconditional (past the
// last tile they repeat it: an L2 hit), a repeated tile's stores are dropped,
// so between a buffer's loads and its use exactly the other buffer's loads and
// one tile's MT stores are issued (on entry w0 has landed already).
template <int G2, bool TAIL, int MT, int LAYOUT>
__device__ __forceinline__ void dn_tiles(DnW<G2, TAIL>& w0, DnW<G2, TAIL>& w1, const uint8_t* wrow, int rb,
                                         int nmine, int wave, const char* a_lds, const f16* s_lds,
                                         const f16* z_lds, __amdgpu_buffer_rsrc_t out, int H, int colw, int mrows,
                                         int col, int c, int fo, const NibConsts& kn) {
    constexpr int kAfter = G2 + (TAIL ? 1 : 0) + MT;
    for (int k = 0; k < nmine; k += 2) {
        const int k1 = k + 1 < nmine ? k + 1 : nmine - 1;
        const int k2 = k + 2 < nmine ? k + 2 : nmine - 1;
        dn_load_w<G2, TAIL, LAYOUT>(w1, wrow + static_cast<int64_t>(wave + k1 * kDnWaves) * 16 * rb, col, c, rb);
        dn_wait_w<kAfter>(w0);
        dn_do_tile<G2, TAIL, MT>(w0, a_lds, s_lds, z_lds, out, H, wave + k * kDnWaves, colw, true, mrows, col, c,
                                 fo, kn);
        // odd count: tile k was the wave's last. w1's repeated load is waited
        // for here, so its registers stay w1's until it has landed
        // (wave-uniform branch)
        if (k + 1 >= nmine) {
            dn_wait_w<0>(w1);
            break;
        }
        dn_load_w<G2, TAIL, LAYOUT>(w0, wrow + static_cast<int64_t>(wave + k2 * kDnWaves) * 16 * rb, col, c, rb);
        dn_wait_w<kAfter>(w1);
        dn_do_tile<G2, TAIL, MT>(w1, a_lds, s_lds, z_lds, out, H, wave + k1 * kDnWaves, colw, k + 1 < nmine, mrows,
                                 col, c, fo, kn);
    }
}

template <int G2, bool TAIL, int LAYOUT>
__global__ __launch_bounds__(kDnThreads) void down_kernel(DnArgs A) {
    constexpr int G = 2 * G2 + (TAIL ? 1 : 0);
    // M tiles per chunk: four need more than the 168 registers of 12 waves
    // once a tile's weights take G2 >= 6 128-K units (I >= 768)
    constexpr int MTX = G2 >= 6 ? 2 : kDnMaxMt;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int bid = xcd_remap(blockIdx.x, gridDim.x);
    const int e = bid / A.nsplit;
    const int h = bid - e * A.nsplit;
    const int start = A.offsets[e];
    const int M = A.offsets[e + 1] - start;
    const int col0 = h * A.tpw * 16;
    const int ncols = A.H - col0 < A.tpw * 16 ? A.H - col0 : A.tpw * 16;
    if (M <= 0 || ncols <= 0) return;
    const int ntiles = ncols >> 4;
    const int wave = wave_id();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int fo = frag_pos(col, c) * 16;
    const NibConsts kn = nib_consts();
    char* a_lds = lds;
    f16* s_lds = reinterpret_cast<f16*>(lds + kDnMaxMt * 2 * G * kBlk);
    f16* z_lds = s_lds + ncols * G;
    const int64_t row0 = static_cast<int64_t>(e) * A.H + col0;  // first dn row of the workgroup
    const int rb = A.I >> 1;
    const uint8_t* wrow = A.dn_q + row0 * rb;  // the workgroup's first tile
    // 1. scale / zero rows and the first chunk's activations into LDS
    {
        const int nq = ncols * G / 8;  // 16-byte chunks per block
        const char* ssrc = reinterpret_cast<const char*>(A.dn_s + row0 * G);
        const char* zsrc = reinterpret_cast<const char*>(A.dn_z + row0 * G);
        for (int q0 = wave * kWave; q0 < 2 * nq; q0 += kDnWaves * kWave) {
            const int q = q0 + lane;
            if (q < 2 * nq) dma16(q < nq ? ssrc + q * 16 : zsrc + (q - nq) * 16, reinterpret_cast<char*>(s_lds) + q0 * 16);
        }
        const int mrows = M < 16 * MTX ? M : 16 * MTX;
        dn_stage_a<G2, TAIL>(A, a_lds, start, 0, mrows, (mrows + 15) >> 4, wave, rr, ch);
    }
    // 2. the first tile's weights, then wait for the LDS copies only
    DnW<G2, TAIL> w0, w1;
    if (wave < ntiles) dn_load_w<G2, TAIL, LAYOUT>(w0, wrow + static_cast<int64_t>(wave) * 16 * rb, col, c, rb);
    vm_wait<0>();
    dma_barrier();
    const int nmine = wave < ntiles ? (ntiles - 1 - wave) / kDnWaves + 1 : 0;
    for (int m0 = 0; m0 < M; m0 += 16 * MTX) {
        const int mrows = M - m0 < 16 * MTX ? M - m0 : 16 * MTX;
        const int mt = (mrows + 15) >> 4;
        if (m0 > 0) {
            __syncthreads();  // every wave is done with the previous chunk's activations
            dn_stage_a<G2, TAIL>(A, a_lds, start, m0, mrows, mt, wave, rr, ch);
            if (wave < ntiles) dn_load_w<G2, TAIL, LAYOUT>(w0, wrow + static_cast<int64_t>(wave) * 16 * rb, col, c, rb);
            vm_wait<0>();
            dma_barrier();
        }
        const __amdgpu_buffer_rsrc_t out =
            raw_rsrc(A.out3 + static_cast<int64_t>(start + m0) * A.H, static_cast<uint32_t>(mrows * A.H * 2));
#define KSL_DN_TILES(MT_)                                                                                      \
    dn_tiles<G2, TAIL, MT_, LAYOUT>(w0, w1, wrow, rb, nmine, wave, a_lds, s_lds, z_lds, out, A.H, col0, mrows, col, c, \
                                    fo, kn)
        if (mt == 1) {
            KSL_DN_TILES(1);
        } else if (MTX == 2 || mt == 2) {
            KSL_DN_TILES(2);
        } else if constexpr (MTX == 4) {
            if (mt == 3) KSL_DN_TILES(3);
            else KSL_DN_TILES(4);
        }
#undef KSL_DN_TILES
    }
    vm_wait<0>();  // the last (repeated) prefetch lands before the wave ends
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
        return launch_gateup_nc<11, 1, 3>(A, E, nrows_hint, act, st);
    }
    if (I % 128 == 0) return launch_gateup_nc<8, 4, 4>(A, E, nrows_hint, act, st);
    return launch_gateup_nc<4, 4, 4>(A, E, nrows_hint, act, st);
}

// Column split of the down launch: each expert's H/16 column tiles go to
// nsplit workgroups of tpw tiles, enough workgroups to fill the CUs and few
// enough tiles that their scale / zero rows fit in LDS beside the
// activations (the static LDS reserved).
struct DnPlan {
    int64_t tpw, nsplit;
    size_t lds;
};
DnPlan plan_down(int64_t E, int64_t H, int64_t I, int cus) {
    const int G = static_cast<int>(I / 64);
    const int64_t te = H / 16;  // 16-column tiles per expert
    const int64_t max_tiles = static_cast<int64_t>((kLdsDynMax - dn_lds_bytes(G, 0)) / (static_cast<size_t>(16) * G * 4));
    int64_t nsplit = std::max<int64_t>((cus + E - 1) / E, (te + max_tiles - 1) / max_tiles);
    nsplit = std::max<int64_t>(1, std::min<int64_t>(nsplit, te));
    const int64_t tpw = (te + nsplit - 1) / nsplit;
    nsplit = (te + tpw - 1) / tpw;
    return DnPlan{tpw, nsplit, dn_lds_bytes(G, static_cast<int>(tpw * 16))};
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
        reinterpret_cast<uintptr_t>(out3) % 8)
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

extern "C" int ksl_moe_repack_down(const uint8_t* dn_q, int64_t E, int64_t H, int64_t I, uint8_t* dn_q_tiled,
                                   void* stream) {
    using namespace ksl;
    if (E <= 0 || H <= 0 || I <= 0 || H % 16 != 0 || I % 64 != 0) return KSL_ERR_SHAPE;
    if (!dn_q || !dn_q_tiled) return KSL_ERR_ARG;
    if (dn_q == dn_q_tiled) return KSL_ERR_ARG;  // out of place
    if (reinterpret_cast<uintptr_t>(dn_q) % 16 || reinterpret_cast<uintptr_t>(dn_q_tiled) % 16) return KSL_ERR_ALIGN;
    const int64_t ntiles = E * (H / 16);
    const int g2n = static_cast<int>(I / 128), tail = (I % 128) != 0;
    const int64_t n = ntiles * (g2n * kWave + (tail ? kWave : 0));
    const int64_t grid = (n + 255) / 256;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipLaunchKernelGGL(repack_down_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dn_q, dn_q_tiled, ntiles, static_cast<int>(I / 2), g2n,
                       tail);
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}
