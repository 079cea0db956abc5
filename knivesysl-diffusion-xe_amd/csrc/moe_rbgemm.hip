// Expert GEMMs of large routings (prefill: more than 8192 routed rows) for
// gfx950, in GEMM form: one workgroup per (block of up to 128 rows of one
// expert, block of 256 weight rows), four waves, each wave owning all 128
// rows x 64 weight rows of the block (8 x 4 tiles of v_mfma_f32_16x16x32_f16),
// two workgroups per CU.
//
// Why this shape: with a 16-column tile per wave every MFMA needs its own
// 1 KB activation fragment from LDS, and at prefill the LDS read port, not
// the matrix cores, sets the pace (each CU would need 256 B per clock at
// full MFMA rate). Four weight tiles per activation fragment and eight M
// tiles per decoded weight fragment cut that to ~70 B per clock and spread
// the nibble decode over 32 MFMAs.
//
// Pipeline: per 128-K quantisation group (one slot) the workgroup needs the
// block's activation fragments (8 M tiles x 4 steps x 1 KB), which go into a
// two-slot LDS ring by direct global -> LDS loads, and each wave its own
// weight fragments (4 tiles x 1 KB), loaded straight into registers. Every
// wave issues its share of the next group (its weight tiles, and the
// activation tiles whose index is its wave number) before computing the
// current one, then waits for its own loads and joins one workgroup barrier
// per group; the loads of group g + 1 are in flight while group g's MFMAs run
// (see `stage`). The scales and zero-points of
// the block's 256 weight rows sit in LDS for the whole K loop (fp16 scales,
// zero-points as nibbles, so that the table fits beside the ring).
//
// Numerics: B = fp16((q - z) * s) per weight as the reference dequantises
// (kernels/fused_moe_w4_v2.py:125-128, :172-175), fp32 MFMA accumulation over
// K in group order, each lane group c taking K offsets 32c + 8i of step i:
// the same operands, order and operand roles as the row-chunk kernels of
// moe_gemm.hip, so a row's bits do not depend on which kernel ran it.
//
// Gate/up: wave w owns I columns c0 + 32w .. +32 as tiles (gate 0-15,
// gate 16-31, up 0-15, up 16-31); the activations are the MFMA's A operand,
// the epilogue computes act(gate) * up in fp32 and stores fp16 in out2's
// fragment order. Down: wave w owns H columns c0 + 64w .. +64; the weights
// are the A operand, so each lane holds 4 consecutive output columns of one
// row (one 8-byte store); a trailing 64-K group (I % 128 == 64) takes two
// 4-byte loads per lane.

#include <algorithm>

#include "ksl_common.h"

namespace ksl {
namespace {

constexpr int kRbWaves = 4;
constexpr int kRbThreads = kRbWaves * kWave;
constexpr int kRbMt = 8;                          // 16-row M tiles per row block
constexpr int kRbRows = 16 * kRbMt;               // rows per row block
constexpr int kRbNt = 4;                          // 16-row weight tiles per wave
constexpr int kRbTabRows = kRbWaves * kRbNt * 16; // weight rows per workgroup (256)
constexpr int kRbHalf = kRbTabRows / 2;           // gate/up: gate rows, then as many up rows
constexpr int kRbSlot = kRbMt * 4 * kBlk;         // activation bytes per slot (32 KB)
constexpr size_t kRbLdsMax = 160 * 1024 - 64;     // LDS per workgroup less find_row_block's static LDS

enum RbKind { kRbGateUp = 0, kRbDown = 1 };

struct RbArgs {
    const f16* act;              // gate/up: a16 [T, H], rows gathered by sorted_rows / topk; down: out2 [rows, I]
    const int32_t* sorted_rows;  // gate/up only
    const int32_t* offsets;
    const uint8_t* wq;
    const f16* ws;
    const f16* wz;
    f16* out;                    // gate/up: out2 [rows, I]; down: out3 [rows, H]
    int topk;
    int K;                       // reduction length: H (gate/up) or I (down)
    int N;                       // output columns: I (gate/up) or H (down)
    int E;
    int ncb;                     // column blocks per row block
    int Gs;                      // scale groups per weight row: K / 128 (gate/up) or K / 64 (down)
};

// Scale table (fp16 [256][Gs]) then zero-point nibbles (element j of the
// [256][Gs] order in byte j / 2, low nibble first).
constexpr size_t rb_tab_bytes(int Gs) {
    return static_cast<size_t>(kRbTabRows) * Gs * 2 + static_cast<size_t>(kRbTabRows) * Gs / 2;
}
constexpr size_t rb_lds_bytes(int Gs) { return 2 * static_cast<size_t>(kRbSlot) + rb_tab_bytes(Gs); }

// Direct global -> LDS copy of 4 bytes per lane: lane L lands at lds_block + 4L.
__device__ __forceinline__ void dma4(const void* src, char* lds_block) {
    __builtin_amdgcn_global_load_lds((gbl_vptr)(const_cast<void*>(src)), (lds_vptr)lds_block, 4, 0, 0);
}

// Zero-point pairs from a nibble z: (1024 + z) and (64 + z) as fp16 bits
// (0x6400 | z, 0x5400 | z << 4), both halves of each pair.
__device__ __forceinline__ ZeroPair zero_pair_nib(uint32_t z) {
    const uint32_t lo = 0x6400u | z, hi = 0x5400u | (z << 4);
    return ZeroPair{__builtin_bit_cast(f16x2, lo | (lo << 16)), __builtin_bit_cast(f16x2, hi | (hi << 16))};
}

template <int KIND, int ACT, int LAYOUT>
__global__ __launch_bounds__(kRbThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void rb_gemm_kernel(RbArgs A) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    constexpr int kWc = KIND == kRbGateUp ? 32 : 64;  // output columns per wave
    const int tile = xcd_remap(blockIdx.x, gridDim.x);
    const int unit = tile / A.ncb;
    const int cb = tile - unit * A.ncb;
    int e, start, M;
    find_row_block(A.offsets, A.E, kRbRows, unit, e, start, M);
    if (M <= 0) return;  // past the last row block (uniform)
    M = __builtin_amdgcn_readfirstlane(M);
    start = __builtin_amdgcn_readfirstlane(start);
    e = __builtin_amdgcn_readfirstlane(e);
    const int mt = (M + 15) >> 4;  // M tiles with rows
    const int wave = wave_id();
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int fo = frag_pos(col, c) * 16;
    const int c0 = cb * kRbWaves * kWc;
    const int ncols = std::min(A.N - c0, kRbWaves * kWc);  // a multiple of kWc
    const bool active = wave * kWc < ncols;                // wave-uniform
    const int K = A.K, Gs = A.Gs;
    const int G2 = K >> 7;                                  // full 128-K groups
    const bool has_tail = KIND == kRbDown && (K & 127) != 0;
    const int NS = G2 + (has_tail ? 1 : 0);                 // slots of the K loop
    const int rowbytes = K >> 1;
    char* s_tab_b = lds + 2 * kRbSlot;  // after the two activation slots
    const f16* s_tab = reinterpret_cast<const f16*>(s_tab_b);
    uint8_t* z_tab = reinterpret_cast<uint8_t*>(s_tab_b + kRbTabRows * Gs * 2);

    // ---- weight rows of the workgroup: local row lr (0..255) -> global row
    // gate/up: lr < 128 the gate rows c0 + lr, else the up rows I + c0 + lr - 128
    // down:    the output columns c0 + lr
    const int64_t erow = KIND == kRbGateUp ? static_cast<int64_t>(e) * 2 * A.N : static_cast<int64_t>(e) * A.N;
    // local row of this lane's weight row in tile n
    auto local_row = [&](int n) {
        if constexpr (KIND == kRbGateUp) return (n >= 2 ? kRbHalf : 0) + wave * 32 + (n & 1) * 16 + col;
        else return wave * 64 + n * 16 + col;
    };
    auto global_row = [&](int lr) -> int64_t {
        if constexpr (KIND == kRbGateUp) return erow + (lr >= kRbHalf ? A.N + c0 + lr - kRbHalf : c0 + lr);
        else return erow + c0 + lr;
    };

    // ---- 1. scale / zero-point table: 16-byte chunks of the [256][Gs] order
    {
        const int half = KIND == kRbGateUp ? kRbHalf * Gs : kRbTabRows * Gs;  // elements per contiguous source range
        const int nvalid = ncols * Gs;
        const int nchunks = kRbTabRows * Gs / 8;
        for (int q = tid; q < nchunks; q += kRbThreads) {
            const int el = q * 8;
            const int hsel = el >= half ? 1 : 0;
            const int eo = el - hsel * half;
            u32x4 sv = u32x4{0u, 0u, 0u, 0u};
            uint32_t zb = 0;
            if (eo < nvalid) {
                const int64_t g0 = (global_row(hsel * kRbHalf) * Gs) + eo;  // the range's first row, then eo elements on
                sv = *reinterpret_cast<const u32x4*>(A.ws + g0);
                const f16x8 zv = *reinterpret_cast<const f16x8*>(A.wz + g0);
#pragma unroll
                for (int j = 0; j < 8; ++j) zb |= (static_cast<uint32_t>(static_cast<float>(zv[j])) & 15u) << (4 * j);
            }
            *reinterpret_cast<u32x4*>(s_tab_b + el * 2) = sv;
            *reinterpret_cast<uint32_t*>(z_tab + el / 2) = zb;
        }
    }

    // ---- 2. loads of one group
    // activations: M tiles `wave` and `wave + 4` into the slot (rows past the
    // block repeat its last row: loaded, never stored)
    const char* arow[2] = {nullptr, nullptr};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int t = wave + h * kRbWaves;
        if (t < mt) {
            int r = t * 16 + rr;
            if (r >= M) r = M - 1;
            int64_t row;
            if constexpr (KIND == kRbGateUp)
                row = A.sorted_rows[start + r] / A.topk;
            else
                row = start + r;
            arow[h] = reinterpret_cast<const char*>(A.act) + (row * K + ch * 8) * 2;
        }
    }
    auto issue_act_p = [&](int g, char* base) {
        const int nst = has_tail && g == G2 ? 2 : 4;  // the 64-K tail group has two steps
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int t = wave + h * kRbWaves;
            if (t < mt) {
                for (int i = 0; i < nst; ++i) dma16(arow[h] + (g * 128 + i * 32) * 2, base + (t * 4 + i) * kBlk);
            }
        }
    };
    auto issue_act = [&](int g, int slot) { issue_act_p(g, lds + slot * kRbSlot); };
    // weights: this lane's 16 bytes of each of its 4 tiles for one 128-K
    // group, straight into registers (lane (col, c): row col, K 32c .. +32);
    // the tail group's 8 bytes (K 16c .. +16)
    const uint8_t* wl[kRbNt];
#pragma unroll
    for (int n = 0; n < kRbNt; ++n) {
        const int lr0 = KIND == kRbGateUp ? (n >= 2 ? kRbHalf : 0) + wave * 32 + (n & 1) * 16 : wave * 64 + n * 16;
        const uint8_t* tb = A.wq + global_row(lr0) * rowbytes;  // the tile's first byte
        wl[n] = LAYOUT == KSL_DN_LAYOUT_TILED ? tb + lane * 16 : tb + col * rowbytes + c * 16;
    }
    auto load_w = [&](int g, u32x4 (&w)[kRbNt]) {
#pragma unroll
        for (int n = 0; n < kRbNt; ++n)
            w[n] = *reinterpret_cast<const u32x4*>(wl[n] + (LAYOUT == KSL_DN_LAYOUT_TILED ? g * 1024 : g * 64));
    };
    auto load_w_tail = [&](u32x2 (&w)[kRbNt]) {
#pragma unroll
        for (int n = 0; n < kRbNt; ++n) {
            const uint8_t* p = LAYOUT == KSL_DN_LAYOUT_TILED ? wl[n] - lane * 16 + G2 * 1024 + lane * 8
                                                             : wl[n] - c * 16 + G2 * 64 + c * 8;
            w[n] = *reinterpret_cast<const u32x2*>(p);
        }
    };

    // ---- 3. K loop and epilogue
    const NibConsts kn = nib_consts();
    int tix[kRbNt];
#pragma unroll
    for (int n = 0; n < kRbNt; ++n) tix[n] = local_row(n) * Gs;

    // FULL: all eight M tiles have rows (no per-tile guards, so a step's
    // activation fragments can be read ahead of its MFMAs). The two forms
    // are separate loops, each with its own accumulators.
    auto run = [&](auto full_c) {
        constexpr bool FULL = decltype(full_c)::value;
        f32x4 acc[kRbMt][kRbNt];
#pragma unroll
        for (int t = 0; t < kRbMt; ++t)
#pragma unroll
            for (int n = 0; n < kRbNt; ++n) acc[t][n] = f32x4{0.f, 0.f, 0.f, 0.f};
        // one slot's MFMAs; wv[n][i]: tile n's weight word of step i
        auto compute_p = [&](int g, const char* sp, const auto& wv, auto nstep_c) {
            constexpr int NSTEP = decltype(nstep_c)::value;
            const bool tail = NSTEP == 2;
            // this lane's scale group in slot g
            const int gs = KIND == kRbGateUp ? g : (tail ? 2 * G2 : 2 * g + (c >> 1));
            f16x2 sc[kRbNt];
            ZeroPair zc[kRbNt];
#pragma unroll
            for (int n = 0; n < kRbNt; ++n) {
                const int idx = tix[n] + gs;
                const f16 sv = s_tab[idx];
                sc[n] = f16x2{sv, sv};
                zc[n] = zero_pair_nib((z_tab[idx >> 1] >> ((idx & 1) * 4)) & 15u);
            }
            {
#pragma unroll
                for (int i = 0; i < NSTEP; ++i) {
                    f16x8 b[kRbNt];
#pragma unroll
                    for (int n = 0; n < kRbNt; ++n) b[n] = nib8_dequant(wv[n][i], zc[n], sc[n], kn);
                    if constexpr (FULL) {
                        // Activation fragments read one M tile ahead of their
                        // MFMAs, by asm: with the accumulators, the weights and
                        // the decoded fragments in registers the compiler keeps
                        // one fragment register and waits for each read right
                        // before its MFMAs. Each read's destination is left
                        // untouched until the wait before its use (checked on
                        // the generated code by tests/test_cpu_codegen.py).
                        const uint32_t ap = static_cast<uint32_t>(
                            reinterpret_cast<uintptr_t>((lds_vptr)const_cast<char*>(sp + i * kBlk + fo)));
                        f16x8 a;
                        asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(a) : "v"(ap) : "memory");
#pragma unroll
                        for (int t = 0; t < kRbMt; ++t) {
                            f16x8 an;
                            if (t + 1 < kRbMt)
                                asm volatile("ds_read_b128 %0, %1 offset:%2 ; ksl-ahead"
                                             : "=v"(an)
                                             : "v"(ap), "i"((t + 1) * 4 * kBlk)
                                             : "memory");
#pragma unroll
                            for (int n = 0; n < kRbNt; ++n) {
                                if constexpr (KIND == kRbGateUp)
                                    acc[t][n] = mfma16x16x32(a, b[n], acc[t][n]);
                                else
                                    acc[t][n] = mfma16x16x32(b[n], a, acc[t][n]);
                            }
                            if (t + 1 < kRbMt) {
                                __builtin_amdgcn_sched_barrier(0);
                                asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(an) : : "memory");
                                a = an;
                            }
                        }
                    } else
#pragma unroll
                    for (int t = 0; t < kRbMt; ++t) {
                        if (t < mt) {
                            const f16x8 a = *reinterpret_cast<const f16x8*>(sp + (t * 4 + i) * kBlk + fo);
#pragma unroll
                            for (int n = 0; n < kRbNt; ++n) {
                                if constexpr (KIND == kRbGateUp)
                                    acc[t][n] = mfma16x16x32(a, b[n], acc[t][n]);
                                else
                                    acc[t][n] = mfma16x16x32(b[n], a, acc[t][n]);
                            }
                        }
                    }
                    // one step's fragments at a time (hoisting the next step's
                    // reads as well would exceed the register budget)
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        };
        auto compute = [&](int g, const auto& wv, auto nstep_c) { compute_p(g, lds + (g & 1) * kRbSlot, wv, nstep_c); };
        // One group of the K loop: the next slot's direct-to-LDS loads, the
        // next group's weights, this slot's MFMAs. The compiler makes an LDS
        // read wait (vmcnt) for every outstanding direct-to-LDS load it cannot
        // tell apart from it; issued and read through two restrict pointers of
        // one inlined call, they carry disjoint alias scopes and the reads of
        // slot g run while slot g + 1 and the weights of group g + 1 are in
        // flight. (With the slot pointers computed in place, the generated
        // code waited for all of them before the first read: load and compute
        // ran one after the other.)
        auto stage = [&](int g, char* __restrict__ dst, const char* __restrict__ src, auto& wc_, auto& wn_) {
            if (g + 1 < NS) issue_act_p(g + 1, dst);
            if (active) {
                if (g + 1 < G2) load_w(g + 1, wn_);
                compute_p(g, src, wc_, std::integral_constant<int, 4>{});
            }
        };
        // weights one group ahead in registers, activations one group ahead
        // in the LDS ring; each wave waits for its own loads, then one
        // barrier per group publishes the slot and frees the other one
        u32x4 wc[kRbNt], wn[kRbNt] = {};
        u32x2 wt[kRbNt];
        issue_act(0, 0);
        // the tail group's weights with the first group's, held in registers
        // through the loop: a load of them inside the loop made the compiler
        // copy (and so wait for) the buffer on every trip
        if (active) {
            if (G2 > 0) load_w(0, wc);
            if (has_tail) load_w_tail(wt);
        }
        vm_wait<0>();
        __syncthreads();  // group 0 and the table are in LDS
        for (int g = 0; g < G2; ++g) {
            stage(g, lds + ((g + 1) & 1) * kRbSlot, lds + (g & 1) * kRbSlot, wc, wn);
            vm_wait<0>();     // this wave's loads of group g + 1 have landed
            __syncthreads();  // everyone's have, and slot g is free
#pragma unroll
            for (int n = 0; n < kRbNt; ++n) wc[n] = wn[n];
        }
        if (!active) return;
        if (has_tail) compute(G2, wt, std::integral_constant<int, 2>{});

        // epilogue (rows past the block take an out-of-range offset: dropped)
        const __amdgpu_buffer_rsrc_t out =
            raw_rsrc(A.out + static_cast<int64_t>(start) * A.N, static_cast<uint32_t>(M * A.N * 2));
        if constexpr (KIND == kRbGateUp) {
            // lane (col, c): I column c0 + 32w + 16n + col (n = 0, 1), rows 16t + 4c + q
            const int i128 = A.N & ~127;
#pragma unroll
            for (int n = 0; n < 2; ++n) {
                const int sci = out2_store_index(c0 + wave * 32 + n * 16 + col, i128);
#pragma unroll
                for (int t = 0; t < kRbMt; ++t) {
                    if (FULL || t < mt) {
#pragma unroll
                        for (int q = 0; q < 4; ++q) {
                            const int row = t * 16 + 4 * c + q;
                            const uint32_t off = row < M ? static_cast<uint32_t>((row * A.N + sci) * 2) : kDropOffset;
                            const f16 v = static_cast<f16>(act_times_up_fast<ACT>(acc[t][n][q], acc[t][n + 2][q]));
                            __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, v), out, off, 0, 0);
                        }
                    }
                }
            }
        } else {
            // lane (col, c): row 16t + col, output columns c0 + 64w + 16n + 4c .. +4
#pragma unroll
            for (int t = 0; t < kRbMt; ++t) {
                if (FULL || t < mt) {
                    const int row = t * 16 + col;
#pragma unroll
                    for (int n = 0; n < kRbNt; ++n) {
                        const uint32_t off =
                            row < M ? static_cast<uint32_t>((row * A.N + c0 + wave * 64 + n * 16 + 4 * c) * 2)
                                    : kDropOffset;
                        const f16x4 v{static_cast<f16>(acc[t][n][0]), static_cast<f16>(acc[t][n][1]),
                                      static_cast<f16>(acc[t][n][2]), static_cast<f16>(acc[t][n][3])};
                        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, v), out, off, 0, 0);
                    }
                }
            }
        }
    };

    if (mt == kRbMt)
        run(std::true_type{});
    else
        run(std::false_type{});
}

template <int KIND, int ACT, int LAYOUT>
int rb_launch(const RbArgs& A, int64_t nrows, hipStream_t st) {
    static const bool attr = [] {
        const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(&rb_gemm_kernel<KIND, ACT, LAYOUT>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize,
                                            static_cast<int>(kRbLdsMax)) == hipSuccess;
        (void)hipGetLastError();
        return ok;
    }();
    (void)attr;
    // row blocks: at most ceil(nrows / 128) + E of them (one partial block per expert)
    const int64_t units = (nrows + kRbRows - 1) / kRbRows + A.E;
    const int64_t grid = units * A.ncb;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipLaunchKernelGGL((rb_gemm_kernel<KIND, ACT, LAYOUT>), dim3(static_cast<unsigned>(grid)), dim3(kRbThreads),
                       rb_lds_bytes(A.Gs), st, A);
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

}  // namespace

// Whether the row-block GEMM kernels take a shape (the caller checked the
// common contract: H % 128 == 0, I % 64 == 0, alignment). Gate/up needs
// I % 32 == 0 and a scale table that fits beside the ring (H <= 3200);
// down needs H % 64 == 0 and I <= 1024.
bool rb_gateup_fits(int64_t H, int64_t I) {
    const int64_t Gs = H / 128;
    return I % 32 == 0 && H % 128 == 0 && rb_lds_bytes(static_cast<int>(Gs)) <= kRbLdsMax;
}
bool rb_down_fits(int64_t H, int64_t I) {
    const int64_t Gs = I / 64;
    return H % 64 == 0 && I % 64 == 0 && Gs <= 16 && rb_lds_bytes(static_cast<int>(Gs)) <= kRbLdsMax;
}

// out2 rows [offsets[0], offsets[E]) = act(a16[rows] gate) * up, row blocks of 128.
int launch_rb_gateup(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
                     const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H, int64_t I,
                     int act, void* out2, hipStream_t st, int64_t nrows) {
    RbArgs A;
    A.act = static_cast<const f16*>(a16);
    A.sorted_rows = sorted_rows;
    A.offsets = offsets;
    A.wq = gu_q;
    A.ws = static_cast<const f16*>(gu_s);
    A.wz = static_cast<const f16*>(gu_z);
    A.out = static_cast<f16*>(out2);
    A.topk = static_cast<int>(topk);
    A.K = static_cast<int>(H);
    A.N = static_cast<int>(I);
    A.E = static_cast<int>(E);
    A.ncb = static_cast<int>((I + kRbWaves * 32 - 1) / (kRbWaves * 32));
    A.Gs = static_cast<int>(H / 128);
    if (act == KSL_ACT_GELU_TANH) return rb_launch<kRbGateUp, KSL_ACT_GELU_TANH, KSL_DN_LAYOUT_REF>(A, nrows, st);
    if (act == KSL_ACT_SILU) return rb_launch<kRbGateUp, KSL_ACT_SILU, KSL_DN_LAYOUT_REF>(A, nrows, st);
    return KSL_ERR_ARG;
}

// out3 rows [offsets[0], offsets[E]) = out2[rows] x dn^T, row blocks of 128.
int launch_rb_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                   const void* dn_z, int64_t E, int64_t H, int64_t I, void* out3, hipStream_t st, int layout,
                   int64_t nrows) {
    RbArgs A;
    A.act = static_cast<const f16*>(out2);
    A.sorted_rows = nullptr;
    A.offsets = offsets;
    A.wq = dn_q;
    A.ws = static_cast<const f16*>(dn_s);
    A.wz = static_cast<const f16*>(dn_z);
    A.out = static_cast<f16*>(out3);
    A.topk = 1;
    A.K = static_cast<int>(I);
    A.N = static_cast<int>(H);
    A.E = static_cast<int>(E);
    A.ncb = static_cast<int>((H + kRbWaves * 64 - 1) / (kRbWaves * 64));
    A.Gs = static_cast<int>(I / 64);
    if (layout == KSL_DN_LAYOUT_TILED) return rb_launch<kRbDown, 0, KSL_DN_LAYOUT_TILED>(A, nrows, st);
    return rb_launch<kRbDown, 0, KSL_DN_LAYOUT_REF>(A, nrows, st);
}

}  // namespace ksl
