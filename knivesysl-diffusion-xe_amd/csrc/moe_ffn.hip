// The expert feed-forward of a small routing (at most 8192 routed rows) as ONE
// persistent launch: gate/up + activation and down for every expert, fed from
// the "pack" weight layout that ksl_moe_pack_gateup / ksl_moe_pack_down write
// at load time. Replaces the _gateup_act_kernel and _down_kernel launches of
// kernels/fused_moe_w4_v2.py:351-366 (same values: the accumulation order of
// every output element is that of the separate gate/up and down kernels of
// moe_gemm.hip, so out2 and out3 are bit-identical to theirs).
//
// Why one launch: at a 256-token canvas the layer streams 412 MB of packed
// weights and does little arithmetic per byte; separate launches lose the
// chip at every boundary (a per-workgroup prologue before the first weight
// byte arrives, a round of workgroups waiting for the slowest expert, the
// gate/up tail before down starts). Here one workgroup per CU streams units of
// work back to back through one LDS ring, so the weight stream never stops at
// a unit boundary, and the down units of an expert start as soon as that
// expert's gate/up units are done, while other CUs are still on gate/up.
//
// Units (all of one expert e, one chunk of at most 16*MTX of its routed rows):
//   gate/up unit (e, cb): columns [176*cb, +176) of I, gate and up: 22 slots
//     of one 128-K group each (11 tiles x (gate, up) fragment blocks + scales);
//   down unit (e, q): output columns [352*q, +352) of H: I/128 slots of one
//     128-K group each (22 tile blocks + scales), then a 64-K tail slot.
// Units are taken from a queue: workgroup b starts with unit b, then pulls
// the next index from a counter. All gate/up units come before all down units,
// chunk 0 of every expert before its later chunks.
//
// Waves of a workgroup (15):
//   0..10  consumers: wave w owns gate/up tile w, or down tiles 2w and 2w+1;
//          they read LDS only (nibble decode, v_mfma_f32_16x16x32_f16) and
//          store out2 / out3 at the end of a chunk;
//   11, 12 weight producers: copy the first and second half of each slot's
//          contiguous pack bytes (1 KB per instruction) into the ring (direct
//          global -> LDS loads);
//   13     activation producer: gathers the chunk's activation rows into the
//          ring in MFMA fragment order (a16 rows for gate/up, out2 rows for
//          down);
//   14     control: pulls units, reads the routing, tracks which experts'
//          gate/up is complete, and writes one plan per ring slot into LDS.
// Waves 11..14 run at raised priority, so that after a barrier their load
// issue is not queued behind the consumers' arithmetic.
// One barrier per slot. In cycle n the consumers compute slot n, the producers
// issue slot n+R-1 and wait for slot n+1, the control wave plans slot n+R.
// A slot whose unit cannot start yet (its expert's gate/up still running
// elsewhere) is planned empty: the barriers keep turning, nothing waits on
// another workgroup while holding the ring.
//
// Cross-workgroup data: out2 rows are written with device-coherent stores
// (sc1) and read by the down units with device-coherent loads (sc1); after a
// consumer's out2 stores of a finished gate/up unit are complete (vmcnt(0))
// it adds 1 to the expert's counter (device-scope atomic). A down unit of
// expert e starts once the counter reaches 11 * (gate/up units of e).
// Deadlock freedom: gate/up units never wait; a down unit waits only on
// gate/up units pulled before it, which are held by running workgroups whose
// cycles keep turning. Every wait is bounded (kMaxIdle empty cycles, then the
// error word is set and the unit proceeds).
#include <algorithm>
#include <atomic>

#include "ksl_common.h"

namespace ksl {
namespace {

constexpr int kNc = 11;                 // consumer waves
constexpr int kWaveW0 = kNc;            // weight producers: each slot's first and second half
constexpr int kWaveW1 = kNc + 1;
constexpr int kWaveA = kNc + 2;         // activation producer
constexpr int kWaveCtl = kNc + 3;       // control wave
constexpr int kFfnWaves = kNc + 4;
constexpr int kFfnThreads = kFfnWaves * kWave;
constexpr int kGuT = kNc;               // gate (and up) tiles per gate/up unit: 176 columns of I
constexpr int kDnT = 2 * kNc;           // tiles per down unit: 352 columns of H
constexpr int kGuTileB = 2 * 1024 + 128;  // per tile and 128-K group: gate + up blocks, then 4 fp16 s/z
constexpr int kDnTileB = 1024 + 128;      // per tile and 128-K slot: one block, then 2 x (s, z)
constexpr int kDnTailB = 512 + 64;        // per tile, trailing 64-K group: half block, then (s, z)
constexpr int kSlotW = 25600;           // pack bytes of a ring slot (>= 11 * 2176, 22 * 1152)
constexpr int kPlanN = 8;               // plan ring entries
constexpr int kMaxIdle = 1 << 18;       // empty cycles a unit may wait for its dependency (default)
constexpr int kMaxE = 512;

static_assert(kSlotW >= kGuT * kGuTileB && kSlotW >= kDnT * kDnTileB, "slot too small");

enum PlanKind { kNone = 0, kGu = 1, kDnFull = 2, kDnTail = 3, kEnd = 4 };
// Counter slots of the ctl array (each kCtlStride int32 words, so that no two
// share a cache line or a memory channel's queue): the unit queue, the error
// word, the exit count, then per expert the number of its finished gate/up units.
enum CtlSlot { kCtlQueue = 0, kCtlError = 1, kCtlExits = 2, kCtlExpert0 = 3 };
__device__ __forceinline__ int32_t* ctl_slot(int32_t* ctl, int i) { return ctl + static_cast<int64_t>(i) * kCtlStride; }
enum PlanFlag { kFirst = 1, kLast = 2, kSignal = 4 };

struct Plan {
    int kind, e, blk, nt, g, row0, mrows, flags;
};

struct FfnArgs {
    const f16* a16;
    const int32_t* sorted_rows;
    const int32_t* offsets;
    const uint8_t* gu_pack;
    const uint8_t* dn_pack;
    f16* out2;
    f16* out3;
    int32_t* ctl;  // counter slots, kCtlStride words apart: unit queue, error word, exits, then one per expert
    int E, H, I, topk;
    int ncb, nq;     // gate/up units and down units per expert chunk
    int G;           // 128-K groups of H (gate/up slots per unit)
    int nfull, tail; // down slots per unit: I / 128 full, one 64-K tail when I % 128 == 64
    int n0;          // units taken statically (= gridDim.x): workgroup b starts with unit b
    int max_idle;    // empty cycles a down unit waits for its expert's gate/up units before giving up
    int force_wait;  // nonzero: every dependency counts as unmet (failure-handling tests)
};

template <int MTX>
struct Lay {
    static constexpr int kAct = MTX * 4 * 1024;  // activation blocks (t, i) of a slot
    static constexpr int kSlot = kSlotW + kAct;
};

// Byte offsets of the pack layouts (ksl_moe_pack_gateup / ksl_moe_pack_down).
__host__ __device__ inline int64_t gu_unit_off(int64_t e, int cb, int I, int H) {
    return e * (static_cast<int64_t>(I) * H / 16 * 17) + static_cast<int64_t>(kGuT) * cb * (H / 128) * kGuTileB;
}
__host__ __device__ inline int64_t dn_unit_off(int64_t e, int q, int I, int H) {
    return e * (static_cast<int64_t>(H) * I / 16 * 9) + static_cast<int64_t>(kDnT) * q * 9 * I;
}

// s_waitcnt vmcnt(n) for a run-time n in [0, 63].
__device__ __forceinline__ void vm_wait_dyn(int n) {
    n = n < 0 ? 0 : (n > 63 ? 63 : n);
    switch (n >> 3) {
#define KSL_VW8(B)                                   \
    case B:                                          \
        switch (n & 7) {                             \
            case 0: vm_wait<B * 8 + 0>(); break;     \
            case 1: vm_wait<B * 8 + 1>(); break;     \
            case 2: vm_wait<B * 8 + 2>(); break;     \
            case 3: vm_wait<B * 8 + 3>(); break;     \
            case 4: vm_wait<B * 8 + 4>(); break;     \
            case 5: vm_wait<B * 8 + 5>(); break;     \
            case 6: vm_wait<B * 8 + 6>(); break;     \
            default: vm_wait<B * 8 + 7>(); break;    \
        }                                            \
        break;
        KSL_VW8(0) KSL_VW8(1) KSL_VW8(2) KSL_VW8(3) KSL_VW8(4) KSL_VW8(5) KSL_VW8(6) KSL_VW8(7)
#undef KSL_VW8
    }
}

__device__ __forceinline__ int ruf(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int wave_id_ffn() { return ruf(threadIdx.x / kWave); }

// LDS reads of the producer waves, as asm with their own lgkmcnt wait: a plain
// LDS read after a direct global -> LDS load makes the compiler wait for every
// load in flight (it cannot tell the plan area from the ring).
__device__ __forceinline__ uint32_t lds_off(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)(p)));
}
__device__ __forceinline__ u32x4 lds_read16_now(const void* p) {
    u32x4 r;
    asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(lds_off(p)) : "memory");
    return r;
}
__device__ __forceinline__ int lds_read4_now(const void* p) {
    int r;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(r) : "v"(lds_off(p)) : "memory");
    return r;
}

// Compute units of the current device (cached per device).
int ffn_cus() {
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

__device__ __forceinline__ Plan read_plan(const Plan* plans, int k) {
    const Plan* p = plans + (k & (kPlanN - 1));
    Plan r;
    r.kind = ruf(p->kind);
    r.e = ruf(p->e);
    r.blk = ruf(p->blk);
    r.nt = ruf(p->nt);
    r.g = ruf(p->g);
    r.row0 = ruf(p->row0);
    r.mrows = ruf(p->mrows);
    r.flags = ruf(p->flags);
    return r;
}

// Plan of slot k as the producers read it (asm LDS reads, see lds_read16_now).
__device__ __forceinline__ Plan read_plan_p(const Plan* plans, int k) {
    const Plan* p = plans + (k & (kPlanN - 1));
    const u32x4 a = lds_read16_now(p), b = lds_read16_now(reinterpret_cast<const char*>(p) + 16);
    Plan r;
    r.kind = ruf(a[0]);
    r.e = ruf(a[1]);
    r.blk = ruf(a[2]);
    r.nt = ruf(a[3]);
    r.g = ruf(b[0]);
    r.row0 = ruf(b[1]);
    r.mrows = ruf(b[2]);
    r.flags = ruf(b[3]);
    return r;
}

// ---------------------------------------------------------------- producers
// Pack bytes of one slot: [src, src + len) of the pack -> the slot's first
// len bytes, 1 KB per instruction (the last one partial). Returns the number
// of instructions issued.
__device__ __forceinline__ int pack_src(const FfnArgs& A, const Plan& p, const uint8_t*& src) {
    if (p.kind == kGu) {
        src = A.gu_pack + gu_unit_off(p.e, p.blk, A.I, A.H) + static_cast<int64_t>(p.g) * p.nt * kGuTileB;
        return p.nt * kGuTileB;
    }
    const uint8_t* u = A.dn_pack + dn_unit_off(p.e, p.blk, A.I, A.H);
    if (p.kind == kDnFull) {
        src = u + static_cast<int64_t>(p.g) * p.nt * kDnTileB;
        return p.nt * kDnTileB;
    }
    src = u + static_cast<int64_t>(A.nfull) * p.nt * kDnTileB;
    return p.nt * kDnTailB;
}

// Half h of a slot's pack bytes: the 1 KB instructions d0 .. d1-1 of the
// slot's nd (wave 0 the first ceil(nd/2), wave 1 the rest with the partial
// last one). Issues them when ISSUE; returns how many there are.
template <bool ISSUE>
__device__ __forceinline__ int issue_pack_half(const FfnArgs& A, const Plan& p, char* slot, int h) {
    if (p.kind < kGu || p.kind > kDnTail) return 0;
    const int lane = threadIdx.x & (kWave - 1);
    const uint8_t* src;
    const int len = pack_src(A, p, src);
    const int nfull = len >> 10, rem = (len & 1023) >> 4;
    const int nd = nfull + (rem ? 1 : 0), half = (nd + 1) >> 1;
    const int d0 = h ? half : 0, d1 = h ? nd : half;
    if constexpr (ISSUE) {
        for (int d = d0; d < d1; ++d) {
            if (d < nfull) dma16(src + d * 1024 + lane * 16, slot + d * 1024);
            else if (lane < rem) dma16(src + d * 1024 + lane * 16, slot + d * 1024);
        }
    }
    return d1 - d0;
}

// Activation blocks of one slot: block (t, i) = 16 rows x 64 bytes (MFMA step
// i of M tile t), fetched row-major (4 lanes per row) into the swizzled
// fragment order of frag_pos. Gate/up rows are token rows of a16 (tokens of the
// chunk in tok[t]); down rows are the chunk's out2 rows, read device-coherent
// (written by other workgroups in this launch).
template <int MTX>
__device__ __forceinline__ int issue_act(const FfnArgs& A, const Plan& p, char* slot, const int (&tok)[MTX]) {
    if (p.kind < kGu || p.kind > kDnTail || p.mrows <= 0) return 0;
    const int lane = threadIdx.x & (kWave - 1);
    const int rr = lane >> 2, ch = (lane & 3) ^ frag_swz(rr);
    const int mt = (p.mrows + 15) >> 4;
    char* ab = slot + kSlotW;
    if (p.kind == kGu) {
#pragma unroll
        for (int t = 0; t < MTX; ++t) {
            if (t < mt) {
                const char* src = reinterpret_cast<const char*>(A.a16) +
                                  (static_cast<int64_t>(tok[t]) * A.H + p.g * 128 + ch * 8) * 2;
#pragma unroll
                for (int i = 0; i < 4; ++i) dma16(src + i * 64, ab + (t * 4 + i) * 1024);
            }
        }
        return 4 * mt;
    }
    const int nstep = p.kind == kDnFull ? 4 : 2;
    const int col0 = p.kind == kDnFull ? p.g * 128 : A.nfull * 128;
#pragma unroll
    for (int t = 0; t < MTX; ++t) {
        if (t < mt) {
            int r = t * 16 + rr;
            if (r >= p.mrows) r = p.mrows - 1;  // rows past the chunk: loaded, never stored
            const char* src = reinterpret_cast<const char*>(A.out2) +
                              (static_cast<int64_t>(p.row0 + r) * A.I + col0 + ch * 8) * 2;
            for (int i = 0; i < nstep; ++i)
                __builtin_amdgcn_global_load_lds((gbl_vptr)(const_cast<char*>(src + i * 64)),
                                                 (lds_vptr)(ab + (t * 4 + i) * 1024), 16, 0, 16 /* sc1 */);
        }
    }
    return nstep * mt;
}

// The three producer waves share this loop (ROLE 0, 1: the two halves of each
// slot's weights; 2: the activations); only the issue differs.
template <int MTX, int R, int ROLE>
__device__ void ffn_produce(const FfnArgs& A, char* lds, const Plan* plans, const int* toks) {
    using L = Lay<MTX>;
    constexpr bool WEIGHTS = ROLE < 2;
    const int lane = threadIdx.x & (kWave - 1);
    const int rr = lane >> 2;
    int tok[MTX];
#pragma unroll
    for (int t = 0; t < MTX; ++t) tok[t] = 0;
    int k_end = 0x7fffffff;
    int win[R];  // instructions of slots n+1 .. n+R-1 (win[0] = slot n+1)
#pragma unroll
    for (int j = 0; j < R; ++j) win[j] = 0;
    auto issue = [&](int k) -> int {
        const Plan p = read_plan_p(plans, k);
        if (p.kind == kEnd) {
            k_end = k < k_end ? k : k_end;
            return 0;
        }
        char* slot = lds + (k % R) * L::kSlot;
        if constexpr (WEIGHTS) {
            return issue_pack_half<true>(A, p, slot, ROLE);
        } else {
            if (p.kind == kGu && (p.flags & kFirst)) {
                const int* tk = toks + (k & (kPlanN - 1)) * kWave;
#pragma unroll
                for (int t = 0; t < MTX; ++t) tok[t] = lds_read4_now(tk + t * 16 + rr);
            }
            return issue_act<MTX>(A, p, slot, tok);
        }
    };
    // early issue: the weight slots of unit blockIdx.x (a chunk-0 gate/up unit,
    // whatever the routing) go out before the plans exist
    int e0 = 0;
    if constexpr (WEIGHTS) {
        const int u = blockIdx.x;
        Plan p;
        p.kind = kGu;
        p.e = u / A.ncb;
        p.blk = u - p.e * A.ncb;
        p.nt = min(kGuT, A.I / 16 - kGuT * p.blk);
        e0 = min(R - 1, A.G);
        for (int g = 0; g < e0; ++g) {
            p.g = g;
            win[g] = issue_pack_half<true>(A, p, lds + g * L::kSlot, ROLE);
        }
    }
    __builtin_amdgcn_s_barrier();  // B_init: plans 0 .. R-1 are written
    asm volatile("" ::: "memory");
    // Issue first, then wait: at most R-1 slots are in flight, so a wave keeps
    // fewer than 64 memory instructions outstanding (vmcnt's range: 3 slots of
    // at most 13 weight or 8 activation instructions).
    for (int k = e0; k < R - 1; ++k)
        if (k < k_end) win[k] = issue(k);
    {
        int after = 0;
#pragma unroll
        for (int j = 1; j < R - 1; ++j) after += win[j];
        vm_wait_dyn(after);  // slot 0 landed
    }
    dma_barrier();  // B_0
    // window: slots n+1 .. n+R-2 in win[0 .. R-3] at the start of cycle n
#pragma unroll
    for (int j = 0; j < R - 1; ++j) win[j] = win[j + 1];
    win[R - 1] = 0;
    for (int n = 0; n < k_end; ++n) {
        const int k = n + R - 1;
        win[R - 2] = k < k_end ? issue(k) : 0;
        if (n + 1 < k_end) {
            int after = 0;
#pragma unroll
            for (int j = 1; j < R - 1; ++j) after += win[j];
            vm_wait_dyn(after);  // slot n+1 landed
        }
        dma_barrier();  // B_{n+1}
#pragma unroll
        for (int j = 0; j < R - 2; ++j) win[j] = win[j + 1];
        win[R - 2] = 0;
    }
    vm_wait<0>();
    __builtin_amdgcn_s_barrier();  // B_exit
}

// ---------------------------------------------------------------- consumers
template <int ACT, int MTX, int MT>
__device__ __forceinline__ void gu_slot(const char* __restrict__ sp, int nt, f32x4 (&acc)[2][MTX],
                                        const NibConsts& kn) {
    const int w = wave_id_ffn();
    (void)nt;
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int fo = frag_pos(col, c) * 16;
    u32x4 wv[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) wv[j] = *reinterpret_cast<const u32x4*>(sp + (2 * w + j) * 1024 + lane * 16);
    const f16x4 sz = *reinterpret_cast<const f16x4*>(sp + nt * 2048 + w * 128 + col * 8);  // sg zg su zu
    const ZeroPair zc[2] = {zero_pair(sz[1]), zero_pair(sz[3])};
    f32x4 part[2][MT];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int t = 0; t < MT; ++t) part[j][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        f16x8 a[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) a[t] = *reinterpret_cast<const f16x8*>(sp + kSlotW + (t * 4 + i) * 1024 + fo);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const f16x8 b = nib8_minus_zero(wv[j][i], zc[j], kn);
#pragma unroll
            for (int t = 0; t < MT; ++t) part[j][t] = mfma16x16x32(a[t], b, part[j][t]);
        }
        if constexpr (MT > 2) __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float sc = static_cast<float>(sz[2 * j]);
#pragma unroll
        for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[j][t][q] = __builtin_fmaf(sc, part[j][t][q], acc[j][t][q]);
    }
}

template <int ACT, int MTX, int MT>
__device__ __forceinline__ void gu_epilogue(const FfnArgs& A, const Plan& p, const f32x4 (&acc)[2][MTX]) {
    const int w = wave_id_ffn();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int sc = out2_store_index(16 * (kGuT * p.blk + w) + col, A.I & ~127);
    uint16_t* o = reinterpret_cast<uint16_t*>(A.out2) + (static_cast<int64_t>(p.row0) + 4 * c) * A.I + sc;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = t * 16 + 4 * c + q;
            if (row < p.mrows) {
                const f16 v = static_cast<f16>(act_times_up<ACT>(acc[0][t][q], acc[1][t][q]));
                // device-coherent: down units on other CUs read it in this launch
                __hip_atomic_store(o + (t * 16 + q) * A.I, f16_bits(v), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
}

// Down slot of a wave that owns NT2 (1 or 2) tiles: 2w and, for 2, 2w+1.
template <int MTX, int MT, bool TAILS, int NT2>
__device__ __forceinline__ void dn_slot(const char* __restrict__ sp, int nt, f32x4 (&acc)[2][MTX],
                                        const NibConsts& kn) {
    const int w = wave_id_ffn();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
    const int fo = frag_pos(col, c) * 16;
    constexpr int NS = TAILS ? 2 : 4;
    u32x4 wq[NT2];
    f16x2 sz[NT2];
#pragma unroll
    for (int v = 0; v < NT2; ++v) {
        const int u = 2 * w + v;
        if constexpr (TAILS) {
            const u32x2 t2 = *reinterpret_cast<const u32x2*>(sp + u * 512 + lane * 8);
            wq[v] = u32x4{t2[0], t2[1], 0u, 0u};
            sz[v] = *reinterpret_cast<const f16x2*>(sp + nt * 512 + u * 64 + col * 4);
        } else {
            wq[v] = *reinterpret_cast<const u32x4*>(sp + u * 1024 + lane * 16);
            sz[v] = *reinterpret_cast<const f16x2*>(sp + nt * 1024 + u * 128 + col * 8 + (c >> 1) * 4);
        }
    }
    ZeroPair zc[NT2];
#pragma unroll
    for (int v = 0; v < NT2; ++v) zc[v] = zero_pair(sz[v][1]);
#pragma unroll
    for (int i = 0; i < NS; ++i) {
        f16x8 a[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) a[t] = *reinterpret_cast<const f16x8*>(sp + kSlotW + (t * 4 + i) * 1024 + fo);
#pragma unroll
        for (int v = 0; v < NT2; ++v) {
            const f16x8 b = nib8_dequant(wq[v][i], zc[v], f16x2{sz[v][0], sz[v][0]}, kn);
#pragma unroll
            for (int t = 0; t < MT; ++t) acc[v][t] = mfma16x16x32(b, a[t], acc[v][t]);
        }
        if constexpr (MT > 2) __builtin_amdgcn_sched_barrier(0);
    }
}

template <int MTX, int MT>
__device__ __forceinline__ void dn_epilogue(const FfnArgs& A, const Plan& p, const f32x4 (&acc)[2][MTX]) {
    const int w = wave_id_ffn();
    const int lane = threadIdx.x & (kWave - 1);
    const int col = lane & 15, c = lane >> 4;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
        const int u = 2 * w + v;
        if (u >= p.nt) continue;
        f16* o = A.out3 + static_cast<int64_t>(p.row0) * A.H + kDnT * 16 * p.blk + 16 * u + 4 * c;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            const int row = t * 16 + col;
            if (row < p.mrows) {
                const f16x4 val{static_cast<f16>(acc[v][t][0]), static_cast<f16>(acc[v][t][1]),
                                static_cast<f16>(acc[v][t][2]), static_cast<f16>(acc[v][t][3])};
                *reinterpret_cast<u32x2*>(o + static_cast<int64_t>(row) * A.H) = __builtin_bit_cast(u32x2, val);
            }
        }
    }
}

template <int ACT, int MTX, int MT>
__device__ __forceinline__ void consume_mt(const FfnArgs& A, const Plan& p, const char* sp, f32x4 (&acc)[2][MTX],
                                           const NibConsts& kn) {
    const int w = wave_id_ffn();
    if (p.kind == kGu) {
        if (w < p.nt) {
            gu_slot<ACT, MTX, MT>(sp, p.nt, acc, kn);
            if (p.flags & kLast) gu_epilogue<ACT, MTX, MT>(A, p, acc);
        }
    } else {
        if (2 * w < p.nt) {
            const bool two = 2 * w + 1 < p.nt;
            if (p.kind == kDnFull) {
                if (two) dn_slot<MTX, MT, false, 2>(sp, p.nt, acc, kn);
                else dn_slot<MTX, MT, false, 1>(sp, p.nt, acc, kn);
            } else {
                if (two) dn_slot<MTX, MT, true, 2>(sp, p.nt, acc, kn);
                else dn_slot<MTX, MT, true, 1>(sp, p.nt, acc, kn);
            }
            if (p.flags & kLast) dn_epilogue<MTX, MT>(A, p, acc);
        }
    }
}

template <int ACT, int MTX, int R>
__device__ void ffn_consume(const FfnArgs& A, const char* lds, const Plan* plans, int* sig) {
    using L = Lay<MTX>;
    const NibConsts kn = nib_consts();
    f32x4 acc[2][MTX];
    int pend_e = -1, pend_age = 0, pend_k = 0;
    // A finished gate/up unit counts once: each consumer wave, its out2 stores
    // complete (device scope), adds 1 to an LDS counter of the unit's last slot;
    // the wave that completes the count adds 1 to the expert's counter.
    auto signal = [&]() {
        vm_wait<0>();
        int old = 0;
        if ((threadIdx.x & (kWave - 1)) == 0)
            old = __hip_atomic_fetch_add(sig + (pend_k & (kPlanN - 1)), 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_WORKGROUP);
        if (ruf(old) == kNc - 1) {
            if ((threadIdx.x & (kWave - 1)) == 0) {
                sig[pend_k & (kPlanN - 1)] = 0;
                __hip_atomic_fetch_add(ctl_slot(A.ctl, kCtlExpert0 + pend_e), 1, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        pend_e = -1;
    };
    __builtin_amdgcn_s_barrier();  // B_init
    __builtin_amdgcn_s_barrier();  // B_0
    asm volatile("" ::: "memory");
    for (int n = 0;; ++n) {
        const Plan p = read_plan(plans, n);
        if (pend_e >= 0 && ++pend_age >= 4) signal();  // four slots later the stores are acknowledged
        if (p.kind == kEnd) break;
        if (p.kind != kNone) {
            if (p.flags & kFirst) {
#pragma unroll
                for (int v = 0; v < 2; ++v)
#pragma unroll
                    for (int t = 0; t < MTX; ++t) acc[v][t] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            if (p.mrows > 0) {
                const char* sp = lds + (n % R) * L::kSlot;
                const int mt = (p.mrows + 15) >> 4;
                if (mt == 1) consume_mt<ACT, MTX, 1>(A, p, sp, acc, kn);
                else if (mt == 2 || MTX == 2) consume_mt<ACT, MTX, 2>(A, p, sp, acc, kn);
                else if constexpr (MTX >= 4) {
                    if (mt == 3) consume_mt<ACT, MTX, 3>(A, p, sp, acc, kn);
                    else consume_mt<ACT, MTX, 4>(A, p, sp, acc, kn);
                }
            }
            if (p.flags & kSignal) {
                if (pend_e >= 0) signal();
                pend_e = p.e;
                pend_k = n;
                pend_age = 0;
            }
        }
        lds_sync();  // B_{n+1}
    }
    if (pend_e >= 0) signal();
    vm_wait<0>();                  // the last counter update is performed
    __builtin_amdgcn_s_barrier();  // B_exit
}

// ------------------------------------------------------------------ control
struct Unit {
    int kind;  // kNone (empty), kGu, kDnFull (a down unit), kEnd
    int e, blk, nt, row0, mrows, nslots;
};

template <int MTX>
__device__ __forceinline__ Unit decode_unit(const FfnArgs& A, int u, const int* offs, const int* xgu,
                                            const int* xdn) {
    constexpr int CH = 16 * MTX;
    const int E = A.E;
    const int n0g = E * A.ncb, XG = ruf(xgu[E]), n0d = E * A.nq, XD = ruf(xdn[E]);
    Unit r;
    r.kind = kEnd;
    int e = 0, blk = 0, c = 0;
    auto search = [&](const int* x, int v) {
        int lo = 0, hi = E - 1;  // largest e with x[e] <= v
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (ruf(x[mid]) <= v) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    if (u < n0g) {
        r.kind = kGu;
        e = u / A.ncb;
        blk = u - e * A.ncb;
    } else if ((u -= n0g) < XG) {
        r.kind = kGu;
        e = search(xgu, u);
        const int rr = u - ruf(xgu[e]);
        c = 1 + rr / A.ncb;
        blk = rr - (c - 1) * A.ncb;
    } else if ((u -= XG) < n0d) {
        r.kind = kDnFull;
        e = u / A.nq;
        blk = u - e * A.nq;
    } else if ((u -= n0d) < XD) {
        r.kind = kDnFull;
        e = search(xdn, u);
        const int rr = u - ruf(xdn[e]);
        c = 1 + rr / A.nq;
        blk = rr - (c - 1) * A.nq;
    } else {
        return r;
    }
    const int o = ruf(offs[e]), M = ruf(offs[e + 1]) - o;
    r.e = e;
    r.blk = blk;
    r.row0 = o + c * CH;
    r.mrows = min(CH, M - c * CH);
    if (r.kind == kGu) {
        r.nt = min(kGuT, A.I / 16 - kGuT * blk);
        r.nslots = A.G;
    } else {
        r.nt = min(kDnT, A.H / 16 - kDnT * blk);
        r.nslots = A.nfull + A.tail;
    }
    return r;
}

template <int MTX, int R>
__device__ void ffn_control(const FfnArgs& A, const Plan* plans_c, int* toks, int* offs, int* xgu, int* xdn) {
    constexpr int CH = 16 * MTX;
    Plan* plans = const_cast<Plan*>(plans_c);
    const int lane = threadIdx.x & (kWave - 1);
    const int E = A.E;
    const int nj = (E + kWave - 1) / kWave;  // experts per lane (<= 8)
    int32_t* qctr = ctl_slot(A.ctl, kCtlQueue);
    int32_t* errw = ctl_slot(A.ctl, kCtlError);

    // ---- startup: routing offsets into LDS, chunk counts, prefix sums of the
    // units beyond chunk 0
    {
        for (int i = lane; i <= E; i += kWave) offs[i] = A.offsets[i];
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
        int rung = 0, rund = 0;
#pragma unroll
        for (int j = 0; j < kMaxE / kWave; ++j) {
            if (j >= nj) continue;
            const int e = j * kWave + lane;
            int M = 0;
            if (e < E) M = offs[e + 1] - offs[e];
            const int ch = (M + CH - 1) / CH;
            const int xg = ch > 1 ? (ch - 1) * A.ncb : 0, xd = ch > 1 ? (ch - 1) * A.nq : 0;
            int ig = xg, id = xd;
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) {
                const int og = __shfl_up(ig, off, kWave), od = __shfl_up(id, off, kWave);
                if (lane >= off) {
                    ig += og;
                    id += od;
                }
            }
            if (e < E) {
                xgu[e] = rung + ig - xg;
                xdn[e] = rund + id - xd;
            }
            rung += __shfl(ig, kWave - 1, kWave);
            rund += __shfl(id, kWave - 1, kWave);
        }
        if (lane == 0) {
            xgu[E] = rung;
            xdn[E] = rund;
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }

    // ---- unit pipeline state (wave-uniform). The control wave's memory
    // operations go out in batches (a unit pull, a chunk's token rows, a poll
    // of one expert's completion counter); one batch is in flight at a time and is
    // read two cycles after it was issued, when nothing younger is in flight,
    // so the waits the compiler places before the reads cost nothing.
    Unit cur, nx;
    cur.kind = kNone;
    cur.nslots = 0;
    int cur_g = 0;
    int cur_tok = 0, nx_tok = 0;     // per lane: token of chunk row `lane`
    enum { kEmpty, kNeedPull, kPulled, kNeedTok, kTokWait, kDepWait, kReady, kEndSt };
    int nx_state = kEmpty;
    int pull_v = 0, tok_v = 0, poll_v = 0;
    bool busy = false, poll_in = false, dep_ok = false;
    // gate/up units of expert e: one per column block and chunk of its rows
    auto gu_units = [&](int e) {
        const int M = ruf(offs[e + 1]) - ruf(offs[e]);
        return A.ncb * ((M + CH - 1) / CH);
    };
    int stamp = 0, idle = 0;

    auto take_batch = [&]() {
        // the batch's results (the compiler's wait lands here)
        if (poll_in) {
            dep_ok = !A.force_wait && ruf(poll_v) >= gu_units(nx.e);
            poll_in = false;
        }
        if (nx_state == kPulled) {
            const int u = ruf(pull_v) + A.n0;
            nx = decode_unit<MTX>(A, u, offs, xgu, xdn);
            if (nx.kind == kEnd) nx_state = kEndSt;
            else if (nx.mrows <= 0) nx_state = kNeedPull;  // an expert without rows: take the next unit
            else nx_state = nx.kind == kGu ? kNeedTok : kDepWait;
            dep_ok = false;
        } else if (nx_state == kTokWait) {
            nx_tok = tok_v / A.topk;
            nx_state = kReady;
        }
        busy = false;
    };
    // issue the next batch if the pipeline needs one
    auto issue_batch = [&](int n) {
        if (busy) return;
        if (nx_state == kDepWait && dep_ok) nx_state = kReady;
        if (nx_state == kNeedPull) {
            int v = 0;
            if (lane == 0) v = __hip_atomic_fetch_add(qctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pull_v = v;  // lane 0's value is read (readfirstlane) when the batch is taken
            nx_state = kPulled;
        } else if (nx_state == kNeedTok) {
            const int r = lane < nx.mrows ? lane : nx.mrows - 1;
            tok_v = A.sorted_rows[nx.row0 + r];
            nx_state = kTokWait;
        } else if (nx_state == kDepWait) {
            // one device-coherent load of the expert's counter
            int v = 0;
            if (lane == 0)
                v = __hip_atomic_load(ctl_slot(A.ctl, kCtlExpert0 + nx.e), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            poll_v = v;
            poll_in = true;
        } else {
            return;
        }
        busy = true;
        stamp = n;
    };
    auto write_plan = [&](int k, int kind, const Unit& u, int g, int flags) {
        Plan* p = plans + (k & (kPlanN - 1));
        if (lane == 0) {
            p->kind = kind;
            p->e = u.e;
            p->blk = u.blk;
            p->nt = u.nt;
            p->g = g;
            p->row0 = u.row0;
            p->mrows = u.mrows;
            p->flags = flags;
        }
    };
    int k_end = 0x7fffffff;
    // plan slot k (blocking: complete the next unit first if it is needed)
    auto plan = [&](int k, int n, bool blocking) {
        if (cur_g >= cur.nslots) {
            if (blocking) {
                for (int it = 0; it < 8 && nx_state != kReady && nx_state != kEndSt; ++it) {
                    issue_batch(n);
                    if (!busy) break;  // waiting for a dependency: not in the prologue
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    take_batch();
                }
            }
            if (nx_state == kReady) {
                cur = nx;
                cur_tok = nx_tok;
                cur_g = 0;
                nx_state = kNeedPull;
                idle = 0;
            } else if (nx_state == kEndSt) {
                Unit z{};
                write_plan(k, kEnd, z, 0, 0);
                k_end = k;
                return;
            } else {
                if (nx_state == kDepWait && ++idle > A.max_idle) {
                    // bounded wait: record the error and let the unit run
                    if (lane == 0) __hip_atomic_store(errw, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    nx_state = kReady;
                }
                Unit z{};
                write_plan(k, kNone, z, 0, 0);
                return;
            }
        }
        const int g = cur_g++;
        int flags = 0;
        if (g == 0) flags |= kFirst;
        if (g == cur.nslots - 1) {
            flags |= kLast;
            if (cur.kind == kGu && cur.mrows > 0) flags |= kSignal;  // every chunk's unit counts
        }
        int kind = cur.kind;
        if (kind == kDnFull && g >= A.nfull) kind = kDnTail;
        if (kind == kGu && g == 0) toks[(k & (kPlanN - 1)) * kWave + lane] = cur_tok;
        write_plan(k, kind, cur, g, flags);
    };

    // ---- startup plans 0 .. R-1 (blocking): the first unit is blockIdx.x
    {
        const int u0 = blockIdx.x;
        cur = decode_unit<MTX>(A, u0, offs, xgu, xdn);  // a chunk-0 gate/up unit
        const int e0 = min(R - 1, A.G);                  // slots the weight producer issued already
        if (cur.mrows <= 0) {
            cur.mrows = 0;
            cur.nslots = e0;  // only the slots already in flight
            cur_tok = 0;
        } else {
            const int r = lane < cur.mrows ? lane : cur.mrows - 1;
            cur_tok = A.sorted_rows[cur.row0 + r] / A.topk;
        }
        cur_g = 0;
        nx_state = kNeedPull;
        issue_batch(0);
        for (int k = 0; k < R && k_end == 0x7fffffff; ++k) plan(k, 0, true);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    __builtin_amdgcn_s_barrier();  // B_init
    __builtin_amdgcn_s_barrier();  // B_0
    asm volatile("" ::: "memory");
    for (int n = 0; n < k_end; ++n) {
        if (busy && n >= stamp + 2) take_batch();
        issue_batch(n);
        const int k = n + R;
        if (k < k_end) plan(k, n, false);
        issue_batch(n);  // a unit that just started pulls its successor
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();  // B_{n+1}
        asm volatile("" ::: "memory");
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();  // B_exit: every counter update of this workgroup is performed
    // The last workgroup to leave clears the counters and the queue for the
    // next launch (the error word stays).
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(ctl_slot(A.ctl, kCtlExits), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (ruf(old) == static_cast<int>(gridDim.x) - 1) {
        for (int i = lane; i < kCtlExpert0 + E; i += kWave)
            if (i != kCtlError) *ctl_slot(A.ctl, i) = 0;
    }
}

template <int ACT, int MTX, int R>
__global__ __launch_bounds__(kFfnThreads) void ffn_kernel(FfnArgs A) {
    using L = Lay<MTX>;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    Plan* plans = reinterpret_cast<Plan*>(lds + R * L::kSlot);
    int* toks = reinterpret_cast<int*>(plans + kPlanN);
    int* offs = toks + kPlanN * kWave;
    int* xgu = offs + (A.E + 1);
    int* xdn = xgu + (A.E + 1);
    int* sig = xdn + (A.E + 1);  // kPlanN counters of finished gate/up units
    if (threadIdx.x < kPlanN) sig[threadIdx.x] = 0;
    const int wave = wave_id_ffn();
    // The producer and control waves issue first on their SIMD: the arbiter
    // favours older waves, and the consumers (waves 0 .. kNc-1) would
    // otherwise delay every load issue after a barrier.
    if (wave >= kNc) __builtin_amdgcn_s_setprio(3);
    if (wave < kNc)
        ffn_consume<ACT, MTX, R>(A, lds, plans, sig);
    else if (wave == kWaveW0)
        ffn_produce<MTX, R, 0>(A, lds, plans, toks);
    else if (wave == kWaveW1)
        ffn_produce<MTX, R, 1>(A, lds, plans, toks);
    else if (wave == kWaveA)
        ffn_produce<MTX, R, 2>(A, lds, plans, toks);
    else if (wave == kWaveCtl)
        ffn_control<MTX, R>(A, plans, toks, offs, xgu, xdn);
}

template <int MTX, int R>
size_t ffn_lds_bytes(int E) {
    return static_cast<size_t>(R) * Lay<MTX>::kSlot + kPlanN * sizeof(Plan) + kPlanN * kWave * 4 +
           static_cast<size_t>(3) * (E + 1) * 4 + kPlanN * 4;
}

// ------------------------------------------------------------ load-time pack
// Gate/up pack: per expert e, unit cb (176 columns of I, nt tiles), 128-K
// group g: nt*2 fragment blocks of 1 KB (block 2w + j: tile w, j = gate/up;
// lane l = c*16 + col holds row j*I + 16*(11*cb + w) + col, bytes
// 64*g + 16*c .. +16), then nt*128 bytes of scales and zero-points (tile w,
// column col: s_gate, z_gate, s_up, z_up of group g, fp16). One thread per
// 16-byte unit of the output.
__global__ __launch_bounds__(256) void pack_gateup_kernel(const uint8_t* __restrict__ q, const f16* __restrict__ s,
                                                          const f16* __restrict__ z, uint8_t* __restrict__ out,
                                                          int E, int H, int I) {
    const int G = H / 128;
    const int64_t per_e = static_cast<int64_t>(I) * H / 16 * 17 / 16;  // 16-byte units per expert
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= per_e * E) return;
    const int e = static_cast<int>(idx / per_e);
    int64_t r = idx - e * per_e;
    const int64_t unit_full = static_cast<int64_t>(kGuT) * G * kGuTileB / 16;
    const int cb = static_cast<int>(r / unit_full);
    r -= cb * unit_full;
    const int nt = min(kGuT, I / 16 - kGuT * cb);
    const int per_slot = nt * kGuTileB / 16;
    const int g = static_cast<int>(r / per_slot);
    const int o = static_cast<int>(r - static_cast<int64_t>(g) * per_slot);
    const int rb = H / 2;
    u32x4 v;
    if (o < nt * 128) {  // weight block
        const int b = o >> 6, l = o & 63, w = b >> 1, j = b & 1, c = l >> 4, col = l & 15;
        const int64_t row = static_cast<int64_t>(e) * 2 * I + (j ? I : 0) + 16 * (kGuT * cb + w) + col;
        v = *reinterpret_cast<const u32x4*>(q + row * rb + 64 * g + 16 * c);
    } else {  // scales / zero-points: two columns per 16 bytes
        const int k = o - nt * 128, w = k >> 3, c2 = (k & 7) * 2;
        f16 h[8];
#pragma unroll
        for (int m = 0; m < 2; ++m) {
            const int64_t rg = static_cast<int64_t>(e) * 2 * I + 16 * (kGuT * cb + w) + c2 + m;
            const int64_t ru = rg + I;
            h[4 * m + 0] = s[rg * G + g];
            h[4 * m + 1] = z[rg * G + g];
            h[4 * m + 2] = s[ru * G + g];
            h[4 * m + 3] = z[ru * G + g];
        }
        v = __builtin_bit_cast(u32x4, f16x8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]});
    }
    *reinterpret_cast<u32x4*>(out + idx * 16) = v;
}

// Down pack: per expert e, unit q (352 columns of H, nt tiles), slot s < I/128:
// nt blocks of 1 KB (tile u; lane l = c*16 + col holds row 16*(22*q + u) + col,
// bytes 64*s + 16*c .. +16), then nt*128 bytes (tile u, column col: s and z of
// group 2s, then of group 2s + 1); for I % 128 == 64 a tail slot: nt half
// blocks of 512 B (lane l: bytes 64*(I/128) + 8*c .. +8), then nt*64 bytes
// (tile u, column col: s and z of the last group).
// Address of bytes b .. of down row `row` in dn_layout (reference: row-major;
// tiled: ksl_moe_repack_down's regrouping inside each 16-row tile, where a
// 16-byte piece at b % 16 == 0, and a tail 8-byte piece, stay contiguous).
__device__ __forceinline__ const uint8_t* dn_byte(const uint8_t* q, int layout, int64_t row, int b, int rb, int g2n) {
    if (layout == KSL_DN_LAYOUT_REF) return q + row * rb + b;
    const uint8_t* tb = q + (row >> 4) * 16 * rb;
    const int col = static_cast<int>(row & 15);
    if (b < 64 * g2n) {
        const int u = b >> 6, c = (b >> 4) & 3;
        return tb + u * 1024 + (c * 16 + col) * 16 + (b & 15);
    }
    const int c = (b - 64 * g2n) >> 3;
    return tb + g2n * 1024 + (c * 16 + col) * 8 + (b & 7);
}

__global__ __launch_bounds__(256) void pack_down_kernel(const uint8_t* __restrict__ q, const f16* __restrict__ s,
                                                        const f16* __restrict__ z, int layout,
                                                        uint8_t* __restrict__ out, int E, int H, int I) {
    const int Gd = I / 64, nfull = I / 128, rb = I / 2;
    const int64_t per_e = static_cast<int64_t>(H) * I / 16 * 9 / 16;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= per_e * E) return;
    const int e = static_cast<int>(idx / per_e);
    int64_t r = idx - e * per_e;
    const int64_t unit_full = static_cast<int64_t>(kDnT) * 9 * I / 16;
    const int qb = static_cast<int>(r / unit_full);
    r -= qb * unit_full;
    const int nt = min(kDnT, H / 16 - kDnT * qb);
    const int full_units = nt * kDnTileB / 16;
    const int64_t row_base = static_cast<int64_t>(e) * H + 16 * kDnT * qb;
    u32x4 v;
    if (r < static_cast<int64_t>(nfull) * full_units) {
        const int sl = static_cast<int>(r / full_units);
        const int o = static_cast<int>(r - static_cast<int64_t>(sl) * full_units);
        if (o < nt * 64) {
            const int u = o >> 6, l = o & 63, c = l >> 4, col = l & 15;
            const int64_t row = row_base + 16 * u + col;
            v = *reinterpret_cast<const u32x4*>(dn_byte(q, layout, row, 64 * sl + 16 * c, rb, nfull));
        } else {
            const int k = o - nt * 64, u = k >> 3, c2 = (k & 7) * 2;
            f16 h[8];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const int64_t row = row_base + 16 * u + c2 + m;
                h[4 * m + 0] = s[row * Gd + 2 * sl];
                h[4 * m + 1] = z[row * Gd + 2 * sl];
                h[4 * m + 2] = s[row * Gd + 2 * sl + 1];
                h[4 * m + 3] = z[row * Gd + 2 * sl + 1];
            }
            v = __builtin_bit_cast(u32x4, f16x8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]});
        }
    } else {
        const int o = static_cast<int>(r - static_cast<int64_t>(nfull) * full_units);
        if (o < nt * 32) {  // two lanes' 8-byte pieces per 16 bytes
            const int u = o >> 5, l2 = (o & 31) * 2;
            u32x2 pc[2];
#pragma unroll
            for (int m = 0; m < 2; ++m) {
                const int l = l2 + m, c = l >> 4, col = l & 15;
                const int64_t row = row_base + 16 * u + col;
                pc[m] = *reinterpret_cast<const u32x2*>(dn_byte(q, layout, row, 64 * nfull + 8 * c, rb, nfull));
            }
            v = u32x4{pc[0][0], pc[0][1], pc[1][0], pc[1][1]};
        } else {
            const int k = o - nt * 32, u = k >> 2, c4 = (k & 3) * 4;
            f16 h[8];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int64_t row = row_base + 16 * u + c4 + m;
                h[2 * m + 0] = s[row * Gd + Gd - 1];
                h[2 * m + 1] = z[row * Gd + Gd - 1];
            }
            v = __builtin_bit_cast(u32x4, f16x8{h[0], h[1], h[2], h[3], h[4], h[5], h[6], h[7]});
        }
    }
    *reinterpret_cast<u32x4*>(out + idx * 16) = v;
}

bool ffn_set_lds(const void* fn) {
    const bool ok = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) == hipSuccess;
    (void)hipGetLastError();
    return ok;
}

constexpr int kFfnMtx = 2;  // rows per chunk: 32
constexpr int kFfnR = 4;    // ring slots (three in flight)

}  // namespace

size_t ffn_ctl_words(int64_t E) { return (static_cast<size_t>(E) + kCtlExpert0) * kCtlStride; }

// The error word of a ctl array: nonzero after a launch whose bounded wait
// gave up (its out2 / out3 are not to be trusted).
const int32_t* ffn_error_word(const int32_t* ctl) { return ctl ? ctl + kCtlError * kCtlStride : nullptr; }

// Process-wide wait limit of the down units' dependency wait, and the
// failure-handling switch that makes every dependency count as unmet.
static std::atomic<int> g_max_idle{kMaxIdle};
static std::atomic<int> g_force_wait{0};

int ffn_set_wait_limit(int64_t cycles, int force_wait) {
    if (cycles < 0) cycles = kMaxIdle;
    if (cycles > (int64_t(1) << 30)) return KSL_ERR_ARG;
    g_max_idle.store(static_cast<int>(cycles), std::memory_order_relaxed);
    g_force_wait.store(force_wait ? 1 : 0, std::memory_order_relaxed);
    return KSL_OK;
}

bool ffn_supported(int64_t E, int64_t H, int64_t I, int64_t nrows) {
    return E > 0 && E <= kMaxE && H % 128 == 0 && I % 64 == 0 && H >= 128 && I >= 64 && nrows > 0 &&
           nrows <= 8192 && H <= 8192 && I <= 8192;
}

// Gate/up + activation and down of every expert in one launch (see above).
// ctl: ffn_ctl_words(E) int32 words, zero on entry (the routing launch clears them).
int launch_ffn(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t topk,
               const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t E, int64_t H, int64_t I, int act,
               void* out2, void* out3, int32_t* ctl, int64_t nrows, hipStream_t st) {
    if (!a16 || !sorted_rows || !offsets || !gu_pack || !dn_pack || !out2 || !out3 || !ctl) return KSL_ERR_ARG;
    if (!ffn_supported(E, H, I, nrows) || topk <= 0) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(gu_pack) % 16 || reinterpret_cast<uintptr_t>(dn_pack) % 16 ||
        reinterpret_cast<uintptr_t>(a16) % 16 || reinterpret_cast<uintptr_t>(out2) % 16 ||
        reinterpret_cast<uintptr_t>(out3) % 8)
        return KSL_ERR_ALIGN;
    FfnArgs A;
    A.a16 = static_cast<const f16*>(a16);
    A.sorted_rows = sorted_rows;
    A.offsets = offsets;
    A.gu_pack = gu_pack;
    A.dn_pack = dn_pack;
    A.out2 = static_cast<f16*>(out2);
    A.out3 = static_cast<f16*>(out3);
    A.ctl = ctl;
    A.E = static_cast<int>(E);
    A.H = static_cast<int>(H);
    A.I = static_cast<int>(I);
    A.topk = static_cast<int>(topk);
    A.ncb = static_cast<int>((I / 16 + kGuT - 1) / kGuT);
    A.nq = static_cast<int>((H / 16 + kDnT - 1) / kDnT);
    A.G = static_cast<int>(H / 128);
    A.nfull = static_cast<int>(I / 128);
    A.tail = (I % 128) != 0;
    A.max_idle = g_max_idle.load(std::memory_order_relaxed);
    A.force_wait = g_force_wait.load(std::memory_order_relaxed);
    const int64_t first = E * A.ncb;  // chunk-0 gate/up units: every workgroup's first unit is one
    const int64_t grid = std::min<int64_t>(ffn_cus(), first);
    A.n0 = static_cast<int>(grid);
    const size_t lds = ffn_lds_bytes<kFfnMtx, kFfnR>(A.E);
    if (lds > 160 * 1024) return KSL_ERR_SHAPE;
    static const bool attr =
        ffn_set_lds(reinterpret_cast<const void*>(&ffn_kernel<KSL_ACT_GELU_TANH, kFfnMtx, kFfnR>)) &&
        ffn_set_lds(reinterpret_cast<const void*>(&ffn_kernel<KSL_ACT_SILU, kFfnMtx, kFfnR>));
    (void)attr;
    if (act == KSL_ACT_GELU_TANH)
        hipLaunchKernelGGL((ffn_kernel<KSL_ACT_GELU_TANH, kFfnMtx, kFfnR>), dim3(static_cast<unsigned>(grid)),
                           dim3(kFfnThreads), lds, st, A);
    else if (act == KSL_ACT_SILU)
        hipLaunchKernelGGL((ffn_kernel<KSL_ACT_SILU, kFfnMtx, kFfnR>), dim3(static_cast<unsigned>(grid)),
                           dim3(kFfnThreads), lds, st, A);
    else
        return KSL_ERR_ARG;
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

}  // namespace ksl

extern "C" size_t ksl_moe_ffn_ctl_bytes(int64_t E) {
    return E > 0 ? ksl::ffn_ctl_words(E) * 4 : 0;
}

extern "C" int ksl_moe_ffn(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t T,
                           int64_t topk, const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t E, int64_t H,
                           int64_t I, int act, void* out2, void* out3, int32_t* ctl, void* stream) {
    if (T < 0 || topk <= 0) return KSL_ERR_SHAPE;
    if (T == 0) return KSL_OK;
    if (!ksl::ffn_supported(E, H, I, T * topk)) return KSL_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(ctl) % 4) return KSL_ERR_ALIGN;
    return ksl::launch_ffn(a16, sorted_rows, offsets, topk, gu_pack, dn_pack, E, H, I, act, out2, out3, ctl, T * topk,
                           static_cast<hipStream_t>(stream));
}

extern "C" int ksl_moe_ffn_set_wait_limit(int64_t cycles, int force_wait) {
    return ksl::ffn_set_wait_limit(cycles, force_wait);
}

extern "C" size_t ksl_moe_pack_gateup_bytes(int64_t E, int64_t H, int64_t I) {
    if (E <= 0 || H <= 0 || I <= 0 || H % 128 != 0 || I % 64 != 0) return 0;
    return static_cast<size_t>(E * I * H / 16 * 17);
}

extern "C" size_t ksl_moe_pack_down_bytes(int64_t E, int64_t H, int64_t I) {
    if (E <= 0 || H <= 0 || I <= 0 || H % 128 != 0 || I % 64 != 0) return 0;
    return static_cast<size_t>(E * H * I / 16 * 9);
}

extern "C" int ksl_moe_pack_gateup(const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H,
                                   int64_t I, uint8_t* gu_pack, void* stream) {
    using namespace ksl;
    if (E <= 0 || H <= 0 || I <= 0 || H % 128 != 0 || I % 64 != 0 || H > 8192 || I > 8192) return KSL_ERR_SHAPE;
    if (!gu_q || !gu_s || !gu_z || !gu_pack) return KSL_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(gu_q) % 16 || reinterpret_cast<uintptr_t>(gu_pack) % 16 ||
        reinterpret_cast<uintptr_t>(gu_s) % 2 || reinterpret_cast<uintptr_t>(gu_z) % 2)
        return KSL_ERR_ALIGN;
    const int64_t n = E * I * H / 16 * 17 / 16;
    const int64_t grid = (n + 255) / 256;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipLaunchKernelGGL(pack_gateup_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), gu_q, static_cast<const f16*>(gu_s),
                       static_cast<const f16*>(gu_z), gu_pack, static_cast<int>(E), static_cast<int>(H),
                       static_cast<int>(I));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

extern "C" int ksl_moe_pack_down(const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout, int64_t E,
                                 int64_t H, int64_t I, uint8_t* dn_pack, void* stream) {
    using namespace ksl;
    if (E <= 0 || H <= 0 || I <= 0 || H % 128 != 0 || I % 64 != 0 || H > 8192 || I > 8192) return KSL_ERR_SHAPE;
    if (!dn_q || !dn_s || !dn_z || !dn_pack) return KSL_ERR_ARG;
    if (dn_layout != KSL_DN_LAYOUT_REF && dn_layout != KSL_DN_LAYOUT_TILED) return KSL_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(dn_q) % 16 || reinterpret_cast<uintptr_t>(dn_pack) % 16 ||
        reinterpret_cast<uintptr_t>(dn_s) % 2 || reinterpret_cast<uintptr_t>(dn_z) % 2)
        return KSL_ERR_ALIGN;
    const int64_t n = E * H * I / 16 * 9 / 16;
    const int64_t grid = (n + 255) / 256;
    if (grid >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    hipLaunchKernelGGL(pack_down_kernel, dim3(static_cast<unsigned>(grid)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dn_q, static_cast<const f16*>(dn_s),
                       static_cast<const f16*>(dn_z), dn_layout, dn_pack, static_cast<int>(E), static_cast<int>(H),
                       static_cast<int>(I));
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}
