// Expert routing metadata on the GPU, plus the fp16 activation copy.
//
// Contract (kernels/fused_moe_w4.py:15-51, moe_align): expanded rows
// i = t*topk + slot are sorted stably by expert id (ids clamped to <= E; E is
// the dropped sentinel), each expert's run is padded to block_m, pad slots hold
// Nexp = T*topk, expert_ids[b] names the expert owning block b (E past the
// last block), and inv[i] is the sorted slot of row i (0 for dropped rows).
//
// One workgroup of 16 waves does the whole job in one launch:
//   1. each wave owns a contiguous range of rows and counts its rows per
//      expert in a private LDS row, 64 rows at a time: lanes holding the same
//      expert find each other with ballots over the id bits, the lowest such
//      lane adds the group size (no atomics);
//   2. one thread per expert turns the 16 per-wave counts into per-wave bases
//      (exclusive prefix over waves) and the expert total; a workgroup scan of
//      the padded block counts gives each expert's first slot;
//   3. each expert fills its own pad slots and block ids (disjoint writes);
//   4. each wave replays its rows in order and scatters slot = expert start +
//      wave base + rank among earlier equal lanes, so the order inside an
//      expert is the original row order (stable).
// Extra workgroups (blockIdx.x > 0) convert hidden to fp16 for the GEMMs,
// in the gate/up activation order (act_store_index<128>).
//
// The compact routing (block_m = 1) of at most kFastRows rows, the layer's
// case, takes a wider route: small workgroups each stage the keys in LDS once,
// then one wave per expert (plus one for the dropped rows) counts the rows
// below its expert (that count is the expert's first slot) and places its own
// rows in row order with one wave scan (stable, the same result), with no
// workgroup-wide scan and one barrier.
#include "ksl_common.h"

namespace ksl {
namespace {

constexpr int kRouteWaves = 16;
constexpr int kRouteThreads = kRouteWaves * kWave;
constexpr int kRouteSeg = 4;  // 64-row segments per wave per key batch
constexpr int kMaxExperts = 512;  // 16 waves x E int32 counters + E int64 starts fit in 64 KB of LDS

__device__ __forceinline__ uint64_t match_key(int key, int nbits) {
    uint64_t peers = ~0ull;
    for (int b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1;
        const uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return peers;
}

// Workgroup-wide exclusive scan of one int64 per thread (kRouteThreads threads).
__device__ int64_t block_exclusive_scan(int64_t v, int64_t* lds_wave, int64_t* total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int64_t incl = v;
    for (int off = 1; off < kWave; off <<= 1) {
        const int64_t o = __shfl_up(incl, off, kWave);
        if (lane >= off) incl += o;
    }
    if (lane == kWave - 1) lds_wave[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        int64_t wv = lane < kRouteWaves ? lds_wave[lane] : 0;
        int64_t wincl = wv;
        for (int off = 1; off < kWave; off <<= 1) {
            const int64_t o = __shfl_up(wincl, off, kWave);
            if (lane >= off) wincl += o;
        }
        if (lane < kRouteWaves) lds_wave[lane] = wincl - wv;
        if (lane == kRouteWaves - 1) *total = wincl;
    }
    __syncthreads();
    return lds_wave[wave] + incl - v;
}

struct RouteOut {
    int64_t Nexp, cap, max_blocks, block_m;
    int E;
    int32_t* zero;  // counters cleared by the routing (the expert FFN's), kCtlStride words apart, or null
    int nzero;
    // token-row mode (the moe_align_cuda contract): a real slot holds its
    // token r / row_div instead of the expanded row r, a padding slot pad_tok
    // (T) instead of Nexp. row_div == 0: expanded rows.
    int64_t row_div = 0, pad_tok = 0;
};

// Clear the n counters (kCtlStride words apart) a following launch expects
// to be zero (the one-launch expert FFN's unit queue and completion counts).
__device__ __forceinline__ void clear_words(int32_t* __restrict__ p, int n, int t, int nt) {
    for (int i = t; i < n; i += nt) p[static_cast<int64_t>(i) * kCtlStride] = 0;
}

template <typename IdxT>
__device__ void route_block(const int64_t* __restrict__ ids, const RouteOut& R, IdxT* __restrict__ sorted_rows,
                           IdxT* __restrict__ expert_ids, IdxT* __restrict__ inv,
                           int32_t* __restrict__ offsets);

// 8 consecutive values (logical columns c0 .. c0+7) as fp16 in K-slot order
// {0,4,1,5,2,6,3,7} at their gate/up activation position.
__device__ __forceinline__ void store_act8(f16* __restrict__ row, int c0, const float (&f)[8]) {
    f16x8 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        o[2 * j] = static_cast<f16>(f[j]);
        o[2 * j + 1] = static_cast<f16>(f[j + 4]);
    }
    *reinterpret_cast<f16x8*>(row + act_store_index<128>(c0)) = o;
}

constexpr int kFastRows = 4096;                           // routed rows of the barrier-free compact routing
constexpr int kFastWaves = 4;                             // waves per workgroup of the fast kernels
constexpr int kFastPad = kFastRows + kWave * 8;           // staged keys incl. padding to 8 per lane
constexpr int kFastPer = kFastPad / (kFastWaves * kWave); // ids loaded per thread at most

// Compact routing by the routing workgroups of the fast kernels. The
// workgroup stages every key in LDS once (key = expert id, E for a dropped
// id, E + 1 for padding past the last row); then wave `e` (0 <= e <= E)
// routes expert e with no further barrier: lane l takes the rows
// l*rpl .. l*rpl + rpl - 1 (rpl = ceil(Nexp / 64) rounded up to 8, read as
// 16-byte groups of 8 keys), so row order is (lane, then position). The
// expert's first slot is the number of rows with a smaller key (a wave sum of
// per-lane counts); a lane's first slot adds the expert's rows held by the
// lanes below it (an exclusive scan by ballots, one per bit of the count);
// each lane then places its own rows in order, walking a mask of them: the
// stable order of the reference. Wave E writes inv = 0 for dropped rows,
// offsets[E] and the unused tail slots (Nexp).
__device__ __forceinline__ void route_fast_wg(const int64_t* __restrict__ ids, int Nexp, int E,
                                              int32_t* __restrict__ sorted_rows, int32_t* __restrict__ inv,
                                              int32_t* __restrict__ offsets, int32_t* __restrict__ zero, int nzero) {
    __shared__ __attribute__((aligned(16))) uint16_t keys[kFastPad];
    const int lane = threadIdx.x & (kWave - 1);
    const int e = blockIdx.x * kFastWaves + threadIdx.x / kWave;
    const int rpl = ((Nexp + kWave - 1) / kWave + 7) & ~7;
    const int npad = rpl * kWave;
    // 1. keys into LDS: batches of 8 loads per thread, all issued before use
    constexpr int kBatch = 8;
    constexpr int kThreads = kFastWaves * kWave;
#pragma unroll
    for (int b = 0; b < kFastPer; b += kBatch) {
        if (b * kThreads >= npad) break;
        int64_t idv[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int r = (b + i) * kThreads + static_cast<int>(threadIdx.x);
            idv[i] = ids[r < Nexp ? r : 0];
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const int r = (b + i) * kThreads + static_cast<int>(threadIdx.x);
            const int64_t id = idv[i];
            const int key = r >= Nexp ? E + 1 : ((id < 0 || id > E) ? E : static_cast<int>(id));
            if (r < npad) keys[r] = static_cast<uint16_t>(key);
        }
    }
    __syncthreads();
    if (e > E) return;
    // 2. this lane's rows: the count below e and a mask of the rows at e
    //    (at most 64 per lane: Nexp <= kFastRows)
    const int r0 = lane * rpl;
    const u32x4* kq = reinterpret_cast<const u32x4*>(keys + r0);
    const int nq = rpl / 8;
    int c_lt = 0;
    uint64_t at_e = 0;
    for (int q = 0; q < nq; ++q) {
        const u32x4 v = kq[q];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int k = static_cast<int>((v[j >> 1] >> (16 * (j & 1))) & 0xFFFFu);
            c_lt += k < e ? 1 : 0;
            at_e |= static_cast<uint64_t>(k == e ? 1u : 0u) << (q * 8 + j);
        }
    }
    const int c_eq = __popcll(at_e);
    const int before = __ockl_wfred_add_i32(c_lt);
    // exclusive prefix of c_eq over the lanes, bit by bit (c_eq <= 64): per
    // bit, a ballot and the count of its lanes below this one
    int excl = 0;
#pragma unroll
    for (int b = 0; b < 7; ++b) {
        const uint64_t bm = __ballot((c_eq >> b) & 1);
        excl += static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bm >> 32),
                                                            __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bm), 0u)))
                << b;
    }
    // 3. scatter in row order: each lane walks only its rows at e
    int slot = before + excl;
    while (at_e != 0ull) {
        const int r = r0 + __ffsll(static_cast<long long>(at_e)) - 1;
        if (e < E) {
            sorted_rows[slot] = r;
            inv[r] = slot;
            ++slot;
        } else {
            inv[r] = 0;
        }
        at_e &= at_e - 1ull;
    }
    if (lane == 0) offsets[e] = before;
    if (e == E) {
        for (int p = before + lane; p < Nexp; p += kWave) sorted_rows[p] = Nexp;
        if (zero) clear_words(zero, nzero, lane, kWave);
    }
}

// Activation prep by workgroup blk of nblk: hidden -> fp16, 8-blocks in K-slot order.
template <int HD>
__device__ __forceinline__ void prep_rows(int blk, int nblk, const void* __restrict__ hidden, int64_t hidden_stride,
                                          int64_t T, int64_t H, f16* __restrict__ a16) {
    typedef typename Elem<HD>::T HT;
    const HT* h = static_cast<const HT*>(hidden);
    const int64_t vec_per_row = H / 8;
    const int64_t nvec = T * vec_per_row;
    const int64_t nthreads = static_cast<int64_t>(nblk) * kRouteThreads;
    for (int64_t v = static_cast<int64_t>(blk) * kRouteThreads + threadIdx.x; v < nvec; v += nthreads) {
        const int64_t t = v / vec_per_row;
        const int64_t c0 = (v - t * vec_per_row) * 8;
        float f[8];
        load8<HD>(h + t * hidden_stride + c0, f);
        store_act8(a16 + t * H, static_cast<int>(c0), f);
    }
}

// RMSNorm rows by workgroup blk of nblk: one wave per row (64 lanes x 8
// columns x NSTEP), the bf16-rounded norm output converted to fp16 in the
// gate/up activation order.
template <int XD, int WD, int NSTEP, bool HAS_W>
__device__ __forceinline__ void norm_rows(int blk, int nblk, const void* __restrict__ xv, int64_t x_stride,
                                          const void* __restrict__ wv, float eps, int64_t T, int64_t H,
                                          f16* __restrict__ a16) {
    typedef typename Elem<XD>::T XT;
    typedef typename Elem<WD>::T WT;
    const XT* x = static_cast<const XT*>(xv);
    const WT* w = static_cast<const WT*>(wv);
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int64_t nworkers = static_cast<int64_t>(nblk) * kRouteWaves;
    for (int64_t row = static_cast<int64_t>(blk) * kRouteWaves + wave; row < T; row += nworkers) {
        f16* arow = a16 + row * H;
        rms_row<XD, WD, NSTEP, HAS_W>(x + row * x_stride, w, static_cast<int>(H), eps, lane, 6, true,
                                      [&](int, int c0, const float (&v)[8]) { store_act8(arow, c0, v); });
    }
}

template <typename IdxT, int HD>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(
    const int64_t* __restrict__ ids, RouteOut R, IdxT* __restrict__ sorted_rows,
    IdxT* __restrict__ expert_ids, IdxT* __restrict__ inv, int32_t* __restrict__ offsets,
    // fused activation prep (blockIdx.x > 0)
    const void* __restrict__ hidden, int64_t hidden_stride, int64_t T, int64_t H,
    f16* __restrict__ a16) {
    if (blockIdx.x > 0) {
        prep_rows<HD>(blockIdx.x - 1, gridDim.x - 1, hidden, hidden_stride, T, H, a16);
        return;
    }
    route_block<IdxT>(ids, R, sorted_rows, expert_ids, inv, offsets);
}

// RMSNorm of each token row fused with the activation prep: one wave per row
// (64 lanes x 8 columns x NSTEP), the bf16-rounded norm output converted to
// fp16 in the gate/up activation order. Workgroup 0 builds the routing.
template <int XD, int WD, int NSTEP, bool HAS_W>
__global__ __launch_bounds__(kRouteThreads) void route_norm_kernel(
    const int64_t* __restrict__ ids, RouteOut R, int32_t* __restrict__ sorted_rows,
    int32_t* __restrict__ inv, int32_t* __restrict__ offsets, const void* __restrict__ xv,
    int64_t x_stride, const void* __restrict__ wv, float eps, int64_t T, int64_t H,
    f16* __restrict__ a16) {
    if (blockIdx.x == 0) {
        route_block<int32_t>(ids, R, sorted_rows, nullptr, inv, offsets);
        return;
    }
    norm_rows<XD, WD, NSTEP, HAS_W>(blockIdx.x - 1, gridDim.x - 1, xv, x_stride, wv, eps, T, H, a16);
}

// Fast compact routing (at most kFastRows rows) and the activation prep in one
// launch of kFastWaves-wave workgroups: workgroups below nrw route (wave =
// expert), the rest convert hidden to fp16 (one row per wave).
template <int HD>
__global__ __launch_bounds__(kFastWaves * kWave) void route_fast_kernel(
    const int64_t* __restrict__ ids, int Nexp, int E, int nrw, int32_t* __restrict__ sorted_rows,
    int32_t* __restrict__ inv, int32_t* __restrict__ offsets, const void* __restrict__ hidden,
    int64_t hidden_stride, int64_t T, int64_t H, f16* __restrict__ a16, int32_t* __restrict__ zero, int nzero) {
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (static_cast<int>(blockIdx.x) < nrw) {
        route_fast_wg(ids, Nexp, E, sorted_rows, inv, offsets, zero, nzero);
        return;
    }
    const int64_t row = static_cast<int64_t>(blockIdx.x - nrw) * kFastWaves + wave;
    if (row >= T) return;
    typedef typename Elem<HD>::T HT;
    const HT* h = static_cast<const HT*>(hidden) + row * hidden_stride;
    for (int c0 = lane * 8; c0 < H; c0 += kWave * 8) {
        float f[8];
        load8<HD>(h + c0, f);
        store_act8(a16 + row * H, c0, f);
    }
}

// Fast compact routing fused with the RMSNorm -> fp16 activations (one row per
// wave in the workgroups from nrw on).
template <int XD, int WD, int NSTEP, bool HAS_W>
__global__ __launch_bounds__(kFastWaves * kWave) void route_norm_fast_kernel(
    const int64_t* __restrict__ ids, int Nexp, int E, int nrw, int32_t* __restrict__ sorted_rows,
    int32_t* __restrict__ inv, int32_t* __restrict__ offsets, const void* __restrict__ xv, int64_t x_stride,
    const void* __restrict__ wv, float eps, int64_t T, int64_t H, f16* __restrict__ a16, int32_t* __restrict__ zero,
    int nzero) {
    const int wave = threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (static_cast<int>(blockIdx.x) < nrw) {
        route_fast_wg(ids, Nexp, E, sorted_rows, inv, offsets, zero, nzero);
        return;
    }
    const int64_t row = static_cast<int64_t>(blockIdx.x - nrw) * kFastWaves + wave;
    if (row >= T) return;
    typedef typename Elem<XD>::T XT;
    typedef typename Elem<WD>::T WT;
    f16* arow = a16 + row * H;
    rms_row<XD, WD, NSTEP, HAS_W>(static_cast<const XT*>(xv) + row * x_stride, static_cast<const WT*>(wv),
                                  static_cast<int>(H), eps, lane, 6, true,
                                  [&](int, int c0, const float (&v)[8]) { store_act8(arow, c0, v); });
}

template <typename IdxT>
__device__ void route_block(const int64_t* __restrict__ ids, const RouteOut& R, IdxT* __restrict__ sorted_rows,
                           IdxT* __restrict__ expert_ids, IdxT* __restrict__ inv,
                           int32_t* __restrict__ offsets) {
    const int64_t Nexp = R.Nexp, cap = R.cap, max_blocks = R.max_blocks, block_m = R.block_m;
    const int E = R.E;
    const IdxT pad_row = static_cast<IdxT>(R.row_div ? R.pad_tok : Nexp);
    extern __shared__ int32_t lds[];
    int32_t* wcnt = lds;                                  // [kRouteWaves][E]
    int64_t* estart = reinterpret_cast<int64_t*>(lds + kRouteWaves * E);  // [E], 8-byte aligned (16*E ints)
    int64_t* scan_tmp = estart + E;                       // [kRouteWaves]
    int64_t* total_blocks = scan_tmp + kRouteWaves;       // [1]

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
    int nbits = 1;
    while ((1 << nbits) < E + 2) ++nbits;  // keys 0..E+1

    for (int i = threadIdx.x; i < kRouteWaves * E; i += kRouteThreads) wcnt[i] = 0;
    __syncthreads();

    // rows owned by this wave: [r_begin, r_end), whole 64-row segments
    const int64_t per_wave = ((Nexp + kRouteWaves - 1) / kRouteWaves + kWave - 1) / kWave * kWave;
    const int64_t r_begin = wave * per_wave;
    const int64_t r_end = r_begin + per_wave < Nexp ? r_begin + per_wave : Nexp;
    int32_t* mycnt = wcnt + wave * E;

    // Keys of this wave's rows, kRouteSeg 64-row segments at a time: all loads of
    // a batch go out together (clamped indices, one round trip); with at most
    // kRouteSeg segments per wave (T * topk <= 4096) the keys stay in registers
    // for the scatter phase.
    const int64_t nrows = r_end > r_begin ? r_end - r_begin : 0;
    const int nseg = static_cast<int>((nrows + kWave - 1) / kWave);
    int keys[kRouteSeg];
    auto load_keys = [&](int seg0) {
#pragma unroll
        for (int s = 0; s < kRouteSeg; ++s) {
            const int64_t r = r_begin + static_cast<int64_t>(seg0 + s) * kWave + lane;
            const bool ok = r < r_end;
            const int64_t id = ids[ok ? r : 0];
            keys[s] = !ok ? E + 1 : ((id < 0 || id > E) ? E : static_cast<int>(id));  // E + 1: not a row
        }
    };

    // ---- 1. per-wave counts ----
    for (int seg0 = 0; seg0 < nseg; seg0 += kRouteSeg) {
        load_keys(seg0);
#pragma unroll
        for (int s = 0; s < kRouteSeg; ++s) {
            if (seg0 + s < nseg) {
                const int key = keys[s];
                const uint64_t peers = match_key(key, nbits);
                const bool leader = (__builtin_ctzll(peers) == lane);
                if (leader && key < E) mycnt[key] += __builtin_popcountll(peers);
            }
        }
    }
    __syncthreads();

    // ---- 2. per-wave bases, totals, expert starts ----
    int64_t cnt = 0, nblk = 0;
    const int e = threadIdx.x;
    if (e < E) {
        int32_t run = 0;
        for (int w = 0; w < kRouteWaves; ++w) {
            const int32_t c = wcnt[w * E + e];
            wcnt[w * E + e] = run;
            run += c;
        }
        cnt = run;
        nblk = (cnt + block_m - 1) / block_m;
    }
    const int64_t blk_start = block_exclusive_scan(e < E ? nblk : 0, scan_tmp, total_blocks);
    if (e < E) estart[e] = blk_start * block_m;
    const int64_t tot_blocks = *total_blocks;

    // ---- 3. pad slots, block ids, offsets (disjoint writes) ----
    if (e < E) {
        if (sorted_rows) {
            for (int64_t p = blk_start * block_m + cnt; p < (blk_start + nblk) * block_m; ++p)
                sorted_rows[p] = pad_row;
        }
        if (expert_ids) {
            for (int64_t b = blk_start; b < blk_start + nblk; ++b) expert_ids[b] = static_cast<IdxT>(e);
        }
        if (offsets) offsets[e] = static_cast<int32_t>(blk_start * block_m);
    }
    if (offsets && threadIdx.x == 0) offsets[E] = static_cast<int32_t>(tot_blocks * block_m);
    if (R.zero) clear_words(R.zero, R.nzero, threadIdx.x, kRouteThreads);
    if (sorted_rows) {
        for (int64_t p = tot_blocks * block_m + threadIdx.x; p < cap; p += kRouteThreads)
            sorted_rows[p] = pad_row;
    }
    if (expert_ids) {
        for (int64_t b = tot_blocks + threadIdx.x; b < max_blocks; b += kRouteThreads)
            expert_ids[b] = static_cast<IdxT>(E);
    }
    __syncthreads();

    // ---- 4. stable scatter ----
    for (int seg0 = 0; seg0 < nseg; seg0 += kRouteSeg) {
        if (nseg > kRouteSeg) load_keys(seg0);  // else the keys are still in registers
#pragma unroll
        for (int s = 0; s < kRouteSeg; ++s) {
            if (seg0 + s < nseg) {
                const int64_t r = r_begin + static_cast<int64_t>(seg0 + s) * kWave + lane;
                const int key = keys[s];
                const uint64_t peers = match_key(key, nbits);
                if (key < E) {
                    const int32_t before = mycnt[key];
                    const int64_t slot = estart[key] + before + __builtin_popcountll(peers & lt_mask);
                    if (sorted_rows) sorted_rows[slot] = static_cast<IdxT>(R.row_div ? r / R.row_div : r);
                    if (inv) inv[r] = static_cast<IdxT>(slot);
                    if (__builtin_ctzll(peers) == lane) mycnt[key] = before + __builtin_popcountll(peers);
                } else if (key == E) {
                    if (inv) inv[r] = 0;
                }
            }
        }
    }
}

// ---- multi-block compact routing (more than kFastRows rows, a workspace for
// the block counts): the single-workgroup algorithm above with its waves
// spread over blocks of kMbRows = 1024 rows. Launch 1: every block counts its
// rows per expert (wave w of block b owns rows b*kMbRows + w*64 .. +64, one
// 64-row segment held in registers) and writes the block's counts to
// bcnt[b*E + e]. Launch 2: every block counts again, adds the counts of the
// blocks before it and of the lower experts (a scan over e of the column sums
// of bcnt) to get each wave's first slot per expert, and places its rows in
// row order, the stable order of the reference; block 0 writes offsets and
// the unused tail slots.
constexpr int kMbSeg = 1;  // 64-row segments per wave
constexpr int kMbRows = kRouteWaves * kMbSeg * kWave;

__device__ __forceinline__ void mb_keys(const int64_t* __restrict__ ids, int64_t Nexp, int E, int64_t r_begin,
                                        int (&keys)[kMbSeg]) {
    const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
    for (int s = 0; s < kMbSeg; ++s) {
        const int64_t r = r_begin + s * kWave + lane;
        const bool ok = r < Nexp;
        const int64_t id = ids[ok ? r : 0];
        keys[s] = !ok ? E + 1 : ((id < 0 || id > E) ? E : static_cast<int>(id));  // E + 1: not a row
    }
}

// Per-wave counts of the block's rows into wcnt[wave][e] (zeroed here).
__device__ __forceinline__ void mb_wave_counts(const int (&keys)[kMbSeg], int E, int nbits, int32_t* wcnt) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    for (int i = threadIdx.x; i < kRouteWaves * E; i += kRouteThreads) wcnt[i] = 0;
    __syncthreads();
    int32_t* mycnt = wcnt + wave * E;
#pragma unroll
    for (int s = 0; s < kMbSeg; ++s) {
        const uint64_t peers = match_key(keys[s], nbits);
        if (__builtin_ctzll(peers) == lane && keys[s] < E) mycnt[keys[s]] += __builtin_popcountll(peers);
    }
    __syncthreads();
}

__device__ __forceinline__ int mb_nbits(int E) {
    int nbits = 1;
    while ((1 << nbits) < E + 2) ++nbits;  // keys 0..E+1
    return nbits;
}

__device__ void route_mb_count(const int64_t* __restrict__ ids, int64_t Nexp, int E, int b,
                               int32_t* __restrict__ bcnt) {
    extern __shared__ int32_t lds[];
    const int wave = threadIdx.x / kWave;
    int keys[kMbSeg];
    mb_keys(ids, Nexp, E, static_cast<int64_t>(b) * kMbRows + wave * (kMbSeg * kWave), keys);
    mb_wave_counts(keys, E, mb_nbits(E), lds);
    for (int e = threadIdx.x; e < E; e += kRouteThreads) {
        int32_t c = 0;
        for (int w = 0; w < kRouteWaves; ++w) c += lds[w * E + e];
        bcnt[static_cast<int64_t>(b) * E + e] = c;
    }
}

__global__ __launch_bounds__(kRouteThreads) void route_mb_scatter_kernel(
    const int64_t* __restrict__ ids, int64_t Nexp, int E, int nb, const int32_t* __restrict__ bcnt,
    int32_t* __restrict__ sorted_rows, int32_t* __restrict__ inv, int32_t* __restrict__ offsets,
    int32_t* __restrict__ zero, int nzero) {
    extern __shared__ int32_t lds[];
    int32_t* wcnt = lds;                                                  // [kRouteWaves][E]
    int64_t* estart = reinterpret_cast<int64_t*>(lds + kRouteWaves * E);  // [E]
    int64_t* scan_tmp = estart + E;                                       // [kRouteWaves]
    int64_t* total = scan_tmp + kRouteWaves;                              // [1]
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int b = blockIdx.x;
    const int nbits = mb_nbits(E);
    const int64_t r_begin = static_cast<int64_t>(b) * kMbRows + wave * (kMbSeg * kWave);
    int keys[kMbSeg];
    mb_keys(ids, Nexp, E, r_begin, keys);
    mb_wave_counts(keys, E, nbits, wcnt);
    // expert e (thread e): rows of all blocks, and of the blocks before b
    const int e = threadIdx.x;
    int64_t tot = 0;
    if (e < E) {
        int32_t pre = 0, all = 0;
#pragma unroll 16
        for (int bb = 0; bb < nb; ++bb) {
            const int32_t c = bcnt[static_cast<int64_t>(bb) * E + e];
            all += c;
            pre += bb < b ? c : 0;
        }
        tot = all;
        int32_t run = pre;
        for (int w = 0; w < kRouteWaves; ++w) {
            const int32_t c = wcnt[w * E + e];
            wcnt[w * E + e] = run;
            run += c;
        }
    }
    const int64_t start = block_exclusive_scan(e < E ? tot : 0, scan_tmp, total);
    if (e < E) estart[e] = start;
    if (b == 0) {
        if (e < E) offsets[e] = static_cast<int32_t>(start);
        if (threadIdx.x == 0) offsets[E] = static_cast<int32_t>(*total);
        for (int64_t p = *total + threadIdx.x; p < Nexp; p += kRouteThreads) sorted_rows[p] = static_cast<int32_t>(Nexp);
        if (zero) clear_words(zero, nzero, threadIdx.x, kRouteThreads);
    }
    __syncthreads();
    int32_t* mycnt = wcnt + wave * E;
    const uint64_t lt_mask = (1ull << lane) - 1ull;
#pragma unroll
    for (int s = 0; s < kMbSeg; ++s) {
        const int64_t r = r_begin + s * kWave + lane;
        const int key = keys[s];
        const uint64_t peers = match_key(key, nbits);
        if (key < E) {
            const int32_t before = mycnt[key];
            const int64_t slot = estart[key] + before + __builtin_popcountll(peers & lt_mask);
            sorted_rows[slot] = static_cast<int32_t>(r);
            inv[r] = static_cast<int32_t>(slot);
            if (__builtin_ctzll(peers) == lane) mycnt[key] = before + __builtin_popcountll(peers);
        } else if (key == E) {
            inv[r] = 0;
        }
    }
}

// Launch 1 of the multi-block routing with the RMSNorm rows (workgroups >= nb).
template <int XD, int WD, int NSTEP, bool HAS_W>
__global__ __launch_bounds__(kRouteThreads) void route_norm_mb_kernel(
    const int64_t* __restrict__ ids, int64_t Nexp, int E, int nb, int32_t* __restrict__ bcnt,
    const void* __restrict__ xv, int64_t x_stride, const void* __restrict__ wv, float eps, int64_t T, int64_t H,
    f16* __restrict__ a16) {
    if (static_cast<int>(blockIdx.x) < nb) {
        route_mb_count(ids, Nexp, E, blockIdx.x, bcnt);
        return;
    }
    norm_rows<XD, WD, NSTEP, HAS_W>(blockIdx.x - nb, gridDim.x - nb, xv, x_stride, wv, eps, T, H, a16);
}

// Launch 1 of the multi-block routing with the activation prep (workgroups >= nb).
template <int HD>
__global__ __launch_bounds__(kRouteThreads) void route_mb_kernel(
    const int64_t* __restrict__ ids, int64_t Nexp, int E, int nb, int32_t* __restrict__ bcnt,
    const void* __restrict__ hidden, int64_t hidden_stride, int64_t T, int64_t H, f16* __restrict__ a16) {
    if (static_cast<int>(blockIdx.x) < nb) {
        route_mb_count(ids, Nexp, E, blockIdx.x, bcnt);
        return;
    }
    if (a16) prep_rows<HD>(blockIdx.x - nb, gridDim.x - nb, hidden, hidden_stride, T, H, a16);
}

size_t route_lds_bytes(int64_t E) {
    return kRouteWaves * E * sizeof(int32_t) + (E + kRouteWaves + 1) * sizeof(int64_t);
}

template <typename IdxT, int HD>
int launch_route(const int64_t* ids, int64_t T, int64_t topk, int64_t E, int64_t block_m,
                 IdxT* sorted_rows, int64_t cap, IdxT* expert_ids, int64_t max_blocks, IdxT* inv,
                 int32_t* offsets, const void* hidden, int64_t hstride, int64_t H, f16* a16,
                 hipStream_t st, int32_t* zero = nullptr, int nzero = 0, bool token_rows = false) {
    const int64_t Nexp = T * topk;
    unsigned grid = 1;
    if (a16) {
        const int64_t nvec = T * (H / 8);
        int64_t want = (nvec + kRouteThreads * 4 - 1) / (kRouteThreads * 4);
        if (want < 1) want = 1;
        if (want > 2048) want = 2048;
        grid += static_cast<unsigned>(want);
    }
    const size_t lds_bytes = route_lds_bytes(E);
    RouteOut R{Nexp, cap, max_blocks, block_m, static_cast<int>(E), zero, nzero};
    if (token_rows) {
        R.row_div = topk;
        R.pad_tok = T;
    }
    hipLaunchKernelGGL((route_kernel<IdxT, HD>), dim3(grid), dim3(kRouteThreads), lds_bytes, st, ids, R,
                       sorted_rows, expert_ids, inv, offsets, hidden, hstride, T, H, a16);
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}

}  // namespace
}  // namespace ksl

extern "C" int ksl_moe_align(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                             int64_t block_m, int64_t* sorted_rows, int64_t* expert_ids,
                             int64_t* inv, void* stream) {
    using namespace ksl;
    if (T < 0 || topk <= 0 || E <= 0 || E > kMaxExperts || block_m <= 0) return KSL_ERR_SHAPE;
    if (T * topk >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    if (T > 0 && !topk_ids) return KSL_ERR_ARG;
    const int64_t Nexp = T * topk;
    const int64_t max_blocks = (Nexp + block_m - 1) / block_m + E;
    const int64_t cap = max_blocks * block_m;
    return launch_route<int64_t, KSL_DTYPE_BF16>(topk_ids, T, topk, E, block_m, sorted_rows, cap,
                                                 expert_ids, max_blocks, inv, nullptr, nullptr, 0, 0,
                                                 nullptr, static_cast<hipStream_t>(stream));
}

// Capacity of the moe_align_cuda contract (kernels/fused_moe_w4_v2.py:59-64):
// mx = Nexp + E*(block_m - 1) slots (at most Nexp*block_m when Nexp < E),
// rounded up to whole blocks. The used blocks never exceed it: an expert with
// c > 0 rows takes at most c + block_m - 1 slots.
extern "C" int64_t ksl_moe_align_i32_capacity(int64_t T, int64_t topk, int64_t E, int64_t block_m) {
    if (T < 0 || topk <= 0 || E <= 0 || block_m <= 0) return -1;
    const int64_t Nexp = T * topk;
    int64_t mx = Nexp + E * (block_m - 1);
    if (Nexp < E && Nexp * block_m < mx) mx = Nexp * block_m;
    return (mx + block_m - 1) / block_m * block_m;
}

extern "C" int ksl_moe_align_i32(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                                 int64_t block_m, int32_t* a_row, int32_t* expert_ids, int32_t* inv,
                                 void* stream) {
    using namespace ksl;
    if (T < 0 || topk <= 0 || E <= 0 || E > kMaxExperts || block_m <= 0) return KSL_ERR_SHAPE;
    if (T * topk >= (int64_t(1) << 31) || T * topk + E * block_m >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    const int64_t cap = ksl_moe_align_i32_capacity(T, topk, E, block_m);
    if (cap == 0) return KSL_OK;  // no rows: nothing to write
    if (!topk_ids || !a_row || !expert_ids || !inv) return KSL_ERR_ARG;
    return launch_route<int32_t, KSL_DTYPE_BF16>(topk_ids, T, topk, E, block_m, a_row, cap, expert_ids,
                                                 cap / block_m, inv, nullptr, nullptr, 0, 0, nullptr,
                                                 static_cast<hipStream_t>(stream), nullptr, 0, true);
}

namespace ksl {
int route_compact(const int64_t* ids, int64_t T, int64_t topk, int64_t E, int32_t* sorted_rows,
                  int32_t* offsets, int32_t* inv, const void* hidden, int hd, int64_t hstride,
                  int64_t H, void* a16, int32_t* bcnt, hipStream_t st, int32_t* zero, int nzero) {
    if (T < 0 || topk <= 0 || E <= 0 || E > kMaxExperts) return KSL_ERR_SHAPE;
    if (T * topk >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    if (T > 0 && !ids) return KSL_ERR_ARG;
    if (a16) {
        if (!hidden || H <= 0 || H % 8 != 0 || hstride < H || hstride % 8 != 0) return KSL_ERR_SHAPE;
        if (reinterpret_cast<uintptr_t>(hidden) % 16 || reinterpret_cast<uintptr_t>(a16) % 16)
            return KSL_ERR_ALIGN;
    }
    const int64_t Nexp = T * topk;
    f16* a = static_cast<f16*>(a16);
    if (Nexp > 0 && Nexp <= kFastRows) {
        const int nrw = static_cast<int>((E + 1 + kFastWaves - 1) / kFastWaves);
        const int64_t nprep = a ? (T + kFastWaves - 1) / kFastWaves : 0;
        const dim3 grid(static_cast<unsigned>(nrw + nprep)), block(kFastWaves * kWave);
        switch (hd) {
            case KSL_DTYPE_BF16:
                hipLaunchKernelGGL(route_fast_kernel<KSL_DTYPE_BF16>, grid, block, 0, st, ids, static_cast<int>(Nexp),
                                   static_cast<int>(E), nrw, sorted_rows, inv, offsets, hidden, hstride, T, H, a, zero, nzero);
                break;
            case KSL_DTYPE_F16:
                hipLaunchKernelGGL(route_fast_kernel<KSL_DTYPE_F16>, grid, block, 0, st, ids, static_cast<int>(Nexp),
                                   static_cast<int>(E), nrw, sorted_rows, inv, offsets, hidden, hstride, T, H, a, zero, nzero);
                break;
            case KSL_DTYPE_F32:
                hipLaunchKernelGGL(route_fast_kernel<KSL_DTYPE_F32>, grid, block, 0, st, ids, static_cast<int>(Nexp),
                                   static_cast<int>(E), nrw, sorted_rows, inv, offsets, hidden, hstride, T, H, a, zero, nzero);
                break;
            default:
                return KSL_ERR_ARG;
        }
        KSL_LAUNCH_CHECK();
        return KSL_OK;
    }
    if (bcnt && Nexp > kFastRows) {
        // multi-block routing: count (+ activation prep), then scatter
        const int nb = static_cast<int>((Nexp + kMbRows - 1) / kMbRows);
        int64_t nprep = 0;
        if (a) {
            nprep = (T * (H / 8) + kRouteThreads * 4 - 1) / (kRouteThreads * 4);
            if (nprep > 2048) nprep = 2048;
        }
        const dim3 grid(static_cast<unsigned>(nb + nprep)), block(kRouteThreads);
        const size_t lds = route_lds_bytes(E);
        const int e = static_cast<int>(E);
        switch (hd) {
            case KSL_DTYPE_BF16:
                hipLaunchKernelGGL(route_mb_kernel<KSL_DTYPE_BF16>, grid, block, lds, st, ids, Nexp, e, nb, bcnt, hidden,
                                   hstride, T, H, a);
                break;
            case KSL_DTYPE_F16:
                hipLaunchKernelGGL(route_mb_kernel<KSL_DTYPE_F16>, grid, block, lds, st, ids, Nexp, e, nb, bcnt, hidden,
                                   hstride, T, H, a);
                break;
            case KSL_DTYPE_F32:
                hipLaunchKernelGGL(route_mb_kernel<KSL_DTYPE_F32>, grid, block, lds, st, ids, Nexp, e, nb, bcnt, hidden,
                                   hstride, T, H, a);
                break;
            default:
                return KSL_ERR_ARG;
        }
        KSL_LAUNCH_CHECK();
        hipLaunchKernelGGL(route_mb_scatter_kernel, dim3(nb), block, lds, st, ids, Nexp, e, nb, bcnt, sorted_rows, inv,
                           offsets, zero, nzero);
        KSL_LAUNCH_CHECK();
        return KSL_OK;
    }
    // compact layout: block_m = 1; slots past offsets[E] hold Nexp, only the
    // first Nexp slots are materialised.
    switch (hd) {
        case KSL_DTYPE_BF16:
            return launch_route<int32_t, KSL_DTYPE_BF16>(ids, T, topk, E, 1, sorted_rows, Nexp, nullptr, 0,
                                                         inv, offsets, hidden, hstride, H, a, st, zero, nzero);
        case KSL_DTYPE_F16:
            return launch_route<int32_t, KSL_DTYPE_F16>(ids, T, topk, E, 1, sorted_rows, Nexp, nullptr, 0,
                                                        inv, offsets, hidden, hstride, H, a, st, zero, nzero);
        case KSL_DTYPE_F32:
            return launch_route<int32_t, KSL_DTYPE_F32>(ids, T, topk, E, 1, sorted_rows, Nexp, nullptr, 0,
                                                        inv, offsets, hidden, hstride, H, a, st, zero, nzero);
    }
    return KSL_ERR_ARG;
}
}  // namespace ksl

namespace ksl {
namespace {
template <int XD, int WD, bool HAS_W>
int launch_route_norm_ns(int nstep, const int64_t* ids, const RouteOut& R, int32_t* sorted_rows, int32_t* inv,
                         int32_t* offsets, const void* x, int64_t xs, const void* w, float eps, int64_t T,
                         int64_t H, f16* a16, int32_t* bcnt, hipStream_t st) {
    if (R.Nexp > 0 && R.Nexp <= kFastRows) {
        const int nrw = (R.E + 1 + kFastWaves - 1) / kFastWaves;
        const dim3 fgrid(static_cast<unsigned>(nrw + (T + kFastWaves - 1) / kFastWaves)), fblock(kFastWaves * kWave);
        const int nexp = static_cast<int>(R.Nexp);
#define KSL_RNF(NS)                                                                                          \
    hipLaunchKernelGGL((route_norm_fast_kernel<XD, WD, NS, HAS_W>), fgrid, fblock, 0, st, ids, nexp, R.E, nrw, \
                       sorted_rows, inv, offsets, x, xs, w, eps, T, H, a16, R.zero, R.nzero)
        if (nstep <= 1) KSL_RNF(1);
        else if (nstep <= 2) KSL_RNF(2);
        else if (nstep <= 4) KSL_RNF(4);
        else if (nstep <= 6) KSL_RNF(6);
        else KSL_RNF(8);
#undef KSL_RNF
        KSL_LAUNCH_CHECK();
        return KSL_OK;
    }
    int64_t want = (T + kRouteWaves - 1) / kRouteWaves;
    if (want < 1) want = 1;
    if (want > 4096) want = 4096;
    const size_t lds = route_lds_bytes(R.E);
    if (bcnt && R.Nexp > kFastRows) {
        // multi-block routing: count + norm rows, then scatter
        const int nb = static_cast<int>((R.Nexp + kMbRows - 1) / kMbRows);
        const dim3 mgrid(static_cast<unsigned>(nb + want));
#define KSL_RNM(NS)                                                                                          \
    hipLaunchKernelGGL((route_norm_mb_kernel<XD, WD, NS, HAS_W>), mgrid, dim3(kRouteThreads), lds, st, ids, R.Nexp, \
                       R.E, nb, bcnt, x, xs, w, eps, T, H, a16)
        if (nstep <= 1) KSL_RNM(1);
        else if (nstep <= 2) KSL_RNM(2);
        else if (nstep <= 4) KSL_RNM(4);
        else if (nstep <= 6) KSL_RNM(6);
        else KSL_RNM(8);
#undef KSL_RNM
        KSL_LAUNCH_CHECK();
        hipLaunchKernelGGL(route_mb_scatter_kernel, dim3(nb), dim3(kRouteThreads), lds, st, ids, R.Nexp, R.E, nb, bcnt,
                           sorted_rows, inv, offsets, R.zero, R.nzero);
        KSL_LAUNCH_CHECK();
        return KSL_OK;
    }
    const unsigned grid = 1 + static_cast<unsigned>(want);
#define KSL_RN(NS)                                                                                         \
    hipLaunchKernelGGL((route_norm_kernel<XD, WD, NS, HAS_W>), dim3(grid), dim3(kRouteThreads), lds, st, ids, R, \
                       sorted_rows, inv, offsets, x, xs, w, eps, T, H, a16)
    if (nstep <= 1) KSL_RN(1);
    else if (nstep <= 2) KSL_RN(2);
    else if (nstep <= 4) KSL_RN(4);
    else if (nstep <= 6) KSL_RN(6);
    else KSL_RN(8);
#undef KSL_RN
    KSL_LAUNCH_CHECK();
    return KSL_OK;
}
template <int XD>
int launch_route_norm_x(int wd, int nstep, const int64_t* ids, const RouteOut& R, int32_t* sorted_rows, int32_t* inv,
                        int32_t* offsets, const void* x, int64_t xs, const void* w, float eps, int64_t T,
                        int64_t H, f16* a16, int32_t* bcnt, hipStream_t st) {
    if (!w) return launch_route_norm_ns<XD, KSL_DTYPE_BF16, false>(nstep, ids, R, sorted_rows, inv, offsets, x, xs, w, eps, T, H, a16, bcnt, st);
    switch (wd) {
        case KSL_DTYPE_BF16: return launch_route_norm_ns<XD, KSL_DTYPE_BF16, true>(nstep, ids, R, sorted_rows, inv, offsets, x, xs, w, eps, T, H, a16, bcnt, st);
        case KSL_DTYPE_F16: return launch_route_norm_ns<XD, KSL_DTYPE_F16, true>(nstep, ids, R, sorted_rows, inv, offsets, x, xs, w, eps, T, H, a16, bcnt, st);
        case KSL_DTYPE_F32: return launch_route_norm_ns<XD, KSL_DTYPE_F32, true>(nstep, ids, R, sorted_rows, inv, offsets, x, xs, w, eps, T, H, a16, bcnt, st);
    }
    return KSL_ERR_ARG;
}
}  // namespace

// Routing plus RMSNorm -> fp16 activations in one launch (the layer path).
int route_norm(const int64_t* ids, int64_t T, int64_t topk, int64_t E, int32_t* sorted_rows,
               int32_t* offsets, int32_t* inv, const void* x, int xd, int64_t xs, const void* w,
               int wd, float eps, int64_t H, void* a16, int32_t* bcnt, hipStream_t st, int32_t* zero, int nzero) {
    if (T < 0 || topk <= 0 || E <= 0 || E > kMaxExperts) return KSL_ERR_SHAPE;
    if (T * topk >= (int64_t(1) << 31)) return KSL_ERR_SHAPE;
    if (H <= 0 || H % 128 != 0 || H > 4096 || xs < H || xs % 8 != 0) return KSL_ERR_SHAPE;
    if (T > 0 && (!ids || !x || !a16)) return KSL_ERR_ARG;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(a16) % 16 ||
        (w && reinterpret_cast<uintptr_t>(w) % 16))
        return KSL_ERR_ALIGN;
    const int64_t Nexp = T * topk;
    RouteOut R{Nexp, Nexp, 0, 1, static_cast<int>(E), zero, nzero};
    const int nstep = static_cast<int>((H / 8 + kWave - 1) / kWave);
    f16* a = static_cast<f16*>(a16);
    switch (xd) {
        case KSL_DTYPE_BF16: return launch_route_norm_x<KSL_DTYPE_BF16>(wd, nstep, ids, R, sorted_rows, inv, offsets, x, xs, w, eps, T, H, a, bcnt, st);
        case KSL_DTYPE_F16: return launch_route_norm_x<KSL_DTYPE_F16>(wd, nstep, ids, R, sorted_rows, inv, offsets, x, xs, w, eps, T, H, a, bcnt, st);
    }
    return KSL_ERR_ARG;
}
}  // namespace ksl

extern "C" int ksl_moe_route(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                             int32_t* sorted_rows, int32_t* offsets, int32_t* inv,
                             const void* hidden, int hidden_dtype, int64_t hidden_stride, int64_t H,
                             void* a16, void* stream) {
    return ksl::route_compact(topk_ids, T, topk, E, sorted_rows, offsets, inv, hidden, hidden_dtype,
                              hidden_stride, H, a16, nullptr, static_cast<hipStream_t>(stream), nullptr, 0);
}
