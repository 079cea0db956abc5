/* CPU restatement of the bit-exact parts of the fused MoE path, in plain C.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for tests/, smoke() and the
 * cpu_baseline leg of bench.py. Nothing in the product links it.
 *
 *  - orc_combine: kernels/fused_moe_w4_v2.py:248-263. y[t,:] is an fp32
 *    fused-multiply-add chain over the top-k slots in fixed order k=0..tk-1,
 *    starting from 0, of fp32(w[t,k]) * fp32(out3[inv[t*tk+k], :]); Triton
 *    contracts `acc += w * x` to an FMA. Stored as bf16 (RNE) or fp16.
 *  - orc_moe_align: kernels/fused_moe_w4.py:15-51, restated as a counting
 *    sort (stable by construction) instead of the reference's argsort, so
 *    that it is an independent check on the numpy restatement.
 *  - orc_philox_first: the first output word of Philox4x32-10 for counters
 *    (c, 0, 0, 0) and one key: the noise source of the Gumbel-max sampler
 *    (kernels/fused_sampler_ops.py:67, tl.rand; Triton's philox_impl), the
 *    same algorithm as oracle/sampler_oracle.py:philox4x32, in C for the
 *    full-vocabulary rows (262144 columns) of the parity tests.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so only the explicit fmaf
 * calls fuse).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: value = man * 2^-24 */
            float v = (float)man * 5.9604644775390625e-08f;
            memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t float_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if (isnan(f)) return 0x7FC0u;
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

static uint16_t float_to_half(float f) {
    /* round-to-nearest-even fp32 -> fp16 */
    uint32_t u;
    memcpy(&u, &f, 4);
    uint32_t sign = (u >> 16) & 0x8000u;
    uint32_t aexp = (u >> 23) & 0xFFu;
    uint32_t man = u & 0x7FFFFFu;
    if (aexp == 0xFF) return (uint16_t)(sign | 0x7C00u | (man ? 0x200u : 0u));
    int e = (int)aexp - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e; /* 24-bit mantissa -> (11+e-1) bits */
        uint32_t hm = man >> shift;
        uint32_t rem = man & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = man >> 13;
    uint32_t rem = man & 0x1FFFu;
    uint32_t out = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) out++;
    return (uint16_t)out;
}

/* out3: fp16 bits [rows, H] row stride H; inv: int64 [T*tk];
 * w: fp32 [T, tk]; y: [T, H] as bf16 (y_bf16=1) or fp16 bits, and yf fp32. */
int orc_combine(const uint16_t* out3, const int64_t* inv, const float* w, int64_t T,
                int64_t tk, int64_t H, int y_bf16, uint16_t* y, float* yf) {
    for (int64_t t = 0; t < T; ++t) {
        for (int64_t h = 0; h < H; ++h) {
            float acc = 0.0f;
            for (int64_t k = 0; k < tk; ++k) {
                int64_t r = inv[t * tk + k];
                float x = half_to_float(out3[r * H + h]);
                acc = fmaf(w[t * tk + k], x, acc);
            }
            if (yf) yf[t * H + h] = acc;
            if (y) y[t * H + h] = y_bf16 ? float_to_bf16(acc) : float_to_half(acc);
        }
    }
    return 0;
}

/* Counting-sort restatement of moe_align.
 * ids int64 [Nexp] (flattened [T, tk]); outputs sized by the caller:
 * sorted_rows [cap], expert_ids [max_blocks], inv [Nexp].
 * cap = max_blocks * block_m, max_blocks = ceil(Nexp/block_m) + E. */
int orc_moe_align(const int64_t* ids, int64_t Nexp, int64_t E, int64_t block_m,
                  int64_t* sorted_rows, int64_t* expert_ids, int64_t* inv) {
    int64_t max_blocks = (Nexp + block_m - 1) / block_m + E;
    int64_t cap = max_blocks * block_m;
    int64_t* counts = (int64_t*)calloc((size_t)E, sizeof(int64_t));
    int64_t* start = (int64_t*)calloc((size_t)E, sizeof(int64_t));
    int64_t* fill = (int64_t*)calloc((size_t)E, sizeof(int64_t));
    if (!counts || !start || !fill) return 1;
    for (int64_t i = 0; i < Nexp; ++i) {
        int64_t e = ids[i] > E ? E : ids[i];
        if (e < 0) { free(counts); free(start); free(fill); return 2; }
        if (e < E) counts[e]++;
    }
    int64_t blk = 0;
    for (int64_t e = 0; e < E; ++e) {
        int64_t nb = (counts[e] + block_m - 1) / block_m;
        start[e] = blk * block_m;
        for (int64_t b = blk; b < blk + nb; ++b) expert_ids[b] = e;
        blk += nb;
    }
    for (int64_t b = blk; b < max_blocks; ++b) expert_ids[b] = E;
    for (int64_t p = 0; p < cap; ++p) sorted_rows[p] = Nexp;
    for (int64_t i = 0; i < Nexp; ++i) inv[i] = 0;
    for (int64_t i = 0; i < Nexp; ++i) {
        int64_t e = ids[i] > E ? E : ids[i];
        if (e == E) continue;
        int64_t p = start[e] + fill[e]++;
        sorted_rows[p] = i;
        inv[i] = p;
    }
    free(counts); free(start); free(fill);
    return 0;
}

/* Sanity probe used by the loader. */
void orc_philox_first(const uint32_t* ctr, int64_t n, uint32_t key0, uint32_t key1, uint32_t* out) {
    for (int64_t i = 0; i < n; ++i) {
        uint32_t c0 = ctr[i], c1 = 0, c2 = 0, c3 = 0, k0 = key0, k1 = key1;
        for (int r = 0; r < 10; ++r) {
            const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
            const uint64_t p2 = (uint64_t)0xCD9E8D57u * c2;
            const uint32_t n0 = (uint32_t)(p2 >> 32) ^ c1 ^ k0;
            const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
            c1 = (uint32_t)p2;
            c3 = (uint32_t)p0;
            c0 = n0;
            c2 = n2;
            k0 += 0x9E3779B9u;
            k1 += 0xBB67AE85u;
        }
        out[i] = c0;
    }
}

int orc_version(void) { return 1; }
