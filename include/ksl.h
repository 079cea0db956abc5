/* C ABI of the MI355X (gfx950) fused layer-kernel library of the DiffusionGemma
 * block-diffusion model: RMSNorm and the W4A16 128-expert fused MoE forward,
 * with the expert router before it, the feed-forward block's tail after it,
 * and the per-step sampler pass (entropy, Gumbel-max sample, argmax).
 *
 * Every entry point takes raw device pointers, element counts and strides and
 * the HIP stream to launch on (hipStream_t passed as void*). Every entry point
 * returns 0 on success or a KSL_ERR_* code, never throws, never synchronises
 * the host and never allocates device memory: buffers come from the caller.
 * Outputs are written in full by the launched kernels.
 *
 * Reference interfaces are cited as path:line in SRSWTI/knivesysl-diffusion-xe.
 */
#ifndef KSL_H_
#define KSL_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define KSL_OK 0
#define KSL_ERR_ARG 1       /* null pointer or bad enum */
#define KSL_ERR_SHAPE 2     /* shape / divisibility contract violated */
#define KSL_ERR_ALIGN 3     /* pointer or stride alignment contract violated */
#define KSL_ERR_LAUNCH 4    /* kernel launch failed */
#define KSL_ERR_WORKSPACE 5 /* workspace too small */
#define KSL_ERR_SCRATCH 6   /* input larger than ksl_moe_layer_forward_noalloc's scratch */
#define KSL_ERR_RUNTIME 7   /* a HIP runtime query failed */

/* storage dtype codes */
#define KSL_DTYPE_F32 0
#define KSL_DTYPE_F16 1
#define KSL_DTYPE_BF16 2

/* activation codes for the gate/up epilogue */
#define KSL_ACT_GELU_TANH 0 /* kernels/fused_moe_w4_v2.py:136-138 */
#define KSL_ACT_SILU 1      /* SiLU-gated variant (act(g) = g * sigmoid(g)) */
#define KSL_ACT_NONE 2      /* ksl_moe_gateup_act only: gate and up themselves, no
                             * activation (the v1 path, kernels/fused_moe_w4.py:117-119);
                             * the forwards reject it */

/* layouts of the down weights dn_q */
#define KSL_DN_LAYOUT_REF 0   /* [E, H, I/2] as packed (kernels/w4a16.py:19-32) */
#define KSL_DN_LAYOUT_TILED 1 /* regrouped per 16-row tile by ksl_moe_repack_down */

/* Library version (bumped on ABI changes). */
int ksl_version(void);

/* Human-readable text of a status code. */
const char* ksl_status_string(int status);

/* RMSNorm over the last dim, one launch.
 * Replaces fused_rmsnorm / _rmsnorm_kernel (kernels/fused_rmsnorm.py:10-32).
 * y[r, :] = to(y_dtype)( bf16( x * (1/sqrt(sum(x^2)/cols + eps)) [* w] ) )
 * x: [rows, cols] with row stride x_stride (elements); w: [cols] or NULL
 * (a norm without scale, kernels/fused_rmsnorm.py:35-36); y: [rows, cols]
 * with row stride y_stride. The value is always rounded to bf16 first, as the
 * reference stores bf16 and then casts to x.dtype (fused_rmsnorm.py:21, :32).
 * fp32 accumulation. */
int ksl_rmsnorm(const void* x, int x_dtype, const void* w, int w_dtype, void* y, int y_dtype,
                int64_t rows, int64_t cols, int64_t x_stride, int64_t y_stride, float eps,
                void* stream);

/* Routing metadata on the GPU, one launch.
 * Replaces moe_align (kernels/fused_moe_w4.py:15-51) with identical outputs:
 *   sorted_rows int64[cap]    expanded row (t*topk + slot) per sorted slot,
 *                             pad slots = T*topk
 *   expert_ids  int64[max_blocks]  expert of each block_m block, pad = E
 *   inv         int64[T*topk] sorted slot of each expanded row (dropped: 0)
 * with max_blocks = ceil(T*topk/block_m) + E and cap = max_blocks*block_m.
 * Ids are clamped to <= E (E marks a dropped row); a negative id is treated
 * as dropped (the reference raises an index error there). E <= 512. */
int ksl_moe_align(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E, int64_t block_m,
                  int64_t* sorted_rows, int64_t* expert_ids, int64_t* inv, void* stream);

/* Routing metadata in the int32 token-row form, one launch.
 * Replaces moe_align_cuda (kernels/fused_moe_w4_v2.py:46-76: marlin's
 * moe_align_block_size followed by _align_finalize, :32-43):
 *   a_row      int32[cap]   token (expanded row / topk) of each sorted slot,
 *                           padding slots = T
 *   expert_ids int32[cap / block_m]  expert of each block, padding = E
 *   inv        int32[T*topk] sorted slot of each expanded row
 * cap = ksl_moe_align_i32_capacity(T, topk, E, block_m), the reference's
 * mx = T*topk + E*(block_m-1) (min(T*topk*block_m, mx) when T*topk < E)
 * rounded up to whole blocks. Rows of an expert keep their expanded-row
 * order (the reference's marlin kernel places them in an unspecified order;
 * every consumer of the layout is indifferent to it). Ids must lie in
 * [0, E) as the reference's contract requires (:48-56); an id outside is
 * treated as dropped (inv 0, no slot). E <= 512. */
int64_t ksl_moe_align_i32_capacity(int64_t T, int64_t topk, int64_t E, int64_t block_m);
int ksl_moe_align_i32(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E, int64_t block_m,
                      int32_t* a_row, int32_t* expert_ids, int32_t* inv, void* stream);

/* Workspace bytes the fused forward needs for these shapes: the routing
 * (sorted rows, offsets, inv), the fp16 activations, out2, out3 and the
 * per-block expert counts of the multi-block routing used above 4096 routed
 * rows. The workspace pointer must be 256-byte aligned (hipMalloc's is). */
size_t ksl_moe_workspace_bytes(int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I);

/* The whole W4A16 MoE forward, four launches (five above 4096 routed rows:
 * the routing then counts and places in two), no host sync.
 * Replaces fused_moe_w4_v2 (kernels/fused_moe_w4_v2.py:319-371):
 *   align -> gate/up + activation -> down -> fixed-order top-k combine.
 * hidden: [T, H] (bf16/fp16/fp32) with row stride hidden_stride;
 * topk_ids int64 [T, topk]; topk_w [T, topk] (fp32/fp16/bf16);
 * gu_q uint8 [E, 2I, H/2], gu_s/gu_z fp16 [E, 2I, H/128];
 * dn_q uint8 [E, H, I/2],  dn_s/dn_z fp16 [E, H, I/64]  (all contiguous;
 * zero-points are integers in [0, 15] as quantize_w4 writes them,
 * kernels/w4a16.py:28);
 * y: [T, H] of y_dtype with row stride y_stride. H % 128 == 0, I % 64 == 0
 * (fused_moe_w4_v2.py:327-328). dn_layout: KSL_DN_LAYOUT_REF, or
 * KSL_DN_LAYOUT_TILED for dn_q regrouped by ksl_moe_repack_down (same
 * results, faster weight stream).
 * gu_pack / dn_pack: the same experts in the pack layout of ksl_moe_pack_gateup
 * and ksl_moe_pack_down (16-byte aligned), or NULL. With both given and at
 * most 8192 routed rows, gate/up and down run as ONE persistent launch over
 * the pack layout (bit-identical results; gu_q .. dn_z are then not read and
 * may be NULL); otherwise the gate/up and down launches read gu_q .. dn_z. */
int ksl_moe_w4a16_forward(const void* hidden, int hidden_dtype, int64_t hidden_stride,
                          const int64_t* topk_ids, const void* topk_w, int w_dtype,
                          const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                          const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout,
                          const uint8_t* gu_pack, const uint8_t* dn_pack,
                          int64_t T, int64_t topk, int64_t E, int64_t H, int64_t I, int act,
                          void* y, int y_dtype, int64_t y_stride,
                          void* workspace, size_t workspace_bytes, void* stream);

/* RMSNorm followed by the W4A16 MoE forward: the layer as the experts see it
 * (DiffusionGemma decoder layer, TF modeling_diffusion_gemma.py:731-733:
 * experts(pre_feedforward_layernorm_2(x), topk_ids, topk_w)), four launches.
 * The norm (kernels/fused_rmsnorm.py:10-21 semantics; norm_w may be NULL) is
 * fused with the routing and the fp16 activation copy (ksl_moe_layer_route);
 * then gate/up, down and combine as in ksl_moe_w4a16_forward. x: bf16 or fp16
 * [T, H], row stride x_stride; H <= 4096. The normalised activations are
 * consumed in fp16 (bf16 norm output -> fp16, as hidden.to(fp16) does in
 * kernels/fused_moe_w4_v2.py:347). Same workspace and weight arguments
 * (gu_pack / dn_pack: three launches instead of four) as ksl_moe_w4a16_forward.
 * Not a reference entry point: the reference runs the two as separate calls. */
int ksl_moe_layer_forward(const void* x, int x_dtype, int64_t x_stride, const void* norm_w,
                          int norm_w_dtype, float eps, const int64_t* topk_ids, const void* topk_w,
                          int w_dtype, const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                          const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout,
                          const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t T,
                          int64_t topk, int64_t E, int64_t H, int64_t I, int act, void* y, int y_dtype,
                          int64_t y_stride, void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the library's own per-GPU scratch array, the workspace of
 * ksl_moe_layer_forward_noalloc: 32 MiB, enough for T * topk = 4096 routed
 * rows at H = 2816, I = 704, E = 128 (ksl_moe_workspace_bytes gives the need
 * of a shape). Every GPU the library runs on holds one until the process ends. */
#define KSL_NOALLOC_SCRATCH_BYTES (32 * 1024 * 1024)

/* ksl_moe_layer_forward without the workspace argument, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same arguments, contracts and results as ksl_moe_layer_forward; its
 * workspace is a static array of KSL_NOALLOC_SCRATCH_BYTES per GPU, found on
 * the current device (hipGetDevice) at the first call there. Returns
 * KSL_ERR_SCRATCH, before any device work, when ksl_moe_workspace_bytes(T,
 * topk, E, H, I) exceeds it, and KSL_ERR_RUNTIME when the array's address
 * cannot be looked up. Allocates nothing (no hipMalloc, no library
 * allocation). All calls on one GPU share its array: calls that overlap on
 * one GPU (other streams, other threads) race; calls on one stream do not. */
int ksl_moe_layer_forward_noalloc(const void* x, int x_dtype, int64_t x_stride, const void* norm_w,
                                  int norm_w_dtype, float eps, const int64_t* topk_ids, const void* topk_w,
                                  int w_dtype, const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                                  const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout,
                                  const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t T,
                                  int64_t topk, int64_t E, int64_t H, int64_t I, int act, void* y, int y_dtype,
                                  int64_t y_stride, void* stream);

/* The first stage of ksl_moe_layer_forward: compact routing (as
 * ksl_moe_route) plus a16 = fp16(bf16(rmsnorm(x) [* norm_w])) in the gate/up
 * activation order. One launch; above 4096 routed rows, when `scratch` holds
 * ksl_moe_route_scratch_bytes(T, topk, E) bytes (4-byte aligned), two
 * launches over many workgroups (per-block counts in scratch, then the stable
 * placement; same results), else one routing workgroup. scratch may be NULL. */
int ksl_moe_layer_route(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                        int32_t* sorted_rows, int32_t* offsets, int32_t* inv, const void* x, int x_dtype,
                        int64_t x_stride, const void* norm_w, int norm_w_dtype, float eps, int64_t H,
                        void* a16, void* scratch, size_t scratch_bytes, void* stream);

/* Scratch bytes of the multi-block routing: ceil(T*topk / 1024) * E int32
 * block counts (0 when T*topk <= 4096). Not a reference entry point. */
size_t ksl_moe_route_scratch_bytes(int64_t T, int64_t topk, int64_t E);

/* ---- the forward's stages, exposed for tests and for callers that fuse
 *      their own pipeline (same kernels as ksl_moe_w4a16_forward) ---------- */

/* Compact routing (moe_align with block_m = 1, int32): rows of expert e occupy
 * sorted slots [offsets[e], offsets[e+1]); sorted_rows int32[T*topk] (tail
 * past offsets[E] = T*topk); inv int32[T*topk]. Plus, in the same launch, the
 * fp16 activation copy a16[T, H] (hidden.to(fp16), fused_moe_w4_v2.py:347)
 * in the gate/up activation order: within each 128-element group, logical
 * offset c*32 + i*8 + j is stored at i*32 + c*8 + s(j), s the inverse of the
 * MFMA K-slot order {0,4,1,5,2,6,3,7}. a16 may be NULL (routing only). */
int ksl_moe_route(const int64_t* topk_ids, int64_t T, int64_t topk, int64_t E,
                  int32_t* sorted_rows, int32_t* offsets, int32_t* inv,
                  const void* hidden, int hidden_dtype, int64_t hidden_stride, int64_t H,
                  void* a16, void* stream);

/* Grouped W4 gate/up GEMM with the activation fused in the epilogue.
 * Replaces _gateup_act_kernel (kernels/fused_moe_w4_v2.py:96-139).
 * out2 fp16 [T*topk, I] row per sorted slot, in the down activation order:
 * the first I128 = I - I % 128 columns in the 128-element group order of a16,
 * a trailing 64-element group (I % 128 == 64) with offset c*16 + i*8 + j
 * stored at i*32 + c*8 + s(j). T: the tokens of a16 (T*topk routed rows;
 * with at least E of them the first weight groups are fetched before the
 * routing is read; above 8192 of them each workgroup takes a block of at most
 * 64 rows of one expert).
 * act KSL_ACT_NONE (the v1 grouped GEMM, kernels/fused_moe_w4.py:54-90 as
 * fused_moe_w4 runs it on gate/up, :117-118): out2 is instead out1 fp16
 * [T*topk, 2I], gate in columns 0..I-1 and up in I..2I-1, plain column order,
 * no activation; every routing size runs the per-expert kernel. */
int ksl_moe_gateup_act(const void* a16, const int32_t* sorted_rows, const int32_t* offsets,
                       int64_t T, int64_t topk, const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                       int64_t E, int64_t H, int64_t I, int act, void* out2, void* stream);

/* Grouped W4 down GEMM. Replaces _down_kernel (kernels/fused_moe_w4_v2.py:146-177).
 * out3 fp16 [T*topk, H] row per sorted slot, natural column order, 16-byte
 * aligned (written 8 columns per store). nrows:
 * the routed rows (T*topk), which size the grid (above 8192 routed rows each
 * workgroup takes a block of at most 64 rows of one expert, so that a heavy
 * expert spreads over many workgroups). dn_layout as in ksl_moe_w4a16_forward. */
int ksl_moe_down(const void* out2, const int32_t* offsets, const uint8_t* dn_q, const void* dn_s,
                 const void* dn_z, int64_t E, int64_t H, int64_t I, int64_t nrows, void* out3, int dn_layout,
                 void* stream);

/* Activation rows fp16 [rows, I] in plain column order (what an activation
 * applied outside the kernels writes, kernels/fused_moe_w4.py:119) -> the same
 * rows in the down activation order of ksl_moe_gateup_act's out2, ready for
 * ksl_moe_down. No reference counterpart: the v1 path's glue. src != dst,
 * both 16-byte aligned, I % 64 == 0. */
int ksl_moe_act_to_down_order(const void* src, int64_t rows, int64_t I, void* dst, void* stream);

/* Dynamic LDS bytes a ksl_moe_down launch requests for an (E, H, I) layer on
 * a device with cus compute units (host-only arithmetic, no device call; 0
 * for a shape outside the contract): the activation blocks of one 64-row
 * chunk (4 x I/64 x 2 KB) and each of the 8 waves' output staging (2.5 KB),
 * at most 148 KB (I = 1024), within gfx950's 160 KB per workgroup. */
size_t ksl_moe_down_lds_bytes(int64_t E, int64_t H, int64_t I, int64_t cus);

/* Asymmetric group-wise 4-bit quantisation (load time): quantize_w4
 * (kernels/w4a16.py:19-32) as pack_experts_module runs it on every expert
 * (kernels/pack_experts.py:34-41, 87-106). w: [rows, K] of w_dtype (bf16,
 * fp16 or fp32; an [E, N, K] expert stack is rows = E*N), contiguous,
 * pairs of elements aligned; per row and group of group_size columns (32,
 * 64 or 128; K % group_size == 0), in fp32: scale = max(max - min, 1e-8) / 15,
 * zero = clamp(round(-min / scale), 0, 15), q = clamp(round(w / scale + zero),
 * 0, 15) with round-half-to-even; qpacked uint8 [rows, K/2] (byte j =
 * q[2j] | q[2j+1] << 4), scale / zero fp16 [rows, K/group_size]. The same
 * bytes, scales and zero-points as the reference. */
int ksl_quantize_w4(const void* w, int w_dtype, int64_t rows, int64_t K, int64_t group_size, uint8_t* qpacked,
                    void* scale, void* zero, void* stream);

/* dequant_w4 (kernels/w4a16.py:35-48): W [rows, K] fp16 = fp16((q - zero) *
 * scale), the difference and the product in fp32 as the reference's torch
 * expression evaluates them (its nibbles promoted against the fp32 scale and
 * zero), rounded once. qpacked uint8 [rows, K/2] (4-byte aligned), scale and
 * zero fp16 [rows, K/group_size], out fp16 [rows, K] (16-byte aligned);
 * group_size % 8 == 0, K % group_size == 0. */
int ksl_dequant_w4(const uint8_t* qpacked, const void* scale, const void* zero, int64_t rows, int64_t K,
                   int64_t group_size, void* out, void* stream);

/* The MOE_NS down pack back to the reference layout (load time, out of
 * place): ns_q uint8 [E, I/2, H], the layout the reference's preshuffle_T_dn
 * writes for its _down_nsT_kernel (kernels/fused_moe_w4_v2.py:187-206; in
 * each 64-K chunk kb, byte row kb*32 + j of column n holds q[kb*64 + j] in
 * the low and q[kb*64 + 32 + j] in the high nibble) -> dn_q uint8 [E, H, I/2]
 * (KSL_DN_LAYOUT_REF, byte b = q[2b] | q[2b+1] << 4). H % 64 == 0,
 * I % 64 == 0, both pointers 8-byte aligned. Follow with ksl_moe_repack_down
 * for the tiled layout. */
int ksl_moe_unshuffle_ns_down(const uint8_t* ns_q, int64_t E, int64_t H, int64_t I, uint8_t* dn_q,
                              void* stream);

/* preshuffle_T_dn (kernels/fused_moe_w4_v2.py:186-197), the forward direction
 * of the above: dn_q uint8 [E, H, I/2] in the reference layout -> ns_q uint8
 * [E, I/2, H], the MOE_NS pack that enable_ns_down installs (:200-206), byte
 * for byte. Out of place; H % 64 == 0, I % 64 == 0, 8-byte aligned. */
int ksl_moe_preshuffle_ns_down(const uint8_t* dn_q, int64_t E, int64_t H, int64_t I, uint8_t* ns_q,
                               void* stream);

/* Load-time repack of the down buffers into the layout the down kernel
 * streams (the reference's precedent is the preshuffled down pack,
 * kernels/fused_moe_w4_v2.py:187-206). Out of place, into
 * ksl_moe_repack_down_bytes(E, H, I) bytes (16-byte aligned):
 *   - first E*H*I/2 bytes: the tiled weights, a pure permutation of dn_q
 *     [E, H, I/2]. Within each 16-row tile (base address unchanged): unit
 *     u < I/128 is 1 KB, 16 bytes per lane l = c*16 + col: row col, bytes
 *     u*64 + c*16 .. +16; then for I % 128 == 64 a 512-byte tail, 8 bytes per
 *     lane: row col, bytes (I/128)*64 + c*8 .. +8;
 *   - then the (scale, zero) pair table: per tile T, group g < I/64 and row
 *     col of the tile, the uint32 (scale bits | zero bits << 16) at index
 *     (T*(I/64) + g)*16 + col.
 * A buffer passed to the forwards as dn_q with KSL_DN_LAYOUT_TILED must be
 * one written by this call (the down kernel reads the pair table behind the
 * E*H*I/2 weight bytes; dn_s and dn_z still serve the other kernels).
 * dn_s / dn_z fp16 [E, H, I/64]. H % 16 == 0, I % 64 == 0. */
size_t ksl_moe_repack_down_bytes(int64_t E, int64_t H, int64_t I);
int ksl_moe_repack_down(const uint8_t* dn_q, const void* dn_s, const void* dn_z, int64_t E, int64_t H, int64_t I,
                        uint8_t* dn_q_tiled, void* stream);

/* Gate/up + activation and down of every expert in ONE persistent launch over
 * the pack layout (the stage that ksl_moe_w4a16_forward runs between routing
 * and combine when given gu_pack / dn_pack). Replaces _gateup_act_kernel and
 * _down_kernel (kernels/fused_moe_w4_v2.py:96-177, launched at :351-366) with
 * the same values: out2 and out3 are bit-identical to ksl_moe_gateup_act and
 * ksl_moe_down. a16, sorted_rows, offsets as produced by ksl_moe_route /
 * ksl_moe_layer_route; out2 fp16 [T*topk, I] (16-byte aligned), out3 fp16
 * [T*topk, H] (8-byte aligned). ctl: ksl_moe_ffn_ctl_bytes(E) bytes of int32
 * counters (one per 256 bytes: the unit queue, an error word, an exit count,
 * one per expert) that must be zero on entry (torch.zeros once); the launch
 * leaves them zero (the last workgroup to finish clears them), except the
 * error word (int32 index 64), which becomes 1 if a down unit's wait for its
 * expert's gate/up units (in other workgroups) ran out of its bound; the unit
 * then runs anyway, so out2 / out3 of that launch are not to be trusted. Here
 * the error word latches: only the caller clears it. Inside the fused
 * forwards (ksl_moe_w4a16_forward, ksl_moe_layer_forward and its no-allocation
 * variant, ksl_moe_block_forward) the routing launch clears it at the start
 * of each call and the combine launch of the same call reads it: when it is
 * set, every element of that call's output y is NaN (the status cannot reach
 * the caller without a host synchronisation). Calls that share one ctl
 * buffer must not overlap. T*topk <= 8192, E <= 512, H % 128 == 0,
 * I % 64 == 0, H, I <= 8192. */
size_t ksl_moe_ffn_ctl_bytes(int64_t E);
int ksl_moe_ffn(const void* a16, const int32_t* sorted_rows, const int32_t* offsets, int64_t T, int64_t topk,
                const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t E, int64_t H, int64_t I, int act,
                void* out2, void* out3, int32_t* ctl, void* stream);

/* Bound of the one-launch FFN's dependency wait, for later launches of this
 * process (no reference counterpart: the reference launches gate/up and down
 * separately and never waits across workgroups). cycles: empty ring cycles a
 * down unit waits before it gives up and sets the error word (< 0: the
 * default, 2^18; at most 2^30). force_wait != 0 makes every dependency count
 * as unmet, so each down unit waits out the bound and the error word is set
 * while every workgroup still finishes normally: the host-forced failure of
 * the failure-handling tests. */
int ksl_moe_ffn_set_wait_limit(int64_t cycles, int force_wait);

/* Load-time pack of the experts for the one-launch expert FFN (the
 * reference's precedent for a kernel-specific load-time repack is the
 * preshuffled down pack, kernels/fused_moe_w4_v2.py:187-206). Out of place;
 * the pack holds the same nibbles, scales and zero-points, regrouped so that
 * each 128-K slot of a unit of work is one contiguous run of bytes:
 *   gate/up, per expert e, unit cb (176 columns of I; the last unit of an
 *   expert may be narrower: nt = min(11, I/16 - 11*cb) tiles), group g < H/128:
 *   nt*2 blocks of 1 KB (block 2w + j, tile w, j = 0 gate / 1 up; lane
 *   l = 16*c + col holds gu_q row j*I + 16*(11*cb + w) + col, bytes
 *   64*g + 16*c .. +16), then nt*128 bytes (tile w, column col: gate scale,
 *   gate zero, up scale, up zero of group g, fp16).
 *   ksl_moe_pack_gateup_bytes(E, H, I) = E*H*I*17/16 bytes.
 * H % 128 == 0, I % 64 == 0, H, I <= 8192. gu_* as ksl_moe_w4a16_forward. */
size_t ksl_moe_pack_gateup_bytes(int64_t E, int64_t H, int64_t I);
int ksl_moe_pack_gateup(const uint8_t* gu_q, const void* gu_s, const void* gu_z, int64_t E, int64_t H, int64_t I,
                        uint8_t* gu_pack, void* stream);

/* Down: per expert e, unit q (352 columns of H; nt = min(22, H/16 - 22*q)
 * tiles), slot s < I/128: nt blocks of 1 KB (tile u; lane l = 16*c + col
 * holds dn_q row 16*(22*q + u) + col, bytes 64*s + 16*c .. +16), then nt*128
 * bytes (tile u, column col: scale and zero of group 2s, then of group
 * 2s + 1); for I % 128 == 64 a tail slot: nt blocks of 512 B (lane l: bytes
 * 64*(I/128) + 8*c .. +8), then nt*64 bytes (scale and zero of the last group).
 * ksl_moe_pack_down_bytes(E, H, I) = E*H*I*9/16 bytes. dn_q in dn_layout
 * (reference or tiled). */
size_t ksl_moe_pack_down_bytes(int64_t E, int64_t H, int64_t I);
int ksl_moe_pack_down(const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout, int64_t E, int64_t H,
                      int64_t I, uint8_t* dn_pack, void* stream);

/* Fixed-order top-k combine, no atomics: y[t,:] = fma-chain over k=0..topk-1
 * of fp32(w[t,k]) * fp32(out3[inv[t*topk+k], :]), rounded once to y_dtype.
 * Replaces _combine_kernel / _combine (kernels/fused_moe_w4_v2.py:248-288).
 * H % 8 == 0. */
int ksl_moe_combine(const void* out3, const int32_t* inv, const void* topk_w, int w_dtype,
                    int64_t T, int64_t topk, int64_t H, void* y, int y_dtype, int64_t y_stride,
                    void* stream);

/* The v1 combine (kernels/fused_moe_w4.py:125-127, (out3[inv].view(T, topk, H)
 * * topk_w.to(fp16)).sum(1).to(y dtype)): per slot k in order, the product
 * fp16(fp16(w[t,k]) * out3[inv[t*topk+k], :]) summed in fp32, the sum rounded
 * to fp16, then to y_dtype. Arguments as ksl_moe_combine. */
int ksl_moe_combine_v1(const void* out3, const int32_t* inv, const void* topk_w, int w_dtype,
                       int64_t T, int64_t topk, int64_t H, void* y, int y_dtype, int64_t y_stride,
                       void* stream);

/* The combine of the stock experts loop that packed_experts_forward runs
 * (kernels/pack_experts.py:44-62; TF modeling_diffusion_gemma.py:578-588):
 * y = 0 in y_dtype, then expert by expert in ascending id, each of its rows
 * adds term = y_dtype(h * w[t,k]) with one rounding to y_dtype per add
 * (index_add_), h = out3[inv[t*topk+k], :] fp16; h * w is taken in fp32 for
 * fp32 or bf16 weights and in fp16 for fp16 weights (torch's type
 * promotion). Per token the slots go in (expert id, slot) order; ids outside
 * [0, E) are skipped. topk_ids int64 [T, topk] (8-byte aligned), topk <= 32;
 * other arguments as ksl_moe_combine. */
int ksl_moe_combine_stock(const void* out3, const int32_t* inv, const int64_t* topk_ids, int64_t E,
                          const void* topk_w, int w_dtype, int64_t T, int64_t topk, int64_t H, void* y,
                          int y_dtype, int64_t y_stride, void* stream);

/* Expert router, the step before the MoE: TF modeling_diffusion_gemma.py:529-548
 * (DiffusionGemmaTextRouter.forward), its scale-free norm being the fused
 * RMSNorm as the reference patches every DiffusionGemmaRMSNorm
 * (kernels/load_w4_checkpoint.py:126-127, kernels/fused_rmsnorm.py:35-48):
 *   h = bf16(bf16(bf16(rmsnorm(x)) * scale) * fp32(H ** -0.5));
 *   scores = bf16(h @ proj_w^T); probs = softmax(fp32(scores));
 *   topk_w, topk_ids = top-k of probs (descending; equal values: lower id),
 *   topk_w = topk_w / sum(topk_w) * per_expert_scale[topk_ids].
 * x bf16 or fp16 [T, H] (row stride x_stride elements); scale [H], proj_w
 * [E, H], per_expert_scale [E] in w_dtype (bf16). probs fp32 [T, E] (the
 * router probabilities; it also holds the scores between the two launches),
 * topk_w fp32 [T, topk], topk_ids int64 [T, topk] (the MoE's inputs).
 * H % 32 == 0, H <= 4096, E % 16 == 0, E <= 256, topk <= min(E, 16). */
int ksl_moe_router(const void* x, int x_dtype, int64_t x_stride, const void* scale, const void* proj_w,
                   const void* per_expert_scale, int w_dtype, float eps, int64_t T, int64_t H, int64_t E,
                   int64_t topk, float* probs, float* topk_w, int64_t* topk_ids, void* stream);

/* The combine fused with the feed-forward block's tail, the step after the
 * MoE: TF modeling_diffusion_gemma.py:734-744 (decoder and encoder layers),
 * every RMSNorm being the fused RMSNorm (kernels/fused_rmsnorm.py:10-21):
 *   m  = bf16(combine as ksl_moe_combine)
 *   s  = bf16(h1 + bf16(m * r(m) * post2_w))           post_feedforward_layernorm_2, + hidden_states_1
 *   o  = bf16(residual + bf16(s * r(s) * post_w))     post_feedforward_layernorm, + residual
 *   y  = bf16(o * layer_scalar)                        hidden_states *= layer_scalar
 * r(v) = 1 / sqrt(sum(v^2) / H + eps) with post2_eps resp. post_eps. One
 * launch, one workgroup per token. h1, residual, post2_w, post_w, y: bf16
 * (the layer's dtype); layer_scalar: one fp32 or bf16 element (ls_dtype), or
 * NULL for 1. H % 8 == 0, H <= 8192. y may be the residual or h1 buffer
 * (same stride): each element is read before it is written, by one thread.
 * Not a reference entry point: the reference runs the tail as five torch
 * calls after _combine (kernels/fused_moe_w4_v2.py:371). */
int ksl_moe_combine_post(const void* out3, const int32_t* inv, const void* topk_w, int w_dtype,
                         int64_t T, int64_t topk, int64_t H, const void* h1, int64_t h1_stride,
                         const void* residual, int64_t residual_stride, const void* post2_w,
                         float post2_eps, const void* post_w, float post_eps, const void* layer_scalar,
                         int ls_dtype, void* y, int64_t y_stride, void* stream);

/* The decoder layer's MoE branch and tail, four launches (TF
 * modeling_diffusion_gemma.py:729-744 after the router): x is the residual
 * (hidden_states_flat), bf16 [T, H];
 *   moe = experts(rmsnorm(x) * pre_norm_w, topk_ids, topk_w)   as ksl_moe_layer_forward
 *   y   = the tail of ksl_moe_combine_post with residual = x.
 * Same workspace and weight arguments as ksl_moe_w4a16_forward; same
 * contracts as ksl_moe_layer_forward (H <= 4096) and ksl_moe_combine_post.
 * Not a reference entry point (see ksl_moe_combine_post). */
int ksl_moe_block_forward(const void* x, int64_t x_stride, const void* pre_norm_w, float pre_eps,
                          const int64_t* topk_ids, const void* topk_w, int w_dtype,
                          const uint8_t* gu_q, const void* gu_s, const void* gu_z,
                          const uint8_t* dn_q, const void* dn_s, const void* dn_z, int dn_layout,
                          const uint8_t* gu_pack, const uint8_t* dn_pack, int64_t T,
                          int64_t topk, int64_t E, int64_t H, int64_t I, int act, const void* h1,
                          int64_t h1_stride, const void* post2_w, float post2_eps, const void* post_w,
                          float post_eps, const void* layer_scalar, int ls_dtype, void* y,
                          int64_t y_stride, void* workspace, size_t workspace_bytes, void* stream);

/* ---- the per-step sampler pass (over [rows, V] logits, one read per call) ---- */

/* Entropy (nats) of softmax(logits) per row, one pass: online running max,
 * sum e^(x-m) and sum x e^(x-m). Replaces _entropy_kernel / fused_entropy
 * (kernels/fused_sampler_ops.py:22-51). logits fp32, bf16 or fp16 [rows, V]
 * (row stride row_stride elements, V < 2^31); entropy fp32 [rows]. Entries
 * equal to -inf contribute nothing (torch's Categorical.entropy; the
 * reference's kernel returns NaN for such rows). */
int ksl_entropy(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride, float* entropy,
                void* stream);

/* Gumbel-max sample and argmax per row. Replaces _gumbel_argmax_kernel /
 * gumbel_argmax_sample (kernels/fused_sampler_ops.py:54-93): sampled = first
 * index of the max of fp32(x + g), g = -log(-log(clamp(u, 1e-10, 1 - 1e-7))),
 * u = tl.rand(seed + row, column), i.e. Triton's Philox4x32-10 stream (counter
 * (column, 0, 0, 0), key = seed + row computed in int32 when seed fits int32,
 * else int64, sign-extended); argmax = first index of the max of x. The same
 * seed gives the reference's draws. sampled, argmax int64 [rows]. */
int ksl_gumbel_argmax(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride,
                      int64_t seed, int64_t* sampled, int64_t* argmax, void* stream);

/* Both of the above in one read of the logits (the reference reads them twice
 * per denoising step: the sample, then the sampler's entropy,
 * kernels/fast_sampler.py:93-96). Not a reference entry point. */
int ksl_sample_step(const void* logits, int dtype, int64_t rows, int64_t V, int64_t row_stride, int64_t seed,
                    int64_t* sampled, int64_t* argmax, float* entropy, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KSL_H_ */
