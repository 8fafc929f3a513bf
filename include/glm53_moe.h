/*
 * glm53_moe.h -- C ABI of libglm53_moe.so, the MI355X (gfx950) implementation
 * of the FP8 block-scaled packed mixture-of-experts path of
 * kiojuvr/glm53-flash-mlx.
 *
 * Conventions
 *   - Plain pointers and sizes only.  Every pointer argument is a device
 *     pointer unless the comment says "host".  BF16 tensors are passed as
 *     `void*` (2 bytes per element, row-major), E4M3 weights as `uint8_t*`,
 *     block scales (`weight_scale_inv`) as `float*` over 128x128 blocks.
 *   - `stream` is a hipStream_t (NULL = default stream).  All work is
 *     enqueued on it; no call synchronises the host except the *_status /
 *     *_error_flag readbacks, which say so.
 *   - Return value: GLM53_OK, or an error code with a message retrievable by
 *     glm53_last_error() (thread-local).  The Python layer maps
 *     GLM53_INVALID_ARGUMENT to ValueError and the others to RuntimeError,
 *     as the reference does (fp8.py:256-273; native_packed_moe_plan.cpp:
 *     127-149).
 *   - Plans own fixed device scratch allocated once at creation and are not
 *     safe for concurrent use (one plan per layer and stream), as the
 *     reference's native plans (native_packed_moe_plan.h:22-146).
 *
 * Reference paths are relative to the kiojuvr/glm53-flash-mlx repository.
 */
#ifndef GLM53_MOE_H
#define GLM53_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GLM53_ABI_VERSION 2

#define GLM53_OK 0
#define GLM53_INVALID_ARGUMENT 1
#define GLM53_BAD_STATE 2
#define GLM53_DEVICE_ERROR 3

/* Reduction order of the prefill combine step. */
#define GLM53_REDUCE_GROUPED 0 /* FP32 slot order, grouped_fp8.py:273-276 */
#define GLM53_REDUCE_DIRECT 1  /* BF16 ascending expert, fp8.py:384-397 */

/* Packed per-layer expert bank (packed.py:782-850):
 *   gate_up_weight    u8  [E, 2I, H]  rows 0..I-1 gate, I..2I-1 up
 *   gate_up_scale_inv f32 [E, 2*ceil(I/128), ceil(H/128)]  (up from row ceil(I/128))
 *   down_weight       u8  [E, H, I]
 *   down_scale_inv    f32 [E, ceil(H/128), ceil(I/128)]
 * Each expert matrix [N, K] of the two weight tensors is stored in the
 * layout row_group_log2 = g names:
 *   g = 0      row-major, byte (n, k) at n K + k: the reference's layout and
 *              the checkpoint's, the import / export format;
 *   g = 1..7   row groups (needs H % 128 == 0 and I % 128 == 0): the 2^g
 *              rows of group n >> g are stored together, their K span as K /
 *              128 consecutive blocks of 2^g rows x 128 bytes, so byte (n, k)
 *              sits at (n >> g) 2^g K + (k >> 7) 2^g 128 + (n mod 2^g) 128 +
 *              k mod 128.  A 128-row MFMA weight stage of the grouped GEMM
 *              then reads 128 / 2^g contiguous runs instead of 128 lines,
 *              and a row group's K span is one contiguous run for the decode
 *              GEMV.  Every kernel gives the same bits on every g.  The
 *              library's own banks default to g = 0 (decode runs 0.6-1.4 us
 *              per layer faster on it; prefill 1-3% slower than on
 *              GLM53_TILED_ROW_GROUP_LOG2, 16-row groups).
 * Block scales have one layout (as above) whatever g is.                     */
#define GLM53_MAX_ROW_GROUP_LOG2 7
#define GLM53_TILED_ROW_GROUP_LOG2 4
typedef struct glm53_bank {
  const uint8_t* gate_up_weight;
  const float* gate_up_scale_inv;
  const uint8_t* down_weight;
  const float* down_scale_inv;
  int64_t experts;
  int64_t hidden;
  int64_t intermediate;
  /* device int32, nonzero when the weights hold E4M3 codes 0x7F / 0xFF
   * (glm53_e4m3_scan_codes); NULL makes every prefill call scan the bank */
  const int32_t* code_flags;
  int32_t row_group_log2; /* weight layout, above (0 = reference row-major) */
} glm53_bank;

/* Bank handle -- the native side of PackedFP8ExpertBank(...)
 * (packed.py:747-876).  Validates `desc` (pointers, dimensions, layout,
 * 16-byte aligned weights), copies it, and owns a device code flag: both
 * weight tensors are scanned once on `stream` for E4M3 codes 0x7F / 0xFF, so
 * calls made with the handle never scan again (desc's own code_flags is
 * ignored).  Weights stay borrowed, in the layout desc names: the caller
 * keeps them alive and unchanged while the handle is in use.  The returned
 * pointer is used wherever a `const glm53_bank*` is taken; destroy it (which
 * frees what the handle owns) only after the work that uses it has
 * completed. */
int glm53_bank_create(const glm53_bank* desc, void* stream, glm53_bank** out);

/* Bank import (PackedFP8ExpertBank.pack, packed.py:782-850, with the re-lay
 * of this build): allocates device buffers owned by the handle, copies the
 * bank of `desc` (any layout, usually the reference row-major one) into
 * them re-laid as row_group_log2 (0 keeps the reference layout,
 * GLM53_TILED_ROW_GROUP_LOG2 makes 16-row groups), copies the block scales,
 * scans the codes, and waits for
 * `stream`, so the caller may free desc's buffers when this returns.  Costs
 * one bank of device memory (5.44 GB at H = 4096, I = 1536, E = 288) beside
 * the caller's copy until that is freed. */
int glm53_bank_import(const glm53_bank* desc, int32_t row_group_log2, void* stream, glm53_bank** out);
void glm53_bank_destroy(glm53_bank* bank);

/* Out-of-place re-lay of `matrices` consecutive E4M3 matrices [rows, cols]
 * (rows * cols bytes apart) from the layout from_log2 to the layout to_log2
 * (glm53_bank): the bank import above, and its export back to the
 * reference layout (to_log2 = 0).  Needs (rows * cols) % 16 == 0, 16-byte
 * aligned, non-overlapping buffers, and for a row-group layout cols % 128 ==
 * 0 and rows a multiple of the group.  HBM-bound: each byte read and written
 * once. */
int glm53_relayout_weights(const uint8_t* src, uint8_t* dst, int64_t matrices, int64_t rows, int64_t cols,
                           int32_t from_log2, int32_t to_log2, void* stream);

/* One BlockFP8Linear (fp8.py:302-326): weight u8 [out, in], scale
 * f32 [ceil(out/128), ceil(in/128)]. */
typedef struct glm53_linear {
  const uint8_t* weight;
  const float* scale_inv;
  int64_t out_features;
  int64_t in_features;
  const int32_t* code_flags; /* as glm53_bank.code_flags; may be NULL */
} glm53_linear;

/* Shared expert = ClampedMLP over block-FP8 linears (patch.py:114-129). */
typedef struct glm53_shared_expert {
  glm53_linear gate;
  glm53_linear up;
  glm53_linear down;
} glm53_shared_expert;

/* FP32 router (patch.py:131-142): weight f32 [E, H], bias f32 [E]
 * (e_score_correction_bias); selection = top_k of sigmoid(logits) + bias
 * ordered (biased score desc, expert id asc); weights = sigmoid of the
 * selected logits, normalised if norm_topk_prob, times
 * routed_scaling_factor. */
typedef struct glm53_router {
  const float* weight;
  const float* bias;
  int64_t experts;
  int64_t hidden;
  int64_t top_k;
  float routed_scaling_factor;
  int32_t norm_topk_prob;
  /* Group-limited selection (patch.py:134-142 passes n_group and
   * topk_group to group_expert_select): the experts form n_group groups of
   * consecutive ids, a group scores the FP32 sum of its two largest biased
   * scores, and the biased scores of all but the topk_group best groups
   * (ties: lower group index kept) become 0.0 before the top-k.  0 or 1 in
   * both: no grouping.  n_group <= 64, dividing experts into groups of at
   * least two; top_k <= topk_group * experts / n_group. */
  int32_t n_group;
  int32_t topk_group;
} glm53_router;

const char* glm53_last_error(void);
int glm53_abi_version(void);

/* Writes 1 to the device int32 *flag when any of the n E4M3 codes is 0x7F
 * or 0xFF, else 0.  The reference's table (fp8.py:22-27) decodes those codes
 * to +-480; OCP E4M3 (the MFMA operand format) reads them as NaN, so the
 * MFMA paths use the flag to switch on an exact fix-up.  The streaming
 * decode kernels decode them exactly without a flag. */
int glm53_e4m3_scan_codes(const uint8_t* codes, int64_t n, int32_t* flag, void* stream);

/* ------------------------------------------------------------------------
 * block_fp8_linear -- replaces fp8.py:254-299 `block_fp8_linear`
 * (kernels fp8.py:41-116).  y[m, n] = T(sum_k x[m,k] * E4M3(w[n,k]) *
 * s[n/128, k/128]).  x bf16 [M, K], y bf16 [M, N].  M == 1 runs the
 * streaming GEMV; M > 1 with K % 128 == 0 runs the FP8 MFMA GEMM and needs
 * `workspace` of glm53_fp8_linear_workspace_bytes(M, N, K) bytes (may be
 * NULL when that is 0).  code_flags (device int32 from glm53_e4m3_scan_codes,
 * may be NULL) lets both paths use the hardware E4M3 decode when the weight
 * holds no 0x7F / 0xFF code; NULL keeps the exact software decode (M == 1)
 * or scans the weight first (M > 1).
 * ---------------------------------------------------------------------- */
size_t glm53_fp8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);
int glm53_fp8_linear(const void* x, int64_t M, int64_t K, const uint8_t* weight, int64_t N,
                     const float* scale_inv, const int32_t* code_flags, void* y, void* workspace,
                     size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Router -- replaces patch.py:131-142 `Float32Gate.__call__` (with the
 * selection half of mlx-vlm dsv32.group_expert_select, group-limited when
 * the router's n_group > 1).
 * x bf16 [tokens, H] -> ids int32 [tokens, top_k], scores f32 [tokens, top_k].
 * The workspace holds, for several tokens, the FP32 partial sums of the
 * BF16-MFMA logits (up to 16 K chunks x tokens x experts floats) and FP32
 * logits (tokens x experts, for shapes the MFMA form does not take); for one
 * token, the logits.
 * ---------------------------------------------------------------------- */
size_t glm53_router_workspace_bytes(int64_t tokens, int64_t hidden, int64_t experts);
int glm53_router_topk(const glm53_router* router, const void* x, int64_t tokens, int32_t* ids,
                      float* scores, void* workspace, size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Batch-1 decode plan -- replaces native_packed_moe_plan.h:22-146
 * `NativePackedMoEDecodePlan` (bindings.cpp:562-632) and the Python
 * composition packed.py:896-923 `PackedFP8MoE.__call__` for one token.
 * ---------------------------------------------------------------------- */
typedef struct glm53_decode_plan glm53_decode_plan;

int glm53_decode_plan_create(int64_t hidden, int64_t intermediate, int64_t shared_intermediate,
                             int64_t experts, int64_t top_k, float swiglu_limit,
                             glm53_decode_plan** out);
void glm53_decode_plan_destroy(glm53_decode_plan* plan);

/* Routed experts + shared expert for given expert ids / scores (the
 * reference's execute(x, ids, scores, weights...), .cpp:151-173).
 * x bf16 [H]; expert_ids int32 [top_k]; scores f32 [top_k]; out bf16 [H].
 * shared may be NULL. */
int glm53_decode_moe_routed(glm53_decode_plan* plan, const glm53_bank* bank,
                            const glm53_shared_expert* shared, const void* x,
                            const int32_t* expert_ids, const float* scores, void* out,
                            void* stream);

/* Router + routed + shared in one call (PackedFP8MoE.__call__ for L = 1).
 * ids_out / scores_out (device, [top_k]) may be NULL. */
int glm53_decode_moe(glm53_decode_plan* plan, const glm53_bank* bank,
                     const glm53_shared_expert* shared, const glm53_router* router,
                     const void* x, void* out, int32_t* ids_out, float* scores_out, void* stream);

/* Decoder-step form with optional residual and stage control:
 * out = T(residual + T(moe(x))) when residual is not NULL (out may alias
 * residual / x), else out = moe(x).  stages selects launches:
 * GLM53_STAGE_ROUTER (router + top-k into the plan), GLM53_STAGE_GATE_UP
 * (routed + shared gate/up/SwiGLU), GLM53_STAGE_DOWN (down, ordered
 * reduction, shared add, residual).  router is required with
 * GLM53_STAGE_ROUTER (and for shapes without the fused step kernels, which
 * run only the whole mask); without that bit the routed launches use the
 * selection the plan holds from an earlier router stage, and router may be
 * NULL.  Partial masks let a caller time each launch; they need the fused
 * path (16-byte aligned pointers, supported widths).  A captured HIP graph
 * of this call replays correctly: it records no memset and resets its own
 * counters. */
#define GLM53_STAGE_ROUTER 1
#define GLM53_STAGE_GATE_UP 2
#define GLM53_STAGE_DOWN 4
#define GLM53_STAGE_ALL 7
int glm53_decode_moe_ex(glm53_decode_plan* plan, const glm53_bank* bank,
                        const glm53_shared_expert* shared, const glm53_router* router,
                        const void* x, const void* residual, void* out, int32_t stages,
                        void* stream);

/* bind_weights (native_packed_moe_plan.h:40-47, .cpp:231-258;
 * bindings.cpp:576-581): record the layer's weights once -- the bank, the
 * shared expert (may be NULL) and, beyond the reference, the router (may be
 * NULL) -- so later calls pass only activations.  The plan keeps the
 * pointers, not the bytes: the caller keeps the weights alive and unchanged
 * while bound (glm53_decode_plan_identities(plan, 1, ...) returns the
 * recorded pointers for an identity re-check).  Binding twice is
 * GLM53_BAD_STATE. */
int glm53_decode_plan_bind(glm53_decode_plan* plan, const glm53_bank* bank,
                           const glm53_shared_expert* shared, const glm53_router* router);

/* execute_bound(x, expert_ids, scores) (native_packed_moe_plan.h:48,
 * .cpp:260-280; bindings.cpp:580): the bound weights with caller-chosen
 * routing, as glm53_decode_moe_routed.  GLM53_BAD_STATE when nothing is
 * bound. */
int glm53_decode_moe_bound_routed(glm53_decode_plan* plan, const void* x, const int32_t* expert_ids,
                                  const float* scores, void* out, void* stream);

/* The bound weights with the bound router, as glm53_decode_moe (no
 * reference counterpart: the reference's router stays in MLX).
 * GLM53_BAD_STATE when nothing, or no router, is bound. */
int glm53_decode_moe_bound(glm53_decode_plan* plan, const void* x, void* out, void* stream);

/* Launch shape of the fused decode kernels: rows of one slot streamed per
 * wavefront in the gate/up kernel (default 8) and output rows per workgroup
 * in the down kernel (default 16, at most 64).  Results do not depend on it. */
int glm53_decode_plan_tune(glm53_decode_plan* plan, int32_t gate_up_rows_per_wave,
                           int32_t down_rows_per_wg);

/* Device scratch of the last call (read-only diagnostics): which = 0 hidden
 * bf16 [top_k + 1, I] (routed SwiGLU rows in slot order, then the shared
 * expert's; the reference's debug_routed_hidden / debug_shared_hidden,
 * native_packed_moe_plan.h:81-85), 1 expert ids int32 [top_k], 2 scores f32
 * [top_k], 3 the router words u64 [E] of the router launch (sigmoid bits <<
 * 32 | selection key), 4 the plan's whole device arena (allocated once at
 * creation; scratch_bytes, native_packed_moe_plan.h:73), 5 the shared
 * expert's output bf16 [H] (debug_shared_down). */
int glm53_decode_plan_scratch(glm53_decode_plan* plan, int32_t which, void** ptr, size_t* bytes);

/* Synchronous: copies the plan's device error flag to *host_value and
 * clears it.  Bit 0 = an expert id was out of range (those slots produce
 * NaN rows and the layer output is NaN); no other bit is used. */
int glm53_decode_plan_error_flag(glm53_decode_plan* plan, int32_t* host_value);

/* Read-only counters of a plan (native_packed_moe_plan.h:55-73;
 * native_prefill_moe_plan.h; bindings.cpp:389-407, 584-632).  Host-side
 * bookkeeping only: reading them touches no device. */
typedef struct glm53_plan_counters {
  uint64_t execution_count;                /* calls that enqueued a forward */
  uint64_t dynamic_allocation_count;       /* device allocations after creation: always 0 */
  uint64_t host_synchronization_count;     /* synchronous readbacks (error flag, status) */
  uint64_t static_input_validation_count;  /* weight-set validations (each unbound call, each bind) */
  uint64_t dynamic_input_validation_count; /* activation / routing validations (every call) */
  uint64_t scratch_bytes;                  /* the plan's device arena */
  int32_t weights_bound;                   /* decode: glm53_decode_plan_bind has run */
  int32_t router_bound;                    /* decode: ... with a router */
} glm53_plan_counters;
int glm53_decode_plan_counters(const glm53_decode_plan* plan, glm53_plan_counters* out);

/* Identities (device addresses) the plan works with, for the reference's
 * buffer_identities / bound_weight_identities checks
 * (native_packed_moe_plan.cpp:382-411): which = 0 its scratch buffers
 * (fixed at creation), 1 the bound weight pointers (bank 4, shared 6 when
 * bound, router 2 when bound; GLM53_BAD_STATE when nothing is bound).
 * Writes min(count, capacity) values to out (host) and the count to *count. */
int glm53_decode_plan_identities(const glm53_decode_plan* plan, int32_t which, uint64_t* out,
                                 int32_t capacity, int32_t* count);

/* Routed-stage diagnostic -- replaces native_packed_moe_plan.h:148-183
 * `NativePackedMoERoutedDiagnostic` (bindings.cpp:634-649): one decode's
 * routed gate/up/SwiGLU boundary with every stage kept, for localising
 * numerics.  execute(x bf16 [H], expert_ids int32 [top_k], the bank's
 * gate_up_weight u8 [E, 2I, H] in the layout row_group_log2 (glm53_bank)
 * and gate_up_scale_inv) fills five bf16
 * [top_k, I] stages owned by the object (fixed addresses from creation):
 * 0 gate = T(x . W_gate[e]^T), 1 up = T(x . W_up[e]^T), 2 sigmoid =
 * T(sigmoid(g')), 3 silu = T(g' * sigmoid), 4 hidden = T(silu * u') with
 * g' = T(min(gate, L)), u' = T(clip(up, -L, L)) (packed.py:146-163).  It is
 * separate from the decode plan and runs the any-shape GEMV, so its gate /
 * up may differ from the fused step's by the FP32 summation order; the
 * stages after gate / up are exact functions of them. */
typedef struct glm53_routed_diagnostic glm53_routed_diagnostic;
int glm53_routed_diagnostic_create(int64_t hidden, int64_t intermediate, int64_t experts, int64_t top_k,
                                   float swiglu_limit, glm53_routed_diagnostic** out);
void glm53_routed_diagnostic_destroy(glm53_routed_diagnostic* diag);
int glm53_routed_diagnostic_execute(glm53_routed_diagnostic* diag, const void* x, const int32_t* expert_ids,
                                    const uint8_t* gate_up_weight, const float* gate_up_scale_inv,
                                    int32_t row_group_log2, void* stream);
int glm53_routed_diagnostic_stage(glm53_routed_diagnostic* diag, int32_t which, void** ptr, size_t* bytes);
int glm53_routed_diagnostic_counters(const glm53_routed_diagnostic* diag, uint64_t* execution_count,
                                     uint64_t* scratch_bytes);

/* Allocation-free decode step.  No counterpart in the reference: this entry
 * point is for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * is glm53_decode_moe_ex with the whole stage mask and a router, without a
 * plan: out = T(residual + T(moe(x))) (residual may be NULL; out may alias x
 * and residual), the same kernels and bits as the plan form.  It calls no
 * hipMalloc / hipFree: its scratch is a static device array of
 * GLM53_DECODE_STATIC_SCRATCH_BYTES, one copy per GPU held until the process
 * ends; the first call on a GPU looks up that copy's address, clears it
 * with a fill kernel on `stream` and waits for the clear, so calls on any
 * stream of that GPU start from it (make that first call outside graph
 * capture: it synchronises `stream`).  `stream` must belong to the current
 * device (GLM53_INVALID_ARGUMENT otherwise).  Limits: the fused step shapes
 * (H, I) in {(4096, 1536), (4096, 2048), (7168, 2048), (6144, 2048),
 * (2048, 1024), (2048, 1536), (1024, 512), (1024, 1024)}, at most 320
 * experts, top_k <= 8, a shared expert (if any) of width I, 16-byte aligned
 * x and weights; other inputs return GLM53_INVALID_ARGUMENT with a message.
 * Every call on one GPU shares that GPU's scratch, so calls that overlap on
 * one GPU (concurrent streams or threads) race; the scratch keeps the last
 * call's contents, and out-of-range expert ids (NaN output) are not
 * reported through a readable flag. */
#define GLM53_DECODE_STATIC_SCRATCH_BYTES 131072
int glm53_decode_moe_static(int64_t hidden, int64_t intermediate, int64_t experts, int64_t top_k,
                            float swiglu_limit, const glm53_bank* bank,
                            const glm53_shared_expert* shared, const glm53_router* router,
                            const void* x, const void* residual, void* out, void* stream);

/* ------------------------------------------------------------------------
 * Prefill building blocks -- replace grouped_fp8.py:157-276.
 * ---------------------------------------------------------------------- */

/* build_route_plan + build_grouped_tile_plan (grouped_fp8.py:157-203;
 * native_indexer_plan.metal:1878-1982).  expert_ids int32 [routes] (flat,
 * token-major), scores f32 [routes] (may be NULL).  Outputs (device):
 * sorted_route/inverse/sorted_expert/sorted_token int32 [routes],
 * sorted_score f32 [routes] (ignored when scores is NULL),
 * route_offsets/tile_offsets u32 [experts + 1], tile_expert/tile_start/
 * tile_len int32 [capacity] with capacity = ceil(routes / tile_rows) +
 * experts, status u32 [2] = {invalid route count, valid descriptors}. */
size_t glm53_route_plan_workspace_bytes(int64_t routes, int64_t experts);
int glm53_route_plan(const int32_t* expert_ids, const float* scores, int64_t routes, int64_t top_k,
                     int64_t experts, int64_t tile_rows, int32_t* sorted_route, int32_t* inverse,
                     int32_t* sorted_expert, int32_t* sorted_token, float* sorted_score,
                     uint32_t* route_offsets, uint32_t* tile_offsets, int32_t* tile_expert,
                     int32_t* tile_start, int32_t* tile_len, int64_t capacity, uint32_t* status,
                     void* workspace, size_t workspace_bytes, void* stream);

/* Activation split feeding the grouped FP8 GEMM.  No counterpart in the
 * reference, which multiplies BF16 activations by the dequantised weights
 * (grouped_fp8.py:206-262); exported so the encoding can be checked bit for
 * bit.  Per row and 128-column block: s = 2^ceil(log2(amax / 448)), so
 * amax / s lies in (224, 448] (s = 1 for an all-zero or non-finite amax);
 * q = x / s; hi = E4M3(q); lo = E4M3(16 (q - hi)), both round to nearest
 * even, saturating at +-448 (never the 0x7F / 0xFF codes); x ~= s (hi +
 * lo / 16).  x bf16 rows of x_row_stride elements (2-byte aligned), hi and
 * lo u8 [rows, cols] (8-byte aligned), scale f32 [rows, cols / 128].
 * Requires cols % 128 == 0. */
int glm53_split_activations(const void* x, int64_t rows, int64_t cols, int64_t x_row_stride, uint8_t* hi,
                            uint8_t* lo, float* scale, void* stream);

/* grouped_fp8_linear (grouped_fp8.py:206-262): y[r] = T(x[row(r)] .
 * W[e(r)]^T) for sorted routes r, where row(r) = row_index[r] (NULL:
 * identity) and e(r) comes from the 32-route descriptors.  x bf16
 * [act_rows, K], weight u8 [E, N, K], scale f32 [E, ceil(N/128), K/128],
 * y bf16 [routes, N].  Requires K % 128 == 0 and N % 16 == 0.  code_flags
 * (device int32, may be NULL = scan the weight first) as in glm53_bank. */
size_t glm53_grouped_linear_workspace_bytes(int64_t act_rows, int64_t K);
int glm53_grouped_linear(const void* x, int64_t act_rows, const int32_t* row_index, int64_t routes,
                         int64_t K, const int32_t* tile_expert, const int32_t* tile_start,
                         const int32_t* tile_len, int64_t descriptors, const uint8_t* weight,
                         const float* scale_inv, const int32_t* code_flags, int64_t experts,
                         int64_t N, void* y, void* workspace, size_t workspace_bytes, void* stream);

/* activate_gate_up (grouped_fp8.py:265-270): gate_up bf16 [rows, 2I] ->
 * h bf16 [rows, I] = T(T(g' * sigmoid(g')) * u'), g' = min(g, L),
 * u' = clip(u, -L, L), MLX BF16 rounding. */
int glm53_activate_gate_up(const void* gate_up, int64_t rows, int64_t intermediate, float limit,
                           void* out, void* stream);

/* restore_and_reduce (grouped_fp8.py:273-276) plus optional BF16 add of
 * `shared` bf16 [tokens, H]: out[t] = T(T(sum_s sorted_out[inverse[t*k+s]]
 * * sorted_score[...]) + shared[t]). */
int glm53_restore_and_reduce(const void* sorted_out, const float* sorted_score,
                             const int32_t* inverse, int64_t tokens, int64_t top_k, int64_t H,
                             const void* shared, void* out, void* stream);

/* Exact Direct accumulation (fp8.py:384-397; native_indexer_plan.metal:
 * 2174-2207): per token, ascending expert id, total = T(total + T(out *
 * score)); expert_ids / scores are the unsorted flat routes. */
int glm53_direct_order_reduce(const void* sorted_out, const int32_t* inverse,
                              const int32_t* expert_ids, const float* scores, int64_t tokens,
                              int64_t top_k, int64_t H, const void* shared, void* out,
                              void* stream);

/* MLX BF16 sigmoid used inside the SwiGLU epilogue (packed.py:155-160),
 * elementwise over n BF16 values, in the form every SwiGLU of the library
 * evaluates (hardware exponential and reciprocal, with the correctly
 * rounding steps where those would change a BF16 result).  Diagnostic: pins
 * the device arithmetic against the reference's exhaustive sweep. */
int glm53_sigmoid_bf16(const void* gate, int64_t n, void* out, void* stream);

/* ------------------------------------------------------------------------
 * Prefill plan -- replaces native_prefill_moe_plan.h:18-96
 * `NativePrefillMoEPlan` and grouped_fp8.py:279-328
 * `SortedGroupedFP8MoE.grouped_from_routes` (+ the shared expert).
 * ---------------------------------------------------------------------- */
typedef struct glm53_prefill_plan glm53_prefill_plan;

int glm53_prefill_plan_create(int64_t hidden, int64_t intermediate, int64_t shared_intermediate,
                              int64_t experts, int64_t top_k, int64_t max_tokens,
                              float swiglu_limit, glm53_prefill_plan** out);
void glm53_prefill_plan_destroy(glm53_prefill_plan* plan);

/* x bf16 [tokens, H] -> out bf16 [tokens, H].  Routes come from `router`
 * when expert_ids is NULL, otherwise from expert_ids int32 [tokens, top_k]
 * and scores f32 [tokens, top_k].  reduction: GLM53_REDUCE_*. */
int glm53_prefill_moe(glm53_prefill_plan* plan, const glm53_bank* bank,
                      const glm53_shared_expert* shared, const glm53_router* router, const void* x,
                      int64_t tokens, const int32_t* expert_ids, const float* scores,
                      int32_t reduction, void* out, void* stream);

/* NativePrefillMoEPlan.execute_indirect_hc (native_prefill_moe_plan.cpp:
 * 101-119, finish_hc 136-161; kernel native_indexer_plan.metal:2362-2388):
 * the MoE of glm53_prefill_moe followed by the hyper-connection expand,
 * fused into the reduction (the MoE output is never written):
 * out_hc[t, b, h] = T(post[t, b] * moe[t, h] + mixed), mixed = fma chain
 * over s = 0..3 of comb[t, s, b] * residual[t, s, h], starting from 0.
 * residual bf16 [tokens, 4, H], post f32 [tokens, 4], comb f32
 * [tokens, 4, 4], out_hc bf16 [tokens, 4, H]. */
int glm53_prefill_moe_hc(glm53_prefill_plan* plan, const glm53_bank* bank,
                         const glm53_shared_expert* shared, const glm53_router* router,
                         const void* x, int64_t tokens, const int32_t* expert_ids,
                         const float* scores, int32_t reduction, const void* residual,
                         const float* post, const float* comb, void* out_hc, void* stream);

/* Synchronous: invalid route count of the last glm53_prefill_moe. */
int glm53_prefill_plan_status(glm53_prefill_plan* plan, uint32_t* invalid_routes);

/* Read-only counters (NativePrefillMoEPlan, bindings.cpp:389-407): as the
 * decode plan's (weights_bound / router_bound stay 0). */
int glm53_prefill_plan_counters(const glm53_prefill_plan* plan, glm53_plan_counters* out);

/* buffer_identities (bindings.cpp:406-407): device addresses of the plan's
 * scratch buffers, fixed at creation; min(count, capacity) values to out
 * (host), the count to *count. */
int glm53_prefill_plan_identities(const glm53_prefill_plan* plan, uint64_t* out, int32_t capacity,
                                  int32_t* count);

/* Device scratch of the last call: which = 0 ids int32 [tokens, top_k],
 * 1 scores f32 [tokens, top_k], 2 sorted route order int32 [routes],
 * 3 descriptors int32 [3, capacity]. */
int glm53_prefill_plan_scratch(glm53_prefill_plan* plan, int32_t which, void** ptr, size_t* bytes);

/* ------------------------------------------------------------------------
 * Seeded synthetic inputs (no reference counterpart: the reference loads a
 * checkpoint).  Element i of stream `seed` is N(0, std) (or U(lo, hi)). */
int glm53_synth_fp8(uint8_t* codes, float* scale_inv, int64_t rows, int64_t cols, uint64_t seed,
                    float std, void* stream);
int glm53_synth_f32(float* out, int64_t n, uint64_t seed, float std, float lo, float hi,
                    int32_t uniform, void* stream);
int glm53_synth_bf16(void* out, int64_t n, uint64_t seed, float std, void* stream);
/* batch matrices at codes + b * codes_stride / scale_inv + b * scale_stride;
 * matrix b draws from a key derived from (seed, b), matrix 0 from seed.  The
 * codes are written in the layout row_group_log2 (glm53_bank); the values
 * do not depend on it. */
int glm53_synth_fp8_batched(uint8_t* codes, float* scale_inv, int64_t rows, int64_t cols, int64_t batch,
                            int64_t codes_stride, int64_t scale_stride, uint64_t seed, float std,
                            int32_t row_group_log2, void* stream);
/* out bf16 [n] = N(0, std) under key (seed, *counter), then ++*counter
 * (device uint32): a fresh decode input per replay of a captured graph. */
int glm53_synth_step_input(void* out, int64_t n, uint64_t seed, float std, uint32_t* counter,
                           void* stream);

/* Streaming-read probe (measurement only): reads every byte of buf once with
 * 16-byte non-temporal loads from `blocks` workgroups of 256 lanes and writes
 * 4 words per workgroup to sink ([4 * blocks] uint32).  Its rate is the
 * achievable-HBM reference of the benchmark's roofline fractions. */
int glm53_probe_read(const void* buf, int64_t bytes, uint32_t* sink, int32_t blocks, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GLM53_MOE_H */
