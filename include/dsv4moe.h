/*
 * dsv4moe.h -- C ABI of the MI355X (gfx950) DeepSeek-V4-Flash MoE hot path.
 *
 * Every entry point is stream-ordered on the HIP stream passed as `stream`
 * (a hipStream_t; NULL = the default stream), allocates no device memory,
 * performs no host<->device synchronisation, and returns DSV4MOE_OK (0) or a
 * nonzero status with a thread-local message in dsv4moe_last_error().
 * Arguments are validated before any launch; on a validation error nothing is
 * launched.  Device pointers are plain addresses of caller-owned buffers.
 *
 * Tensor conventions (row-major, contiguous):
 *   bf16 values are passed as uint16_t bit patterns;
 *   route ids int32 [T, k]; route weights fp32 [T, k];
 *   int4 weights in the "tiled" layout produced by dsv4moe_pack_int4_g128.
 *
 * Reference interfaces replaced (gaiban-lite, paths from its repo root) are
 * cited per entry point.
 */
#ifndef DSV4MOE_H
#define DSV4MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DSV4MOE_OK 0
#define DSV4MOE_EINVAL 1   /* contract violation detected before launch */
#define DSV4MOE_EHIP 2     /* HIP runtime error (launch / device state) */

#define DSV4MOE_SCORE_SIGMOID 0
#define DSV4MOE_SCORE_SOFTMAX 1
#define DSV4MOE_SCORE_SQRTSOFTPLUS 2

#define DSV4MOE_GROUP 128  /* int4 quantisation group along K */

/* Element-type codes of the `*_dtype` arguments. */
#define DSV4MOE_DTYPE_BF16 0
#define DSV4MOE_DTYPE_FP16 1
#define DSV4MOE_DTYPE_FP32 2
#define DSV4MOE_DTYPE_FP8_E4M3 3  /* OCP E4M3FN (torch.float8_e4m3fn) */

/* Message of the last failing call on this thread ("" if none). */
const char* dsv4moe_last_error(void);

/* ABI revision of this library. */
int32_t dsv4moe_abi_version(void);

/*
 * Per-kernel timing of the next `max_calls` calls of dsv4moe_layer_w4a16 /
 * dsv4moe_experts_w4a16, recorded with HIP events on the launch stream at 7
 * stamps (begin, after route, after align, after row sums, after stage 1,
 * after stage 2, after combine).  No counterpart in the reference (its benches
 * time with CUDA events from Python, experiments/A3F-marlin-moe-flash/common.py:220-234).
 * dsv4moe_profile_end synchronises on the last event and writes the mean
 * duration in ms of the 6 intervals (route, align, row sums, stage 1, stage 2,
 * combine) to mean_ms[6].  Process-global; use from one host thread.
 */
int dsv4moe_profile_begin(int32_t max_calls);
int dsv4moe_profile_end(float* mean_ms, int32_t n_intervals, int32_t* calls_recorded);
/*
 * As dsv4moe_profile_begin, recording only the stamps whose bit is set in
 * stamp_mask (bit i = stamp i in the order above), so that a timed loop can
 * measure one kernel with two events instead of seven.  Intervals whose two
 * stamps are not both recorded read -1 in dsv4moe_profile_end.
 */
int dsv4moe_profile_begin_stamps(int32_t max_calls, uint32_t stamp_mask);

/*
 * Block-size policy for the expert alignment.
 * Replaces _marlin_block_size_m (runtime/dsv4_direct/moe_runtime.py:276-300):
 * first of (8,16,32,48,64) with rows*topk/experts/bs < 0.9, else 64; at least
 * 16 for 1-byte activations.  Returns -1 on invalid arguments.
 */
int32_t dsv4moe_block_size_m(int64_t rows, int32_t topk, int32_t experts, int32_t act_itemsize);

/*
 * Capacity of sorted_token_ids.
 * Replaces max_padded_tokens (runtime/dsv4_direct/deterministic_moe_align.py:17-32).
 * Returns -1 on invalid arguments.
 */
int64_t dsv4moe_max_padded_tokens(int64_t num_assignments, int32_t num_experts, int32_t block_size);

/*
 * Router: scores, top-(k+1) selection, renormalised weights, margin.
 * Replaces the score/top-k half of gate_forward_with_boundary
 * (runtime/dsv4_direct/moe_forward.py:52-94) and Gate.forward
 * (reference/inference/model.py:564-584) for pre-computed logits.
 *
 *   logits   fp32 [tokens, experts]
 *   bias     fp32 [experts] or NULL (shifts selection only)
 *   ids      int32 [tokens, topk]      out
 *   weights  fp32  [tokens, topk]      out (score/sum*route_scale; softmax: score*route_scale)
 *   margin   fp32  [tokens] or NULL    out (sel[k-1]-sel[k]; 0 if topk == experts)
 *   selection_ids    int32 [tokens, min(topk+1,experts)] or NULL   out
 *   selection_scores fp32  [tokens, min(topk+1,experts)] or NULL   out
 * Ordering: biased score descending, expert id ascending.  experts <= 1024,
 * 1 <= topk <= min(experts, 16).
 */
int dsv4moe_route_topk(const float* logits, const float* bias, int64_t tokens, int32_t experts,
                       int32_t topk, int32_t score_func, float route_scale, int32_t* ids,
                       float* weights, float* margin, int32_t* selection_ids,
                       float* selection_scores, void* stream);

/*
 * Hash router: ids = tid2eid[input_ids], weights from sqrt-softplus scores.
 * Replaces hash_gate_forward (runtime/dsv4_direct/moe_forward.py:186-231).
 *   tid2eid int64 [vocab, topk]; input_ids int64 [tokens].
 *   selected_scores fp32 [tokens, topk] or NULL: the unnormalised gathered scores.
 *   An id or token outside its table is written as expert id -1.
 */
int dsv4moe_route_hash(const float* logits, const int64_t* tid2eid, int64_t vocab,
                       const int64_t* input_ids, int64_t tokens, int32_t experts, int32_t topk,
                       float route_scale, int32_t* ids, float* weights,
                       float* selected_scores, void* stream);

/*
 * Router logits from hidden states: logits = x . Wg^T with fp32 accumulation
 * (bf16 products are exact in fp32).  Replaces F.linear(x.float(), W.float())
 * (runtime/dsv4_direct/moe_forward.py:80; reference/inference/model.py:565).
 *   x bf16 [tokens, hidden]; wg bf16 [experts, hidden]; logits fp32 [tokens, experts].
 *   hidden % 32 == 0, experts % 16 == 0.
 */
int dsv4moe_gate_logits(const uint16_t* x, const uint16_t* wg, int64_t tokens, int32_t hidden,
                        int32_t experts, float* logits, void* stream);

/*
 * Deterministic expert alignment.
 * Replaces deterministic_moe_align_block_size
 * (runtime/dsv4_direct/deterministic_moe_align.py:58-133) and the Triton
 * fixed_b240_moe_align_block8 (runtime/dsv4_direct/fixed_moe_align.py:407-421).
 *   ids int32 [tokens, topk], every id in [0, experts)
 *   sorted_token_ids int32 [capacity]  out (capacity = dsv4moe_max_padded_tokens)
 *   expert_ids int32 [ceil(capacity/block_size)]  out
 *   num_tokens_post_padded int32 [1]  out; -1 if an id was out of range
 * experts <= 1024.
 */
int dsv4moe_align(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts,
                  int32_t block_size, int32_t* sorted_token_ids, int64_t capacity,
                  int32_t* expert_ids, int64_t num_blocks, int32_t* num_tokens_post_padded,
                  void* stream);

/*
 * The same alignment (same outputs, bit for bit) split over workgroups when
 * tokens * topk >= 8192: one launch counts chunks of the ids into the
 * workspace, a second scatters each chunk from the summed counts.  The
 * workspace replaces the reference's torch temporaries of
 * deterministic_moe_align_block_size (deterministic_moe_align.py:95-106); its
 * size is dsv4moe_align_workspace_bytes (0 below the split threshold, then the
 * call is dsv4moe_align and workspace may be NULL; at most 262400 bytes).
 * The workspace needs no initial contents.
 */
size_t dsv4moe_align_workspace_bytes(int64_t tokens, int32_t topk, int32_t experts);
int dsv4moe_align_ws(const int32_t* ids, int64_t tokens, int32_t topk, int32_t experts,
                     int32_t block_size, int32_t* sorted_token_ids, int64_t capacity,
                     int32_t* expert_ids, int64_t num_blocks, int32_t* num_tokens_post_padded,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Repack int4 group-128 weights from the checkpoint layout into the
 * pair-interleaved tiled layout the expert kernels stream.  Replaces the
 * load-time Marlin repack (runtime/dsv4_direct/ops/marlin_moe.py:173-223).
 *   canon        uint8 [batch, n, k/2]   (low nibble = even k, two's complement)
 *   canon_scales bf16  [batch, n, k/128]
 *   pairing      DSV4MOE_PAIR_PLAIN: strip pair p = rows 32p..32p+31 (w2);
 *                DSV4MOE_PAIR_GATED: pair p = rows 16p.. and n/2+16p.. (w13:
 *                the gate row strip and its up row strip)
 *   packed       uint8 [batch, n*k/2]  out: tile (p, g, m) of 16 rows x 128 k
 *                at byte ((p*(k/128) + g)*2 + m)*1024
 *   packed_scales bf16 [batch, n*k/128] out: [p][g][quad][m][4 rows]
 * A group whose scale is +-0 is stored with all codes q = 0 and the nearest
 * nonzero scale of its row (previous group first, else next, else 1.0), which
 * leaves every product q * s unchanged and every packed scale nonzero.
 * n % 32 == 0, k % 128 == 0.
 */
#define DSV4MOE_PAIR_PLAIN 0
#define DSV4MOE_PAIR_GATED 1
int dsv4moe_pack_int4_g128(const uint8_t* canon, const uint16_t* canon_scales, int64_t batch,
                           int64_t n, int64_t k, int32_t pairing, uint8_t* packed,
                           uint16_t* packed_scales, void* stream);

/*
 * Group-scale ratios of the W4A16 prefill kernels, from packed scales
 * (dsv4moe_pack_int4_g128's packed_scales [batch, n*k/128] bf16) into
 * ratios fp32 [batch, n*k/128] in the same element order: the ratio of a
 * row's scale of group g-1 to its scale of group g (fp32, correctly rounded;
 * 0 for g = 0).  The prefill kernels keep each accumulator divided by the
 * current group's scale: a <- a * ratio + (next group's partial sums), and
 * multiply by the last group's scale at the end.  Computed once per packed
 * weight set; no counterpart in the reference (its Marlin kernels scale each
 * dequantised weight).  n a multiple of 32, k of 128.
 * Guard: a matrix (one expert) with a row whose running-sum amplification
 * max_g (s_0 + ... + s_g) / s_g exceeds 2^64 (e.g. a 2^100 group scale
 * before a 2^-100 one) gets 1.0 in its element 0, and element 1 of the first
 * matrix of the call gets 1.0 when any matrix is marked (both are group-0
 * ratios, otherwise 0 and never multiplied into a nonzero sum); the expert
 * entries then compute the marked experts' prefill blocks with exact
 * per-group scaling.  One call must cover the whole expert stack passed to
 * the expert entries as w13r / w2r.
 */
int dsv4moe_pack_int4_ratios(const uint16_t* packed_scales, int64_t batch, int64_t n, int64_t k, float* ratios,
                             void* stream);

/*
 * Workspace needed by dsv4moe_experts_w4a16 / _w4a8 (bytes).
 */
size_t dsv4moe_experts_workspace_bytes(int64_t tokens, int32_t topk, int32_t hidden,
                                       int32_t inter, int32_t has_shared);

/*
 * Routed + shared experts with the fused combine, W4A16.
 * Replaces the vLLM _fused_marlin_moe call (runtime/dsv4_direct/moe_runtime.py:1829-1856),
 * the top-k sum (:1857), shared_bf16_partial (:246-263) and the combine add (:1873).
 *   x        bf16 [tokens, hidden]
 *   w13q/w13s  tiled int4 + scales (DSV4MOE_PAIR_GATED), experts(+1 shared) x
 *              [2*inter, hidden] (rows [0,inter) = gate w1, [inter,2*inter) = up w3)
 *   w2q/w2s    tiled int4 + scales (DSV4MOE_PAIR_PLAIN), experts(+1 shared) x [hidden, inter]
 *   w13r/w2r   fp32 scale ratios of w13s / w2s (dsv4moe_pack_int4_ratios), read by
 *              the prefill kernels (block_size >= 32); required, 16-byte aligned
 *   has_shared 1: expert index `experts` is the always-on shared expert
 *   weights  fp32 [tokens, topk]  (route weights, applied to the w2 output)
 *   sorted_token_ids / expert_ids / num_tokens_post_padded: dsv4moe_align output
 *   clamp_limit > 0: gate = min(gate, L), up = clamp(up, -L, L) before SiLU(gate)*up
 *   out      bf16 [tokens, hidden] = bf16( sum_j routed_j + shared ), fp32 accumulation
 * hidden % 256 == 0, inter % 256 == 0, block_size in {8,16,32,48,64}.
 */
int dsv4moe_experts_w4a16(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                          int32_t experts, int32_t topk, const uint8_t* w13q,
                          const uint16_t* w13s, const uint8_t* w2q, const uint16_t* w2s,
                          const float* w13r, const float* w2r, int32_t has_shared, const float* weights,
                          const int32_t* sorted_token_ids, int64_t capacity,
                          const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                          int32_t block_size, float clamp_limit, uint16_t* out,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * Whole MoE layer, W4A16: route (from logits) -> align -> experts -> combine.
 * Replaces TP4MoE.compute_partial (runtime/dsv4_direct/moe_runtime.py:1714-1888)
 * at world size 1.  Route and alignment outputs are caller-owned and written.
 * bias may be NULL; margin may be NULL.  Weights, scales and scale ratios as
 * in dsv4moe_experts_w4a16.
 */
int dsv4moe_layer_w4a16(const uint16_t* x, const float* logits, const float* bias,
                        int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                        int32_t topk, int32_t score_func, float route_scale,
                        const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q,
                        const uint16_t* w2s, const float* w13r, const float* w2r, int32_t has_shared,
                        float clamp_limit,
                        int32_t block_size, int32_t* ids, float* weights, float* margin,
                        int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                        int32_t* num_tokens_post_padded, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * No counterpart in the reference.  The fused W4A16 layer call for callers
 * that cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc): the arguments and results of
 * dsv4moe_layer_w4a16 without the workspace, which the library keeps in a
 * static device array of DSV4MOE_NOALLOC_SCRATCH_BYTES on each GPU it runs
 * on (held until the process ends).  Calls whose workspace need
 * (dsv4moe_experts_workspace_bytes) exceeds it fail with DSV4MOE_EINVAL before
 * any launch: at H=4096, I=2048, top-6 with the shared expert that is above
 * 464 tokens.  Calls that overlap on one GPU share the array and race.  The
 * stream must belong to the current device.  Allocates nothing.
 */
#define DSV4MOE_NOALLOC_SCRATCH_BYTES (64u << 20)
int dsv4moe_layer_w4a16_noalloc(const uint16_t* x, const float* logits, const float* bias,
                                int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                                int32_t topk, int32_t score_func, float route_scale,
                                const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q,
                                const uint16_t* w2s, const float* w13r, const float* w2r, int32_t has_shared,
                                float clamp_limit, int32_t block_size, int32_t* ids, float* weights,
                                float* margin, int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                                int32_t* num_tokens_post_padded, uint16_t* out, void* stream);

/*
 * MXFP4 experts: E2M1 codes with one E8M0 scale per 32 K, the checkpoint
 * format of the reference's routed experts (runtime/dsv4_direct/moe_forward.py:
 * 23-40,115-155; the MXFP4 Marlin path of ops/marlin_moe.py:173-223 and
 * moe_runtime.py:1829-1856; dense restatement ops/dense_moe.py:41-68,336-354).
 *
 * dsv4moe_pack_mxfp4_g32 repacks checkpoint-layout weights:
 *   canon        uint8 [batch, n, k/2]  (E2M1, low nibble = even k)
 *   canon_scales uint8 [batch, n, k/32] (E8M0: 2^(e-127); 255 is reserved)
 *   packed       uint8 [batch, n*k/2]   out: the tile geometry and pairing of
 *                dsv4moe_pack_int4_g128; lane L's dword d of a tile holds the 4
 *                checkpoint bytes of row L%16 for k = 128g + 32d + 8*(L/16) ..
 *   packed_scales uint8 [batch, n*k/32] out: 128 bytes per (pair, group),
 *                byte (r16*2 + m)*4 + d = scale of row r16 of member m for
 *                k in [128g + 32d, +32)
 *   n % 32 == 0, k % 128 == 0.
 * dsv4moe_experts_mxfp4: as dsv4moe_experts_w4a16 (same routing, alignment,
 * workspace from dsv4moe_experts_workspace_bytes, combine and output) with
 * MXFP4-packed weights: W = code * 2^(e-127) exactly, bf16 MFMA with fp32
 * accumulation.  hidden % 512 == 0, inter % 512 == 0.
 */
int dsv4moe_pack_mxfp4_g32(const uint8_t* canon, const uint8_t* canon_scales, int64_t batch,
                           int64_t n, int64_t k, int32_t pairing, uint8_t* packed,
                           uint8_t* packed_scales, void* stream);
int dsv4moe_experts_mxfp4(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                          int32_t experts, int32_t topk, const uint8_t* w13q, const uint8_t* w13s,
                          const uint8_t* w2q, const uint8_t* w2s, int32_t has_shared,
                          const float* weights, const int32_t* sorted_token_ids, int64_t capacity,
                          const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                          int32_t block_size, float clamp_limit, uint16_t* out, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * W4A8 over MXFP4 experts: the reference's W4A8 mode on its checkpoint
 * format, _fused_marlin_moe(input_dtype=float8_e4m3fn) over MXFP4 weights
 * with the is_a_8bit repack (runtime/dsv4_direct/ops/marlin_moe.py:197-222,
 * moe_runtime.py:207-235,1829-1856).
 *
 * dsv4moe_pack_mxfp4_g32_w4a8 repacks checkpoint-layout weights as
 * dsv4moe_pack_mxfp4_g32 (same arguments, tile geometry, pairing and
 * packed_scales), except inside a tile: lane L holds the 16 checkpoint bytes
 * of row L%16 for k = 128g + 32*(L/16) .. +31, i.e. one 32-K scale group.
 * dsv4moe_experts_w4a8_mxfp4: as dsv4moe_experts_w4a8 (workspace from
 * dsv4moe_experts_w4a8_workspace_bytes) with those weights: x and the
 * SwiGLU output h are quantised per row to e4m3 (s = max(amax, 1e-12) / 448),
 * each 32-K product of E2M1 codes and e4m3 codes is scaled by the group's
 * E8M0 byte inside the block-scaled fp8 x fp4 MFMA, fp32 accumulation, the
 * row scale applied to the result.  hidden % 512 == 0, inter % 512 == 0.
 */
int dsv4moe_pack_mxfp4_g32_w4a8(const uint8_t* canon, const uint8_t* canon_scales, int64_t batch,
                                int64_t n, int64_t k, int32_t pairing, uint8_t* packed,
                                uint8_t* packed_scales, void* stream);
int dsv4moe_experts_w4a8_mxfp4(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                               int32_t experts, int32_t topk, const uint8_t* w13q, const uint8_t* w13s,
                               const uint8_t* w2q, const uint8_t* w2s, int32_t has_shared,
                               const float* weights, const int32_t* sorted_token_ids, int64_t capacity,
                               const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                               int32_t block_size, float clamp_limit, uint16_t* out, void* workspace,
                               size_t workspace_bytes, void* stream);

/*
 * Whole MoE layer over MXFP4 experts: route (from logits) -> align ->
 * experts (dsv4moe_experts_mxfp4) -> combine, as dsv4moe_layer_w4a16 (same
 * arguments; w13s / w2s are the packed E8M0 bytes).  Replaces
 * TP4MoE.compute_partial (runtime/dsv4_direct/moe_runtime.py:1714-1888) for
 * the checkpoint's routed-expert format at world size 1.
 */
int dsv4moe_layer_mxfp4(const uint16_t* x, const float* logits, const float* bias,
                        int64_t tokens, int32_t hidden, int32_t inter, int32_t experts,
                        int32_t topk, int32_t score_func, float route_scale,
                        const uint8_t* w13q, const uint8_t* w13s, const uint8_t* w2q,
                        const uint8_t* w2s, int32_t has_shared, float clamp_limit,
                        int32_t block_size, int32_t* ids, float* weights, float* margin,
                        int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                        int32_t* num_tokens_post_padded, uint16_t* out, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * Whole MoE layer in the W4A8 mode (marlin_input_dtype = float8_e4m3fn):
 * route (from logits) -> align -> W4A8 experts -> combine, with the per-row
 * e4m3 quantisation of x done by the alignment launch's other workgroups.
 * Arguments as dsv4moe_layer_w4a16 without the ratios; the workspace size is
 * dsv4moe_experts_w4a8_workspace_bytes.  dsv4moe_layer_w4a8 takes the int4
 * weights of dsv4moe_experts_w4a8, dsv4moe_layer_w4a8_mxfp4 the MXFP4 weights
 * of dsv4moe_experts_w4a8_mxfp4 (w13s / w2s the packed E8M0 bytes); the
 * results are bit-identical to route, align and that experts entry called in
 * turn.  Replaces TP4MoE.compute_partial
 * (runtime/dsv4_direct/moe_runtime.py:1714-1888) with
 * _preset_w4a8_activation_quant (moe_runtime.py:207-235) at world size 1.
 */
int dsv4moe_layer_w4a8(const uint16_t* x, const float* logits, const float* bias, int64_t tokens, int32_t hidden,
                       int32_t inter, int32_t experts, int32_t topk, int32_t score_func, float route_scale,
                       const uint8_t* w13q, const uint16_t* w13s, const uint8_t* w2q, const uint16_t* w2s,
                       int32_t has_shared, float clamp_limit, int32_t block_size, int32_t* ids, float* weights,
                       float* margin, int32_t* sorted_token_ids, int64_t capacity, int32_t* expert_ids,
                       int32_t* num_tokens_post_padded, uint16_t* out, void* workspace, size_t workspace_bytes,
                       void* stream);
int dsv4moe_layer_w4a8_mxfp4(const uint16_t* x, const float* logits, const float* bias, int64_t tokens,
                             int32_t hidden, int32_t inter, int32_t experts, int32_t topk, int32_t score_func,
                             float route_scale, const uint8_t* w13q, const uint8_t* w13s, const uint8_t* w2q,
                             const uint8_t* w2s, int32_t has_shared, float clamp_limit, int32_t block_size,
                             int32_t* ids, float* weights, float* margin, int32_t* sorted_token_ids,
                             int64_t capacity, int32_t* expert_ids, int32_t* num_tokens_post_padded, uint16_t* out,
                             void* workspace, size_t workspace_bytes, void* stream);

/*
 * Weight layouts of the dense linears (argument weight_layout):
 *   DSV4MOE_WEIGHT_ROWMAJOR  the checkpoint's bytes as stored, row-major [n, k]
 *                            (what the reference's entry points take);
 *   DSV4MOE_WEIGHT_TILED     the load-time repack of dsv4moe_pack_int8 /
 *                            dsv4moe_pack_fp8 (1 KiB tiles, below).
 * Both feed the same kernels and give the same bits.
 */
#define DSV4MOE_WEIGHT_TILED 0
#define DSV4MOE_WEIGHT_ROWMAJOR 1

/*
 * W8A16 dense linear: out[M,N] = bf16( a[M,K] . (q[N,K] * s[N])^T ), int8
 * symmetric per-output-channel weights, bf16 scales, fp32 accumulation.
 * Replaces w8a16_gemm_into / make_gemm_plan / _automatic_split_k
 * (experiments/C1F-integrated-block/weight_only_linear.py:794-823, :181-221,
 * :168-179) and its kernels (:537-702) for the int8 per-channel format.
 *
 * dsv4moe_pack_int8: row-major int8 [n, k] -> 1 KiB tiles of 16 rows x 64 k,
 *   tile (strip, window) at byte (strip*(k/64) + window)*1024, lane l's 16 bytes
 *   = row 16*strip + l%16, k 64*window + 16*(l/16) ..+15.  n % 16 == 0, k % 128 == 0.
 * dsv4moe_w8a16_split_k: this library's split-K policy for (m, n, k), 1..16.
 * dsv4moe_w8a16_workspace_bytes: split*m*n*4 when split > 1, else 0.
 * dsv4moe_w8a16_linear:
 *   a       bf16 [m, k]
 *   wq      int8 [n, k] in weight_layout (row-major, or packed by dsv4moe_pack_int8)
 *   ws      bf16 [n]
 *   split_k 1, 2, 4, 8 or 16 (<= k/128); > 1 uses workspace fp32 [split, m, n],
 *           partials reduced in split order before the single bf16 rounding
 *   out     bf16 [m, n]
 * m >= 0, n % 16 == 0, k % 128 == 0, m*k*2 and n*k below 2^31.
 */
int dsv4moe_pack_int8(const int8_t* w, int64_t n, int64_t k, uint8_t* packed, void* stream);
int32_t dsv4moe_w8a16_split_k(int64_t m, int64_t n, int64_t k);
size_t dsv4moe_w8a16_workspace_bytes(int64_t m, int64_t n, int32_t split_k);
int dsv4moe_w8a16_linear(const uint16_t* a, int64_t m, int64_t n, int64_t k, const uint8_t* wq,
                         int32_t weight_layout, const uint16_t* ws, int32_t split_k, float* workspace,
                         size_t workspace_bytes, uint16_t* out, void* stream);

/*
 * W8A16 dense linear over the reference checkpoint's weight format: FP8 E4M3
 * codes with one E8M0 scale per 128 x 128 block,
 *   out[M,N] = bf16( a[M,K] . bf16(q[N,K] * 2^(e[n/128][k/128] - 127))^T ),
 * fp32 accumulation.  Replaces w8a16_gemm_into with its checkpoint FP8
 * weights (experiments/C1F-integrated-block/weight_only_linear.py:537-598,
 * E8M0 decode :488-513: byte 0 is 2^-127, 255 reserved) and
 * dequant_fp8_block (runtime/dsv4_direct/moe_forward.py:158-176).
 *   wq      the E4M3 bytes [n, k] in weight_layout: as stored in the
 *           checkpoint (row-major), or packed by dsv4moe_pack_int8 (a byte
 *           permutation; it packs any 1-byte format)
 *   ws8     E8M0 bytes [ceil(n/128), k/128], row-major; 255 must not occur
 *           (the reference rejects it in a cold preflight; the Python wrapper
 *           does the same at load time)
 *   split_k, workspace, out: as dsv4moe_w8a16_linear (same split policy).
 * m >= 0, n % 16 == 0, k % 128 == 0, k <= 32768, m*k*2 and n*k below 2^31.
 */
int dsv4moe_w8a16_fp8_linear(const uint16_t* a, int64_t m, int64_t n, int64_t k, const uint8_t* wq,
                             int32_t weight_layout, const uint8_t* ws8, int32_t split_k, float* workspace,
                             size_t workspace_bytes, uint16_t* out, void* stream);

/*
 * Block-FP8 W8A8 activation quantiser.  Replaces activation_quant_into
 * (runtime/dsv4_direct/fp8_linear.py:523-569, kernel :354-392).
 *   x      [m, k] row-major, x_dtype 0 = bf16, 1 = fp16, 2 = fp32
 *   q      E4M3 bytes [m, k] row-major (out)
 *   scale  E8M0 bytes [m, k/128] (out): per row and 128-K block,
 *          e = ceil-to-power-of-two exponent of max(amax, 1e-4) * fp32(1/448),
 *          clamped to [1, 254]; q = e4m3(clamp(x / 2^(e-127), -448, 448))
 * k a multiple of 128.
 */
int dsv4moe_act_quant_block_fp8(const void* x, int32_t x_dtype, int64_t m, int64_t k, uint8_t* q,
                                uint8_t* scale, void* stream);

/*
 * Block-FP8 W8A8 GEMM.  Replaces block_fp8_gemm_into
 * (runtime/dsv4_direct/fp8_linear.py:572-684, kernels :395-497) and the
 * automatic split of make_gemm_plan (:206-251):
 *   out[m, n] = bf16( sum over 128-K blocks kb of
 *                     (A_kb . W_kb^T) * 2^(a_scale[m, kb] - 127) * 2^(w_scale[n/128, kb] - 127) )
 *   a        E4M3 [m, k] row-major, a_scale E8M0 [m, k/128] (dsv4moe_act_quant_block_fp8)
 *   wq       E4M3 weights [n, k] in weight_layout (the checkpoint's row-major
 *            bytes, or packed by dsv4moe_pack_int8 into 1 KiB tiles)
 *   w_scale  E8M0 [ceil(n/128), k/128] (the checkpoint's block scales; byte 0 = 2^-127)
 *   split_k  1, 2, 4 or 8; > 1 needs dsv4moe_block_fp8_workspace_bytes bytes of
 *            fp32 [split, m, n] workspace, reduced in split order
 * n a multiple of 16, k a multiple of 128 up to 32768, m*k and n*k below 2^31.
 * dsv4moe_block_fp8_split_k returns this library's split for (m, n, k).
 */
int32_t dsv4moe_block_fp8_split_k(int64_t m, int64_t n, int64_t k);
size_t dsv4moe_block_fp8_workspace_bytes(int64_t m, int64_t n, int32_t split_k);
int dsv4moe_block_fp8_gemm(const uint8_t* a, const uint8_t* a_scale, int64_t m, int64_t n, int64_t k,
                           const uint8_t* wq, int32_t weight_layout, const uint8_t* w_scale, int32_t split_k,
                           float* workspace, size_t workspace_bytes, uint16_t* out, void* stream);

/*
 * Shared expert over the checkpoint's FP8 E4M3 / E8M0 128x128-block weights,
 * added into the routed output:
 *   out[T,H] <- bf16( out + shared(x) ),
 *   shared(x) = bf16( bf16( silu(min(g, L)) * clamp(u, -L, L) ) . W2^T ),
 *   g | u     = bf16( x . W13^T ),  W13 = [W1; W3] (gate rows, then up rows),
 * bf16 products of the exactly dequantised weights with fp32 accumulation,
 * no clamp when L = 0.  Replaces prepare_shared_bf16 / shared_bf16_partial
 * and the routed + shared add (runtime/dsv4_direct/moe_runtime.py:238-263,
 * 1865-1873; dequant_fp8_block, moe_forward.py:158-176): the same three
 * bf16 roundings and the same final torch.add of two bf16 tensors.
 *   w13q   E4M3 bytes of W13 [2I, H] packed by dsv4moe_pack_int8
 *   w13s8  E8M0 bytes [2I/128, H/128] (rows of W1's blocks, then W3's)
 *   w2q    E4M3 bytes of W2 [H, I] packed by dsv4moe_pack_int8
 *   w2s8   E8M0 bytes [H/128, I/128]
 *   out    bf16 [T, H], read and written (holds the routed sum on entry)
 *   workspace  dsv4moe_shared_fp8_workspace_bytes(T, H, I) bytes, 256-byte aligned
 * hidden and inter: multiples of 128 up to 32768.  Four to six launches
 * (two W8A16 linears with their split-K reductions, one SwiGLU).
 */
size_t dsv4moe_shared_fp8_workspace_bytes(int64_t tokens, int32_t hidden, int32_t inter);
int dsv4moe_shared_fp8_add(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter, const uint8_t* w13q,
                           const uint8_t* w13s8, const uint8_t* w2q, const uint8_t* w2s8, float clamp_limit,
                           uint16_t* out, void* workspace, size_t workspace_bytes, void* stream);

/*
 * W4A8 variant of dsv4moe_experts_w4a16 on the gfx950 fp8 MFMA
 * (v_mfma_scale_f32_16x16x128_f8f6f4, unit block scales).  Replaces the vLLM
 * _fused_marlin_moe call with input_dtype = float8_e4m3fn
 * (runtime/dsv4_direct/moe_runtime.py:1829-1856) and its per-token activation
 * quantiser (_preset_w4a8_activation_quant, :207-235): x and the bf16 SwiGLU
 * output h are each quantised per row to OCP e4m3 (s = max(amax, 1e-12)/448,
 * q = e4m3(clamp(v/s, -448, 448)), round to nearest even) before their GEMM.
 * Same arguments, weights (the tiled int4 layout) and output as the W4A16
 * entry point; workspace from dsv4moe_experts_w4a8_workspace_bytes.
 * hidden % 512 == 0, inter % 512 == 0.
 */
size_t dsv4moe_experts_w4a8_workspace_bytes(int64_t tokens, int32_t topk, int32_t hidden,
                                            int32_t inter, int32_t has_shared);
int dsv4moe_experts_w4a8(const uint16_t* x, int64_t tokens, int32_t hidden, int32_t inter,
                         int32_t experts, int32_t topk, const uint8_t* w13q, const uint16_t* w13s,
                         const uint8_t* w2q, const uint16_t* w2s, int32_t has_shared,
                         const float* weights, const int32_t* sorted_token_ids, int64_t capacity,
                         const int32_t* expert_ids, const int32_t* num_tokens_post_padded,
                         int32_t block_size, float clamp_limit, uint16_t* out, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * Per-row fp8 activation quantiser used by dsv4moe_experts_w4a8
 * (moe_runtime.py:229-232):
 *   x           bf16 [rows, k]
 *   q           e4m3 [rows, k] out, each 128-column group stored in the fp8
 *               MFMA order: byte j*32 + d*8 + b holds column 32d + 8j + P[b],
 *               P = {0,4,1,5,2,6,3,7}, j, d in 0..3
 *   scale       fp32 [rows] out: max(amax, 1e-12) / 448
 *   group_sums  fp32 [rows, k/128] out: sum of the decoded e4m3 values of
 *               each group (the kernels' offset correction)
 * k % 512 == 0.
 */
int dsv4moe_act_quant_fp8(const uint16_t* x, int64_t rows, int32_t k, uint8_t* q, float* scale,
                          float* group_sums, void* stream);

/*
 * Checkpoint-format dequantisers to dense fp32 [rows, k] / [rows, cols]
 * (HBM-bound streaming kernels off the layer's hot path).  Replace the host
 * helpers _decoded_e8m0, dequant_mxfp4 and dequant_fp8_block
 * (runtime/dsv4_direct/moe_forward.py:115-176); the products are the same
 * fp32 multiplications, so the outputs are bit-identical to those helpers'.
 *
 * dsv4moe_decode_e8m0: codes[n] E8M0 bytes -> out[n] fp32 2^(c-127); byte 0
 *   gives 2^-127, byte 255 NaN (torch float8_e8m0fnu -> float).
 * dsv4moe_dequant_mxfp4: packed [rows, k/2] E2M1 codes (low nibble = even
 *   K), scale fp32 [rows, k/32] (decoded) -> out fp32 [rows, k] = value *
 *   scale; k a positive multiple of 32; packed and out 16-byte aligned.
 * dsv4moe_dequant_fp8_block: w [rows, cols] of w_dtype (a DSV4MOE_DTYPE_*),
 *   scale fp32 [ceil(rows/128), ceil(cols/128)] (decoded) -> out fp32
 *   [rows, cols] = w * scale of the 128 x 128 block; out 16-byte aligned
 *   when cols % 4 == 0.
 */
int dsv4moe_decode_e8m0(const uint8_t* codes, int64_t n, float* out, void* stream);
int dsv4moe_dequant_mxfp4(const uint8_t* packed, const float* scale, int64_t rows, int64_t k, float* out,
                          void* stream);
int dsv4moe_dequant_fp8_block(const void* w, int32_t w_dtype, const float* scale, int64_t rows, int64_t cols,
                              float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSV4MOE_H */
