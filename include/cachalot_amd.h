/*
 * cachalot_amd.h -- C ABI of libcachalot_amd.so, the MI355X (gfx950) routed-expert
 * MoE path.
 *
 * Conventions
 *   - every pointer argument is a device pointer unless the comment says "host";
 *   - bf16 tensors are passed as uint16_t bit patterns;
 *   - all work is stream-ordered on `stream` (a hipStream_t; NULL = default
 *     stream) and asynchronous; nothing allocates device memory -- scratch
 *     space comes in through `workspace` (size from the *_workspace_bytes
 *     query); a workspace must be zero-filled once before its first use (its
 *     first 256 bytes hold a completion counter that every call leaves at
 *     zero; the rest is scratch and nothing in it survives a call); calls
 *     that share one workspace must not overlap (same stream, or ordered);
 *   - return 0 on success or a negative CACHALOT_E* code; the message is in
 *     cachalot_last_error() (thread-local).  The Python layer maps EINVAL to
 *     ValueError, ENOTFOUND to KeyError, EHIP to RuntimeError, the exception
 *     types the reference raises for the same conditions
 *     (src/cachalot/model/router_mlx.py:40-66, moe_layer_metal.py:279-283).
 *
 * Reference citations are paths relative to the prooshani/cachalot checkout.
 */
#ifndef CACHALOT_AMD_H
#define CACHALOT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* cachalot_stream_t; /* == hipStream_t */

#define CACHALOT_OK 0
#define CACHALOT_EINVAL (-1)    /* shape / argument contract violated        */
#define CACHALOT_ENOTFOUND (-2) /* expert not resident (slot table -1)       */
#define CACHALOT_EHIP (-3)      /* HIP runtime / launch error                */
#define CACHALOT_ESPACE (-4)    /* workspace too small                       */

/* Router score functions and output orders. */
#define CACHALOT_SCORE_SQRT_SOFTPLUS 0 /* DeepSeek: router_mlx.py:189-191          */
#define CACHALOT_SCORE_SIGMOID 1       /* MiniMax / GLM: minimax/language.py:280-283 */
#define CACHALOT_ORDER_ASCENDING 0     /* argsort(sel)[-k:]: router_mlx.py:197-202    */
#define CACHALOT_ORDER_RANK 1          /* argpartition(-sel): minimax/gpu_select.py:81-106 */

/* Storage type of a 2-bit affine bank's scales and biases: the bank's
 * ExpertFormat.dtypes entry ("bfloat16" / "float16", src/cachalot/storage/index.py:18,153;
 * oQ3e banks carry fp16, src/cachalot/model/expert_affine.py:1-10). */
#define CACHALOT_SCALE_BF16 0
#define CACHALOT_SCALE_F16 1

/* Byte layout of one expert record inside an HBM slot pool.  A slot's record
 * starts at pool + slot * record_bytes; tensor t sits at offset[t].
 * Tensor order: w1.weight, w1.scale(s), w1.biases, w2.weight, w2.scale(s),
 * w2.biases, w3.weight, w3.scale(s), w3.biases (biases unused for FP4).
 * scale_dtype: CACHALOT_SCALE_BF16 or CACHALOT_SCALE_F16 for 2-bit banks;
 * 0 for FP4 banks (their scales are E8M0).
 * Mirrors SlabSlotPool's fixed per-tensor record offsets
 * (src/cachalot/cache/slots.py:185-216). */
typedef struct cachalot_expert_layout {
  int64_t record_bytes;
  int64_t offset[9];
  int32_t scale_dtype;
} cachalot_expert_layout;

/* Library identity and last error (thread-local). */
int cachalot_version(void);
const char* cachalot_last_error(void);

/* Seeded synthetic fill of `n` elements (kinds 0..4: uint32 words, E8M0 bytes
 * uniform in [p0, p1], bf16 uniform p0 + p1*t, bf16 / fp32 Irwin-Hall normal
 * scaled by p1 = sigma / sqrt((65536^2 - 1) / 3)), element i
 * from counter `start + i`.  Test/bench data only -- the reference has no
 * counterpart (it loads checkpoints, storage/reader.py). */
int cachalot_fill_synthetic(void* dst, int64_t n, int64_t start, uint64_t key, int kind,
                            double p0, double p1, int64_t row_total, int64_t row_valid,
                            cachalot_stream_t stream);

/* Router: logits = W x / gate_temp (fixed fp32 order), scores = score_fn(logits),
 * selection = scores + bias (bias_vl where image_mask[t] != 0), top-k with the
 * chosen order and tie rule, weights = scores[idx] normalised (norm != 0 and
 * k > 1) and scaled by route_scale.
 *   x [T, D] bf16, W [E, D] bf16, bias/bias_vl [E] fp32, image_mask [T] u8 or NULL
 *   idx [T, k] int32, w [T, k] fp32, scores [T, E] fp32.
 * Replaces route_topk / route_topk_fused / route_topk_rows / route_topk_batch
 * (src/cachalot/model/router_mlx.py:16-211, router_fused_metal.py:111-148,
 * moe_prefill_batched.py:128-178) and the sigmoid route tail
 * (minimax/gpu_select.py:80-133). */
int cachalot_router_topk(const uint16_t* x, const uint16_t* W, const float* bias,
                         const float* bias_vl, const uint8_t* image_mask,
                         int T, int D, int E, int k, int score_fn, float gate_temp,
                         float route_scale, int norm, int order,
                         int32_t* idx, float* w, float* scores, cachalot_stream_t stream);

/* Decode, one token, top-k routed experts on a 2-bit affine bank
 * (MLX layout: weight [N, Kp/16] u32, scales/biases [N, Kp/group] bf16):
 *   g = bf16(W1 x), u = bf16(W3 x), h = bf16(silu(min(g,L)) * clip(u,-L,L) * w_e),
 *   y_e = bf16(W2 h), routed = sum_e y_e (route order, fp32),
 *   out = bf16(routed + addend).
 * Experts are addressed on the device: slot = slot_table[idx[e]], record at
 * pool + slot * layout.record_bytes; a negative slot contributes zero rows.
 *   x [D] bf16; idx [k] int32; w [k] fp32; slot_table [E] int32;
 *   addend [D] bf16 or NULL; routed [D] fp32 or NULL; out [D] bf16 or NULL.
 * Replaces affine_routed_experts / topk_core / the traced MoE block
 * (src/cachalot/model/expert_affine.py:117-206, moe_layer_metal.py:93-130). */
size_t cachalot_moe_decode_q2_workspace_bytes(int D, int F, int k);
int cachalot_moe_decode_q2(const uint16_t* x, const uint8_t* pool,
                           const cachalot_expert_layout* layout /* host */,
                           const int32_t* slot_table, const int32_t* idx, const float* w,
                           int D, int F, int E, int k, int group, float swiglu_limit,
                           const uint16_t* addend, float* routed, uint16_t* out,
                           void* workspace, size_t workspace_bytes, cachalot_stream_t stream);

/* Decode, one token, top-k routed experts on an FP4 E2M1 / E8M0-block-32 bank:
 *   g = W1 x, u = W3 x (fp32), h = silu(min(g,L)) * clip(u,-L,L) * w_e (fp32),
 *   routed = sum_e W2_e h_e (fp32, route order); out = bf16(routed + addend).
 * Same addressing and optional outputs as cachalot_moe_decode_q2.
 * Replaces fused_routed_experts (src/cachalot/model/moe_fused_metal.py:189-233)
 * and the unfused loop (moe_metal.py:8-37, expert_metal.py:9-64). */
size_t cachalot_moe_decode_fp4_workspace_bytes(int D, int F, int k);
int cachalot_moe_decode_fp4(const uint16_t* x, const uint8_t* pool,
                            const cachalot_expert_layout* layout /* host */,
                            const int32_t* slot_table, const int32_t* idx, const float* w,
                            int D, int F, int E, int k, float swiglu_limit,
                            const uint16_t* addend, float* routed, uint16_t* out,
                            void* workspace, size_t workspace_bytes, cachalot_stream_t stream);

/* Whole decode MoE layer for one token, routing on the device: router scores
 * (as cachalot_router_topk with T = 1, bias only), top-k, slot lookup, gate/up,
 * down and route-order combine in three launches (router with the top-k as
 * its last workgroup's tail, gate/up, down), no host synchronisation.
 *   gate_weight [E, D] bf16, gate_bias [E] fp32; idx_out [k] int32, w_out [k]
 *   fp32 (either may be NULL), scores [E] fp32 (required: it is the hand-off
 *   between the first two launches).  Other arguments as cachalot_moe_decode_*.
 * Replaces moe_layer_forward's routed part for a fully resident bank
 * (src/cachalot/model/moe_layer_metal.py:133-405): the reference's host sync
 * for store addressing (:220-300) becomes a device-side slot-table lookup,
 * the pattern of minimax/gpu_select.py:1-30. */
int cachalot_moe_layer_decode_q2(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                 int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                 int order, const uint8_t* pool, const cachalot_expert_layout* layout /* host */,
                                 const int32_t* slot_table, int D, int F, int group, float swiglu_limit,
                                 const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                 float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                 cachalot_stream_t stream);
/* cachalot_moe_layer_decode_q2_shared: cachalot_moe_layer_decode_q2 with the
 * layer's FP8 shared expert (the arguments of cachalot_shared_expert_fp8 for one
 * token: shared_w1 / shared_w3 [shared_F, D], shared_w2 [D, shared_F] E4M3 with
 * their E8M0 block-32 scales) in place of `addend`: out = bf16(routed + y_sh),
 * y_sh the shared expert's bf16 output, bit for bit what the two calls give.
 * Where the shapes allow (D, shared_F <= 4096 on the matrix-core decode), the
 * shared expert's tiles run inside the routed gate/up and down launches, so its
 * weights stream together with the experts' (three launches in all).  out is
 * required; shared_F a multiple of 32, D and shared_F <= 5120.  Workspace from
 * cachalot_moe_layer_decode_q2_shared_workspace_bytes.  Replaces the shared and
 * routed halves of moe_layer_forward (src/cachalot/model/moe_layer_metal.py:
 * 133-405, the shared expert at :381-397, shared_expert_metal.py:44-188). */
size_t cachalot_moe_layer_decode_q2_shared_workspace_bytes(int D, int F, int k, int shared_F);
int cachalot_moe_layer_decode_q2_shared(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                        int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                        int order, const uint8_t* pool,
                                        const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                        int D, int F, int group, float swiglu_limit, const uint8_t* shared_w1,
                                        const uint8_t* shared_w1_scales, const uint8_t* shared_w3,
                                        const uint8_t* shared_w3_scales, const uint8_t* shared_w2,
                                        const uint8_t* shared_w2_scales, int shared_F, int32_t* idx_out,
                                        float* w_out, float* scores, float* routed, uint16_t* out, void* workspace,
                                        size_t workspace_bytes, cachalot_stream_t stream);
/* cachalot_moe_layer_decode_q2_static: cachalot_moe_layer_decode_q2 with the
 * same arguments minus the workspace, which allocates nothing.  No counterpart
 * in the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Its scratch is a file-scope device array of
 * cachalot_moe_layer_decode_q2_static_max_bytes() bytes (256 KiB) that each GPU
 * holds until the process ends; shapes whose workspace
 * (cachalot_moe_decode_q2_workspace_bytes) exceeds it return CACHALOT_ESPACE.
 * All calls on one GPU share that array: calls that overlap on one GPU race. */
size_t cachalot_moe_layer_decode_q2_static_max_bytes(void);
int cachalot_moe_layer_decode_q2_static(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                        int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                        int order, const uint8_t* pool,
                                        const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                        int D, int F, int group, float swiglu_limit, const uint16_t* addend,
                                        int32_t* idx_out, float* w_out, float* scores, float* routed, uint16_t* out,
                                        cachalot_stream_t stream);
int cachalot_moe_layer_decode_fp4(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                  int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                  int order, const uint8_t* pool, const cachalot_expert_layout* layout /* host */,
                                  const int32_t* slot_table, int D, int F, float swiglu_limit,
                                  const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                  float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                  cachalot_stream_t stream);
/* cachalot_moe_layer_decode_fp4_shared: cachalot_moe_layer_decode_fp4 with the
 * layer's FP8 shared expert in place of `addend`, as cachalot_moe_layer_decode_q2_shared
 * (same shared arguments, out required, bit for bit the two-call form).  The FP4
 * launches carry the shared tiles for D <= 4096, shared_F <= 3072, 3 <= k <= 6 and
 * k * F <= 17280; other shapes run the shared expert first.  Workspace from
 * cachalot_moe_layer_decode_fp4_shared_workspace_bytes.  Replaces moe_layer_forward
 * over an FP4 bank with shared_* (src/cachalot/model/moe_layer_metal.py:133-405,
 * :381-397; shared_expert_metal.py:44-188). */
size_t cachalot_moe_layer_decode_fp4_shared_workspace_bytes(int D, int F, int k, int shared_F);
int cachalot_moe_layer_decode_fp4_shared(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                         int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                         int order, const uint8_t* pool,
                                         const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                         int D, int F, float swiglu_limit, const uint8_t* shared_w1,
                                         const uint8_t* shared_w1_scales, const uint8_t* shared_w3,
                                         const uint8_t* shared_w3_scales, const uint8_t* shared_w2,
                                         const uint8_t* shared_w2_scales, int shared_F, int32_t* idx_out,
                                         float* w_out, float* scores, float* routed, uint16_t* out, void* workspace,
                                         size_t workspace_bytes, cachalot_stream_t stream);

/* Many tokens (prefill chunk, batched decode), expert-major.
 *
 * cachalot_permute: routes idx/w [T, k] -> rows grouped by expert id
 * (ascending), tokens ascending inside an expert: offsets [E+1] (rows of
 * expert e are offsets[e] .. offsets[e+1]-1), row_token / row_slot / row_w
 * [T*k].  A route whose id lies outside [0, E) is dropped: such routes fill
 * rows offsets[E] .. T*k-1, in route order, with row_w 0, and the grouped
 * entry points write zero y rows for them (the decode entry points likewise
 * give such an id zero rows).  Replaces the host-side assignment build of moe_prefill_grouped
 * (src/cachalot/model/moe_prefill_grouped.py:199-225) and the per-expert
 * x[token_idx] gather lists (:420-437).
 *
 * cachalot_grouped_experts_{q2,fp4}: for every expert with rows, the SwiGLU
 * expert on its rows (x gathered by row_token): g = bf16(x W1), u = bf16(x W3),
 * h = bf16(silu(min(g,L)) * clip(u,-L,L) * row_w), y = bf16(h W2), written to
 * y[row_token, row_slot, :] ([T, k, D] bf16).  Experts whose slot_table entry
 * is negative give zero rows, and so do the dropped routes (rows offsets[E]
 * .. T*k-1, as cachalot_permute lays them out).  Workspace from
 * cachalot_grouped_experts_workspace_bytes (scratch, no state across calls).
 * Replaces affine_expert_forward_batched (expert_affine.py:84-99),
 * routed_expert_forward_sgmm (fp4_sgmm_metal.py:318-333) and
 * routed_expert_forward_batched (moe_prefill_batched.py:31-61) called per
 * expert from moe_prefill_grouped.py:420-467.
 *
 * cachalot_unpermute_combine: routed[t] = 0 + y[t,0] + ... + y[t,k-1] (fp32),
 * out[t] = bf16(routed[t] + addend[t]) (addend NULL: no add).  Replaces the
 * slot-buffer sum of moe_prefill_grouped.py:526-545. */
int cachalot_permute(const int32_t* idx, const float* w, int T, int k, int E, int32_t* offsets,
                     int32_t* row_token, int32_t* row_slot, float* row_w, cachalot_stream_t stream);
size_t cachalot_grouped_experts_workspace_bytes(int T, int k, int E, int D, int F);
int cachalot_grouped_experts_q2(const uint16_t* x, const uint8_t* pool,
                                const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                const int32_t* offsets, const int32_t* row_token, const int32_t* row_slot,
                                const float* row_w, int T, int D, int F, int E, int k, int group,
                                float swiglu_limit, uint16_t* y, void* workspace, size_t workspace_bytes,
                                cachalot_stream_t stream);
/* cachalot_grouped_experts_q2_routes: cachalot_permute(idx, w, ...) followed by
 * cachalot_grouped_experts_q2 (the same routes, rows and y), with offsets / row_*
 * as outputs.  A batched decode of up to 1,024 routes permutes them inside its prep
 * launch, one launch fewer.  Replaces the assignment + per-expert loop of
 * moe_prefill_grouped.py:199-225,420-467 for 2-bit banks. */
int cachalot_grouped_experts_q2_routes(const uint16_t* x, const uint8_t* pool,
                                       const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                       const int32_t* idx, const float* w, int32_t* offsets, int32_t* row_token,
                                       int32_t* row_slot, float* row_w, int T, int D, int F, int E, int k, int group,
                                       float swiglu_limit, uint16_t* y, void* workspace, size_t workspace_bytes,
                                       cachalot_stream_t stream);
int cachalot_grouped_experts_fp4(const uint16_t* x, const uint8_t* pool,
                                 const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                 const int32_t* offsets, const int32_t* row_token, const int32_t* row_slot,
                                 const float* row_w, int T, int D, int F, int E, int k, float swiglu_limit,
                                 uint16_t* y, void* workspace, size_t workspace_bytes, cachalot_stream_t stream);
int cachalot_unpermute_combine(const uint16_t* y, const uint16_t* addend, int T, int k, int D, float* routed,
                               uint16_t* out, cachalot_stream_t stream);

/* FP8 (E4M3FN values, E8M0 power-of-two scales per 32-element block).
 *
 * cachalot_fp8_act_quant: per 32-element block of each row of x [M, K] bf16,
 * amax = max(max|x|, 1e-4), e = ceil(log2(fl32(amax / 448))),
 * q = E4M3(clip(x / 2^e, -448, 448)) rounded to nearest even -> q [M, K] u8,
 * scales [M, K/32] u8 (E8M0, e + 127).  K a multiple of 32.  Replaces
 * quantize_fp8_activation / quantize_activation_fp8
 * (src/cachalot/model/fp8_linear_metal.py:30-53, fp8_ref.py:28-93).
 *
 * cachalot_fp8_linear_quantized: y[t, n] = bf16(sum_kb dot(q[t, kb], w[n, kb])
 * * 2^(q_scales[t, kb]-127) * 2^(w_scales[n/32, kb]-127)), fp32 accumulation;
 * w [N, K] u8 E4M3, w_scales [ceil(N/32), K/32] u8; N a multiple of 16.
 * Replaces fp8_linear_quantized (fp8_linear_metal.py:56-89) and
 * fp8_gemv_reference (fp8_ref.py:96-231).
 *
 * cachalot_shared_expert_fp8: the shared expert for M tokens x [M, D] bf16:
 * q = act_quant(x); g = bf16(w1 q), u = bf16(w3 q); if swiglu_limit > 0,
 * u = clip(u, -L, L), g = min(g, L); h = bf16(silu(g) * u);
 * y = bf16(w2 act_quant(h)) [M, D] bf16.  w1, w3 [F, D] with scales
 * [ceil(F/32), D/32]; w2 [D, F] with scales [ceil(D/32), F/32].  D and F
 * multiples of 32 and of 16.  Workspace from
 * cachalot_shared_expert_fp8_workspace_bytes (scratch only).  The layer
 * combine adds y through the `addend` argument of the decode / combine calls:
 * out = bf16(routed + y), the reference's order (moe_layer_metal.py:381-397,
 * moe_prefill_grouped.py:532-545).  Replaces shared_expert_forward /
 * shared_expert_forward_fused (shared_expert_metal.py:44-188) and
 * shared_expert_forward_batched (moe_prefill_batched.py:104-125). */
int cachalot_fp8_act_quant(const uint16_t* x, int M, int K, uint8_t* q, uint8_t* scales,
                           cachalot_stream_t stream);
int cachalot_fp8_linear_quantized(const uint8_t* q, const uint8_t* q_scales, const uint8_t* w,
                                  const uint8_t* w_scales, int M, int K, int N, uint16_t* y,
                                  cachalot_stream_t stream);
size_t cachalot_shared_expert_fp8_workspace_bytes(int M, int D, int F);
int cachalot_shared_expert_fp8(const uint16_t* x, const uint8_t* w1, const uint8_t* w1_scales,
                               const uint8_t* w3, const uint8_t* w3_scales, const uint8_t* w2,
                               const uint8_t* w2_scales, int M, int D, int F, float swiglu_limit,
                               uint16_t* y, void* workspace, size_t workspace_bytes,
                               cachalot_stream_t stream);

/* Bank loading: n experts' bytes of one tensor ([n, tensor_bytes] contiguous at
 * src, pinned host or device memory) into the slot records first_slot ..
 * first_slot + n - 1 of a pool (record stride record_bytes), at byte `offset`
 * inside each record, as one asynchronous 2-D copy on `stream`.  Replaces the
 * per-expert read_expert_into(entry, slot.views) scatter into slab memory
 * (src/cachalot/storage/reader.py:182-250, cache/slots.py:240-251) for a
 * stacked bank tensor [n_experts, rows, cols] (storage/index.py:120-179). */
int cachalot_copy_records(uint8_t* pool, int64_t record_bytes, int64_t offset, int64_t first_slot,
                          const void* src, int64_t tensor_bytes, int64_t n, cachalot_stream_t stream);

/* Measurement aid (no reference counterpart): a plain streaming read of `bytes`
 * (a multiple of 16) at device address `src` by `blocks` workgroups of 256
 * threads, 16-byte loads; sink [blocks] u32 receives one XOR per workgroup.
 * bench.py times it to measure the HBM read ceiling the expert kernels are
 * judged against. */
int cachalot_stream_read(const void* src, size_t bytes, uint32_t* sink, int blocks, cachalot_stream_t stream);

/* FP4 -> 2-bit affine g128 requantization (the searched fit) of one weight
 * matrix: w_fp4 [N, K/2] packed E2M1 + s_fp4 [N, K/32] E8M0 -> q [N, Kp/16] u32
 * codes (16 per word, low field first), scales / biases [N, Kp/128] bf16 or fp16
 * (scale_dtype, CACHALOT_SCALE_*), Kp = K rounded up to 128.  Per group: the
 * min/max fit, then 24 shrunk ranges (SHRINKS x SHRINKS), the least squared
 * error kept (strictly smaller wins, error summed in index order), scale and
 * bias rounded (RNE) to the storage type, codes
 * recomputed against them; a partial last group fits its real elements and
 * pads with code 0.  Replaces quantize_affine(fit=fit_search) over the FP4
 * checkpoint (benchmarks/quant_affine.py:138-186,303-329,
 * build_affine_bank.py:162-189). */
int cachalot_requant_fp4_to_q2(const uint8_t* w_fp4, const uint8_t* s_fp4, int N, int K, uint32_t* q,
                               uint16_t* scales, uint16_t* biases, int scale_dtype,
                               cachalot_stream_t stream);

/* The bank tool's fits (benchmarks/build_affine_bank.py:74-75, FITS; "mlx",
 * MLX's own quantizer, is not offered). */
#define CACHALOT_FIT_MINMAX 0     /* fit_minmax, quant_affine.py:138-149 */
#define CACHALOT_FIT_SEARCH 1     /* fit_search over SHRINKS (5 x 5), :155-186 */
#define CACHALOT_FIT_SEARCH_LSQ 2 /* fit_search, then 4 least-squares refits, :207-261 */
#define CACHALOT_FIT_WIDE_LSQ 3   /* fit_search over SHRINKS_WIDE (9 x 9), then the refits, :281-287 */

/* FP4 -> affine requantization at every width the bank tool writes: bits 2, 3
 * or 4, groups of 32, 64 or 128, fit CACHALOT_FIT_*, optionally weighted per
 * column by importance [K] fp32 (device; null = unweighted), the activation
 * weighting of quantize_affine(importance=...) (quant_affine.py:126-135,303-329).
 * q [N, Kp*bits/32] u32 (each row one little-endian bit stream), scales /
 * biases [N, Kp/group] bf16 or fp16 (scale_dtype), Kp = K rounded up to the
 * group.  A refit step rounds its pair to the storage type and keeps the
 * previous pair where the normal equations are singular or the new scale is not
 * positive; the best iterate (strictly smaller error) is the fit.  Replaces
 * quantize_affine(w, group, bits, FITS[fit], importance) over the FP4
 * checkpoint (build_affine_bank.py:162-189). */
int cachalot_requant_fp4_to_affine(const uint8_t* w_fp4, const uint8_t* s_fp4, int N, int K, int bits, int group,
                                   int fit, const float* importance, uint32_t* q, uint16_t* scales,
                                   uint16_t* biases, int scale_dtype, cachalot_stream_t stream);

/* Affine banks of the other widths the reference's bank tool writes
 * (benchmarks/build_affine_bank.py:266-267): bits 2, 3 or 4 per code, groups of
 * 32, 64 or 128 (the 2-bit g128 bank has the dedicated entry points above), bf16
 * or fp16 scales and biases (layout->scale_dtype) -- e.g. oQ3e, 3-bit g64 fp16
 * (src/cachalot/model/expert_affine.py:1-10).  Codes: each row one little-endian
 * bit stream, code i at bits [i*bits, (i+1)*bits) (benchmarks/quant_affine.py:
 * 69-105), K padded to whole groups with zero codes.  Same rounding points,
 * outputs and errors as cachalot_moe_decode_q2 / cachalot_moe_layer_decode_q2 /
 * cachalot_grouped_experts_q2, the group formula s*sum(x q) + b*sum(x) in fp32
 * (replacing mx.quantized_matmul at these widths, expert_affine.py:65-99,
 * 117-152).  Workspaces from the *_workspace_bytes functions. */
size_t cachalot_moe_decode_affine_workspace_bytes(int D, int F, int k);
int cachalot_moe_decode_affine(const uint16_t* x, const uint8_t* pool,
                               const cachalot_expert_layout* layout /* host */,
                               const int32_t* slot_table, const int32_t* idx, const float* w,
                               int D, int F, int E, int k, int bits, int group, float swiglu_limit,
                               const uint16_t* addend, float* routed, uint16_t* out,
                               void* workspace, size_t workspace_bytes, cachalot_stream_t stream);
int cachalot_moe_layer_decode_affine(const uint16_t* x, const uint16_t* gate_weight, const float* gate_bias,
                                     int E, int k, int score_fn, float gate_temp, float route_scale, int norm,
                                     int order, const uint8_t* pool,
                                     const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                     int D, int F, int bits, int group, float swiglu_limit,
                                     const uint16_t* addend, int32_t* idx_out, float* w_out, float* scores,
                                     float* routed, uint16_t* out, void* workspace, size_t workspace_bytes,
                                     cachalot_stream_t stream);
size_t cachalot_grouped_experts_affine_workspace_bytes(int T, int k, int E, int D, int F);
int cachalot_grouped_experts_affine(const uint16_t* x, const uint8_t* pool,
                                    const cachalot_expert_layout* layout /* host */, const int32_t* slot_table,
                                    const int32_t* offsets, const int32_t* row_token, const int32_t* row_slot,
                                    const float* row_w, int T, int D, int F, int E, int k, int bits, int group,
                                    float swiglu_limit, uint16_t* y, void* workspace, size_t workspace_bytes,
                                    cachalot_stream_t stream);
/* Dense dequantisation of one affine matrix of any bank width: w [N, row_words]
 * u32, scales / biases [N, groups] (scale_dtype) -> out [N, K] fp32, fl(fl(s*q)+b)
 * (replaces mx.dequantize on the affine views, expert_affine.py:26-51). */
int cachalot_dequant_affine(const uint32_t* w, const uint16_t* scales, const uint16_t* biases, int N, int K,
                            int row_words, int groups, int group, int bits, int scale_dtype, float* out,
                            cachalot_stream_t stream);

/* Dense dequantisation (bit-exact weight checks and debugging).
 * FP4: packed [N, K/2] u8, scales [N, K/32] u8 -> out [N, K] fp32
 *   (replaces dequantize_fp4_weight / dequantize_fp4_dense,
 *    src/cachalot/model/fp4.py:67-109, fp4_dequant_metal.py:43-69);
 *   as_bf16 != 0 converts through the bf16 path the GEMV/GEMM kernels use.
 * 2-bit: w [N, row_words] u32, scales/biases [N, groups] bf16 or fp16
 *   (scale_dtype, CACHALOT_SCALE_*) -> out [N, K] fp32, value fl(fl(s*q)+b)
 *   (replaces mx.dequantize on the affine views,
 *   src/cachalot/model/expert_affine.py:26-51). */
int cachalot_dequant_fp4(const uint8_t* packed, const uint8_t* scales, int N, int K, int as_bf16,
                         float* out, cachalot_stream_t stream);
int cachalot_dequant_q2(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        int N, int K, int row_words, int groups, int group, int scale_dtype,
                        float* out, cachalot_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* CACHALOT_AMD_H */
