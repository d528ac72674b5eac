/*
 * mi355x_attn.h - C ABI of the gfx950 attention hot path (libmi355x_attn.so).
 *
 * Drop-in boundary for the reference server's native attention, KV-store and
 * norm bridges (MabinogiX/llm_infer_rust). Every function takes raw device
 * pointers, element strides, a dtype code (0 = bfloat16, 1 = float16) and a
 * hipStream_t passed as void*. No ATen/torch types cross this boundary.
 *
 * Error convention (same as the reference's raw sglang_native_* launchers):
 * functions returning `const char*` return NULL on success and otherwise a
 * message that stays valid until the next failing call on the same thread.
 * Plan-returning functions return NULL on failure; mi355x_attn_error() then
 * holds the message (the reference's thread-local last_error,
 * src/models/attention/flashinfer_bridge.cpp:13,59).
 *
 * Threading: a plan is owned by one host thread (the reference's plans are
 * Rc, not Send). All work is enqueued on the given stream; nothing blocks
 * except where stated.
 */
#ifndef MI355X_ATTN_H
#define MI355X_ATTN_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#pragma GCC visibility push(default)

/* Last error of a plan-returning call on this thread.
 * Replaces sglang_flashinfer_error / sglang_layers_error / sglang_store_kv_error
 * (flashinfer_bridge.cpp:59, fused_ops_bridge.cpp:56, kv_store_bridge.cpp:11). */
const char* mi355x_attn_error(void);

/* ABI revision of this header (currently 1). No reference counterpart. */
int mi355x_attn_abi_version(void);

/* ------------------------------------------------------------------------
 * K/V store. kc[loc[t]] = k[t], vc[loc[t]] = v[t] bitwise for 16-bit
 * elements. k/v are [tokens, heads, width] with strides (kt, kh, 1); caches
 * are contiguous [capacity, heads, width]. loc is int32 or int64 (index64).
 * A slot equal to `reserved` is skipped. A slot outside [0, capacity) is not
 * written; if `error_count` (device int32) is non-NULL it is incremented once
 * per such token, so the caller can raise the error the reference raises.
 * Replaces sglang_native_store_kv (src/models/attention/kv_store.cu:65-68).
 * ------------------------------------------------------------------------ */
const char* mi355x_store_kv(const void* k, const void* v, void* kc, void* vc, const void* loc,
                            int64_t tokens, int64_t heads, int64_t width, int64_t capacity,
                            int64_t kt, int64_t kh, int64_t vt, int64_t vh, int64_t reserved,
                            bool index64, int32_t* error_count, void* stream);

/* ------------------------------------------------------------------------
 * Norms (fp32 accumulation, output rounded to the activation dtype).
 * ------------------------------------------------------------------------ */

/* out[(t*heads+h), :] = x[t,h,:] * rsqrt(mean(x^2) + eps) * weight; out contiguous.
 * Replaces sglang_layers_native_norm (src/layers/fused_ops.cu:210-213). */
const char* mi355x_rms_norm(const void* x, const void* weight, void* out, int64_t tokens,
                            int64_t heads, int64_t width, int64_t token_stride,
                            int64_t head_stride, double eps, int dtype, void* stream);

/* In place: s = x + residual (fp32); residual <- round(s); x <- round(rms(s) * w).
 * x and residual must not alias.
 * Replaces sglang_layers_native_add_norm (src/layers/fused_ops.cu:300-303). */
const char* mi355x_add_rms_norm(void* x, void* residual, const void* weight, int64_t tokens,
                                int64_t width, int64_t x_stride, int64_t residual_stride,
                                double eps, int dtype, void* stream);

/* In place per-head RMSNorm of q [tokens, q_heads, width] with q_weight and of
 * k [tokens, k_heads, width] with k_weight. Nothing else is written.
 * Replaces sglang_layers_native_qk_norm (src/layers/fused_ops.cu:254-259). */
const char* mi355x_qk_norm(void* q, void* k, const void* q_weight, const void* k_weight,
                           int64_t tokens, int64_t q_heads, int64_t k_heads, int64_t width,
                           int64_t q_token_stride, int64_t q_head_stride,
                           int64_t k_token_stride, int64_t k_head_stride, double eps, int dtype,
                           void* stream);

/* ------------------------------------------------------------------------
 * Paged decode attention (head_dim 128, q heads per kv head in {1,2,4,8}).
 * ------------------------------------------------------------------------ */

/* Build or refresh a decode plan once per forward; every layer reuses it.
 * block_table: device int32 [batch, columns] with row stride table_stride;
 * seq_lens: device int32 [batch]. host_lengths (nullable, host_rows entries)
 * is the scheduler's host copy of seq_lens; without it the lengths are read
 * back once (blocking). The plan packs the reference page metadata
 * (indptr / indices / last_page_len) and a split-KV work list sized for the
 * device's CU count. `existing` must have the same geometry; with graph=true
 * the rows/columns are fixed and workspaces never move.
 * Replaces sglang_flashinfer_prepare (flashinfer_bridge.cpp:61-65). */
void* mi355x_decode_prepare(void* existing, const int32_t* block_table, int64_t batch,
                            int64_t columns, int64_t table_stride, const int32_t* seq_lens,
                            int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                            int64_t page_size, int64_t dtype, bool graph,
                            const int32_t* host_lengths, int64_t host_rows, void* stream);

/* out[b, h, :] = softmax(q[b,h] K^T / sqrt(128)) V over the request's pages.
 * q/out: [batch, num_q_heads, 128] with the given strides (16-byte aligned
 * rows); caches: contiguous [pages, page_size, num_kv_heads, 128].
 * Replaces sglang_flashinfer_decode (flashinfer_bridge.cpp:201-203) and
 * sglang_flashinfer_native_run (flashinfer_plan_run.cu:222-227). */
const char* mi355x_decode_run(const void* plan, const void* q, int64_t q_stride_n,
                              int64_t q_stride_h, const void* k_cache, const void* v_cache,
                              void* out, int64_t out_stride_n, int64_t out_stride_h,
                              int64_t batch, int64_t num_q_heads, int64_t num_kv_heads,
                              int64_t page_size, int64_t dtype, void* stream);

/* Frees a plan after waiting for its pending uploads.
 * Replaces sglang_flashinfer_plan_drop (flashinfer_bridge.cpp:192-199). */
void mi355x_decode_plan_drop(void* plan);

/* Number of workspace (re)allocations made by the plan so far.
 * Replaces sglang_flashinfer_workspace_allocations (flashinfer_bridge.cpp:187-190). */
uint64_t mi355x_decode_workspace_allocations(const void* plan);

/* Plan facts: out6 = {batch, total_pages, num_items, chunk_tokens,
 * items_capacity, cus}. Introspection; no reference counterpart. */
const char* mi355x_decode_plan_info(const void* plan, int64_t* out6);

/* Blocking copy of the plan's page metadata and work list to host memory
 * (indptr batch+1, indices total_pages, last_len batch, work 4*num_items,
 * merge 2*batch ints; any pointer may be NULL). Introspection for parity
 * tests; no reference counterpart. */
const char* mi355x_decode_plan_read(const void* plan, int32_t* indptr, int32_t* indices,
                                    int32_t* last_len, int32_t* work, int32_t* merge,
                                    void* stream);

/* Host-only split-KV scheduler used by mi355x_decode_prepare (page size 1 view):
 * every workgroup of the grid takes an equal share of the batch's kernel tiles plus
 * a fixed cost per work item, cut on tile boundaries (`chunk_tokens` receives the
 * share's tiles in tokens); each request a share touches becomes one work item.
 * Fills `work` (4 ints per item: request, token_begin, token_end, partial slot
 * or -1) and `merge` (2 ints per request: first partial slot or -1, item count).
 * Returns the item count, or -1 on invalid input / insufficient capacity.
 * Stands in for FlashInfer's DecodePlan work estimation
 * (flashinfer_plan_run.cu:74-112). */
int64_t mi355x_decode_schedule(const int32_t* lengths, int64_t batch, int64_t cus,
                               int64_t num_kv_heads, int32_t* work, int64_t work_capacity,
                               int32_t* merge, int64_t* chunk_tokens);

/* Work-list capacity mi355x_decode_schedule needs for `rows` requests. */
int64_t mi355x_decode_items_capacity(int64_t rows, int64_t cus, int64_t num_kv_heads);

/* ------------------------------------------------------------------------
 * Causal prefill attention (head_dim 128, q heads per kv head in {1,2,4,8}).
 * ------------------------------------------------------------------------ */

/* Build or refresh a prefill plan once per forward. q_indptr: device int32
 * [batch+1] (cu_seqlens_q); block_table: device int32 [batch, columns] with
 * row stride table_stride (may be NULL when every prefix is 0); q_host /
 * prefix_host: the scheduler's host snapshots of cu_seqlens_q and
 * prefix_lens. The plan is paged iff some prefix > 0 and then packs the
 * reference page metadata over kv length = prefix + extend.
 * Replaces sglang_flashinfer_prepare_prefill (flashinfer_bridge.cpp:250-253)
 * and PrefillPlan (flashinfer_plan_run.cu:243-274). */
void* mi355x_prefill_prepare(void* existing, const int32_t* q_indptr, const int32_t* block_table,
                             int64_t batch, int64_t columns, int64_t table_stride,
                             const int32_t* q_host, const int32_t* prefix_host,
                             int64_t num_q_heads, int64_t num_kv_heads, int64_t page_size,
                             int64_t dtype, void* stream);

/* out[t, h, :] = causal softmax attention of query row t. q: [total_q,
 * num_q_heads, 128] with strides (q_sn, q_sh, 1). Ragged plans read k/v as
 * [total_q, num_kv_heads, 128] with strides (k_sn, k_sh, 1) (packed QKV views
 * are fine); paged plans read k/v as the contiguous caches [pages,
 * page_size, num_kv_heads, 128] (pass k_sn = num_kv_heads*128, k_sh = 128).
 * Rows must be 16-byte aligned. out may be caller-owned static storage.
 * Replaces sglang_flashinfer_prefill (flashinfer_bridge.cpp:312-314) and
 * sglang_flashinfer_native_prefill_run (flashinfer_plan_run.cu:331-335). */
const char* mi355x_prefill_run(const void* plan, const void* q, int64_t q_sn, int64_t q_sh,
                               const void* k, int64_t k_sn, int64_t k_sh, const void* v,
                               int64_t v_sn, int64_t v_sh, void* out, int64_t o_sn, int64_t o_sh,
                               int64_t total_q, int64_t num_q_heads, int64_t num_kv_heads,
                               int64_t page_size, int64_t dtype, void* stream);

/* Frees a prefill plan after its pending uploads.
 * Replaces sglang_flashinfer_plan_drop for prefill plans (flashinfer_bridge.cpp:192-199). */
void mi355x_prefill_plan_drop(void* plan);

/* Workspace (re)allocations made by a prefill plan so far. */
uint64_t mi355x_prefill_workspace_allocations(const void* plan);

/* Plan facts: out6 = {batch, total_q, paged, num_items, total_pages, split_items}:
 * num_items counts launched work items (chunks included), split_items the items cut
 * along their keys and merged by a second launch. Introspection; no reference counterpart. */
const char* mi355x_prefill_plan_info(const void* plan, int64_t* out6);

/* Blocking copy of kv_indptr (batch+1) and, for paged plans, indices
 * (total_pages) and last_page_len (batch). Introspection for parity tests. */
const char* mi355x_prefill_plan_read(const void* plan, int32_t* kv_indptr, int32_t* indices,
                                     int32_t* last_len, void* stream);

/* Host-only prefill work list: 4 ints per item {request, q_begin, kv_head,
 * head_group}, longest causal horizon first. work may be NULL to count.
 * Returns the item count or -1. Stands in for FlashInfer's PrefillPlan
 * tiling (flashinfer_plan_run.cu:243-274). mi355x_prefill_prepare further cuts
 * items along their keys when the batch is too small to fill the device (when the
 * longest item exceeds twice the mean per-CU share of 64-key tiles). */
int64_t mi355x_prefill_schedule(const int32_t* q_host, const int32_t* prefix_host, int64_t batch,
                                int64_t num_q_heads, int64_t num_kv_heads, int32_t* work,
                                int64_t capacity);

/* ------------------------------------------------------------------------
 * Decoder-layer elementwise ops (dtype 0 = bf16, 1 = fp16).
 * ------------------------------------------------------------------------ */

/* Half-split rotary embedding of every q and k head, in place:
 *   x[i] <- x[i] cos - x[i+W/2] sin,  x[i+W/2] <- x[i+W/2] cos + x[i] sin,
 * cos/sin fp32 [max_positions, W/2], positions int64 [tokens]; a position
 * outside [0, max_positions) leaves its token untouched.
 * Replaces sglang_layers_native_rope (src/layers/fused_ops.cu:340-346). */
const char* mi355x_rope(void* q, void* k, const int64_t* positions, const float* cos,
                        const float* sin, int64_t tokens, int64_t q_heads, int64_t k_heads,
                        int64_t width, int64_t q_token_stride, int64_t q_head_stride,
                        int64_t k_token_stride, int64_t k_head_stride, int64_t max_positions,
                        int dtype, void* stream);

/* One pass of the decoder layer's qk_norm -> rope -> K/V store
 * (src/models/qwen3/model.rs:478-514; base.rs:62-152), width 128 only.
 * Each stage is optional: q_weight/k_weight NULL skips the norm, positions
 * NULL skips the rotation, k_cache NULL skips the store. q and k are updated
 * in place; the stored K row is the rotated one and V is copied unchanged.
 * Results equal mi355x_qk_norm, mi355x_rope and mi355x_store_kv run in turn
 * (the normalised value is rounded before it is rotated). Store semantics
 * (reserved slot, out-of-range slot, error_count) are those of
 * mi355x_store_kv with heads = k_heads. No single reference counterpart: it
 * fuses sglang_layers_native_qk_norm, _rope and sglang_native_store_kv. */
const char* mi355x_qk_norm_rope_store(
    void* q, void* k, const void* v, const void* q_weight, const void* k_weight,
    const int64_t* positions, const float* cos, const float* sin, int64_t max_positions,
    void* k_cache, void* v_cache, const void* loc, bool index64, int64_t capacity,
    int64_t reserved, int32_t* error_count, int64_t tokens, int64_t q_heads, int64_t k_heads,
    int64_t width, int64_t q_token_stride, int64_t q_head_stride, int64_t k_token_stride,
    int64_t k_head_stride, int64_t v_token_stride, int64_t v_head_stride, double eps, int dtype,
    void* stream);

/* out[t, c] = silu(gate_up[t, c]) * gate_up[t, W + c]; gate_up [tokens, 2W]
 * and out [tokens, W] contiguous.
 * Replaces sglang_layers_native_silu_mul (src/layers/fused_ops.cu:364-366). */
const char* mi355x_silu_mul(const void* gate_up, void* out, int64_t tokens, int64_t width,
                            int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Decode-batch projections.
 * ------------------------------------------------------------------------ */

/* out[M, N] = x[M, K] . w[N, K]^T (row strides ldx, ldw, ldo in elements),
 * fp32 accumulation, one rounding. Meant for decode batches (M up to a few
 * hundred rows); K % 64 == 0, N % 4 == 0, 16-byte aligned rows. When the
 * chosen tiling splits K, the fp32 partials go to `workspace`
 * (mi355x_linear_workspace_bytes tells how much). config / splits < 0 pick
 * the tiling for `cus` compute units; otherwise they force one (tuning).
 * Replaces the decode-time x.matmul(w.T) of src/layers/linear.rs:5-7. */
const char* mi355x_linear(const void* x, int64_t ldx, const void* w, int64_t ldw, void* out,
                          int64_t ldo, int64_t M, int64_t N, int64_t K, void* workspace,
                          int64_t workspace_bytes, int32_t cus, int32_t config, int32_t splits,
                          int64_t dtype, void* stream);

/* The projection fused with the residual RMSNorm that follows it in a decoder
 * layer (o_proj -> post-attention norm, down -> next layer's input norm):
 *   y = x . w^T (rounded once), residual <- round(y + residual),
 *   out <- round(rms(y + residual) * norm_weight)   (norm on the fp32 sum).
 * Equal bit for bit to mi355x_linear followed by mi355x_add_rms_norm; the
 * split-K partials are reduced inside the norm pass instead of a separate
 * launch. Width N: a multiple of 8 in 1032..8192 (rows of 16-byte chunks);
 * library-chosen tiling, workspace as for mi355x_linear (config = splits = -1).
 * ldr >= N; out and residual must not alias (the norm pass reads and writes both).
 * Replaces linear.rs:5-7 followed by ops.rs:22-35 (fused_ops.cu:300-338). */
const char* mi355x_linear_add_rms_norm(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                       void* residual, int64_t ldr, const void* norm_weight,
                                       double eps, void* out, int64_t ldo, int64_t M, int64_t N,
                                       int64_t K, void* workspace, int64_t workspace_bytes,
                                       int32_t cus, int64_t dtype, void* stream);

/* The QKV projection fused with the qk_norm -> rope -> K/V store pass that reads it
 * (decode batches): qkv[M, (Hq + 2 Hkv) * 128] = x . w^T, then mi355x_qk_norm_rope_store
 * on its q, k and v head views (token stride ldo, head stride 128) with every stage on
 * (norm weights, positions and a cache are required). When the product is split along K
 * the pass sums the fp32 partials itself (split order, rounded once) instead of a separate
 * reduce launch, and writes the v rows into qkv too, so qkv and the cache equal
 * mi355x_linear (library tiling) followed by mi355x_qk_norm_rope_store bit for bit.
 * Workspace as for mi355x_linear with config = splits = -1 (N = (Hq + 2 Hkv) * 128).
 * Replaces linear.rs:5-7 followed by model.rs:478-514 (fused_ops.cu, base.rs:62-152). */
const char* mi355x_linear_qk_norm_rope_store(
    const void* x, int64_t ldx, const void* w, int64_t ldw, void* qkv, int64_t ldo, int64_t M,
    int64_t K, int64_t q_heads, int64_t k_heads, void* workspace, int64_t workspace_bytes,
    int32_t cus, const void* q_weight, const void* k_weight, const int64_t* positions,
    const float* cos, const float* sin, int64_t max_positions, void* k_cache, void* v_cache,
    const void* loc, bool index64, int64_t capacity, int64_t reserved, int32_t* error_count,
    double eps, int dtype, void* stream);

/* A gate_up projection fused with SiLU x mul (the MLP's first two steps):
 *   y = x . w^T with w = [gate rows (width); up rows (width)] of [2 width, K],
 *   out[m, j] = round(silu(g) * u), g = round(y[m, j]), u = round(y[m, width + j]),
 * computed without writing y: equal bit for bit to mi355x_linear (unsplit, the
 * same tiling) followed by mi355x_silu_mul. K is never split, so no workspace.
 * config < 0 lets the library choose the tile shape by M (0, 6 and 7 are fused);
 * cus is accepted for the same call shape as mi355x_linear.
 * M <= 4096, K % 64 == 0, width % 4 == 0, 16-byte aligned x / w rows.
 * Replaces linear.rs:5-7 (gate_up, mlp.rs) followed by ops.rs:53-61
 * (fused_ops.cu:135-171). */
const char* mi355x_linear_silu_mul(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                   void* out, int64_t ldo, int64_t M, int64_t width, int64_t K,
                                   int32_t cus, int32_t config, int64_t dtype, void* stream);

/* Workspace bytes mi355x_linear needs for this shape and tiling (0 when K is
 * not split, -1 for an invalid shape). Host-only. */
int64_t mi355x_linear_workspace_bytes(int64_t M, int64_t N, int64_t K, int32_t cus,
                                      int32_t config, int32_t splits);

/* mi355x_linear without a workspace argument and without any allocation: the
 * split-K partials go to a 32 MiB device array held by the library on each GPU
 * it runs on (until the process ends). No counterpart in the reference: it is
 * for callers that cannot allocate (code under hipGraph capture without a
 * memory pool, serving loops that forbid hipMalloc). Same arguments, tiling and
 * results as mi355x_linear; fails with an error when the chosen tiling needs
 * more than 32 MiB of partials (mi355x_linear_workspace_bytes tells). All calls
 * on one GPU share that array, so calls that overlap on one GPU (different
 * streams, or host threads) race; calls ordered on one stream are safe. */
const char* mi355x_linear_noalloc(const void* x, int64_t ldx, const void* w, int64_t ldw,
                                  void* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                                  int32_t cus, int32_t config, int32_t splits, int64_t dtype,
                                  void* stream);

/* ------------------------------------------------------------------------
 * Sampling.
 * ------------------------------------------------------------------------ */

/* One token id per logits row (dtype 0 = bf16, 1 = fp16, 2 = fp32; row
 * stride in elements). temperature/top_k/top_p are per-row device arrays,
 * normalised as SamplingParams::normalized: temperature <= 0 or top_p == 0
 * gives the argmax; otherwise joint top-k/top-p filtering on the original
 * softmax(logits / temperature) and one draw from the survivors. An invalid
 * distribution (NaN, or no finite logit) gives -1. The draw is a function of
 * (seed, offset, row, logits) only: equal arguments give equal tokens.
 * Replaces sglang_sampling_native (src/engine/sampling_flashinfer.cu:4-6)
 * plus the temperature/softmax/argmax steps of Sampler::sample
 * (src/engine/sampling.rs:239-269), for a whole heterogeneous batch at once. */
const char* mi355x_sample(const void* logits, int64_t rows, int64_t vocab, int64_t row_stride,
                          int dtype, const float* temperature, const int32_t* top_k,
                          const float* top_p, uint64_t seed, uint64_t offset, int64_t* out,
                          void* stream);

#pragma GCC visibility pop

#ifdef __cplusplus
}
#endif

#endif /* MI355X_ATTN_H */
