/*
 * C ABI of the MI355X (gfx950) AB-Attention library, libab_attention_hip.so.
 *
 * Drop-in boundary for the reference's native ops and its FlashInfer prefill
 * (paths relative to the reference checkout):
 *   _C.ibcs(q, k) -> scores          csrc/bindings.cpp:4-5, csrc/ops.h:5, csrc/ibcs.cu:549-617
 *   _C.sip(scores, offsets, ids, logs)  csrc/bindings.cpp:6-7, csrc/ops.h:7-8, csrc/sip.cu:170-199
 *   FlashInfer paged prefill run     ab_attention/flashinfer_backend.py:164-242
 *
 * Conventions:
 *   - tensors are plain device pointers, row-major and contiguous, with int64
 *     sizes; bf16 and fp16 data are passed as raw 16-bit storage;
 *   - `stream` is a hipStream_t (NULL is the null stream); work is enqueued on
 *     it, nothing synchronises and nothing allocates: the caller owns every
 *     buffer, including IBCS workspace sized by ab_ibcs_workspace_bytes();
 *   - every function returns AB_OK (0) or a nonzero status and then
 *     ab_last_error() describes the failure (thread local). Validation
 *     happens before any launch.
 * Geometry is fixed as in the reference: head dim 128, query blocks of 128
 * tokens (rows = batch_heads * ceil(tokens / 128)), KV4 blocks of 4 keys
 * (kv_blocks = tokens / 4), 8 centroids per query block.
 */
#ifndef AB_ATTENTION_H
#define AB_ATTENTION_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define AB_ABI_VERSION 4

enum ab_status {
    AB_OK = 0,
    AB_ERR_INVALID = 1, /* bad shape, pointer, alignment or size */
    AB_ERR_LAUNCH = 3   /* the HIP runtime rejected a launch */
};

/* Message for the last failure on this thread (empty if none). */
const char *ab_last_error(void);
int ab_abi_version(void);

/* ---- IBCS: population-weighted KV4 block masses ---------------------------
 * Replaces _C.ibcs (csrc/ibcs.cu:549-617): q, k bf16 [batch_heads, tokens, 128]
 * -> scores f32 [rows, kv_blocks], each row summing to 1. `workspace` holds
 * every intermediate (256-byte aligned, ab_ibcs_workspace_bytes() bytes). */
size_t ab_ibcs_workspace_bytes(int64_t batch_heads, int64_t tokens);
int ab_ibcs(const void *q, const void *k, int64_t batch_heads, int64_t tokens, void *workspace,
            size_t workspace_bytes, float *scores, void *stream);

/* IBCS stages, for callers that keep the intermediates.
 * cluster_pool (csrc/ibcs.cu:106-266): centroids bf16 [rows, 8, 128], already
 *   multiplied by 128^-0.5 * log2(e) and rounded to bf16 (csrc/ibcs.cu:293-295);
 *   populations f32 [rows, 8]; pooled_keys bf16 [batch_heads, kv_blocks, 2, 128].
 * lse (csrc/ibcs.cu:370-489): block_lse fp16 [rows, 8, ld] with
 *   ld = ab_ibcs_lse_stride(tokens) >= kv_blocks; lse_max, lse_den f32 [rows, 8].
 * masses (csrc/ibcs.cu:495-538): scores f32 [rows, kv_blocks]. */
int64_t ab_ibcs_lse_stride(int64_t tokens);
int ab_ibcs_cluster_pool(const void *q, const void *k, int64_t batch_heads, int64_t tokens, void *centroids,
                         float *populations, void *pooled_keys, void *stream);
int ab_ibcs_lse(const void *centroids, const void *pooled_keys, int64_t batch_heads, int64_t tokens,
                void *block_lse, float *lse_max, float *lse_den, void *stream);
int ab_ibcs_masses(const void *block_lse, const float *populations, const float *lse_max, const float *lse_den,
                   int64_t rows, int64_t kv_blocks, float *scores, void *stream);

/* ---- SIP: systematic inclusion-probability sampling ----------------------
 * Replaces _C.sip (csrc/sip.cu:170-199): scores f32 [rows, population],
 * offsets f32 [rows] (uniforms in [0,1)) -> ids int32 [rows, samples] (per-head
 * KV4 ids: certain blocks first, ascending) and log_weights f32 [rows, samples]
 * = log2(1/pi). Requires 0 < samples < population. Bit-exact with the
 * reference algorithm given the same scores and offsets. */
int ab_sip(const float *scores, const float *offsets, int64_t rows, int64_t population, int64_t samples,
           int32_t *ids, float *log_weights, void *stream);

/* ---- Fused plan: IBCS + SIP without materialised scores -------------------
 * build_plan's per-chunk work (ab_attention/attention.py:65-75: _C.ibcs then
 * _C.sip) in one call: q, k bf16 [batch_heads, tokens, 128] (tokens read
 * through `order` when it is not NULL, as ab_ibcs_ordered), offsets f32
 * [rows] -> ids int32 / log_weights f32 [rows, samples], the same bits as
 * ab_ibcs followed by ab_sip. Every row is scored and sampled by one kernel
 * that computes its masses straight into LDS (rows over ~26,000 blocks keep
 * two fp64 prefixes per chunk instead of all bucket prefixes); the scores are
 * never written. `workspace` is ab_ibcs_sip_workspace_bytes() bytes, 256-byte
 * aligned. */
size_t ab_ibcs_sip_workspace_bytes(int64_t batch_heads, int64_t tokens);
int ab_ibcs_sip(const void *q, const void *k, const int32_t *order, int64_t batch_heads, int64_t tokens,
                const float *offsets, int64_t samples, void *workspace, size_t workspace_bytes, int32_t *ids,
                float *log_weights, void *stream);

/* Testing variant of ab_ibcs_sip; no counterpart in the reference. Every
 * row that is sampled with kept prefixes takes the reference's binary-search
 * probes (each prefix rebuilt from the kept ones), the path otherwise taken
 * only when a threshold lands in a rounding drop of the prefix array, which
 * no test input can be built to hit. The ids and weights are the same bits
 * as ab_ibcs_sip's; the tests compare the two. */
int ab_ibcs_sip_exact_draws(const void *q, const void *k, const int32_t *order, int64_t batch_heads,
                            int64_t tokens, const float *offsets, int64_t samples, void *workspace,
                            size_t workspace_bytes, int32_t *ids, float *log_weights, void *stream);

/* ---- Weighted paged prefill ------------------------------------------------
 * Replaces the FlashInfer FA3 run with the ABSipAttention variant
 * (ab_attention/flashinfer_backend.py:30-59, :164-242): q, k, v bf16
 * [batch_heads, tokens, 128]; ids/log_weights [rows, samples] (a SamplePlan's
 * descriptor and log_weights, samples = 32 * sample_pages) -> out bf16
 * [batch_heads, tokens, 128] and, if lse != NULL, the base-2 log-sum-exp
 * f32 [batch_heads, tokens]. No page-table translation is needed: ids are
 * used as per-head KV4 ids directly. */
int ab_paged_prefill(const void *q, const void *k, const void *v, int64_t batch_heads, int64_t tokens,
                     const int32_t *ids, const float *log_weights, int64_t samples, void *out, float *lse,
                     void *stream);

/* The same prefill with a K/V length of its own (kv_tokens, divisible by 4)
 * and any positive multiple of 8 for samples (a listed block may carry a
 * -inf weight, which removes it; a query whose every listed block is at -inf
 * gets o = 0 and lse = -inf). With a plan's ids plus the text blocks at
 * weight 0 it computes _hunyuan_attention's video state and its merge with
 * the exact text state in one pass (ab_attention/video.py:129-142). */
int ab_paged_prefill_kv(const void *q, const void *k, const void *v, int64_t batch_heads, int64_t q_tokens,
                        int64_t kv_tokens, const int32_t *ids, const float *log_weights, int64_t samples,
                        void *out, float *lse, void *stream);

/* Dense attention of q [batch_heads, q_tokens, 128] over every key of k, v
 * [batch_heads, kv_tokens, 128] (kv_tokens divisible by 4), with the base-2
 * lse if lse != NULL: the attention ab_paged_prefill_kv computes with every
 * KV4 block listed at weight 0 (within bf16 rounding of it: a kernel of its
 * own, on 16x16x32 MFMA tiles), without a page list in memory (the kernel
 * walks the blocks in order). Replaces the FA3 single prefill of _exact
 * (ab_attention/video.py:13-28), which runs steps 1-10 and layer 0 of a
 * video (README.md:132-133). */
int ab_dense_prefill(const void *q, const void *k, const void *v, int64_t batch_heads, int64_t q_tokens,
                     int64_t kv_tokens, void *out, float *lse, void *stream);

/* How the prefill entry points split a call's rows into launches; no
 * counterpart in the reference (FlashInfer runs one kernel). The rows of
 * head h, query block b are dealt to 8 groups (one per XCD) of
 * ceil(q_blocks / 8) consecutive blocks: group b / ceil(q_blocks / 8), row
 * slot h * ceil(q_blocks / 8) + b % ceil(q_blocks / 8) within the group.
 * Launch i covers the row slots [i * S, (i + 1) * S) of every group, where
 * S = ab_prefill_launch_slots(batch_heads, q_tokens) (a multiple of 64;
 * 0 for a non-positive size). Callers need this only to account for
 * per-launch timings. */
int64_t ab_prefill_launch_slots(int64_t batch_heads, int64_t q_tokens);

/* ---- Attention-state merge -------------------------------------------------
 * Replaces FlashInfer's merge_state as used by _merge
 * (ab_attention/video.py:31-40): two states over disjoint key sets, o bf16
 * [count, 128] with base-2 lse f32 [count] -> merged o bf16 [count, 128] and,
 * if lse_out != NULL, the merged lse. */
int ab_merge_states(const void *o_a, const float *lse_a, const void *o_b, const float *lse_b, int64_t count,
                    void *out, float *lse_out, void *stream);

/* ---- Permuted token layouts (cube layout) ----------------------------------
 * The reference's use_cube_layout (ab_attention/video.py:90-126) gathers the
 * hidden states into 4x4x4-cube order before the first block and scatters
 * them back after the last, so attention sees tensors in cube order. These
 * entry points compute the same attention on tensors kept in their stored
 * order: order int32 [tokens] gives, for cube position t, the stored token
 * order[t] (a permutation; the same for every head).
 * ab_ibcs_ordered: ab_ibcs of the permuted q, k (scores over cube-order KV4
 *   blocks), reading tokens through `order`.
 * ab_remap_ids: out[i] = map[ids[i]] (ids clamped into [0, map_len)); with
 *   map[j] = order[4j] / 4 it turns cube-order KV4 ids into stored-order ones,
 *   which is valid when every cube-order KV4 block is 4 consecutive stored
 *   tokens starting at a multiple of 4 (true for the cube layout when the
 *   latent width is a multiple of 4).
 * ab_paged_prefill_ordered: ab_paged_prefill of the permuted q with stored
 *   k, v, ids already remapped to stored-order KV4 pages; query t is read from
 *   and written to stored row order[t] (out and lse in stored order). */
int ab_ibcs_ordered(const void *q, const void *k, const int32_t *order, int64_t batch_heads, int64_t tokens,
                    void *workspace, size_t workspace_bytes, float *scores, void *stream);
int ab_remap_ids(const int32_t *ids, int64_t count, const int32_t *map, int64_t map_len, int32_t *out,
                 void *stream);
int ab_paged_prefill_ordered(const void *q, const void *k, const void *v, const int32_t *order,
                             int64_t batch_heads, int64_t tokens, const int32_t *ids, const float *log_weights,
                             int64_t samples, void *out, float *lse, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* AB_ATTENTION_H */
