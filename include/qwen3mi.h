/*
 * qwen3mi.h - C ABI of the MI355X (gfx950) kernels for the Qwen3 GRPO
 * rollout-and-loss path.
 *
 * Every entry point:
 *   - takes plain device pointers, element strides and sizes (no torch types);
 *   - launches asynchronously on `stream` (a hipStream_t passed as void*;
 *     NULL means the legacy default stream) and never synchronises, reads
 *     device data on the host or allocates, so it can be captured into a
 *     HIP graph;
 *   - returns QMI_OK (0), a negative QMI_E* code when an argument is
 *     rejected before launch (nothing is launched then), or a positive
 *     hipError_t value when the launch itself failed.
 *
 * bf16 tensors are passed as raw 16-bit words.  Integer index tensors are
 * int32 unless a parameter says int64.
 */
#ifndef QWEN3MI_H
#define QWEN3MI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMI_OK 0
#define QMI_E_NULL_POINTER (-1)
#define QMI_E_BAD_SHAPE (-2)
#define QMI_E_BAD_STRIDE (-3)
#define QMI_E_UNSUPPORTED (-4)
#define QMI_E_WORKSPACE_TOO_SMALL (-5)
#define QMI_E_SCRATCH_LIMIT (-6)

/* Human-readable text for a return code of any entry point. */
const char* qmi_error_string(int code);

/* Library version: major * 10000 + minor * 100 + patch. */
int qmi_version(void);

/*
 * Slot-mapped KV store.
 * Replaces `store_kvcache` / `_store_kvcache_kernel`
 * (qwen3_naive.py:20-41), called from Qwen3Attention.forward_prefill
 * (qwen3_naive.py:626) and forward_decode (qwen3_naive.py:668).
 *
 * For every token i < n_tokens with s = slot_mapping[i]:
 *   k_cache[s*row_elems : (s+1)*row_elems] = key[i*key_row_stride : +row_elems]
 *   v_cache[...same...]                    = value[i*value_row_stride : +row_elems]
 * s == -1 skips the token, as in the reference.  Slots outside
 * [0, n_slots) are also skipped instead of writing out of bounds.
 * row_elems = kv_heads * head_dim (1024 for Qwen3-0.6B); n_slots =
 * num_blocks * block_size.  Strides are in elements.
 */
int qmi_store_kvcache(const uint16_t* key, int64_t key_row_stride,
                      const uint16_t* value, int64_t value_row_stride,
                      uint16_t* k_cache, uint16_t* v_cache,
                      const int32_t* slot_mapping, int64_t n_tokens,
                      int64_t row_elems, int64_t n_slots, void* stream);

/*
 * Paged GQA decode attention (one query token per sequence).
 * Replaces `flash_attn_with_kvcache(q.unsqueeze(1), k_cache, v_cache,
 * cache_seqlens=context_lens + 1, block_table=block_tables,
 * softmax_scale=scale, causal=True)` in Qwen3Attention.forward_decode
 * (qwen3_naive.py:672-680).
 *
 * q      : [batch, num_q_heads, head_dim] bf16, element strides
 *          q_seq_stride / q_head_stride, unit stride along head_dim.
 * caches : [num_blocks, block_size, num_kv_heads, head_dim] bf16, contiguous.
 * seqlens: int32 [batch]; sequence b attends to keys 0 .. seqlens[b] +
 *          seqlen_bias - 1 (flash-attn's cache_seqlens = seqlens + bias;
 *          forward_decode passes context_lens with bias 1).
 * block_table: int32 [batch, bt_width] (row stride bt_stride), -1 padded.
 * out    : [batch, num_q_heads, head_dim] bf16 with its own strides.
 * workspace: fp32 scratch of at least qmi_paged_decode_workspace_bytes().
 * q head h reads KV head h / (num_q_heads / num_kv_heads).
 * Supported: head_dim 128, block_size 256, num_q_heads / num_kv_heads in
 * {1, 2, 4, 8}.  pages_per_split <= 0 selects the balanced schedule (two
 * workgroups per CU each stream an equal share of the keys over all KV
 * heads; num_kv_heads in {2, 4, 8, 16}, ratio in {1, 2, 4}, batch <= 1024,
 * out 16-byte aligned with strides a multiple of 8) when it applies, else an
 * automatic per-(sequence, KV head) split; pages_per_split > 0 forces the
 * per-(sequence, KV head) split with that many pages.  pages_per_split == -1
 * selects the balanced schedule's whole-unit form: each workgroup takes one
 * whole (sequence, KV-head group) unit, empty sequences are written as zeros
 * and no merge launch follows; it is correct for any lengths and pays off
 * when the context lengths are near-equal (the caller's choice: the default
 * form detects that case on the device too, but still launches its merge).
 * With pages_per_split <= 0 the workspace size covers either schedule.
 * Pages whose table entry is outside [0, num_blocks) contribute nothing;
 * num_blocks == 0 is rejected (QMI_E_BAD_SHAPE).
 */
int64_t qmi_paged_decode_workspace_bytes(int64_t batch, int64_t num_kv_heads,
                                         int64_t num_q_heads, int64_t bt_width,
                                         int64_t pages_per_split);

int qmi_paged_decode_attention(const uint16_t* q, int64_t q_seq_stride, int64_t q_head_stride,
                               const uint16_t* k_cache, const uint16_t* v_cache,
                               int64_t num_blocks, int64_t block_size,
                               int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                               const int32_t* seqlens, int32_t seqlen_bias,
                               const int32_t* block_table, int64_t bt_stride, int64_t bt_width,
                               int64_t batch, float scale,
                               uint16_t* out, int64_t out_seq_stride, int64_t out_head_stride,
                               float* workspace, int64_t workspace_bytes,
                               int64_t pages_per_split, void* stream);

/*
 * The decode step's attention with the per-head QK-RMSNorm, RoPE and KV
 * store folded in: the same results as qmi_qk_norm_rope_store(qkv, ...)
 * (k and v heads to cache row slot_mapping[b]) followed by
 * qmi_paged_decode_attention(q, ..., seqlen_bias = 1) on the balanced
 * schedule, with one launch less and no q tensor.  Replaces q_norm / k_norm
 * -> rotary_emb -> store_kvcache -> flash_attn_with_kvcache of
 * Qwen3Attention.forward_decode (qwen3_naive.py:661-680).
 *
 * qkv    : [batch, qkv_stride] bf16 rows holding num_q_heads q heads, then
 *          num_kv_heads k heads, then num_kv_heads v heads of 128 dims
 *          (qkv_proj's packed output); 16-byte aligned, qkv_stride % 8 == 0.
 * q_norm_weight / k_norm_weight: bf16 [128], 16-byte aligned.
 * positions: int64 [batch] (clamped to [0, max_position)); cos_sin_cache:
 *          fp32 [max_position, 128] (cos at i, sin at 64 + i), 16-byte aligned.
 * slot_mapping: int32 [batch]; the new token's rows go to cache slot
 *          slot_mapping[b] (outside [0, num_blocks * 256): not stored).  It
 *          must be -1 or the slot of key seqlens[b] that the table maps (the
 *          engine's decode step); key seqlens[b] is then read from the new
 *          rows.  Sequences with seqlens[b] < 0 store nothing.
 * The rest as qmi_paged_decode_attention with seqlen_bias 1; pages_per_split
 * 0 (balanced split + merge) or -1 (whole units, no merge launch); the
 * workspace is qmi_paged_decode_workspace_bytes(.., pages_per_split = 0).
 * Supported: head_dim 128, block_size 256, num_kv_heads in {2, 4, 8, 16},
 * ratio in {1, 2, 4}, batch <= 1024, out 16-byte aligned, strides % 8 == 0.
 * q and k match the two-call form up to the fp32 order of each head's sum of
 * squares (v rows bit-identical).
 */
int qmi_paged_decode_attention_qkv(const uint16_t* qkv, int64_t qkv_stride, int64_t num_q_heads,
                                   int64_t num_kv_heads, int64_t head_dim,
                                   const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                                   const int64_t* positions, const float* cos_sin_cache,
                                   int64_t max_position, float eps, uint16_t* k_cache,
                                   uint16_t* v_cache, int64_t num_blocks, int64_t block_size,
                                   const int32_t* slot_mapping, const int32_t* seqlens,
                                   const int32_t* block_table, int64_t bt_stride,
                                   int64_t bt_width, int64_t batch, float scale, uint16_t* out,
                                   int64_t out_seq_stride, int64_t out_head_stride,
                                   float* workspace, int64_t workspace_bytes,
                                   int64_t pages_per_split, void* stream);

/*
 * Paged GQA decode attention that allocates nothing: no counterpart in the
 * reference.  For callers that cannot allocate device memory or take a
 * workspace (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and results as
 * qmi_paged_decode_attention without the workspace pair; the kernels use a
 * 16 MiB static device array instead (one per device, held until the
 * process ends; its address is looked up on the first call on a device, so
 * make that first call outside a graph capture).  Problems whose schedule
 * needs more than 16 MiB of workspace are rejected with QMI_E_SCRATCH_LIMIT
 * before anything is launched: the balanced schedule needs at most
 * 2 x CUs x 2 x num_q_heads x 528 B + 4 (batch + 2) B (Qwen3-0.6B's 16 query
 * heads: 8.7 MB on 256 CUs at any batch up to 1024); the per-split schedule
 * (pages_per_split > 0, or layouts the balanced one does not take) needs
 * batch x num_q_heads x splits x 528 B.  The array keeps
 * the last call's contents and needs no clearing, but calls that overlap on
 * one device share it and race: serialise them (one stream, or events).
 */
int qmi_paged_decode_attention_noalloc(const uint16_t* q, int64_t q_seq_stride,
                                       int64_t q_head_stride, const uint16_t* k_cache,
                                       const uint16_t* v_cache, int64_t num_blocks,
                                       int64_t block_size, int64_t num_q_heads,
                                       int64_t num_kv_heads, int64_t head_dim,
                                       const int32_t* seqlens, int32_t seqlen_bias,
                                       const int32_t* block_table, int64_t bt_stride,
                                       int64_t bt_width, int64_t batch, float scale,
                                       uint16_t* out, int64_t out_seq_stride,
                                       int64_t out_head_stride, int64_t pages_per_split,
                                       void* stream);

/*
 * Varlen paged causal prefill attention (bf16 MFMA).
 * Replaces `flash_attn_varlen_func(q, k_cache, v_cache, cu_seqlens_q,
 * cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale, causal=True,
 * block_table=block_tables)` in Qwen3Attention.forward_prefill
 * (qwen3_naive.py:631-637).
 *
 * q   : [total_q, num_q_heads, head_dim] bf16 (element strides; unit stride
 *       along head_dim); out has the same shape and its own strides.
 * Sequence b owns query rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 and
 * Lk = cu_seqlens_k[b+1] - cu_seqlens_k[b] keys, all already stored in the
 * paged caches (key j at row j % 256 of page block_table[b, j / 256]).
 * Causal masking is bottom-right aligned: query i of the Lq new ones sees
 * keys j <= i + Lk - Lq (new tokens see the whole cached prefix).
 * max_seqlen_q bounds Lq (it sizes the grid).  Query rows outside
 * [0, total_q) are never read or written.  Supported: head_dim 128,
 * block_size 256, num_q_heads / num_kv_heads in {1, 2, 4}.  Keys on pages
 * whose table entry is outside [0, num_blocks) contribute nothing (as in
 * decode); num_blocks == 0 is rejected (QMI_E_BAD_SHAPE).
 *
 * Scheduling (split_keys == 0).  A work item is one (query block of 128 / G
 * queries, sequence, KV head).  Launches with at least 256 and fewer than
 * 4 per CU items run on a persistent grid (two workgroups per CU, each
 * serving one KV head) that takes items from per-KV-head counters in the
 * workspace, long causal blocks first; a thin launch (no more items per KV
 * head than workgroups per head, e.g. a chunk after a long cached prefix)
 * also cuts its long items into pieces of about two balanced shares, whose
 * partial results (bf16 rows + fp32 max / sum) are merged by a second
 * kernel on the same stream.  Launches with fewer than 256 items split key
 * ranges across workgroups (fp32 partials, at most 16 pieces per item) and
 * thicker ones run one workgroup per item.  split_keys > 0 (a multiple of
 * 64) instead cuts key ranges into pieces of that many keys (at most 16 per
 * item) whatever the launch size.  max_seqlen_k (the longest Lk) only sizes
 * the split; any value gives the same result up to the rounding of merged
 * pieces.
 *
 * Workspace: at least qmi_varlen_prefill_workspace_bytes(...) bytes,
 * 16-byte aligned.  Its first bytes hold the work-queue counters: zero the
 * workspace once before its first use (e.g. hipMemset after allocating it);
 * every call leaves the counters at zero.  With a smaller workspace (or
 * NULL) the persistent grid and all splits are off (one workgroup per item,
 * same result).  Calls that share one workspace must not overlap (order
 * them on one stream).
 */
int64_t qmi_varlen_prefill_workspace_bytes(int64_t batch, int64_t max_seqlen_q,
                                           int64_t max_seqlen_k, int64_t num_q_heads,
                                           int64_t num_kv_heads, int64_t bt_width,
                                           int64_t split_keys);

int qmi_varlen_prefill_attention(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                 const uint16_t* k_cache, const uint16_t* v_cache,
                                 int64_t num_blocks, int64_t block_size,
                                 int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                 const int32_t* block_table, int64_t bt_stride, int64_t bt_width,
                                 int64_t batch, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                 int64_t total_q, float scale, uint16_t* out,
                                 int64_t out_tok_stride, int64_t out_head_stride,
                                 float* workspace, int64_t workspace_bytes, int64_t split_keys,
                                 void* stream);

/*
 * RMSNorm over rows of n bf16 elements with bf16 weight[n]:
 *   y = bf16(x * rsqrt(mean(x^2) + eps) * w), all math in fp32.
 * Replaces RMSNorm._rms_norm (qwen3_naive.py:156-161).  n % 8 == 0, n <= 4096.
 */
int qmi_rms_norm(const uint16_t* x, int64_t x_stride, const uint16_t* weight, uint16_t* y,
                 int64_t y_stride, int64_t n_rows, int64_t n, float eps, void* stream);

/*
 * Fused residual add + RMSNorm.  Replaces RMSNorm._add_rms_norm
 * (qwen3_naive.py:163-169): s = x + residual (fp32); residual_out = bf16(s);
 * y = bf16(s * rsqrt(mean(s^2) + eps) * w).  residual_out may alias residual.
 */
int qmi_add_rms_norm(const uint16_t* x, int64_t x_stride, const uint16_t* residual,
                     int64_t residual_stride, uint16_t* residual_out, int64_t residual_out_stride,
                     const uint16_t* weight, uint16_t* y, int64_t y_stride, int64_t n_rows,
                     int64_t n, float eps, void* stream);

/*
 * Fused per-head QK-RMSNorm + RoPE on the fused qkv projection.
 * Replaces q_norm / k_norm (qwen3_naive.py:661-662, RMSNorm over head_dim)
 * followed by RotaryEmbedding / _apply_rope_kernel (qwen3_naive.py:44-80,
 * :390-404).  qkv: [n_tok, (Hq + 2*Hkv) * 128] bf16 rows (q heads, then k
 * heads, then v heads).  For every q and k head: RMSNorm with the bf16
 * weight (rounded to bf16 as the reference does), then the half-split
 * rotation with cos/sin from the fp32 cos_sin_cache[max_position, 128]
 * (first 64 columns cos, last 64 sin) at positions[tok] (int64, clamped to
 * [0, max_position)).  Writes q_out [n_tok, Hq, 128] and k_out
 * [n_tok, Hkv, 128] (row strides q_stride / k_stride).  head_dim 128 only.
 * Alignment (else QMI_E_BAD_STRIDE): qkv and cos_sin_cache 16-byte aligned
 * with qkv_stride % 8 == 0; q_out, k_out and the weights 8-byte aligned with
 * q_stride % 4 == 0 and k_stride % 4 == 0.
 */
int qmi_qk_norm_rope(const uint16_t* qkv, int64_t qkv_stride, int64_t n_tok, int64_t num_q_heads,
                     int64_t num_kv_heads, int64_t head_dim, const uint16_t* q_norm_weight,
                     const uint16_t* k_norm_weight, const int64_t* positions,
                     const float* cos_sin_cache, int64_t max_position, uint16_t* q_out,
                     int64_t q_stride, uint16_t* k_out, int64_t k_stride, float eps,
                     void* stream);

/*
 * qmi_qk_norm_rope with the KV store fused in: q goes to q_out as above; the
 * rotated k head and the token's v head (the last Hkv heads of the qkv row,
 * unchanged) go to row slot_mapping[tok] of k_cache / v_cache ([n_slots,
 * Hkv * 128] bf16 rows, i.e. [num_blocks * 256] slots of the paged pool);
 * slots outside [0, n_slots) are skipped.  Replaces q_norm / k_norm + RoPE +
 * store_kvcache(k, v, ...) in Qwen3Attention.forward_prefill
 * (qwen3_naive.py:611-626) and forward_decode (:655-668); results are
 * bit-identical to qmi_qk_norm_rope followed by qmi_store_kvcache.  Same
 * alignment rules, and the caches 16-byte aligned.
 */
int qmi_qk_norm_rope_store(const uint16_t* qkv, int64_t qkv_stride, int64_t n_tok,
                           int64_t num_q_heads, int64_t num_kv_heads, int64_t head_dim,
                           const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                           const int64_t* positions, const float* cos_sin_cache,
                           int64_t max_position, uint16_t* q_out, int64_t q_stride,
                           uint16_t* k_cache, uint16_t* v_cache, const int32_t* slot_mapping,
                           int64_t n_slots, float eps, void* stream);

/*
 * SwiGLU activation of the fused gate_up projection.  Replaces
 * `silu(gate) * up` of Qwen3MLP.forward (qwen3_naive.py:695-702):
 * out[r, j] = bf16(silu(g) * u) with g = gate_up[r, j], u = gate_up[r, inter + j].
 */
int qmi_silu_mul(const uint16_t* gate_up, int64_t gate_up_stride, int64_t n_rows, int64_t inter,
                 uint16_t* out, int64_t out_stride, void* stream);

/*
 * Decode-batch projection y = x W^T (bf16 in and out, fp32 accumulation, one
 * rounding per output) for at most 256 rows.  Replaces the bf16 nn.Linear
 * calls of a decode step: qkv_proj (qwen3_naive.py:427, :654) and, with
 * activation 1, gate_up_proj followed by silu(gate) * up (qwen3_naive.py:692,
 * :699-701).  x [m, k] (row stride x_stride), w [n, k] (row stride w_stride),
 * y [m, n] (row stride y_stride).  activation 1 (SwiGLU): w is the packed
 * [2n, k] = [gate; up] weight and y[i, j] = bf16(silu(g) * u) with
 * g = bf16(x_i . gate_j), u = bf16(x_i . up_j) — the rounding points of a bf16
 * gate_up GEMM followed by qmi_silu_mul.  Requires m <= 256, k % 128 == 0,
 * n % 16 == 0; x and w 16-byte aligned with strides % 8 == 0 (>= k); y
 * 8-byte aligned, y_stride % 4 == 0 (>= n).
 */
int qmi_linear_rows(const uint16_t* x, int64_t x_stride, const uint16_t* w, int64_t w_stride,
                    int64_t m, int64_t n, int64_t k, int32_t activation, uint16_t* y,
                    int64_t y_stride, void* stream);

/*
 * Split-K form of qmi_linear_rows for the narrow projections that feed a
 * residual add + RMSNorm (o_proj, qwen3_naive.py:428, :683; down_proj,
 * :693, :702): writes parts[s][m][n] fp32 (contiguous) with
 * sum_s parts[s] = x W^T, so that few rows still spread over the GPU.
 * n_parts must equal qmi_linear_rows_parts_count(m, n, k) (0: unsupported
 * shape).  Same layout rules as qmi_linear_rows; parts 16-byte aligned.
 */
int64_t qmi_linear_rows_parts_count(int64_t m, int64_t n, int64_t k);
int qmi_linear_rows_parts(const uint16_t* x, int64_t x_stride, const uint16_t* w,
                          int64_t w_stride, int64_t m, int64_t n, int64_t k, float* parts,
                          int64_t n_parts, void* stream);

/*
 * Residual add + RMSNorm over a projection given as its partial products:
 * x = bf16(sum_s parts[s]) (the projection's bf16 output), then as
 * qmi_add_rms_norm: s = x + residual (fp32), residual_out = bf16(s),
 * y = bf16(s * rsqrt(mean(s^2) + eps) * w).  Replaces the o_proj / down_proj
 * output feeding RMSNorm._add_rms_norm (qwen3_naive.py:163-169).
 * parts [n_parts][m][n] fp32 contiguous, n_parts in {1, 2, 4, 8} (the counts
 * qmi_linear_rows_parts_count returns); n % 8 == 0, n <= 4096; rows and the
 * weight 16-byte aligned with strides % 8 == 0.
 */
int qmi_add_rms_norm_parts(const float* parts, int64_t n_parts, int64_t m,
                           const uint16_t* residual, int64_t residual_stride,
                           uint16_t* residual_out, int64_t residual_out_stride,
                           const uint16_t* weight, uint16_t* y, int64_t y_stride, int64_t n,
                           float eps, void* stream);

/*
 * Row-wise log-softmax gathered at one token per row.
 * Replaces `F.log_softmax(logits.float(), -1).gather(-1, ids)` of
 * forward_logprob (qwen3_grpo_train.py:46-53) and the rollout's
 * `log_softmax(last_logits).gather(next_tokens)` (qwen3_naive.py:1649-1650).
 *
 * Rows are (b, t) for b < n_seq, t < n_tok; row (b, t) starts at
 * logits + b*logit_seq_stride + t*logit_tok_stride and holds vocab bf16
 * values with unit stride.  Its token is ids[b*id_seq_stride +
 * t*id_tok_stride] (int64).  Outputs are fp32 [n_seq, n_tok] contiguous:
 *   out_lp[b,t]  = logits[b,t,id] - logsumexp(logits[b,t,:])
 *   out_lse[b,t] = logsumexp(logits[b,t,:])        (out_lse may be NULL)
 * An id outside [0, vocab) yields NaN for that row.
 */
int qmi_logprob_gather(const uint16_t* logits, int64_t logit_seq_stride, int64_t logit_tok_stride,
                       const int64_t* ids, int64_t id_seq_stride, int64_t id_tok_stride,
                       int64_t n_seq, int64_t n_tok, int64_t vocab,
                       float* out_lp, float* out_lse, void* stream);

/*
 * Group-normalised advantages.
 * Replaces compute_grpo_advantage (qwen3_grpo_train.py:162-173):
 *   A[i] = (r[i] - mean_g) / (std_g + eps)
 * over the rows whose prompt_ids equal prompt_ids[i]; std is the unbiased
 * (n-1) estimate, so a group of one row gives NaN as torch does.
 * rewards fp32 [n], prompt_ids int64 [n], out fp32 [n].
 */
int qmi_grpo_advantage(const float* rewards, const int64_t* prompt_ids, int64_t n,
                       float eps, float* out_adv, void* stream);

#define QMI_REDUCE_TOKEN_MEAN 0   /* sum(l*m) / (sum(m) + 1e-8), qwen3_grpo_train.py:198 */
#define QMI_REDUCE_SEQ_MEAN 1     /* mean_b( sum_t(l*m) / (sum_t(m) + 1e-8) ) */

/*
 * PPO clipped surrogate on given log-probabilities.
 * Replaces ppo_clipped_loss (qwen3_grpo_train.py:184-199):
 *   r = exp(new - old); l = -min(r*A, clamp(r, 1-clip, 1+clip)*A)
 * new_lp / old_lp / mask: fp32 [n_seq, n_tok] contiguous.  adv is fp32
 * addressed as adv[b*adv_seq_stride + t*adv_tok_stride]: strides (n_tok, 1)
 * for the reference's per-token advantages (qwen3_grpo_train.py:269),
 * (1, 0) for one advantage per sequence.
 * Masked tokens (mask == 0) are skipped.  out_loss: fp32 scalar.
 * out_dlp (may be NULL): fp32 [n_seq, n_tok], d loss / d new_lp, using
 * torch's subgradients of min (ties split 1/2) and clamp (pass-through
 * on the closed interval).
 */
int qmi_ppo_clipped_loss(const float* new_lp, const float* old_lp, const float* mask,
                         const float* adv, int64_t adv_seq_stride, int64_t adv_tok_stride,
                         int64_t n_seq, int64_t n_tok,
                         float clip_eps, int32_t reduction,
                         float* out_loss, float* out_dlp, void* stream);

/*
 * Fused GRPO loss step: log-softmax gather + group advantages + clipped
 * masked loss, one streaming pass over the logits (the dominant cost).
 * Combines qwen3_grpo_train.py:46-53 (forward_logprob's gather), :162-173
 * (advantages), :269 (token expansion) and :184-199 (loss).
 *
 * Logit/id addressing as qmi_logprob_gather (pass shifted views for the
 * logits[t-1] <-> ids[t] alignment).  old_lp, mask: fp32 [n_seq, n_tok]
 * contiguous; rewards fp32 [n_seq]; prompt_ids int64 [n_seq].
 * Outputs: out_lp, out_lse fp32 [n_seq, n_tok]; out_adv fp32 [n_seq];
 * out_dlp fp32 [n_seq, n_tok] (d loss / d lp); out_loss fp32 scalar.
 * workspace: qmi_grpo_fused_workspace_bytes(n_seq, n_tok) bytes, 16-byte
 * aligned (per-sequence sums; no initial contents needed, nothing kept
 * between calls).  Concurrent calls must not share one.
 * Launches: the row pass, one workgroup per sequence for the loss terms,
 * and one more small launch that applies the token-mean denominator.
 */
int64_t qmi_grpo_fused_workspace_bytes(int64_t n_seq, int64_t n_tok);

int qmi_grpo_fused_loss(const uint16_t* logits, int64_t logit_seq_stride, int64_t logit_tok_stride,
                        const int64_t* ids, int64_t id_seq_stride, int64_t id_tok_stride,
                        int64_t n_seq, int64_t n_tok, int64_t vocab,
                        const float* old_lp, const float* mask,
                        const float* rewards, const int64_t* prompt_ids,
                        float adv_eps, float clip_eps, int32_t reduction,
                        float* out_lp, float* out_lse, float* out_adv, float* out_dlp,
                        float* out_loss, void* workspace, int64_t workspace_bytes,
                        void* stream);

/*
 * Backward of the log-softmax gather through the bf16 logits: for every
 * row (b, t) and vocab entry v,
 *   grad[b,t,v] = g * coef[b,t] * (1[v == id] - exp(logits[b,t,v] - lse[b,t]))
 * rounded to bf16, where g = *grad_scale (a device fp32 scalar, e.g. the
 * incoming gradient of the loss; NULL means 1).  Rows with coef == 0 are
 * written as zeros without reading their logits.  This is the gradient
 * that loss.backward() (qwen3_grpo_train.py:281) sends through
 * log_softmax(logits.float()) back to the bf16 logits.
 * grad is [n_seq, n_tok, vocab] bf16 with strides grad_seq_stride /
 * grad_tok_stride; coef and lse are fp32 [n_seq, n_tok] contiguous.
 */
int qmi_logprob_gather_backward(const uint16_t* logits, int64_t logit_seq_stride, int64_t logit_tok_stride,
                                const int64_t* ids, int64_t id_seq_stride, int64_t id_tok_stride,
                                int64_t n_seq, int64_t n_tok, int64_t vocab,
                                const float* lse, const float* coef, const float* grad_scale,
                                uint16_t* grad, int64_t grad_seq_stride, int64_t grad_tok_stride,
                                void* stream);

/*
 * Token sampling with the drawn token's log-probability, one pass over bf16
 * logits rows.  Replaces, for top_k = None, the sampling step of
 * generate_continuous (qwen3_naive.py:1413-1423) and of
 * generate_continuous_with_logprobs (:1636-1650):
 *   x = logits.float() / temperature; tok ~ Categorical(softmax(x));
 *   lp = log_softmax(x)[tok].
 * Draw: Gumbel-max with Philox4x32-10 uniforms; element i of row r uses word
 * i % 4 of the block at counter (i / 4, r, offset_lo, offset_hi), key
 * (seed_lo, seed_hi); a given (seed, offset) reproduces the same tokens.
 * logits: [n_rows, vocab] bf16 with row stride row_stride (elements).
 * out_tokens: int64 [n_rows]; out_logprobs: fp32 [n_rows] or NULL.
 * temperature must be finite and > 0.
 */
int qmi_sample_tokens(const uint16_t* logits, int64_t row_stride, int64_t n_rows, int64_t vocab,
                      float temperature, uint64_t seed, uint64_t offset, int64_t* out_tokens,
                      float* out_logprobs, void* stream);

/*
 * Top-k token sampling from bf16 logits with the drawn token's log-probability.
 * Replaces, for top_k = k, the sampling step of generate_continuous
 * (qwen3_naive.py:1413-1422, the reference default k = 20) and of
 * generate_continuous_with_logprobs (:1641-1650):
 *   x = logits.float() / T; keep the k largest of x (the rest -inf);
 *   tok ~ Categorical(softmax(x)); lp = log_softmax(x)[tok].
 * Of entries tied at the k-th largest value the lowest indices are kept.
 * Draw: inverse transform sampling over the kept entries in vocabulary order
 * with u as in qmi_lm_head_sample (Philox4x32-10, counter (0, row, offset)).
 * logits: [n_rows, vocab] bf16 (row stride row_stride); 1 <= top_k <= 1024
 * and <= vocab.  out_tokens int64 [n_rows]; out_logprobs fp32 or NULL.
 */
int qmi_sample_tokens_topk(const uint16_t* logits, int64_t row_stride, int64_t n_rows,
                           int64_t vocab, int64_t top_k, float temperature, uint64_t seed,
                           uint64_t offset, int64_t* out_tokens, float* out_logprobs,
                           void* stream);

/*
 * Fused lm_head + sampling: logits = hidden_states . weight^T accumulated in
 * fp32 and rounded to bf16 (the reference's bf16 lm_head output), never
 * materialised; then one token per row drawn from softmax(logits / T), or,
 * with 0 < top_k < vocab, from the softmax of the top_k largest of
 * logits / T (the rest -inf; of entries tied at the k-th value the lowest
 * indices are kept), with the drawn token's log-probability under that
 * distribution.  Replaces `logits = self.lm_head(h)` (qwen3_naive.py:1387,
 * :1607) and the sampling step of generate_continuous (:1413-1423) and
 * generate_continuous_with_logprobs (:1636-1650), for top_k = None (pass 0)
 * and for top_k = k <= 64 (the reference default is 20).
 * hidden_states: [n_rows, hidden] bf16 (row stride h_stride); weight:
 * [vocab, hidden] bf16 (row stride w_stride); hidden a multiple of 64 and at
 * most 16384, pointers 16-byte aligned, strides multiples of 8.
 * Draw: inverse transform sampling over the kept entries in vocabulary
 * order -- the first index whose cumulative probability exceeds u, with
 * u = (53 bits of words 0 and 1 of Philox4x32-10 at counter
 * (0, lo32(q), lo32(offset) + hi32(q), hi32(offset)), key (seed_lo,
 * seed_hi)) + 0.5, scaled by 2^-53, where q is the row's counter value:
 * row_counters[r] (uint64 [n_rows], device memory), or r when row_counters
 * is NULL.  Equal (seed, offset, q) reproduce a row's token, whatever the
 * other rows.  out_tokens int64 [n_rows]; out_logprobs fp32 [n_rows] or NULL.
 * workspace: qmi_lm_head_workspace_bytes(n_rows, vocab, top_k) bytes, 16-byte
 * aligned (per-row softmax pairs over 32-, 64- or 128-entry slices of the
 * vocabulary, by row count, and, with top-k, each
 * tile's four largest logits; no initial contents).  top_k above 64, or top-k
 * over a vocabulary above 262,144 entries, returns QMI_E_UNSUPPORTED (top-k
 * sampling from materialised logits: qmi_sample_tokens_topk), as does a call
 * whose ceil(vocab / 128) x ceil(n_rows / 64) x hidden / 64 exceeds 2^31 - 1
 * (about 7 million rows at Qwen3-0.6B's shape: split such a call by rows).
 */
int64_t qmi_lm_head_workspace_bytes(int64_t n_rows, int64_t vocab, int64_t top_k);

int qmi_lm_head_sample(const uint16_t* hidden_states, int64_t h_stride, int64_t n_rows,
                       const uint16_t* weight, int64_t w_stride, int64_t vocab, int64_t hidden,
                       float temperature, int64_t top_k, uint64_t seed, uint64_t offset,
                       const uint64_t* row_counters, int64_t* out_tokens, float* out_logprobs,
                       void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Fused lm_head + log-softmax gather: out_logprobs[r] =
 * log_softmax(bf16(hidden_states[r] . weight^T))[targets[r * target_stride]]
 * and out_lse[r] (may be NULL) its log-sum-exp, the logits rounded to bf16 as
 * the reference's lm_head output and never materialised.  A target outside
 * [0, vocab) gives a NaN log-probability.  Replaces `model(input_ids)`'s
 * lm_head (qwen3_naive.py:826-835) plus forward_logprob's gather
 * (qwen3_grpo_train.py:46-53) for the rows given.  Layout as
 * qmi_lm_head_sample; workspace qmi_lm_head_workspace_bytes(n_rows, vocab, 0).
 */
int qmi_lm_head_logprob(const uint16_t* hidden_states, int64_t h_stride, int64_t n_rows,
                        const uint16_t* weight, int64_t w_stride, int64_t vocab, int64_t hidden,
                        const int64_t* targets, int64_t target_stride, float* out_logprobs,
                        float* out_lse, void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QWEN3MI_H */
