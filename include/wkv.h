/*
 * wkv.h — C ABI of libwkv.so, the MI355X (gfx950) paged KV-cache decode path.
 *
 * The reference engine never touches KV memory itself: every append, block
 * table read and paged attention happens inside the vLLM engine it drives
 * (wavelet/inference/engine.py:818 builds it, :887 / :1045 / :1274 call
 * llm.generate; wavelet/inference/server.py:323 / :1006 on the OpenAI
 * backend). The entry points below replace the KV operations of that engine;
 * each comment names the reference call site and the engine operation
 * (vLLM's public custom-op name) it stands in for.
 *
 * Conventions
 *   - All pointers are device pointers; sizes and strides are in elements.
 *   - The library allocates nothing: caches, scales, block tables, outputs and
 *     workspaces are owned by the caller (PyTorch in this repository).
 *   - Every call is asynchronous on `stream` (a hipStream_t, NULL = default
 *     stream) and never synchronises the host.
 *   - Return value: 0 (WKV_OK) or a wkv_status_t. Arguments are validated on
 *     the host before any launch; wkv_last_error() returns a thread-local
 *     message for the last failure on the calling thread.
 *   - Slot convention: slot = block_id * block_size + offset; slot -1 marks a
 *     padded token that is skipped.
 *
 * Cache layout (one layer; x = 16 / element bytes, 8 for bf16, 16 for fp8):
 *   k        [num_blocks, num_kv_heads, head_dim / x, block_size, x]
 *   v        [num_blocks, num_kv_heads, head_dim, block_size]
 *   k_scale, v_scale  [num_blocks, num_kv_heads] fp32, fp8 caches only
 *   MLA latent [num_blocks, block_size, kv_lora_rank + rope_dim] bf16
 * This is the paged-attention layout of the engine's ROCm backend: 16-byte
 * runs of K along head_dim for one token, V transposed so one head_dim row of
 * a block is contiguous.
 */
#ifndef WKV_H
#define WKV_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WKV_ABI_VERSION 1

typedef enum {
  WKV_OK = 0,
  WKV_ERR_INVALID = 1,     /* bad argument: shape, dtype, alignment, size */
  WKV_ERR_UNSUPPORTED = 2, /* valid but not implemented (e.g. head_dim 96) */
  WKV_ERR_LAUNCH = 3       /* the HIP runtime rejected a launch */
} wkv_status_t;

typedef enum { WKV_KV_BF16 = 0, WKV_KV_FP8_E4M3 = 1 } wkv_kv_dtype_t;

/* One layer of a paged K/V cache. Replaces the per-layer KV tensors vLLM
 * allocates from gpu_memory_utilization (engine.py:790-813; num_gpu_blocks x
 * block_size is the capacity the reference reads back at
 * wavelet/orchestrator/inference_metrics.py:125-133). */
typedef struct {
  void *k;
  void *v;
  float *k_scale; /* fp8 only, else NULL */
  float *v_scale; /* fp8 only, else NULL */
  int64_t num_blocks;
  int32_t block_size;   /* multiple of 16 */
  int32_t num_kv_heads;
  int32_t head_dim;     /* 64 or 128 */
  int32_t kv_dtype;     /* wkv_kv_dtype_t */
  int32_t flags;        /* WKV_CACHE_* bits, 0 = none */
  int32_t reserved;     /* 0 */
} wkv_cache_t;

/* wkv_cache_t.flags: blocks of this cache are read by several sequences
 * (prefix caching, GRPO groups sharing prompt blocks). The decode then reads
 * K/V with the default cache policy, so a shared block read by one sequence
 * stays cached for the next; without the flag it reads them as streamed,
 * read-once data (non-temporal loads: 3-9% faster on unshared blocks,
 * about 15% slower when blocks are shared). The group-aware decode sets its
 * own policy per role and ignores the flag. */
#define WKV_CACHE_SHARED_BLOCKS 1

/* One layer of an MLA latent cache (bf16). */
typedef struct {
  void *latent;
  int64_t num_blocks;
  int32_t block_size;   /* multiple of 16 */
  int32_t kv_lora_rank; /* 512 */
  int32_t rope_dim;     /* 64 */
} wkv_mla_cache_t;

/* ---- append -------------------------------------------------------------
 * bf16 slot-mapped append: cache[slot[t]] = (key[t], value[t]) for slot >= 0.
 * key/value: [num_tokens, num_kv_heads, head_dim] bf16, head_dim contiguous,
 * strides multiples of 8 and base pointers 16-byte aligned.
 * Replaces vLLM reshape_and_cache (reached through llm.generate,
 * engine.py:887; HF analogue past_key_values.update,
 * wavelet/kernels/patch.py:173-180). */
int wkv_append(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
               const void *value, int64_t value_stride_t, int64_t value_stride_h,
               const int64_t *slot_mapping, int64_t num_tokens, void *stream);

/* fp8-e4m3 append with one power-of-two fp32 scale per (block, head) for K
 * and for V. Tokens are taken in runs (consecutive tokens of the call whose
 * slots share a block); a run starting at offset 0 starts the block afresh,
 * otherwise the scale may only grow and the block's earlier entries are
 * re-encoded by the exact power-of-two ratio. Quantisation follows
 * _fp8_roundtrip (wavelet/trainer/models/deepseek_v4/attention.py:41-50).
 * A block may appear in at most one run per call.
 * Replaces vLLM reshape_and_cache with kv_cache_dtype="fp8_e4m3" (enabled
 * through inference.vllm.extra_args, wavelet/inference/server.py:1201-1212). */
int wkv_append_fp8(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                   const void *value, int64_t value_stride_t, int64_t value_stride_h,
                   const int64_t *slot_mapping, int64_t num_tokens, void *stream);

/* MLA latent append: latent[slot[t]] = concat(kv_c[t], k_pe[t]).
 * kv_c [T, kv_lora_rank], k_pe [T, rope_dim] bf16, row strides multiples of 8.
 * Replaces vLLM concat_and_cache_mla (the MLA backend the reference patches
 * at wavelet/inference/deepseek_v4.py:15-66). */
int wkv_mla_append(const wkv_mla_cache_t *cache, const void *kv_c, int64_t kv_c_stride,
                   const void *k_pe, int64_t k_pe_stride, const int64_t *slot_mapping,
                   int64_t num_tokens, void *stream);

/* ---- gather / block copy -------------------------------------------------
 * Contiguous copy of each sequence's context:
 *   out[cu_seq_lens[i] + t] = cache[block_table[i, t / bs], t % bs], t < seq_lens[i]
 * out_k/out_v: [sum(seq_lens), num_kv_heads, head_dim]. With dequant = 0 the
 * raw stored elements are copied (bf16, or fp8 codes); with dequant = 1 an fp8
 * cache is written as bf16 code * scale (exact). block_table [batch, bt_stride]
 * int32; seq_lens [batch] int32 <= max_blocks_per_seq * block_size;
 * cu_seq_lens [batch] int64 exclusive prefix sums.
 * Replaces vLLM gather_cache / gather_and_maybe_dequant_cache (prefix-cache
 * reads inside llm.generate, engine.py:887; index semantics of
 * attention.py:85-88 / :320-360). */
int wkv_gather(const wkv_cache_t *cache, const int32_t *block_table, int64_t bt_stride,
               int32_t max_blocks_per_seq, const int32_t *seq_lens, const int64_t *cu_seq_lens,
               int32_t batch, void *out_k, void *out_v, int32_t dequant, void *stream);

/* Copy whole blocks (K, V and fp8 scales): for i < n, block mapping[2i+1]
 * becomes a copy of block mapping[2i]. The pairs are copied concurrently, so
 * they must be independent: no block may be the destination of one pair and
 * the source or destination of another (the block manager's copy-on-write
 * pairs -- a shared block, a fresh one -- never are). Copy-on-write of a
 * partially filled shared block when a GRPO group forks (n = num_generations
 * sampling, engine.py:69-90). Replaces vLLM copy_blocks. */
int wkv_copy_blocks(const wkv_cache_t *cache, const int64_t *block_mapping, int64_t n, void *stream);

/* MLA latent gather: contiguous copy of each sequence's latent rows,
 *   out[cu_seq_lens[i] + t] = latent[block_table[i, t / bs], t % bs], t < seq_lens[i]
 * out: [sum(seq_lens), kv_lora_rank + rope_dim] bf16, rows as stored (c_kv
 * then k_pe). Table arguments as for wkv_gather; an entry outside
 * [0, num_blocks) leaves its rows unwritten. Replaces vLLM gather_cache on the
 * MLA latent cache (the cached-context read of MLA chunked prefill and of
 * prefix-cache hits inside llm.generate, engine.py:887); index semantics of
 * the latent gather at wavelet/trainer/models/deepseek_v4/attention.py:85-88
 * and :320-360. */
int wkv_mla_gather(const wkv_mla_cache_t *cache, const int32_t *block_table, int64_t bt_stride,
                   int32_t max_blocks_per_seq, const int32_t *seq_lens, const int64_t *cu_seq_lens, int32_t batch,
                   void *out, void *stream);

/* Copy whole latent blocks: for i < n, block mapping[2i+1] becomes a copy of
 * block mapping[2i] (pairs naming a block outside [0, num_blocks) are
 * skipped; pairs independent, as for wkv_copy_blocks). Copy-on-write of a
 * shared, partly filled latent block before a
 * GRPO group member appends into it (n = num_generations sampling,
 * engine.py:69-90). Replaces vLLM copy_blocks on an MLA cache. */
int wkv_mla_copy_blocks(const wkv_mla_cache_t *cache, const int64_t *block_mapping, int64_t n, void *stream);

/* ---- paged decode attention ---------------------------------------------
 * o[b, h] = softmax(q[b, h] . K_b^T * scale) . V_b over seq_lens[b] tokens read
 * through block_table[b]; query head h reads KV head h / (num_q_heads /
 * num_kv_heads). q: [batch, num_q_heads, head_dim] bf16 (head_dim contiguous,
 * strides multiples of 8); out: [batch, num_q_heads, head_dim] bf16
 * contiguous. max_seq_len must be >= every seq_lens[b]. partition_size
 * (tokens, multiple of 16 spanning at most 64 blocks; 0 = library choice)
 * splits long contexts into partitions; a second kernel merges them by
 * log-sum-exp, using `workspace` (wkv_decode_workspace_size() bytes of
 * scratch; unused when every context fits one partition). A zero-length
 * sequence gives zeros.
 * Replaces vLLM paged_attention_v1/v2 and the ROCm paged-attention op (decode
 * step of llm.generate, engine.py:887; semantics of attention.py:89-96 and the
 * attention_interface call at wavelet/kernels/patch.py:182-196). */
int64_t wkv_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                  int32_t max_seq_len, int32_t partition_size);

int wkv_paged_decode_gqa(const wkv_cache_t *cache, const void *q, int64_t q_stride_b, int64_t q_stride_h,
                         void *out, int32_t num_q_heads, const int32_t *block_table, int64_t bt_stride,
                         int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                         int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                         int64_t workspace_bytes, const int32_t *seq_order, void *stream);

/* seq_order (optional, NULL = batch order) for the two GQA decode calls: a
 * permutation of 0..batch-1 in device memory giving the order in which
 * sequences are dispatched (entries outside 0..batch-1 are skipped, leaving
 * that output unwritten). The result does not depend on it, bit for bit;
 * dispatching long contexts first shortens a launch over mixed lengths.
 * wkv_decode_order writes that order -- sequence indices by seq_lens, longest
 * first, ties by index -- into order[batch]: one call per step serves every
 * layer. No reference counterpart (vLLM's decode launch takes sequences in
 * batch order); an addition of this library's. */
int wkv_decode_order(const int32_t *seq_lens, int32_t batch, int32_t *order, void *stream);

/* The dispatch order for wkv_paged_decode_gqa_grouped over GRPO groups of
 * group_size consecutive sequences, for the decode geometry the call will get
 * (num_kv_heads, max_seq_len, block_size, partition_size as passed to it):
 * longest first, ties by index, within classes of whole groups that the decode
 * launch maps to the same XCDs, the classes interleaved -- a group's members
 * then read its prompt through one L2, in the same longest-first rhythm. When
 * the classes cannot be of equal size (batch not a multiple of group_size
 * times their number) it is wkv_decode_order's order. One call per step serves
 * every layer. No reference counterpart; an addition of this library's. */
int wkv_grouped_decode_order(const int32_t *seq_lens, int32_t batch, int32_t group_size, int32_t num_kv_heads,
                             int32_t max_seq_len, int32_t block_size, int32_t partition_size, int32_t *order,
                             void *stream);

/* The launch shape the two GQA decode calls use for this geometry (host
 * only, no GPU): the partition size (partition_size, or the library's choice
 * when 0), the waves per workgroup and the workgroups (chunks) per sequence
 * and KV head; more than one chunk leaves partials for the merge kernel. For
 * planning and labelling; no reference counterpart. max_seq_len is the one
 * the decode call will get, clipped to the block-table width. */
int wkv_decode_plan(int32_t batch, int32_t num_kv_heads, int32_t max_seq_len, int32_t block_size,
                    int32_t partition_size, int32_t *out_partition, int32_t *out_waves, int32_t *out_chunks);

/* One whole decode step of one layer in one launch: append token b of
 * key/value ([batch, num_kv_heads, head_dim] bf16) at slot_mapping[b] (-1 =
 * none) -- bf16 as wkv_append, fp8 as wkv_append_fp8 with runs of one -- then
 * the attention of wkv_paged_decode_gqa over contexts that include it.
 * slot_mapping[b] must address position seq_lens[b] - 1 of sequence b, and
 * partition_size (when given) must be a multiple of block_size. A slot of -1
 * stores nothing, and what the attention then sees at that position is
 * unspecified (meant for padding entries whose output is discarded). Equivalent to
 * wkv_append (or wkv_append_fp8) followed by wkv_paged_decode_gqa; the append
 * and attention the reference runs back to back per layer in its decode step
 * (past_key_values.update then attention_interface, patch.py:173-196). */
int wkv_append_paged_decode_gqa(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                const int32_t *seq_order, void *stream);

/* The two GQA decode calls with a per-head attention sink: sinks[h] (fp32,
 * device memory, one per query head, natural-log units like the scaled
 * scores; -inf = none) is one more logit in head h's softmax whose value
 * vector is zero, so o[b, h] = sum_t e^(s_t) v_t / (sum_t e^(s_t) + e^(sinks[h]))
 * and a zero-length sequence still gives zeros. Otherwise the arguments and
 * behaviour of wkv_paged_decode_gqa / wkv_append_paged_decode_gqa. Replaces
 * the learned sink of the reference's sparse attention
 * (wavelet/trainer/models/deepseek_v4/attention.py:89-95: torch.cat of the
 * scores with the sink, softmax, sink column dropped; the sinks parameter of
 * attention.py:703), which its decode backend must honour. */
int wkv_paged_decode_gqa_sinks(const wkv_cache_t *cache, const void *q, int64_t q_stride_b, int64_t q_stride_h,
                               void *out, int32_t num_q_heads, const int32_t *block_table, int64_t bt_stride,
                               int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                               int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                               int64_t workspace_bytes, const int32_t *seq_order, const float *sinks, void *stream);

int wkv_append_paged_decode_gqa_sinks(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                      int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                      int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                      int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                      const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                      const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                      int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                      const int32_t *seq_order, const float *sinks, void *stream);

/* Allocation-free variant of wkv_append_paged_decode_gqa, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc): the same arguments and result
 * without workspace / workspace_bytes. The split-K partials go to a static
 * device array of WKV_NOALLOC_SCRATCH_BYTES per GPU, held until the process
 * ends; the call allocates nothing. Geometries needing more scratch than that
 * (wkv_decode_workspace_size at the launch's partition) fail with
 * WKV_ERR_INVALID before any launch. The current device must be the one
 * `stream` belongs to. Every call on a GPU shares that GPU's array: calls that
 * overlap on one GPU race. No counterpart in the reference. */
#define WKV_NOALLOC_SCRATCH_BYTES (32ll << 20)

int wkv_append_paged_decode_gqa_noalloc(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                        int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                        int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                        int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                        const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                        const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                        int32_t partition_size, const int32_t *seq_order, void *stream);

/* Group-aware decode for GRPO groups (the n samples of one prompt):
 * sequences g*group_size .. g*group_size+group_size-1 form group g (the last
 * group may be short), and the first prefix_lens[g] tokens of every member are
 * stored in the same physical blocks -- identical block-table entries, as
 * SamplingParams(n=num_generations) leaves them (engine.py:69-90) and
 * BlockManager.share_prefix builds them. The attention is wkv_paged_decode_gqa's
 * (or, with key, value and slot_mapping given, wkv_append_paged_decode_gqa's),
 * bit for bit; what the groups change is how the cache is read: the group's
 * prompt blocks keep the default cache policy, so its members' reads of one
 * block meet in the L2 and the last-level cache, while each member's own tokens
 * are streamed past them (non-temporal loads). With seq_order from
 * wkv_grouped_decode_order, the members' workgroups of one KV head also run
 * on one XCD (one L2). key, value and slot_mapping are all NULL for attention
 * only. prefix_lens values above max_prefix_len are read as max_prefix_len;
 * prefix_lens only steers the read policy (any values give the same result).
 * workspace: wkv_grouped_decode_workspace_size() bytes (the plain decode's).
 * seq_order as for wkv_paged_decode_gqa. No reference counterpart computes
 * this (vLLM decodes each member separately); the group semantics are the
 * reference's (engine.py:69-90, :1034-1038). */
int64_t wkv_grouped_decode_workspace_size(int32_t batch, int32_t num_q_heads, int32_t head_dim,
                                          int32_t max_seq_len, int32_t max_prefix_len, int32_t partition_size);

int wkv_paged_decode_gqa_grouped(const wkv_cache_t *cache, const void *key, int64_t key_stride_t,
                                 int64_t key_stride_h, const void *value, int64_t value_stride_t,
                                 int64_t value_stride_h, const int64_t *slot_mapping, const void *q,
                                 int64_t q_stride_b, int64_t q_stride_h, void *out, int32_t num_q_heads,
                                 const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                 const int32_t *seq_lens, int32_t batch, int32_t max_seq_len,
                                 const int32_t *prefix_lens, int32_t group_size, int32_t max_prefix_len,
                                 float scale, int32_t partition_size, void *workspace, int64_t workspace_bytes,
                                 const int32_t *seq_order, void *stream);

/* Varlen GQA prefill / chunked prefill over the paged cache. Sequence b
 * brings n_b = cu_seqlens_q[b+1] - cu_seqlens_q[b] new tokens (rows of q
 * [num_tokens, num_q_heads, head_dim] and out, bf16, last dim contiguous) at
 * positions seq_lens[b] - n_b .. seq_lens[b] - 1; new token j attends to
 * positions 0 .. seq_lens[b] - n_b + j (causal, aligned to the end of the
 * context: cached context -- an earlier chunk or a prefix-cache hit -- is
 * attended in full). With key/value/slot_mapping given (num_tokens rows) the
 * new tokens are first appended exactly as wkv_append / wkv_append_fp8 would,
 * then attended from the cache; with all three NULL the cache must already
 * hold them. max_query_len >= every n_b; no workspace.
 * Replaces the prompt step of llm.generate (engine.py:887): vLLM's
 * reshape_and_cache followed by its varlen flash-attention over the paged
 * cache (the prefix-cache path reads cached blocks, engine.py:1034-1038). */
int wkv_prefill_gqa(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                    const void *value, int64_t value_stride_t, int64_t value_stride_h, const int64_t *slot_mapping,
                    int64_t num_tokens, const void *q, int64_t q_stride_t, int64_t q_stride_h, void *out,
                    int64_t out_stride_t, int64_t out_stride_h, int32_t num_q_heads, const int32_t *cu_seqlens_q,
                    const int32_t *seq_lens, const int32_t *block_table, int64_t bt_stride,
                    int32_t max_blocks_per_seq, int32_t batch, int32_t max_query_len, int32_t max_seq_len,
                    float scale, void *stream);

/* wkv_prefill_gqa with per-head attention sinks (sinks as for
 * wkv_paged_decode_gqa_sinks: one zero-value logit per query head, fp32,
 * natural-log units, -inf = none), the sinks of the reference's sparse
 * attention (wavelet/trainer/models/deepseek_v4/attention.py:89-95). */
int wkv_prefill_gqa_sinks(const wkv_cache_t *cache, const void *key, int64_t key_stride_t, int64_t key_stride_h,
                          const void *value, int64_t value_stride_t, int64_t value_stride_h,
                          const int64_t *slot_mapping, int64_t num_tokens, const void *q, int64_t q_stride_t,
                          int64_t q_stride_h, void *out, int64_t out_stride_t, int64_t out_stride_h,
                          int32_t num_q_heads, const int32_t *cu_seqlens_q, const int32_t *seq_lens,
                          const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq, int32_t batch,
                          int32_t max_query_len, int32_t max_seq_len, float scale, const float *sinks, void *stream);

/* Token sampler: the step after decode, producing what the engine records per
 * generated token -- the token, its processed logprob and the sampling mask
 * (llm.generate with logprobs_mode="processed_logprobs" and
 * return_sampling_mask, engine.py:795-805, consumed at engine.py:187-256).
 * logits [batch, vocab] (row_stride elements apart; logits_dtype 0 = fp32,
 * 1 = bf16). Per row, in order (NULL arrays = the default):
 *   repetition penalty on tokens set in seen_tokens (bitmap, [batch,
 *   ceil(vocab/32)] uint32): l > 0 ? l / r : l * r (default r = 1);
 *   x = l / temperature (temperature < 1e-5: greedy, x = l; default 1);
 *   min_p: keep x >= max(x) + ln(min_p) (default 0: off);
 *   top_k: keep the top_k largest, ties kept (<= 0 or >= vocab: off);
 *   top_p: keep token i iff the softmax mass of tokens strictly larger than
 *     x_i is < top_p (>= 1: off);
 *   sample: exponential race over the kept set, E_i ~ Exp(1) from a hash of
 *     (seeds[b], step, i) -- a draw from softmax(x) restricted to the kept set;
 *     greedy rows take the largest x (ties: lowest index).
 * Outputs: out_tokens [batch] int64; out_logprobs [batch] (log-softmax of x
 * over the kept set at the token; may be NULL); out_mask [batch,
 * ceil(vocab/32)] bitmap of the kept set and out_counts [batch] its size
 * (each may be NULL). Deterministic for given inputs and step.
 * Replaces vLLM's sampler (vllm.v1 Sampler; parameters from
 * vllm_sampling_kwargs, engine.py:69-90). */
int wkv_sample(const void *logits, int32_t logits_dtype, int64_t row_stride, int32_t batch, int32_t vocab,
               const float *temperature, const int32_t *top_k, const float *top_p, const float *min_p,
               const float *repetition_penalty, const uint32_t *seen_tokens, const uint64_t *seeds, int64_t step,
               int64_t *out_tokens, float *out_logprobs, uint32_t *out_mask, int32_t *out_counts, void *stream);

/* Weight-absorbed MLA decode over the latent cache:
 *   s = (q_nope . c_kv + q_pe . k_pe) * scale; o = softmax(s) . c_kv
 * q_nope [batch, num_heads, kv_lora_rank], q_pe [batch, num_heads, rope_dim]
 * bf16 (last dim contiguous); out [batch, num_heads, kv_lora_rank] bf16.
 * Replaces the vLLM MLA decode backend (FlashMLA, named at
 * wavelet/inference/deepseek_v4.py:17, :64-66). */
int64_t wkv_mla_workspace_size(int32_t batch, int32_t num_heads, int32_t kv_lora_rank,
                               int32_t max_seq_len, int32_t partition_size);

int wkv_paged_decode_mla(const wkv_mla_cache_t *cache, const void *q_nope, int64_t qn_stride_b,
                         int64_t qn_stride_h, const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h,
                         void *out, int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                         int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                         int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                         int64_t workspace_bytes, void *stream);

/* One MLA decode step of one layer in one launch: latent[slot_mapping[b]] =
 * concat(kv_c[b], k_pe[b]) (as wkv_mla_append; -1 = none), then the
 * attention of wkv_paged_decode_mla over contexts that include that token.
 * kv_c [batch, kv_lora_rank], k_pe [batch, rope_dim] bf16, row strides
 * multiples of 8; slot_mapping[b] must address position seq_lens[b] - 1 of
 * sequence b. The new token is attended from kv_c / k_pe (so nothing waits
 * for its cache write). Equivalent to wkv_mla_append followed by
 * wkv_paged_decode_mla: the latent append and MLA attention the engine runs
 * back to back per layer (concat_and_cache_mla, then the MLA decode backend
 * named at wavelet/inference/deepseek_v4.py:17, :64-66). */
int wkv_append_paged_decode_mla(const wkv_mla_cache_t *cache, const void *kv_c, int64_t kv_c_stride,
                                const void *k_pe, int64_t k_pe_stride, const int64_t *slot_mapping,
                                const void *q_nope, int64_t qn_stride_b, int64_t qn_stride_h, const void *q_pe,
                                int64_t qp_stride_b, int64_t qp_stride_h, void *out, int32_t num_heads,
                                const int32_t *block_table, int64_t bt_stride, int32_t max_blocks_per_seq,
                                const int32_t *seq_lens, int32_t batch, int32_t max_seq_len, float scale,
                                int32_t partition_size, void *workspace, int64_t workspace_bytes, void *stream);

/* The two MLA decode calls with a per-head attention sink: sinks[h] (fp32,
 * device memory, one per query head, natural-log units like the scaled
 * scores; -inf = none) is one more logit in head h's softmax whose value
 * vector is zero, so o[b, h] = sum_t e^(s_t) c_t / (sum_t e^(s_t) + e^(sinks[h]))
 * and a zero-length sequence still gives zeros. Otherwise the arguments and
 * behaviour of wkv_paged_decode_mla / wkv_append_paged_decode_mla. Replaces
 * the learned per-head sink of the reference's shared-KV MQA attention
 * (wavelet/trainer/models/deepseek_v4/attention.py:703 declares it, :89-95
 * and :763 add it to the softmax), which its MLA decode backend must honour. */
int wkv_paged_decode_mla_sinks(const wkv_mla_cache_t *cache, const void *q_nope, int64_t qn_stride_b,
                               int64_t qn_stride_h, const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h,
                               void *out, int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                               int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                               int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                               int64_t workspace_bytes, const float *sinks, void *stream);

int wkv_append_paged_decode_mla_sinks(const wkv_mla_cache_t *cache, const void *kv_c, int64_t kv_c_stride,
                                      const void *k_pe, int64_t k_pe_stride, const int64_t *slot_mapping,
                                      const void *q_nope, int64_t qn_stride_b, int64_t qn_stride_h,
                                      const void *q_pe, int64_t qp_stride_b, int64_t qp_stride_h, void *out,
                                      int32_t num_heads, const int32_t *block_table, int64_t bt_stride,
                                      int32_t max_blocks_per_seq, const int32_t *seq_lens, int32_t batch,
                                      int32_t max_seq_len, float scale, int32_t partition_size, void *workspace,
                                      int64_t workspace_bytes, const float *sinks, void *stream);

/* ---- measurement --------------------------------------------------------
 * Read `bytes` (a multiple of 16) of device memory at `buf` once, with
 * `blocks` workgroups of 256 threads streaming 16-byte loads, and discard
 * it: the practical HBM read ceiling a benchmark sets beside a kernel's
 * achieved bandwidth. sink: `blocks` uint32 of device memory the kernel may
 * write (it does not, for any data but one 1-in-2^32 checksum). No reference
 * counterpart: a measuring aid of this library. */
int wkv_hbm_read_probe(const void *buf, int64_t bytes, int32_t blocks, uint32_t *sink, void *stream);

/* ---- misc ---------------------------------------------------------------- */
const char *wkv_last_error(void);
int wkv_version(void);

#ifdef __cplusplus
}
#endif
#endif /* WKV_H */
