/*
 * damendaemon_amd — C ABI of the MI355X (gfx950) paged-attention hot path.
 *
 * Conventions (mirroring the reference's ctypes-loaded native libraries,
 * damendaemon/native_q4.py:9-47):
 *   - every entry point returns int: 0 on success, a DD_E* code otherwise;
 *     dd_error_string() names the code;
 *   - buffers are plain device pointers owned by the caller (PyTorch);
 *     the library never allocates device memory;
 *   - `stream` is a hipStream_t passed as void* (NULL = legacy default);
 *     every launch is asynchronous on that stream and no entry point
 *     synchronises, so all of them can be recorded into a HIP graph;
 *   - dtype codes are DD_F32 / DD_F16 / DD_BF16 / DD_I8.
 *
 * KV page layout (damendaemon/paged.py:31-34): one layer's cache is
 * (2, capacity, kv_heads, page_size, dim); K and V are the two planes.
 * A slotted (non-paged) cache is (slots, kv_heads, context, dim)
 * (damendaemon/kernels.py:152-154).
 */
#ifndef DAMENDAEMON_AMD_H
#define DAMENDAEMON_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DD_ABI_VERSION 5

enum dd_dtype { DD_F32 = 0, DD_F16 = 1, DD_BF16 = 2, DD_I8 = 3 };

enum dd_error {
  DD_OK = 0,
  DD_EINVAL = 1,       /* bad shape, dtype or argument combination */
  DD_EUNSUPPORTED = 2, /* valid request this build has no kernel for */
  DD_ELAUNCH = 3,      /* HIP launch error (hipGetLastError after launch) */
  DD_ESCRATCH = 4      /* caller scratch buffers too small */
};

/* ABI version; callers refuse a library whose version differs
 * (native_q4.py:12-15 does the same for the reference's Q4 library). */
int dd_abi_version(void);
const char *dd_error_string(int code);

/*
 * Split-KV size the decode kernel will use for a given maximum context
 * (page-table width * page size, or the slotted context).  The caller sizes
 * `partial` as (batch*heads, splits, dim) fp32 and `lse` as
 * (batch*heads, splits) fp32 from it.  Replaces the host-side split choice
 * of damendaemon/kernels.py:231-236 (BLOCK/splits).
 * Returns the number of splits (>=1), or -DD_EINVAL for bad arguments;
 * *split_tokens receives the tokens per split (a multiple of 64).
 * `batch_kv` = batch * kv_heads.
 */
int dd_decode_splits(int max_context, int batch_kv, int *split_tokens);

/*
 * The same policy for a given head size and page dtype (no counterpart in
 * the reference, whose split choice ignores both): dd_decode_splits, except
 * that int8 pages take longer splits (about a third of the context, at most
 * 2,752 keys, while the launch keeps 512 workgroups), and that at head sizes
 * 160-256 with 16-bit pages, at least 128 (sequence, KV head) pairs and
 * fewer than four splits per resident workgroup (2 per CU), splits hold at
 * most 768 keys (a longer split is a long unit of work for those kernels,
 * and too few of them leave CUs idle at the end).
 * Same return values.
 */
int dd_decode_splits_for(int max_context, int batch_kv, int dim, int kv_dtype, int *split_tokens);

/*
 * Ragged decode attention, one query row per sequence.
 * Replaces damendaemon/kernels.py:213-267 (`attention` with the `_attention`
 * and `_merge` Triton kernels), paged (page_table != NULL) or slotted.
 *
 *   q          (batch, heads, dim)           q_dtype (F32/F16/BF16)
 *   k, v       paged: (capacity, kv_heads, page_size, dim) planes,
 *              slotted: (slots, kv_heads, context, dim)     kv_dtype
 *   k_scale,   int8 KV only: fp16 scales (..., page_size|context, dim/group)
 *   v_scale    with the same leading layout as k/v; NULL otherwise
 *   group      int8 channel group (a divisor of dim, multiple of 32 or ==dim)
 *   positions  int64 (batch,)  index of the current token; keys 0..pos
 *   slots      int64 (batch,)  slot / page-table row per sequence, or NULL
 *   page_table int32 (table_rows, table_width); NULL selects slotted mode;
 *              a slot outside [0, table_rows) reads no keys
 *   page_size  tokens per page (paged, a multiple of 16) or context (slotted)
 *   capacity   physical pages (paged) or slots (slotted): table entries or
 *              slot ids outside [0, capacity) are treated as unallocated
 *   window     0 = full causal history, else keys > pos - window only
 *   scale      softmax scale applied to q.k
 *   alibi      fp32 (heads,) slope per head or NULL       (kernels.py:160-161)
 *   rel_bias   fp32 (heads, rel_buckets) T5 bias or NULL   (kernels.py:162-167)
 *   rel_denom  log(max_distance / (rel_buckets/2))
 *   sinks      fp32 (heads,) sink logit per head or NULL   (kernels.py:170-175)
 *   out        (batch, heads, dim) q_dtype
 *   partial    fp32 (batch*heads, splits, dim)  scratch (unused if splits==1)
 *   lse        fp32 (batch*heads, splits)       scratch (unused if splits==1)
 *   splits, split_tokens  from dd_decode_splits() or dd_decode_splits_for()
 */
int dd_decode_attention(const void *q, int q_dtype, const void *k,
                        const void *v, int kv_dtype, const void *k_scale,
                        const void *v_scale, int group,
                        const int64_t *positions, const int64_t *slots,
                        const int32_t *page_table, int table_rows,
                        int table_width, int batch, int heads, int kv_heads, int dim,
                        int page_size, int64_t capacity, int window,
                        float scale,
                        const float *alibi, const float *rel_bias,
                        int rel_buckets, float rel_denom, const float *sinks,
                        void *out, float *partial, float *lse, int splits,
                        int split_tokens, void *stream);

/*
 * The two launches of dd_decode_attention, callable one at a time with the
 * same arguments: dd_decode_partials runs the split kernel (with splits==1
 * it writes `out` directly); dd_decode_merge runs the log-sum-exp combine
 * of kernels.py:191-210 (a no-op when splits==1).  Calling both in order
 * on one stream equals dd_decode_attention; they exist so a caller can
 * time or overlap the phases separately.
 */
int dd_decode_partials(const void *q, int q_dtype, const void *k,
                       const void *v, int kv_dtype, const void *k_scale,
                       const void *v_scale, int group,
                       const int64_t *positions, const int64_t *slots,
                       const int32_t *page_table, int table_rows,
                       int table_width, int batch, int heads, int kv_heads,
                       int dim, int page_size, int64_t capacity, int window,
                       float scale, const float *alibi, const float *rel_bias,
                       int rel_buckets, float rel_denom, const float *sinks,
                       void *out, float *partial, float *lse, int splits,
                       int split_tokens, void *stream);
int dd_decode_merge(const void *q, int q_dtype, const void *k, const void *v,
                    int kv_dtype, const void *k_scale, const void *v_scale,
                    int group, const int64_t *positions, const int64_t *slots,
                    const int32_t *page_table, int table_rows,
                    int table_width, int batch, int heads, int kv_heads,
                    int dim, int page_size, int64_t capacity, int window,
                    float scale, const float *alibi, const float *rel_bias,
                    int rel_buckets, float rel_denom, const float *sinks,
                    void *out, float *partial, float *lse, int splits,
                    int split_tokens, void *stream);

/*
 * dd_decode_attention without the partial / lse arguments, for callers that
 * cannot allocate device memory (code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The split scratch is a file-scope device array of
 * DD_STATIC_SCRATCH_FLOATS fp32 per GPU (32 MiB), held until the process
 * ends; batch*heads*splits*(dim+1) must fit in it (else DD_ESCRATCH, e.g.
 * at dim 128 about 65k (sequence, head, split) rows).  Calls share that
 * array per GPU: calls that overlap on one GPU race.  Allocates nothing.
 */
#define DD_STATIC_SCRATCH_FLOATS (8 * 1024 * 1024)
int dd_decode_attention_static(const void *q, int q_dtype, const void *k,
                               const void *v, int kv_dtype,
                               const void *k_scale, const void *v_scale,
                               int group, const int64_t *positions,
                               const int64_t *slots,
                               const int32_t *page_table, int table_rows,
                               int table_width, int batch, int heads,
                               int kv_heads, int dim, int page_size,
                               int64_t capacity, int window, float scale,
                               const float *alibi, const float *rel_bias,
                               int rel_buckets, float rel_denom,
                               const float *sinks, void *out, int splits,
                               int split_tokens, void *stream);

/*
 * Q8_0 KV codec (damendaemon/kv_quant.py:48-76), bit-exact with the
 * reference's torch arithmetic.  x / out: (rows, dim) in x_dtype/out_dtype
 * (F32/F16/BF16); q: (rows, dim) int8; scale: (rows, dim/group) fp16.
 */
int dd_quantize_q8(const void *x, int x_dtype, int64_t rows, int dim,
                   int group, void *q, void *scale, void *stream);
int dd_dequantize_q8(const void *q, const void *scale, int64_t rows, int dim,
                     int group, void *out, int out_dtype, void *stream);

/*
 * Ragged-batch packer (replaces the host list comprehensions of
 * damendaemon/paged.py:149-159 / batch.py:133-136, the segment ends of
 * paged.py:118-120 and the slot computation of kernels.py:279-281).
 * Inputs, int64 (n,): lengths, starts (tokens already cached), slots.
 * Outputs (bit-exact with the reference's Python arithmetic):
 *   cu_seqlens int64 (n+1), ends int64 (n) = cu_seqlens[1:]-1,
 *   context_lens int64 (n) = starts+lengths,
 *   positions/slot_ids int64 (total_tokens),
 *   slot_map int64 (total_tokens) = table[slot, pos/P]*P + pos%P (optional),
 *   cu_pages int32 (n+1) and gather_pages int32 (total_pages): the physical
 *   pages of each segment's whole history in logical order (optional).
 * total_tokens = sum(lengths) and total_pages = sum(ceil(context/P)) are
 * given by the caller (they size the outputs).
 */
int dd_pack_batch(const int64_t *lengths, const int64_t *starts,
                  const int64_t *slots, int n, int64_t total_tokens,
                  int64_t total_pages, const int32_t *page_table,
                  int table_rows, int table_width, int page_size,
                  int64_t *cu_seqlens, int64_t *ends, int64_t *context_lens,
                  int64_t *positions, int64_t *slot_ids, int64_t *slot_map,
                  int32_t *cu_pages, int32_t *gather_pages, void *stream);

/*
 * Write new K/V rows (tokens, kv_heads, dim) into their page slots
 * (slot_map from dd_pack_batch; negative entries are skipped): the page
 * write half of damendaemon/kernels.py:312-319 without the rotation.
 * elem_bytes is the cache element size (K/V already in the cache dtype).
 */
int dd_store_kv_pages(const void *key, const void *value, int elem_bytes,
                      const int64_t *slot_map, int64_t tokens, int kv_heads,
                      int dim, int page_size, int64_t capacity, void *cache_k,
                      void *cache_v, void *stream);

/*
 * Same, quantising each (token, KV head, group) row to Q8_0 on the way into
 * int8 pages with fp16 scale rows (..., page, dim/group).  No reference
 * counterpart: the reference's Q8_0 cache (kv_quant.py:79-107) is dense.
 */
int dd_store_kv_pages_q8(const void *key, const void *value, int dtype,
                         const int64_t *slot_map, int64_t tokens,
                         int kv_heads, int dim, int group, int page_size,
                         int64_t capacity, void *cache_k, void *cache_v,
                         void *k_scale, void *v_scale, void *stream);

/*
 * Page gather (restore=0) or restore (restore=1) of one slot's first
 * `tokens` tokens between a paged layer (2, capacity, heads, page, dim) and
 * a dense (2, heads, tokens, dim) snapshot; replaces `_copy` of
 * damendaemon/paged_kernels.py:8-47.  Page tails are never touched.
 */
int dd_copy_pages(void *cache, const int32_t *table, int table_rows,
                  int table_width, void *dense, int elem_bytes, int64_t slot,
                  int64_t tokens, int64_t capacity, int heads, int page,
                  int dim, int restore, void *stream);

/*
 * Rotary embedding (+ optional QK RMS norm) of a packed (tokens,
 * (heads + 2*kv_heads)*dim) projection, writing queries to `query`
 * (tokens, heads, 1, dim) and rotated keys / raw values into the cache at
 * each token's position; replaces `_rope_batch` of
 * damendaemon/kernels.py:271-340.  page_table NULL = slotted cache of
 * context `cache_len`; otherwise cache_len is the page size.  key_out /
 * value_out (tokens, kv_heads, dim), optional, receive the dense copies of
 * the `materialize` path.
 */
int dd_rope_batch(const void *qkv, int qkv_dtype, const void *cos,
                  const void *sin, int cos_dtype, int rotary_dim,
                  const int64_t *positions, const int64_t *slots,
                  int64_t tokens, int heads, int kv_heads, int dim,
                  const void *q_norm, const void *k_norm, int norm_dtype,
                  float eps, int precise, const int32_t *page_table,
                  int table_rows, int table_width, void *query, void *cache_k,
                  void *cache_v, int cache_dtype, int64_t capacity,
                  int cache_len, void *key_out, void *value_out,
                  void *stream);

/*
 * Chunked-prefill attention over the paged cache (the attention half of
 * damendaemon/paged.py:97-111: copy_pages gather + lower-right causal SDPA
 * of qwen2.py:754-770), without materialising the gathered K/V.
 *   q, out        (T, heads, dim) packed query / output rows, bf16, fp16 or
 *                 fp32 (bf16/fp16 at 64/128/256 take the 16-bit MFMA kernel;
 *                 fp32, and 16-bit at other head sizes, the fp32-arithmetic
 *                 MFMA kernel when dim is a multiple of 16 up to 256; other
 *                 head sizes up to 256 in steps of 4 a vector-ALU kernel)
 *   k, v          (capacity, kv_heads, page_size, dim) pages holding every
 *                 segment's history including the chunk itself
 *   cu_seqlens    int64 (n+1), context_lens int64 (n) = start+len, slots int64 (n)
 *   max_len       the longest segment (sizes the grid)
 *   max_context   the longest start+len (informational; any length)
 *   scale         any finite value (non-finite: DD_EINVAL); 0 gives uniform
 *                 weights over each row's allowed keys, as SDPA does
 *   plan          NULL, or the device copy of dd_prefill_plan's output for
 *                 these same segments, plan_len = its workgroup count G:
 *                 the schedule; NULL uses a fixed XCD-aware order
 *   flags         device int32 workspace of dd_prefill_flag_count(...)
 *                 entries (NULL allowed when that count is 0).  The bf16
 *                 kernel at dim 64/128 multiplies V in fp16; a work item
 *                 whose output shows V outside fp16's normal range flags
 *                 itself there and a second launch recomputes it in fp32
 *                 arithmetic.  Overwritten on every call; needs no clearing.
 * Row j of segment i attends keys 0 .. start_i + j (and > that - window).
 */
int dd_prefill_attention(const void *q, const void *k, const void *v,
                         int dtype, const int64_t *cu_seqlens,
                         const int64_t *context_lens, const int64_t *slots,
                         int n, int max_len, int max_context,
                         const int32_t *page_table,
                         int table_rows, int table_width, int heads,
                         int kv_heads, int dim, int page_size,
                         int64_t capacity, int window, float scale,
                         const int32_t *plan, int plan_len, int32_t *flags,
                         void *out, void *stream);

/*
 * dd_prefill_attention in two launches (same arguments): phase 1 runs the
 * attention kernel, phase 2 the exact re-run of the work items the bf16
 * kernel flagged (a no-op for calls without a flags workspace); 3 = both,
 * as dd_prefill_attention.  For timing the attention kernel on its own.
 */
int dd_prefill_attention_phase(const void *q, const void *k, const void *v,
                               int dtype, const int64_t *cu_seqlens,
                               const int64_t *context_lens, const int64_t *slots,
                               int n, int max_len, int max_context,
                               const int32_t *page_table, int table_rows,
                               int table_width, int heads, int kv_heads,
                               int dim, int page_size, int64_t capacity,
                               int window, float scale, const int32_t *plan,
                               int plan_len, int32_t *flags, void *out,
                               int phase, void *stream);

/*
 * Entries of dd_prefill_attention's flags workspace for these arguments (0
 * when the call needs none); negative = -DD_E*.  No reference counterpart:
 * the exactness guard of the fp16 P.V product of bf16 pages.
 */
int dd_prefill_flag_count(int n, int max_len, int heads, int kv_heads,
                          int dim, int dtype);

/*
 * Host-side schedule for dd_prefill_attention (no reference counterpart:
 * the reference runs one SDPA per segment, paged.py:97-111).  lengths,
 * starts and slots are HOST int64 arrays (n), the same segments as the
 * call's device metadata.  Writes the schedule to plan (host int32,
 * DD_PREFILL_PLAN_INTS per entry, capacity entries): each entry holds a
 * work item (-1: none), its segment's first packed token, length, start
 * and slot, and the number of rounds R (the same in every entry).  Entry
 * r * G + b is round r of workgroup b; G = (entries returned) / R is the
 * plan_len dd_prefill_attention takes.  workgroups <= 0: one item per
 * workgroup (R = 1); otherwise at most that many workgroups, each running
 * its items one after another (give the number of CUs: one workgroup fits
 * per CU).  Returns the number of entries; with plan == NULL or too small a
 * capacity it only returns that number.  Negative = -DD_E*.
 */
#define DD_PREFILL_PLAN_INTS 8
int dd_prefill_plan(const int64_t *lengths, const int64_t *starts,
                    const int64_t *slots, int n, int heads, int kv_heads,
                    int dim, int window, int workgroups, int32_t *plan,
                    int capacity);

/*
 * Tile geometry of dd_prefill_attention for head size dim: (query row,
 * head) columns per workgroup and keys per tile (host-side query).
 */
int dd_prefill_geometry(int dim, int *columns, int *keys_per_tile);

/*
 * Index plans of damendaemon/cache_indices.py:24-80 (DeepSeek-style
 * windowed + compressed-block attention), int64, -1 = padding.
 * dd_prefill_indices: out (query_stop - query_start, min(window, seq_len)
 *   + (ratio ? query_stop / ratio : 0)).
 * dd_ring_decode_indices: positions int64 (rows); out (rows, window +
 *   compressed) with compressed = (max(positions) + 1) / ratio (0 without
 *   a ratio), computed by the caller.
 */
int dd_prefill_indices(int64_t seq_len, int window, int ratio,
                       int64_t query_start, int64_t query_stop, int64_t *out,
                       void *stream);
int dd_ring_decode_indices(const int64_t *positions, int64_t rows, int window,
                           int ratio, int compressed, int64_t *out,
                           void *stream);

#ifdef __cplusplus
}
#endif

#endif /* DAMENDAEMON_AMD_H */
