// C entry points of the decode path.  The kernels are instantiated per
// dtype pair in decode_<dtype>.hip so the library compiles in parallel.
#include "decode_impl.h"

#include <mutex>

using namespace dd_decode;

extern template int dd_decode::dispatch_d<DD_BF16, DD_BF16>(const DecodeParams &, int, hipStream_t, int);
extern template int dd_decode::dispatch_d<DD_F16, DD_F16>(const DecodeParams &, int, hipStream_t, int);
extern template int dd_decode::dispatch_d<DD_F32, DD_F32>(const DecodeParams &, int, hipStream_t, int);
extern template int dd_decode::dispatch_d<DD_I8, DD_BF16>(const DecodeParams &, int, hipStream_t, int);
extern template int dd_decode::dispatch_d<DD_I8, DD_F16>(const DecodeParams &, int, hipStream_t, int);

#ifndef DD_DECODE_MIN_WG
#define DD_DECODE_MIN_WG 512
#endif

extern "C" int dd_decode_splits(int max_context, int batch_kv, int *split_tokens) {
  if (max_context <= 0 || batch_kv <= 0) return -DD_EINVAL;
  // About six splits over the longest possible context, 256..2048 keys each
  // (a multiple of 64): long enough that the per-split setup and the merge
  // stay small, short enough that ragged batches balance over the 256 CUs.
  // Splits are dispatched split-major, so unused trailing splits cost one
  // early exit.  (Measured on 64 sequences of U[512, 8192] keys: 1408-key
  // splits beat 1024 by 2 % for bf16 pages and 5 % for int8 pages; 2048 is
  // best for 16 x 32768.  With few (sequence, KV head) pairs, e.g. 64 x 1 KV
  // head, at least 512 workgroups: 34 us vs 41 us at 16 heads per KV head.)
  long st = dd_cdiv(dd_cdiv(max_context, 6), 64) * 64;
  st = st < 256 ? 256 : (st > 2048 ? 2048 : st);
  // Few (sequence, KV head) pairs: more splits, so that the launch has at
  // least DD_DECODE_MIN_WG workgroups.
  const long want = dd_cdiv(DD_DECODE_MIN_WG, batch_kv);
  if (dd_cdiv(max_context, st) < want) {
    const long s2 = dd_cdiv(dd_cdiv(max_context, want), 64) * 64;
    st = s2 < 256 ? 256 : (s2 < st ? s2 : st);
  }
  if (split_tokens) *split_tokens = (int)st;
  return (int)dd_cdiv(max_context, st);
}

extern "C" int dd_decode_splits_for(int max_context, int batch_kv, int dim, int kv_dtype, int *split_tokens) {
  int st = 0;
  const int n = dd_decode_splits(max_context, batch_kv, &st);
  if (n <= 0) return n;
  // int8 pages carry about half the bytes per key, so a split of the same
  // keys is half the work: about a third of the context per split, at most
  // 2,752 keys, while the launch keeps DD_DECODE_MIN_WG workgroups (C3:
  // 2,752-key splits 0.646-0.651 of 8 TB/s vs 0.635-0.637 with 1,408; the
  // reference's group-32 scales 0.587 vs 0.574).
  if (kv_dtype == DD_I8) {
    long st8 = dd_cdiv(dd_cdiv(max_context, 3), 64) * 64;
    if (st8 > 2752) st8 = 2752;
    if (st8 > st && (long)batch_kv * dd_cdiv(max_context, st8) >= DD_DECODE_MIN_WG) {
      if (split_tokens) *split_tokens = (int)st8;
      return (int)dd_cdiv(max_context, st8);
    }
  }
  // Head sizes 160-256 on 16-bit pages, many (sequence, KV head) pairs and
  // few splits per resident workgroup: a longer split is a long unit of work
  // for those kernels and too few of them leave CUs idle at the end, so
  // splits of at most 768 keys.  Measured on 64 sequences of U[512, 8192]
  // keys, bf16, 4 KV heads, with 768 / 1,024 / 1,408-key splits: D 256 182 /
  // 186 / 195 us, D 224 175 / 180 / 186 us, D 160 125 / 127 / 131 us.  8 KV
  // heads (not capped by this rule): 342 us either way at D 256; 16 x 32768
  // keys on 2 KV heads keeps its 2,048 (174 us vs 183 us with 1,024).
  constexpr long kSlots = 2L * 256;   // about two resident workgroups per CU
  if (dim >= 160 && (kv_dtype == DD_BF16 || kv_dtype == DD_F16) && batch_kv >= 128 &&
      (long)batch_kv * n < 4 * kSlots && st > 768) {
    if (split_tokens) *split_tokens = 768;
    return (int)dd_cdiv(max_context, 768);
  }
  if (split_tokens) *split_tokens = st;
  return n;
}

static int decode_entry(int phase, const void *q, int q_dtype, const void *k, const void *v, int kv_dtype,
                                   const void *k_scale, const void *v_scale, int group,
                                   const int64_t *positions, const int64_t *slots, const int32_t *page_table,
                                   int table_rows, int table_width, int batch, int heads, int kv_heads, int dim, int page_size,
                                   int64_t capacity, int window, float scale, const float *alibi, const float *rel_bias,
                                   int rel_buckets, float rel_denom, const float *sinks, void *out,
                                   float *partial, float *lse, int splits, int split_tokens, void *stream) {
  if (!q || !k || !v || !positions || !out || batch < 0 || capacity <= 0 || heads <= 0 || kv_heads <= 0 ||
      heads % kv_heads || page_size <= 0 || splits <= 0 || split_tokens <= 0 || split_tokens % 64)
    return DD_EINVAL;
  if (batch == 0) return DD_OK;
  if (splits > 1 && (!partial || !lse)) return DD_ESCRATCH;
  DecodeParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.ks = (const unsigned short *)k_scale;
  p.vs = (const unsigned short *)v_scale;
  p.pos = positions;
  p.slots = slots;
  p.table = page_table;
  p.out = out;
  p.part = partial;
  p.lse = lse;
  p.alibi = alibi;
  p.rel = rel_bias;
  p.sinks = sinks;
  p.B = batch;
  p.H = heads;
  p.KH = kv_heads;
  p.G = heads / kv_heads;
  p.DR = dim;
  p.gsub = 1;
  p.table_w = table_width;
  p.table_rows = table_rows;
  p.page = page_size;
  p.paged = page_table != nullptr;
  p.window = window > 0 ? window : 0;
  p.splits = splits;
  p.split_tokens = split_tokens;
  p.rel_buckets = rel_bias ? rel_buckets : 0;
  p.rel_denom = rel_denom;
  p.scale_log2 = scale * kLog2e;
  p.group = group;
  p.ngroups = group > 0 ? dim / group : 0;
  if (p.paged) {
    if (table_width <= 0 || page_size % 16) return DD_EUNSUPPORTED;
    p.ctx_limit = table_width * page_size;
    p.chunk_shift = 0;
    while ((16 << p.chunk_shift) < page_size) ++p.chunk_shift;
    if ((16 << p.chunk_shift) != page_size) return DD_EUNSUPPORTED;
  } else {
    p.ctx_limit = page_size;
  }
  if ((long)p.ctx_limit > (long)splits * split_tokens) return DD_ESCRATCH;
  p.capacity = capacity;
  hipStream_t s = (hipStream_t)stream;
  if (kv_dtype == DD_I8) {
    if (!k_scale || !v_scale || group <= 0 || dim % group || (group % 32 && group != dim)) return DD_EINVAL;
    if (q_dtype == DD_BF16) return dispatch_d<DD_I8, DD_BF16>(p, dim, s, phase);
    if (q_dtype == DD_F16) return dispatch_d<DD_I8, DD_F16>(p, dim, s, phase);
    return DD_EUNSUPPORTED;
  }
  if (q_dtype != kv_dtype) return DD_EINVAL;
  if (kv_dtype == DD_BF16) return dispatch_d<DD_BF16, DD_BF16>(p, dim, s, phase);
  if (kv_dtype == DD_F16) return dispatch_d<DD_F16, DD_F16>(p, dim, s, phase);
  if (kv_dtype == DD_F32) return dispatch_d<DD_F32, DD_F32>(p, dim, s, phase);
  return DD_EUNSUPPORTED;
}

extern "C" int dd_decode_attention(const void *q, int q_dtype, const void *k, const void *v, int kv_dtype,
                                   const void *k_scale, const void *v_scale, int group,
                                   const int64_t *positions, const int64_t *slots, const int32_t *page_table,
                                   int table_rows, int table_width, int batch, int heads, int kv_heads, int dim, int page_size,
                                   int64_t capacity, int window, float scale, const float *alibi, const float *rel_bias,
                                   int rel_buckets, float rel_denom, const float *sinks, void *out,
                                   float *partial, float *lse, int splits, int split_tokens, void *stream) {
  return decode_entry(3, q, q_dtype, k, v, kv_dtype, k_scale, v_scale, group, positions, slots, page_table, table_rows, table_width, batch, heads, kv_heads, dim, page_size, capacity, window, scale, alibi, rel_bias, rel_buckets, rel_denom, sinks, out, partial, lse, splits, split_tokens, stream);
}

extern "C" int dd_decode_partials(const void *q, int q_dtype, const void *k, const void *v, int kv_dtype,
                                   const void *k_scale, const void *v_scale, int group,
                                   const int64_t *positions, const int64_t *slots, const int32_t *page_table,
                                   int table_rows, int table_width, int batch, int heads, int kv_heads, int dim, int page_size,
                                   int64_t capacity, int window, float scale, const float *alibi, const float *rel_bias,
                                   int rel_buckets, float rel_denom, const float *sinks, void *out,
                                   float *partial, float *lse, int splits, int split_tokens, void *stream) {
  return decode_entry(1, q, q_dtype, k, v, kv_dtype, k_scale, v_scale, group, positions, slots, page_table, table_rows, table_width, batch, heads, kv_heads, dim, page_size, capacity, window, scale, alibi, rel_bias, rel_buckets, rel_denom, sinks, out, partial, lse, splits, split_tokens, stream);
}

extern "C" int dd_decode_merge(const void *q, int q_dtype, const void *k, const void *v, int kv_dtype,
                                   const void *k_scale, const void *v_scale, int group,
                                   const int64_t *positions, const int64_t *slots, const int32_t *page_table,
                                   int table_rows, int table_width, int batch, int heads, int kv_heads, int dim, int page_size,
                                   int64_t capacity, int window, float scale, const float *alibi, const float *rel_bias,
                                   int rel_buckets, float rel_denom, const float *sinks, void *out,
                                   float *partial, float *lse, int splits, int split_tokens, void *stream) {
  return decode_entry(2, q, q_dtype, k, v, kv_dtype, k_scale, v_scale, group, positions, slots, page_table, table_rows, table_width, batch, heads, kv_heads, dim, page_size, capacity, window, scale, alibi, rel_bias, rel_buckets, rel_denom, sinks, out, partial, lse, splits, split_tokens, stream);
}

// ---- allocation-free variant ----------------------------------------------
// The split partials and log-sum-exps live in this file-scope device array
// instead of caller buffers.  Each GPU the library runs on holds its own copy
// (DD_STATIC_SCRATCH_FLOATS fp32, 32 MiB) until the process ends.  Every
// call on a GPU shares that GPU's copy: calls that overlap on one GPU (two
// streams, or two threads) race.  No element needs clearing between calls:
// the merge reads only the splits that the split kernel of the same call
// wrote for each (sequence, head).
static __device__ __align__(256) float scratch[DD_STATIC_SCRATCH_FLOATS];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
float *g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device, set once

// Device address of this GPU's `scratch`, looked up on the first call on
// each device with that device current (the array's host-side name is not a
// device address).  nullptr on failure.
float *static_scratch(hipStream_t stream) {
  int dev = -1;
  if (hipStreamGetDevice(stream, &dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev]) return g_scratch_ptr[dev];
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) return nullptr;
  if (cur != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
  void *addr = nullptr;
  const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
  if (cur != dev) (void)hipSetDevice(cur);
  if (e != hipSuccess || !addr) return nullptr;
  g_scratch_ptr[dev] = (float *)addr;
  return g_scratch_ptr[dev];
}

}  // namespace

extern "C" int dd_decode_attention_static(const void *q, int q_dtype, const void *k, const void *v, int kv_dtype,
                                          const void *k_scale, const void *v_scale, int group,
                                          const int64_t *positions, const int64_t *slots,
                                          const int32_t *page_table, int table_rows, int table_width, int batch,
                                          int heads, int kv_heads, int dim, int page_size, int64_t capacity,
                                          int window, float scale, const float *alibi, const float *rel_bias,
                                          int rel_buckets, float rel_denom, const float *sinks, void *out,
                                          int splits, int split_tokens, void *stream) {
  if (batch < 0 || heads <= 0 || dim <= 0 || splits <= 0) return DD_EINVAL;
  // partials (batch*heads, splits, dim) then lse (batch*heads, splits)
  const long rows = (long)batch * heads * splits;
  const long need = rows * (dim + 1L);
  if (splits > 1 && need > (long)DD_STATIC_SCRATCH_FLOATS) return DD_ESCRATCH;
  float *part = nullptr, *lse = nullptr;
  if (splits > 1 && batch > 0) {
    float *base = static_scratch((hipStream_t)stream);
    if (!base) return DD_ELAUNCH;
    part = base;
    lse = base + rows * dim;
  }
  return decode_entry(3, q, q_dtype, k, v, kv_dtype, k_scale, v_scale, group, positions, slots, page_table,
                      table_rows, table_width, batch, heads, kv_heads, dim, page_size, capacity, window, scale,
                      alibi, rel_bias, rel_buckets, rel_denom, sinks, out, part, lse, splits, split_tokens, stream);
}
