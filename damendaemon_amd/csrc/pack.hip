// Ragged-batch packer and K/V page writer for gfx950.
//
// The packer replaces the host-side list comprehensions of
// damendaemon/paged.py:149-159 (and batch.py:133-136), the segment ends of
// paged.py:118-120 and the in-kernel slot computation of kernels.py:279-281.
// For n segments (slot_i, start_i, len_i) it writes, bit-exactly:
//   cu_seqlens[i]  = len_0 + ... + len_{i-1}          (n+1 entries)
//   ends[i]        = cu_seqlens[i+1] - 1
//   context[i]     = start_i + len_i
//   positions[t]   = start_i + (t - cu_seqlens[i])    for t in segment i
//   slot_ids[t]    = slot_i
//   slot_map[t]    = table[slot_i, pos / P] * P + pos % P
//   cu_pages[i]    = sum_{j<i} ceil(context_j / P)    (n+1 entries)
//   gather[k]      = table[slot_i, k - cu_pages[i]]   (physical pages of each
//                    segment's whole history, in logical order)
// Segment-level prefix sums run in one workgroup (wave-level scans through
// LDS); the per-token and per-page outputs are filled by a grid of
// workgroups that locate their segment by binary search in the prefix.
#include "common.h"
#include "q8.h"

namespace {

constexpr int kScanThreads = 1024;

// Inclusive scan of one int64 per thread across the workgroup.
DD_DEV long block_scan(long x, long *s_tmp) {
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const long y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  if (lane == 63) s_tmp[w] = x;
  __syncthreads();
  if (w == 0) {
    long t = lane < (int)(blockDim.x >> 6) ? s_tmp[lane] : 0;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const long y = __shfl_up(t, off, 64);
      if (lane >= off) t += y;
    }
    if (lane < (int)(blockDim.x >> 6)) s_tmp[lane] = t;
  }
  __syncthreads();
  if (w > 0) x += s_tmp[w - 1];
  __syncthreads();
  return x;
}

__global__ __launch_bounds__(kScanThreads) void scan_kernel(const int64_t *lengths, const int64_t *starts, int n,
                                                            int page, int64_t *cu, int64_t *ends,
                                                            int64_t *context, int32_t *cu_pages) {
  __shared__ long s_tmp[16];
  __shared__ long s_carry[2];
  if (threadIdx.x == 0) {
    s_carry[0] = 0;
    s_carry[1] = 0;
    cu[0] = 0;
    if (cu_pages) cu_pages[0] = 0;
  }
  __syncthreads();
  for (int base = 0; base < n; base += kScanThreads) {
    const int i = base + threadIdx.x;
    const long len = i < n ? lengths[i] : 0;
    const long ctx = i < n ? starts[i] + len : 0;
    const long np = (ctx + page - 1) / page;
    const long c0 = s_carry[0], c1 = s_carry[1];
    __syncthreads();
    const long inc_t = block_scan(len, s_tmp) + c0;
    const long inc_p = block_scan(i < n ? np : 0, s_tmp) + c1;
    if (i < n) {
      cu[i + 1] = inc_t;
      ends[i] = inc_t - 1;
      context[i] = ctx;
      if (cu_pages) cu_pages[i + 1] = (int32_t)inc_p;
    }
    if (threadIdx.x == kScanThreads - 1) {
      s_carry[0] = inc_t;
      s_carry[1] = inc_p;
    }
    __syncthreads();
  }
}

// Index of the segment whose [cu[i], cu[i+1]) holds t (cu ascending).
template <typename T>
DD_DEV int find_segment(const T *cu, int n, long t) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if ((long)cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

__global__ __launch_bounds__(256) void fill_tokens_kernel(const int64_t *cu, const int64_t *starts,
                                                          const int64_t *slots, int n, long total,
                                                          const int32_t *table, int table_rows, int table_w,
                                                          int page, int64_t *positions, int64_t *slot_ids,
                                                          int64_t *slot_map) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  int i = find_segment(cu, n, t);
  // empty segments share their cu value with the next one: skip forward
  while (i + 1 < n && cu[i + 1] <= t) ++i;
  const long pos = starts[i] + (t - cu[i]);
  const long slot = slots[i];
  positions[t] = pos;
  slot_ids[t] = slot;
  if (slot_map) {
    const long entry = pos / page;
    long phys = -1;
    if (slot >= 0 && slot < table_rows && entry < table_w) phys = table[slot * table_w + entry];
    slot_map[t] = phys * page + pos % page;
  }
}

__global__ __launch_bounds__(256) void fill_pages_kernel(const int32_t *cu_pages, const int64_t *slots, int n,
                                                         long total, const int32_t *table, int table_rows,
                                                         int table_w, int32_t *gather) {
  const long k = (long)blockIdx.x * 256 + threadIdx.x;
  if (k >= total) return;
  int i = find_segment(cu_pages, n, k);
  while (i + 1 < n && cu_pages[i + 1] <= k) ++i;
  const long slot = slots[i];
  const long entry = k - cu_pages[i];
  gather[k] = (slot >= 0 && slot < table_rows && entry < table_w) ? table[slot * table_w + entry] : -1;
}

// One thread moves 16 bytes of one (token, KV head) row into its page slot.
__global__ __launch_bounds__(256) void store_pages_kernel(const char *key, const char *value,
                                                          const int64_t *slot_map, long tokens, int kv_heads,
                                                          int row_bytes, int page, long capacity, char *ck,
                                                          char *cv) {
  const int per_row = row_bytes / 16;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const long per_token = (long)kv_heads * per_row;
  if (g >= tokens * per_token) return;
  const long t = g / per_token;
  const int rem = (int)(g - t * per_token);
  const int kh = rem / per_row;
  const int chunk = rem - kh * per_row;
  const long s = slot_map[t];
  if (s < 0) return;
  const long phys = s / page;
  if (phys >= capacity) return;
  const long dst = ((phys * kv_heads + kh) * page + (s % page)) * (long)row_bytes + 16L * chunk;
  const long src = (t * kv_heads + kh) * (long)row_bytes + 16L * chunk;
  *(u32x4 *)(ck + dst) = *(const u32x4 *)(key + src);
  *(u32x4 *)(cv + dst) = *(const u32x4 *)(value + src);
}

// One thread quantises one (token, KV head, channel group) of K and of V
// straight into int8 pages and their fp16 scale rows.
template <int DT>
__global__ __launch_bounds__(256) void store_pages_q8_kernel(const void *key, const void *value,
                                                             const int64_t *slot_map, long tokens, int kv_heads,
                                                             int dim, int group, int page, long capacity,
                                                             signed char *ck, signed char *cv,
                                                             unsigned short *ks, unsigned short *vs) {
  const int ng = dim / group;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const long per_token = (long)kv_heads * ng;
  if (g >= tokens * per_token) return;
  const long t = g / per_token;
  const int rem = (int)(g - t * per_token);
  const int kh = rem / ng;
  const int gi = rem - kh * ng;
  const long s = slot_map[t];
  if (s < 0 || s / page >= capacity) return;
  const long row = ((s / page) * kv_heads + kh) * page + (s % page);
  const long src = (t * kv_heads + kh) * (long)dim + (long)gi * group;
  const long dst = row * dim + (long)gi * group;
  ks[row * ng + gi] = q8_group<DT>(key, src, group, ck + dst);
  vs[row * ng + gi] = q8_group<DT>(value, src, group, cv + dst);
}

}  // namespace

extern "C" int dd_pack_batch(const int64_t *lengths, const int64_t *starts, const int64_t *slots, int n,
                             int64_t total_tokens, int64_t total_pages, const int32_t *page_table,
                             int table_rows, int table_width, int page_size, int64_t *cu_seqlens, int64_t *ends,
                             int64_t *context_lens, int64_t *positions, int64_t *slot_ids, int64_t *slot_map,
                             int32_t *cu_pages, int32_t *gather_pages, void *stream) {
  if (n < 0 || total_tokens < 0 || page_size <= 0 || !cu_seqlens) return DD_EINVAL;
  if (n > 0 && (!lengths || !starts || !slots || !ends || !context_lens)) return DD_EINVAL;
  if ((slot_map || gather_pages) && (!page_table || table_width <= 0)) return DD_EINVAL;
  if (gather_pages && !cu_pages) return DD_EINVAL;
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(scan_kernel, dim3(1), dim3(kScanThreads), 0, s, lengths, starts, n, page_size, cu_seqlens,
                     ends, context_lens, cu_pages);
  DD_LAUNCH_CHECK();
  if (n > 0 && total_tokens > 0) {
    if (!positions || !slot_ids) return DD_EINVAL;
    hipLaunchKernelGGL(fill_tokens_kernel, dim3((unsigned)dd_cdiv(total_tokens, 256)), dim3(256), 0, s,
                       cu_seqlens, starts, slots, n, (long)total_tokens, page_table, table_rows, table_width,
                       page_size, positions, slot_ids, slot_map);
    DD_LAUNCH_CHECK();
  }
  if (n > 0 && gather_pages && total_pages > 0) {
    hipLaunchKernelGGL(fill_pages_kernel, dim3((unsigned)dd_cdiv(total_pages, 256)), dim3(256), 0, s, cu_pages,
                       slots, n, (long)total_pages, page_table, table_rows, table_width, gather_pages);
    DD_LAUNCH_CHECK();
  }
  return DD_OK;
}

extern "C" int dd_store_kv_pages(const void *key, const void *value, int elem_bytes, const int64_t *slot_map,
                                 int64_t tokens, int kv_heads, int dim, int page_size, int64_t capacity,
                                 void *cache_k, void *cache_v, void *stream) {
  if (!key || !value || !slot_map || !cache_k || !cache_v || tokens < 0 || kv_heads <= 0 || dim <= 0 ||
      page_size <= 0 || capacity <= 0 || (elem_bytes != 1 && elem_bytes != 2 && elem_bytes != 4))
    return DD_EINVAL;
  const int row_bytes = dim * elem_bytes;
  if (row_bytes % 16) return DD_EUNSUPPORTED;
  const long work = (long)tokens * kv_heads * (row_bytes / 16);
  if (work == 0) return DD_OK;
  hipLaunchKernelGGL(store_pages_kernel, dim3((unsigned)dd_cdiv(work, 256)), dim3(256), 0, (hipStream_t)stream,
                     (const char *)key, (const char *)value, slot_map, (long)tokens, kv_heads, row_bytes,
                     page_size, (long)capacity, (char *)cache_k, (char *)cache_v);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

extern "C" int dd_store_kv_pages_q8(const void *key, const void *value, int dtype, const int64_t *slot_map,
                                    int64_t tokens, int kv_heads, int dim, int group, int page_size,
                                    int64_t capacity, void *cache_k, void *cache_v, void *k_scale, void *v_scale,
                                    void *stream) {
  if (!key || !value || !slot_map || !cache_k || !cache_v || !k_scale || !v_scale || tokens < 0 ||
      kv_heads <= 0 || dim <= 0 || group <= 0 || dim % group || page_size <= 0 || capacity <= 0)
    return DD_EINVAL;
  const long work = (long)tokens * kv_heads * (dim / group);
  if (work == 0) return DD_OK;
  const dim3 grid((unsigned)dd_cdiv(work, 256));
  hipStream_t s = (hipStream_t)stream;
  auto *ck = (signed char *)cache_k;
  auto *cv = (signed char *)cache_v;
  auto *ks = (unsigned short *)k_scale;
  auto *vs = (unsigned short *)v_scale;
#define DD_Q8_STORE(DT)                                                                                    \
  hipLaunchKernelGGL(store_pages_q8_kernel<DT>, grid, dim3(256), 0, s, key, value, slot_map, (long)tokens, \
                     kv_heads, dim, group, page_size, (long)capacity, ck, cv, ks, vs)
  switch (dtype) {
    case DD_F32: DD_Q8_STORE(DD_F32); break;
    case DD_F16: DD_Q8_STORE(DD_F16); break;
    case DD_BF16: DD_Q8_STORE(DD_BF16); break;
    default: return DD_EUNSUPPORTED;
  }
#undef DD_Q8_STORE
  DD_LAUNCH_CHECK();
  return DD_OK;
}
