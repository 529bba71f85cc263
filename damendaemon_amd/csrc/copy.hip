// Page gather / restore between a paged KV layer and a dense snapshot.
//
// Same contract as the reference's `_copy` (damendaemon/paged_kernels.py:8-47):
//   dense[kv, h, t, :] <-> cache[kv, table[slot, t / P], h, t % P, :]
// for t < tokens only; page tails and unused pages are never touched.
#include "common.h"

namespace {

// One workgroup per (page-table entry, plane, head): the P rows of that
// entry are one contiguous block on both sides -- page block (phys, head) of
// the plane in the cache, rows t0 .. t0+P-1 of (plane, head) in the dense
// tensor -- so the copy is a flat move of rows * row_bytes bytes, 16 per
// lane-access, kUnroll accesses in flight per lane (all loads of a round
// before its stores).  No per-element index arithmetic beyond the block
// bases; the page lookup is one scalar load.
constexpr int kUnroll = 4;

__global__ __launch_bounds__(256) void copy_pages_kernel(char *cache, const int32_t *table, char *dense,
                                                         long slot, long tokens, int heads, int row_bytes,
                                                         int page, long capacity, int table_w, int restore) {
  const int entry = blockIdx.x;
  const int ph = blockIdx.y;                  // plane * heads + head
  const int plane = ph / heads;
  const int h = ph - plane * heads;
  const long phys = table[slot * table_w + entry];
  if (phys < 0 || phys >= capacity) return;
  const long t0 = (long)entry * page;
  const long rows = tokens - t0 < page ? tokens - t0 : page;
  const int n = (int)(rows * (row_bytes >> 4));   // 16-byte pieces of this block
  char *cblk = cache + (((plane * capacity + phys) * heads + h) * (long)page) * row_bytes;
  char *dblk = dense + ((long)ph * tokens + t0) * row_bytes;
  const char *src = restore ? dblk : cblk;
  char *dst = restore ? cblk : dblk;
  for (int i0 = threadIdx.x; i0 < n; i0 += 256 * kUnroll) {
    u32x4 x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = i0 + 256 * u;
      if (i < n) x[u] = __builtin_nontemporal_load((const u32x4 *)src + i);
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int i = i0 + 256 * u;
      if (i < n) __builtin_nontemporal_store(x[u], (u32x4 *)dst + i);
    }
  }
}

}  // namespace

extern "C" int dd_copy_pages(void *cache, const int32_t *table, int table_rows, int table_width, void *dense,
                             int elem_bytes, int64_t slot, int64_t tokens, int64_t capacity, int heads, int page,
                             int dim, int restore, void *stream) {
  if (!cache || !table || !dense || slot < 0 || slot >= table_rows || tokens <= 0 ||
      tokens > (int64_t)table_width * page || capacity <= 0 || heads <= 0 || page <= 0 || dim <= 0 ||
      elem_bytes <= 0)
    return DD_EINVAL;
  const int row_bytes = dim * elem_bytes;
  if (row_bytes % 16) return DD_EUNSUPPORTED;
  const long entries = dd_cdiv(tokens, page);
  if (2L * heads > 65535 || entries > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL(copy_pages_kernel, dim3((unsigned)entries, (unsigned)(2 * heads)), dim3(256), 0,
                     (hipStream_t)stream,
                     (char *)cache, table, (char *)dense, (long)slot, (long)tokens, heads, row_bytes, page,
                     (long)capacity, table_width, restore);
  DD_LAUNCH_CHECK();
  return DD_OK;
}
