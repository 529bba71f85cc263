// Page gather / restore between a paged KV layer and a dense snapshot.
//
// Same contract as the reference's `_copy` (damendaemon/paged_kernels.py:8-47):
//   dense[kv, h, t, :] <-> cache[kv, table[slot, t / P], h, t % P, :]
// for t < tokens only; page tails and unused pages are never touched.
// One thread moves 16 bytes, so each (token, head) row is moved by
// row_bytes/16 adjacent threads and both sides stay coalesced.
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void copy_pages_kernel(char *cache, const int32_t *table, char *dense,
                                                         long slot, long tokens, int heads, int row_bytes,
                                                         int page, long capacity, int table_w, int restore) {
  const int per_row = row_bytes >> 4;
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  const long total = 2L * heads * tokens * per_row;
  if (g >= total) return;
  const int chunk = (int)(g % per_row);
  const long row = g / per_row;              // (plane, head, token) in dense order
  const long t = row % tokens;
  const long ph = row / tokens;
  const int h = (int)(ph % heads);
  const long plane = ph / heads;
  const long phys = table[slot * table_w + t / page];
  if (phys < 0 || phys >= capacity) return;
  const long c_off = (((plane * capacity + phys) * heads + h) * page + t % page) * row_bytes + 16L * chunk;
  const long d_off = row * row_bytes + 16L * chunk;
  if (restore) {
    *(u32x4 *)(cache + c_off) = *(const u32x4 *)(dense + d_off);
  } else {
    *(u32x4 *)(dense + d_off) = *(const u32x4 *)(cache + c_off);
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
  const long work = 2L * heads * tokens * (row_bytes / 16);
  hipLaunchKernelGGL(copy_pages_kernel, dim3((unsigned)dd_cdiv(work, 256)), dim3(256), 0, (hipStream_t)stream,
                     (char *)cache, table, (char *)dense, (long)slot, (long)tokens, heads, row_bytes, page,
                     (long)capacity, table_width, restore);
  DD_LAUNCH_CHECK();
  return DD_OK;
}
