// Arguments of the vector-ALU chunked-prefill kernel (prefill_generic.hip),
// which dd_prefill_attention uses for fp32 pages and for head sizes the MFMA
// kernel is not built for.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

struct PrefillGenericArgs {
  const void *q;        // (T, heads, dim)
  const void *k;        // (capacity, kv_heads, page, dim)
  const void *v;
  const int64_t *cu;    // (n+1) cu_seqlens
  const int64_t *ctx;   // (n) start + len
  const int64_t *slots;
  const int32_t *table;
  void *out;            // (T, heads, dim)
  long capacity;
  int n, max_len, max_tiles;
  int heads, kv_heads, dim;
  int page, page_shift;
  int table_w, table_rows;
  int window;
  float scale_log2;     // scale * log2(e), any finite sign
  // Re-run mode (flags != NULL): a workgroup computes its rows only if one of
  // the 16-bit kernel's work items covering them flagged its result (item
  // group * flag_tiles + r / flag_rows for query row r of group (segment,
  // KV head)); otherwise it exits at once.
  const int32_t *flags;
  int flag_rows, flag_tiles;
};

// Whether the 16-bit kernel flagged any of the work items that cover query
// rows r0 .. r0 + rows - 1 of group grp (always true without flags).
__device__ inline bool rerun_wanted(const PrefillGenericArgs &p, int grp, int r0, int rows) {
  if (!p.flags) return true;
  int any = 0;
  const long base = (long)grp * p.flag_tiles;
  for (int t = r0 / p.flag_rows; t <= (r0 + rows - 1) / p.flag_rows; ++t) any |= p.flags[base + t];
  return any != 0;
}

int dd_prefill_generic(const PrefillGenericArgs &args, int dtype, hipStream_t stream);

// fp32 arithmetic on the matrix cores (prefill_f32.hip): fp32 pages, and
// bf16 / fp16 pages at head sizes without a 16-bit MFMA kernel; D a multiple
// of 16 up to 256, at most 128 query heads per KV head.  DD_EUNSUPPORTED for anything else.
int dd_prefill_f32(const PrefillGenericArgs &args, int dtype, hipStream_t stream);
