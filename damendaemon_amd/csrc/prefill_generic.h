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
};

int dd_prefill_generic(const PrefillGenericArgs &args, int dtype, hipStream_t stream);

// fp32 arithmetic on the matrix cores (prefill_f32.hip): fp32 pages, and
// bf16 / fp16 pages at head sizes without a 16-bit MFMA kernel; D a multiple
// of 16 up to 256, at most 128 query heads per KV head.  DD_EUNSUPPORTED for anything else.
int dd_prefill_f32(const PrefillGenericArgs &args, int dtype, hipStream_t stream);
