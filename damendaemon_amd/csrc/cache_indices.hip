// Causal index plans for windowed + compressed-block attention
// (damendaemon/cache_indices.py:24-80), one thread per plan entry.
//
// prefill: row r is position p = query_start + r of a sequence of length L;
//   cols [0, keys): local key max(p - window + 1, 0) + j if <= p, else -1
//   cols [keys, keys + compressed): block b -> L + b if b < (p + 1) / ratio, else -1
// ring decode: row r is the logical position p = positions[r];
//   cols [0, window): t = max(p - window + 1, 0) + j -> t % window if t <= p, else -1
//   cols [window, window + compressed): block b -> window + b if b < (p + 1) / ratio, else -1
#include "common.h"

namespace {

__global__ __launch_bounds__(256) void prefill_plan_kernel(long rows, int cols, int keys, long seq_len, int window,
                                                           int ratio, long query_start, int64_t *out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cols) return;
  const long r = i / cols;
  const int c = (int)(i - r * cols);
  const long p = query_start + r;
  long v;
  if (c < keys) {
    const long start = p - window + 1 > 0 ? p - window + 1 : 0;
    v = start + c <= p ? start + c : -1;
  } else {
    const long b = c - keys;
    v = b < (p + 1) / ratio ? b + seq_len : -1;
  }
  out[i] = v;
}

__global__ __launch_bounds__(256) void ring_plan_kernel(const int64_t *positions, long rows, int cols, int window,
                                                        int ratio, int64_t *out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cols) return;
  const long r = i / cols;
  const int c = (int)(i - r * cols);
  const long p = positions[r];
  long v;
  if (c < window) {
    const long t = (p - window + 1 > 0 ? p - window + 1 : 0) + c;
    v = t <= p ? t % window : -1;
  } else {
    const long b = c - window;
    v = b < (p + 1) / ratio ? b + window : -1;
  }
  out[i] = v;
}

}  // namespace

extern "C" int dd_prefill_indices(int64_t seq_len, int window, int ratio, int64_t query_start, int64_t query_stop,
                                  int64_t *out, void *stream) {
  if (!out || seq_len <= 0 || window <= 0 || ratio < 0 || query_start < 0 || query_stop <= query_start ||
      query_stop > seq_len)
    return DD_EINVAL;
  const int keys = (int)(window < seq_len ? window : seq_len);
  const int compressed = ratio ? (int)(query_stop / ratio) : 0;
  const long rows = query_stop - query_start;
  const int cols = keys + compressed;
  hipLaunchKernelGGL(prefill_plan_kernel, dim3((unsigned)dd_cdiv(rows * cols, 256)), dim3(256), 0,
                     (hipStream_t)stream, rows, cols, keys, (long)seq_len, window, ratio ? ratio : 1,
                     (long)query_start, out);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

extern "C" int dd_ring_decode_indices(const int64_t *positions, int64_t rows, int window, int ratio,
                                      int compressed, int64_t *out, void *stream) {
  if (!positions || !out || rows <= 0 || window <= 0 || ratio < 0 || compressed < 0 || (compressed && !ratio))
    return DD_EINVAL;
  const int cols = window + compressed;
  hipLaunchKernelGGL(ring_plan_kernel, dim3((unsigned)dd_cdiv(rows * cols, 256)), dim3(256), 0, (hipStream_t)stream,
                     positions, (long)rows, cols, window, ratio ? ratio : 1, out);
  DD_LAUNCH_CHECK();
  return DD_OK;
}
