// Q8_0 KV codec (damendaemon/kv_quant.py:48-76) for gfx950.
//
// Per group of `group` consecutive channels of a row:
//   scale = fp16(absmax / 127)                       (fp32 divide, RNE to fp16)
//   inv   = scale == 0 ? 0 : 1 / float(scale)        (correctly rounded)
//   q     = clamp(sign(x*inv) * floor(|x*inv| + 0.5), -127, 127)
// Dequantisation is int8 * float(scale), rounded once to the output dtype.
// Every step is a single correctly-rounded fp32 operation, so the result is
// bit-identical to the reference's torch arithmetic.  The two divisions are
// done in double and rounded once to float, which yields the correctly
// rounded fp32 quotient (53 >= 2*24+2 bits), independent of the compiler's
// fp32 division mode.
//
// One thread owns one channel group.
#include "common.h"
#include "q8.h"

namespace {

template <int DT>
__global__ __launch_bounds__(256) void quantize_kernel(const void *x, long groups, int group,
                                                       signed char *q, unsigned short *scale) {
  const long g = (long)blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  scale[g] = q8_group<DT>(x, g * group, group, q + g * group);
}

template <int DT>
__global__ __launch_bounds__(256) void dequantize_kernel(const signed char *q, const unsigned short *scale,
                                                         long n, int group, void *out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  store_as<DT>(out, i, (float)q[i] * half_bits_to_float(scale[i / group]));
}

}  // namespace

extern "C" int dd_quantize_q8(const void *x, int x_dtype, int64_t rows, int dim, int group, void *q, void *scale,
                              void *stream) {
  if (!x || !q || !scale || rows < 0 || dim <= 0 || group <= 0 || dim % group) return DD_EINVAL;
  const long groups = rows * (long)(dim / group);
  if (groups == 0) return DD_OK;
  const dim3 grid((unsigned)dd_cdiv(groups, 256));
  hipStream_t s = (hipStream_t)stream;
  auto *qq = (signed char *)q;
  auto *ss = (unsigned short *)scale;
  switch (x_dtype) {
    case DD_F32: hipLaunchKernelGGL(quantize_kernel<DD_F32>, grid, dim3(256), 0, s, x, groups, group, qq, ss); break;
    case DD_F16: hipLaunchKernelGGL(quantize_kernel<DD_F16>, grid, dim3(256), 0, s, x, groups, group, qq, ss); break;
    case DD_BF16: hipLaunchKernelGGL(quantize_kernel<DD_BF16>, grid, dim3(256), 0, s, x, groups, group, qq, ss); break;
    default: return DD_EUNSUPPORTED;
  }
  DD_LAUNCH_CHECK();
  return DD_OK;
}

extern "C" int dd_dequantize_q8(const void *q, const void *scale, int64_t rows, int dim, int group, void *out,
                                int out_dtype, void *stream) {
  if (!q || !scale || !out || rows < 0 || dim <= 0 || group <= 0 || dim % group) return DD_EINVAL;
  const long n = rows * (long)dim;
  if (n == 0) return DD_OK;
  const dim3 grid((unsigned)dd_cdiv(n, 256));
  hipStream_t s = (hipStream_t)stream;
  auto *qq = (const signed char *)q;
  auto *ss = (const unsigned short *)scale;
  switch (out_dtype) {
    case DD_F32: hipLaunchKernelGGL(dequantize_kernel<DD_F32>, grid, dim3(256), 0, s, qq, ss, n, group, out); break;
    case DD_F16: hipLaunchKernelGGL(dequantize_kernel<DD_F16>, grid, dim3(256), 0, s, qq, ss, n, group, out); break;
    case DD_BF16: hipLaunchKernelGGL(dequantize_kernel<DD_BF16>, grid, dim3(256), 0, s, qq, ss, n, group, out); break;
    default: return DD_EUNSUPPORTED;
  }
  DD_LAUNCH_CHECK();
  return DD_OK;
}
