// Q8_0 quantisation of one channel group (damendaemon/kv_quant.py:55-64).
#pragma once
#include "common.h"

// Quantises x[base .. base+group) into q[0 .. group) and returns the fp16
// scale bits.  scale = fp16(absmax / 127); inv = 0 for a zero scale, else
// 1 / float(scale); q = clamp(sign(y) * floor(|y| + 0.5), +-127), y = x*inv.
// Both divisions are done in double and rounded once to float, which gives
// the correctly rounded fp32 quotient (53 >= 2*24 + 2 bits), so the result
// is bit-identical to fp32 torch arithmetic whatever the fp32 divide mode.
template <int DT>
DD_DEV unsigned short q8_group(const void *x, long base, int group, signed char *q) {
  float amax = 0.f;
  for (int i = 0; i < group; ++i) amax = fmaxf(amax, fabsf(load_as<DT>(x, base + i)));
  const unsigned short sbits = float_to_f16_bits((float)((double)amax / 127.0));
  const float s = half_bits_to_float(sbits);
  const float inv = s == 0.f ? 0.f : (float)(1.0 / (double)s);
  for (int i = 0; i < group; ++i) {
    const float y = load_as<DT>(x, base + i) * inv;
    const float r = fminf(floorf(fabsf(y) + 0.5f), 127.f);
    q[i] = (signed char)(y < 0.f ? -r : r);
  }
  return sbits;
}
