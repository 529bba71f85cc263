// Shared device helpers for the gfx950 kernels: dtype conversion, vector
// types, cross-lane reductions and the status plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/damendaemon_amd.h"

#define DD_DEV __device__ __forceinline__

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- scalar conversions -------------------------------------------------

DD_DEV float bf16_lo(unsigned w) { return __uint_as_float(w << 16); }
DD_DEV float bf16_hi(unsigned w) { return __uint_as_float(w & 0xffff0000u); }

DD_DEV float f16_lo(unsigned w) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
}
DD_DEV float f16_hi(unsigned w) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
}

DD_DEV float half_bits_to_float(unsigned short h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// fp32 -> bf16 with round-to-nearest-even (torch's Tensor.to(bfloat16)).
// Written without a branch (NaNs keep their payload, made quiet): as a
// select it costs a few instructions per value; with an early return the
// compiler puts every conversion behind its own divergent branch.
DD_DEV unsigned short float_to_bf16_bits(float f) {
  const unsigned u = __float_as_uint(f);
  const unsigned rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const unsigned quiet = (u >> 16) | 0x40u;
  return (unsigned short)((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}
DD_DEV unsigned short float_to_f16_bits(float f) {
  return __builtin_bit_cast(unsigned short, (_Float16)f);
}

// Store one fp32 value as the given dtype code.
template <int DT>
DD_DEV void store_as(void *base, long idx, float x) {
  if constexpr (DT == DD_F32) {
    ((float *)base)[idx] = x;
  } else if constexpr (DT == DD_BF16) {
    ((unsigned short *)base)[idx] = float_to_bf16_bits(x);
  } else {
    ((unsigned short *)base)[idx] = float_to_f16_bits(x);
  }
}

template <int DT>
DD_DEV float load_as(const void *base, long idx) {
  if constexpr (DT == DD_F32) {
    return ((const float *)base)[idx];
  } else if constexpr (DT == DD_BF16) {
    return __uint_as_float(((unsigned)((const unsigned short *)base)[idx]) << 16);
  } else {
    return half_bits_to_float(((const unsigned short *)base)[idx]);
  }
}

// ---- cross-lane ----------------------------------------------------------

// DPP controls used inside one 16-lane row.
constexpr int kDppQuadXor1 = 0xB1;  // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;  // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;  // row_ror:4
constexpr int kDppRowRor8 = 0x128;  // row_ror:8

template <int CTRL>
DD_DEV float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                         0xf, 0xf, false));
}

// Max / sum over the 16 lanes of a DPP row; every lane gets the result.
DD_DEV float row16_max(float x) {
  x = fmaxf(x, dpp<kDppQuadXor1>(x));
  x = fmaxf(x, dpp<kDppQuadXor2>(x));
  x = fmaxf(x, dpp<kDppRowRor4>(x));
  x = fmaxf(x, dpp<kDppRowRor8>(x));
  return x;
}
DD_DEV float row16_sum(float x) {
  x += dpp<kDppQuadXor1>(x);
  x += dpp<kDppQuadXor2>(x);
  x += dpp<kDppRowRor4>(x);
  x += dpp<kDppRowRor8>(x);
  return x;
}

DD_DEV float read_lane(float x, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), lane));
}
DD_DEV int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

// Lane index within the 64-wide wavefront.
DD_DEV int lane_id() { return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)); }

DD_DEV float shfl(float x, int src_lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_ds_bpermute(src_lane << 2, __builtin_bit_cast(int, x)));
}

// A wave-uniform pointer, made provably scalar (SGPR pair) for the compiler.
DD_DEV const char *uniform_ptr(const char *p) {
  const unsigned long long v = (unsigned long long)p;
  const unsigned lo = __builtin_amdgcn_readfirstlane((unsigned)v);
  const unsigned hi = __builtin_amdgcn_readfirstlane((unsigned)(v >> 32));
  return (const char *)(((unsigned long long)hi << 32) | lo);
}

// Reductions of x over lane pairs (l, l ^ 16) and (l, l ^ 32) with the
// gfx950 permlane swaps (VALU, no LDS round trip).  A swap of a register
// with itself leaves, in the two results, x of this lane and x of the
// partner lane (in an order that depends on the lane), so the commutative
// combination of the pair is the same in both lanes.
DD_DEV float xor16_max(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
DD_DEV float xor32_max(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
DD_DEV float xor16_sum(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
DD_DEV float xor32_sum(float x) {
  const unsigned u = __float_as_uint(x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ---- host side -----------------------------------------------------------

#define DD_LAUNCH_CHECK()                                   \
  do {                                                      \
    if (hipGetLastError() != hipSuccess) return DD_ELAUNCH; \
  } while (0)

static inline long dd_cdiv(long a, long b) { return (a + b - 1) / b; }
