// Fused rotary embedding + K/V page write (damendaemon/kernels.py:271-340).
//
// For token b and head h of the packed (T, (H + 2KH) * D) projection:
//   * query and key heads: optional RMS norm with a learned weight
//     (QK-norm), then rotate-half RoPE over the first RD channels:
//       out[j] = x[j]*cos[pos, j] + sgn(j) * x[(j + RD/2) % RD]*sin[pos, j]
//     with sgn = -1 for j < RD/2; channels j >= RD pass through (cos 1, sin 0);
//   * queries go to query[b, h, 0, :]; rotated keys and raw values go to the
//     cache row of position pos: page table[slot, pos / P], row pos % P (paged)
//     or slot / position (slotted); `materialize` also writes them densely.
// Without `precise`, the reference rounds to fp16 after each of the norm's
// two multiplies and after each of the two rotation products; every product
// and sum here is a separate correctly-rounded fp32 operation (no FMA
// contraction), as in the reference's enable_fp_fusion=False build.
//
// Two kernels.  rope_vec_kernel, for full-width rotation of 16-bit rows into a
// cache of the same dtype at head sizes 64/128/256 (the common case): one
// workgroup per token, so the position, slot and page lookups are done once
// per token; a lane owns 8 consecutive channels of a head (16-byte loads and
// stores), and the rotate-half partner channels come from the lane D/16 away
// within the head's lane group.  rope_kernel, for everything else: one
// wavefront per (token, head), lanes striding over the channels.  Both apply
// the same per-element sequence of fp32 operations and fp16 roundings.
#include "common.h"

// Every fp16 rounding below takes an fp32 value that has already been
// rounded: the reference rounds a product to fp32 and then to fp16, and the
// compiler would otherwise fold "fp32 multiply, then convert to fp16" into
// one mixed-precision FMA (v_fma_mix*) that rounds the exact product once --
// a different result whenever the fp32 product is an fp16 tie.
#pragma clang fp contract(off)

namespace {

DD_DEV float load_code(const void *p, long i, int code) {
  switch (code) {
    case DD_F32: return load_as<DD_F32>(p, i);
    case DD_F16: return load_as<DD_F16>(p, i);
    default: return load_as<DD_BF16>(p, i);
  }
}

DD_DEV float round_f16(float x) {
  asm("" : "+v"(x));   // x is an fp32 value here, not an expression the conversion may absorb
  return half_bits_to_float(float_to_f16_bits(x));
}

struct RopeParams {
  const void *x;
  const void *cos;
  const void *sin;
  const int64_t *pos;
  const int64_t *slots;
  const void *qw;
  const void *kw;
  const int32_t *table;
  void *q;
  void *ck;
  void *cv;
  void *tk;
  void *tv;
  long tokens;
  long capacity;
  int H, KH, D, RD;
  int C;  // page size (paged) or context (slotted)
  int table_w, table_rows;
  int cos_code, w_code;
  int precise;
  float eps;
};

template <int XT, int CT>
__global__ __launch_bounds__(256) void rope_kernel(RopeParams p) {
  const int lane = threadIdx.x & 63;
  const long item = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int heads = p.H + 2 * p.KH;
  if (item >= p.tokens * heads) return;
  const long b = item / heads;
  const int head = (int)(item - b * heads);
  const long pos = p.pos[b];
  const long slot = p.slots[b];
  long cslot = slot, cpos = pos;
  if (p.table) {
    const long entry = pos / p.C;
    cslot = (slot >= 0 && slot < p.table_rows && entry < p.table_w) ? p.table[slot * p.table_w + entry] : -1;
    cpos = pos % p.C;
  }
  const bool cache_ok = cslot >= 0 && cslot < p.capacity;
  const long base = (b * heads + head) * (long)p.D;
  const int D = p.D, RD = p.RD, half = RD / 2;

  if (head >= p.H + p.KH) {  // value head: stored as is
    const int kh = head - p.H - p.KH;
    for (int j = lane; j < D; j += 64) {
      const float x = load_as<XT>(p.x, base + j);
      if (cache_ok) store_as<CT>(p.cv, ((cslot * p.KH + kh) * p.C + cpos) * D + j, x);
      if (p.tv) store_as<CT>(p.tv, (b * p.KH + kh) * (long)D + j, x);
    }
    return;
  }
  const bool is_q = head < p.H;
  const void *w = is_q ? p.qw : p.kw;
  float inv = 1.f;
  if (w) {
    float ss = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float x = load_as<XT>(p.x, base + j);
      ss += x * x;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
    inv = 1.f / sqrtf(__fadd_rn(ss / (float)D, p.eps));
  }
  for (int j = lane; j < D; j += 64) {
    const int oj = (j + half) % RD;
    float x = load_as<XT>(p.x, base + j);
    float o = load_as<XT>(p.x, base + oj);
    if (w) {
      x = __fmul_rn(x, inv);
      o = __fmul_rn(o, inv);
      if (!p.precise) { x = round_f16(x); o = round_f16(o); }
      x = __fmul_rn(x, load_code(w, j, p.w_code));
      o = __fmul_rn(o, load_code(w, oj, p.w_code));
      if (!p.precise) { x = round_f16(x); o = round_f16(o); }
    }
    if (j < half) o = -o;
    const float c = j < RD ? load_code(p.cos, pos * RD + j, p.cos_code) : 1.f;
    const float s = j < RD ? load_code(p.sin, pos * RD + j, p.cos_code) : 0.f;
    float a = __fmul_rn(x, c);
    float bb = __fmul_rn(o, s);
    if (!p.precise) { a = round_f16(a); bb = round_f16(bb); }
    const float r = __fadd_rn(a, bb);
    if (is_q) {
      store_as<XT>(p.q, (b * p.H + head) * (long)D + j, r);
    } else {
      const int kh = head - p.H;
      if (cache_ok) store_as<CT>(p.ck, ((cslot * p.KH + kh) * p.C + cpos) * D + j, r);
      if (p.tk) store_as<CT>(p.tk, (b * p.KH + kh) * (long)D + j, r);
    }
  }
}

// 16-bit <-> fp32 for the 16-bit row formats (bit patterns in the low half)
template <int XT>
DD_DEV float h2f(unsigned h) {
  if constexpr (XT == DD_BF16) return __uint_as_float(h << 16);
  else return half_bits_to_float((unsigned short)h);
}
template <int XT>
DD_DEV unsigned f2h(float x) {
  if constexpr (XT == DD_BF16) return float_to_bf16_bits(x);
  else return float_to_f16_bits(x);
}

template <int XT, int CS>
__global__ __launch_bounds__(256) void rope_vec_kernel(RopeParams p) {
  const long b = blockIdx.x;
  const int D = p.D;
  const int lph = D / 8;                 // lanes per head
  const int hl = threadIdx.x % lph;      // lane within the head's group
  const int hpp = 256 / lph;             // heads per pass of the workgroup
  const int heads = p.H + 2 * p.KH;
  const long pos = p.pos[b];
  const long slot = p.slots[b];
  long cslot = slot, cpos = pos;
  if (p.table) {
    const long entry = pos / p.C;
    cslot = (slot >= 0 && slot < p.table_rows && entry < p.table_w) ? p.table[slot * p.table_w + entry] : -1;
    cpos = pos % p.C;
  }
  const bool cache_ok = cslot >= 0 && cslot < p.capacity;
  const int j0 = 8 * hl;
  // cos / sin of this lane's channels at the token's position
  float c[8], sn[8];
  if constexpr (CS == DD_F32) {
    const f32x4 *cp = (const f32x4 *)((const float *)p.cos + pos * D + j0);
    const f32x4 *sp = (const f32x4 *)((const float *)p.sin + pos * D + j0);
    const f32x4 c0 = cp[0], c1 = cp[1], s0 = sp[0], s1 = sp[1];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      c[k] = c0[k];
      c[k + 4] = c1[k];
      sn[k] = s0[k];
      sn[k + 4] = s1[k];
    }
  } else {
    const u32x4 cw = *(const u32x4 *)((const unsigned short *)p.cos + pos * D + j0);
    const u32x4 sw = *(const u32x4 *)((const unsigned short *)p.sin + pos * D + j0);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      c[2 * k] = h2f<CS>(cw[k] & 0xffffu);
      c[2 * k + 1] = h2f<CS>(cw[k] >> 16);
      sn[2 * k] = h2f<CS>(sw[k] & 0xffffu);
      sn[2 * k + 1] = h2f<CS>(sw[k] >> 16);
    }
  }
  const bool lower = hl < lph / 2;       // channels below D/2: the partner enters negated
  for (int h = (int)threadIdx.x / lph; h < heads; h += hpp) {
    const long base = (b * heads + h) * (long)D + j0;
    const u32x4 xw = *(const u32x4 *)((const unsigned short *)p.x + base);
    if (h >= p.H + p.KH) {  // value head: stored as is
      const int kh = h - p.H - p.KH;
      if (cache_ok) *(u32x4 *)((unsigned short *)p.cv + ((cslot * p.KH + kh) * p.C + cpos) * D + j0) = xw;
      if (p.tv) *(u32x4 *)((unsigned short *)p.tv + (b * p.KH + kh) * (long)D + j0) = xw;
      continue;
    }
    const bool is_q = h < p.H;
    const void *wt = is_q ? p.qw : p.kw;
    float x[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = h2f<XT>(xw[k] & 0xffffu);
      x[2 * k + 1] = h2f<XT>(xw[k] >> 16);
    }
    if (wt) {
      float ss = 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k) ss += x[k] * x[k];
      for (int off = lph / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
      const float inv = 1.f / sqrtf(__fadd_rn(ss / (float)D, p.eps));
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        float v = __fmul_rn(x[k], inv);
        if (!p.precise) v = round_f16(v);
        v = __fmul_rn(v, load_code(wt, j0 + k, p.w_code));
        if (!p.precise) v = round_f16(v);
        x[k] = v;
      }
    }
    float o[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float v = __shfl_xor(x[k], lph / 2, 64);
      o[k] = lower ? -v : v;
    }
    u32x4 r;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      unsigned pr = 0;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int i = 2 * k + e;
        float a = __fmul_rn(x[i], c[i]);
        float bb = __fmul_rn(o[i], sn[i]);
        if (!p.precise) {
          a = round_f16(a);
          bb = round_f16(bb);
        }
        pr |= f2h<XT>(__fadd_rn(a, bb)) << (16 * e);
      }
      r[k] = pr;
    }
    if (is_q) {
      *(u32x4 *)((unsigned short *)p.q + (b * p.H + h) * (long)D + j0) = r;
    } else {
      const int kh = h - p.H;
      if (cache_ok) *(u32x4 *)((unsigned short *)p.ck + ((cslot * p.KH + kh) * p.C + cpos) * D + j0) = r;
      if (p.tk) *(u32x4 *)((unsigned short *)p.tk + (b * p.KH + kh) * (long)D + j0) = r;
    }
  }
}

template <int XT>
int launch_rope_vec(const RopeParams &p, hipStream_t s) {
  if (p.tokens > 0x7fffffffL) return DD_EUNSUPPORTED;
  const dim3 grid((unsigned)p.tokens);
  switch (p.cos_code) {
    case DD_F32: hipLaunchKernelGGL((rope_vec_kernel<XT, DD_F32>), grid, dim3(256), 0, s, p); break;
    case DD_F16: hipLaunchKernelGGL((rope_vec_kernel<XT, DD_F16>), grid, dim3(256), 0, s, p); break;
    case DD_BF16: hipLaunchKernelGGL((rope_vec_kernel<XT, DD_BF16>), grid, dim3(256), 0, s, p); break;
    default: return DD_EUNSUPPORTED;
  }
  DD_LAUNCH_CHECK();
  return DD_OK;
}

template <int XT>
int launch_rope(const RopeParams &p, int ct, hipStream_t s) {
  const long items = p.tokens * (p.H + 2 * p.KH);
  const dim3 grid((unsigned)dd_cdiv(items, 4));
  switch (ct) {
    case DD_F32: hipLaunchKernelGGL((rope_kernel<XT, DD_F32>), grid, dim3(256), 0, s, p); break;
    case DD_F16: hipLaunchKernelGGL((rope_kernel<XT, DD_F16>), grid, dim3(256), 0, s, p); break;
    case DD_BF16: hipLaunchKernelGGL((rope_kernel<XT, DD_BF16>), grid, dim3(256), 0, s, p); break;
    default: return DD_EUNSUPPORTED;
  }
  DD_LAUNCH_CHECK();
  return DD_OK;
}

}  // namespace

extern "C" int dd_rope_batch(const void *qkv, int qkv_dtype, const void *cos, const void *sin, int cos_dtype,
                             int rotary_dim, const int64_t *positions, const int64_t *slots, int64_t tokens,
                             int heads, int kv_heads, int dim, const void *q_norm, const void *k_norm,
                             int norm_dtype, float eps, int precise, const int32_t *page_table, int table_rows,
                             int table_width, void *query, void *cache_k, void *cache_v, int cache_dtype,
                             int64_t capacity, int cache_len, void *key_out, void *value_out, void *stream) {
  if (!qkv || !cos || !sin || !positions || !slots || !query || !cache_k || !cache_v || tokens < 0 ||
      heads <= 0 || kv_heads <= 0 || dim <= 0 || rotary_dim <= 0 || rotary_dim > dim || rotary_dim % 2 ||
      cache_len <= 0 || capacity <= 0 || ((q_norm || k_norm) && rotary_dim != dim))
    return DD_EINVAL;
  if (tokens == 0) return DD_OK;
  RopeParams p{};
  p.x = qkv;
  p.cos = cos;
  p.sin = sin;
  p.pos = positions;
  p.slots = slots;
  p.qw = q_norm;
  p.kw = k_norm;
  p.table = page_table;
  p.q = query;
  p.ck = cache_k;
  p.cv = cache_v;
  p.tk = key_out;
  p.tv = value_out;
  p.tokens = tokens;
  p.capacity = capacity;
  p.H = heads;
  p.KH = kv_heads;
  p.D = dim;
  p.RD = rotary_dim;
  p.C = cache_len;
  p.table_w = table_width;
  p.table_rows = table_rows;
  p.cos_code = cos_dtype;
  p.w_code = norm_dtype;
  p.precise = precise;
  p.eps = eps;
  hipStream_t s = (hipStream_t)stream;
  // the 16-byte accesses of the vector kernel need 16-byte aligned rows
  auto a16 = [](const void *q) { return ((uintptr_t)q & 15) == 0; };
  const bool aligned = a16(qkv) && a16(cos) && a16(sin) && a16(query) && a16(cache_k) && a16(cache_v) &&
                       a16(key_out) && a16(value_out);
  if (aligned && rotary_dim == dim && (dim == 64 || dim == 128 || dim == 256) && cache_dtype == qkv_dtype) {
    if (qkv_dtype == DD_BF16) return launch_rope_vec<DD_BF16>(p, s);
    if (qkv_dtype == DD_F16) return launch_rope_vec<DD_F16>(p, s);
  }
  switch (qkv_dtype) {
    case DD_F32: return launch_rope<DD_F32>(p, cache_dtype, s);
    case DD_F16: return launch_rope<DD_F16>(p, cache_dtype, s);
    case DD_BF16: return launch_rope<DD_BF16>(p, cache_dtype, s);
    default: return DD_EUNSUPPORTED;
  }
}
