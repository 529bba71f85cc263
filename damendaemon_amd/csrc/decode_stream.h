// Streamed split-KV decode (gfx950) for bf16 / f16 / fp32 KV pages at every
// head size up to 256 that is a multiple of 8 (LDS layouts of 64, 96, 128,
// 160, 192, 224 and 256 dims; a smaller head size takes the smallest layout
// that holds it, its rows of the real length in memory and the layout's
// extra dims zeros), and for int8 pages (stream_i8_kernel below: one scale
// per row at every head size that is a multiple of 16, in layouts of 64, 128
// and 256 dims; group-32 scales at 64, 128 and 256).
//
// Same contract as decode_kernel (the reference's `_attention`,
// damendaemon/kernels.py:134-187): one query row per sequence, keys
// [t_lo, pos] read through the page table, fp32 softmax, optional ALiBi,
// T5 relative bias, window and sinks; split partials are combined by
// merge_kernel.
//
// Memory path.  Each of the NW waves of a workgroup (sequence, KV head,
// split) owns every NW-th 16-token chunk and a private ring of NB LDS
// stages (16-bit pages: 8 waves x 1 stage up to D = 128, 4 x 1 from 160;
// fp32 at D = 64 / 128: 8 x 1, measured 1 % (16-bit) and 7 % (fp32) faster
// on 64 ragged contexts than 4 waves x 2; fp32 at 96 and from 160: 4 x 1).  A chunk's K
// and V rows are copied HBM -> LDS by direct-to-LDS buffer loads (no VGPRs
// held while in flight), marked nontemporal because
// every KV byte is read exactly once per step.  A stage is refilled as soon
// as its chunk has been read into registers, so NB chunks per wave are in
// flight while one is computed.  A chunk's buffer resource covers only its
// live rows, so rows past the split or the context, and chunks whose page is
// unallocated, land as zeros.
//
// fp32 pages: Q, K, V and P enter v_mfma_f32_16x16x4_f32 unrounded (exact
// fp32 products, one MFMA per dim of S^T and per key of O^T); O^T tile md
// row m holds dim (D/16) m + md so that V is read 16 contiguous bytes at a
// time.
//
// Math.  S^T = K Q^T with v_mfma_f32_16x16x32 (rows = the chunk's 16
// tokens, columns = the GQA group's heads); the accumulator already has the
// register layout of the P^T operand of O^T += V^T P^T, which runs on
// v_mfma_f32_16x16x16 (P^T split into a high and a residual 16-bit part, two
// MFMAs, so p keeps ~17 bits) with V^T read from LDS by transposing reads
// (ds_read_b64_tr_b16).  Each lane owns one head column, so the online
// softmax needs only two permlane steps per chunk; the running max moves
// only when a chunk's max exceeds it by more than 2^8 (p <= 256, exact in
// fp32 and representable in bf16/f16), so O is rarely rescaled.
//
// LDS layout of a stage: K rows then V rows, 2D bytes per token row, with
// the 16-byte chunks of row r stored at position (chunk ^ swz(r)); the
// DMA lanes fetch the permuted chunks (each instruction still reads 1 KiB
// of contiguous HBM), and the MFMA operand reads of K (16 rows, one column)
// and of V^T (4 rows x 32 bytes per 16 lanes) hit distinct LDS banks.
#pragma once
#include <type_traits>
#include <utility>

namespace dd_decode {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void;

#ifndef DD_STREAM_NB128
#define DD_STREAM_NB128 1
#endif
#ifndef DD_STREAM_NB_F32
#define DD_STREAM_NB_F32 1
#endif
#ifndef DD_STREAM_NW_F32
#define DD_STREAM_NW_F32 8
#endif
#ifndef DD_STREAM_NW_F32_96
#define DD_STREAM_NW_F32_96 4
#endif
#ifndef DD_STREAM_NB_F32_256
#define DD_STREAM_NB_F32_256 1
#endif
#ifndef DD_STREAM_NW_F32_256
#define DD_STREAM_NW_F32_256 4
#endif
#ifndef DD_STREAM_I8_NB128
#define DD_STREAM_I8_NB128 2
#endif
#ifndef DD_STREAM_I8_NW128
#define DD_STREAM_I8_NW128 4
#endif
#ifndef DD_STREAM_NB128G
#define DD_STREAM_NB128G 2
#endif
#ifndef DD_STREAM_NB96
#define DD_STREAM_NB96 1
#endif
#ifndef DD_STREAM_NW96
#define DD_STREAM_NW96 8
#endif
// D = 64, 16-bit pages: 8 waves x 1 stage (C2 contexts, H32/KH8, bf16:
// 93.5-93.9 us vs 99.0-102.8 us with 4 x 4; H64/KH8 97.5 vs 103-105 us).
#ifndef DD_STREAM_NB64
#define DD_STREAM_NB64 1
#endif
#ifndef DD_STREAM_NW64
#define DD_STREAM_NW64 8
#endif
// int8 pages at D = 64 (two chunks per step; its ring needs two stages):
// 4 waves x 2 stages (C2 contexts, H32/KH8: 60.1-60.6 us vs 75.4 us with 4 x 4;
// 2 x 8 67-68, 3 x 4 66, 2 waves x 2 63-64 us)
#ifndef DD_STREAM_I8_NB64
#define DD_STREAM_I8_NB64 2
#endif
#ifndef DD_STREAM_I8_NW64
#define DD_STREAM_I8_NW64 4
#endif
// D = 256, 16-bit pages: 4 waves x 1 stage (C2 contexts, bf16: H16/KH8 341-342 us vs
// 352-353 us with 2 x 2, H16/KH4 187 vs 190 us; C5 176.7 vs 178.5 us)
#ifndef DD_STREAM_NB256
#define DD_STREAM_NB256 1
#endif
// int8 pages at D = 256 (two stages, as every int8 shape)
#ifndef DD_STREAM_I8_NB256
#define DD_STREAM_I8_NB256 2
#endif
#ifndef DD_STREAM_I8_NW256
#define DD_STREAM_I8_NW256 2
#endif

// f(integral_constant<int, I>) for I = 0 .. N-1, unrolled at compile time.
template <typename F, int... I>
DD_DEV void static_for_impl(F &&f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
DD_DEV void static_for(F &&f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}


#ifndef DD_STREAM_NW128
#define DD_STREAM_NW128 8
#endif
#ifndef DD_STREAM_NW256
#define DD_STREAM_NW256 4
#endif
// D = 160, 192, 224 (16-bit pages; rows padded like D = 96): 4 waves x 1 stage
// (C2 contexts, H16/KH8: 0.73-0.76 of 8 TB/s; 8 x 1 0.69-0.72; the general
// kernel 0.51-0.58)
#ifndef DD_STREAM_NB_MID
#define DD_STREAM_NB_MID 1
#endif
#ifndef DD_STREAM_NW_MID
#define DD_STREAM_NW_MID 4
#endif

// Word 3 of a raw buffer resource (no swizzle, dword data format).
constexpr int kRawBufferWord3 = 0x00020000;
// Cache-policy bits of the K/V loads: nontemporal.
constexpr int kStreamLoadAux = 2;
// Running-max slack in the exp2 domain (see the header comment).
constexpr float kStreamSlack = 8.f;

// Position XOR of token row r within its stage (see the layout note).
template <int D>
DD_DEV constexpr int stream_swz(int r) {
  if constexpr (D == 64) {
    const int h = r >> 1;
    return ((h & 3) << 1) | ((h >> 2) & 1);
  } else {
    return ((r & 7) << 1) | ((r >> 3) & 1);
  }
}

// fp32 rows (4 D bytes, 16 or 32 chunks): the K operand reads 16 rows at
// one logical chunk, so the low four chunk bits are XORed with the row.
template <int DT, int D>
DD_DEV constexpr int stream_swz_of(int r) {
  if constexpr ((D & (D - 1)) != 0) {
    return 0;  // rows padded by 16 bytes instead (see stream_kernel)
  } else if constexpr (DT == DD_F32) {
    return r & 15;
  } else {
    return stream_swz<D>(r);
  }
}

template <int DT>
DD_DEV f32x4 mfma16x16x16(u32x2 a, u32x2 b, f32x4 c) {
  if constexpr (DT == DD_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                     0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                 0, 0);
  }
}

template <int DT>
DD_DEV unsigned pack_pair(float a, float b) {
  if constexpr (DT == DD_BF16) {
    return (unsigned)float_to_bf16_bits(a) | ((unsigned)float_to_bf16_bits(b) << 16);
  } else {
    return (unsigned)float_to_f16_bits(a) | ((unsigned)float_to_f16_bits(b) << 16);
  }
}

// LDS reads issued as inline assembly: the compiler cannot relate them to
// the direct-to-LDS loads still in flight into other stages, so it would
// otherwise wait for all of them.  Completion is waited for explicitly.
// (The host pass of the single-source build sees empty bodies: its target
// has no such registers, and these functions never run there.)
template <int OFF>
DD_DEV u32x4 lds_read_b128(unsigned addr) {
  u32x4 r = {};
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
#endif
  return r;
}
template <int OFF>
DD_DEV u32x2 lds_read_tr16(unsigned addr) {
  u32x2 r = {};
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
#endif
  return r;
}
template <int OFF>
DD_DEV u32x2 lds_read_b64(unsigned addr) {
  u32x2 r = {};
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
#endif
  return r;
}
// Transposing byte read (ds_read_b64_tr_b8): within each 16-lane group,
// lane i receives byte i % 8 of the 8-byte chunks addressed by lanes
// i / 8 + 2 j, j = 0..7, in that order.
template <int OFF>
DD_DEV u32x2 lds_read_tr8(unsigned addr) {
  u32x2 r = {};
#if __HIP_DEVICE_COMPILE__
  asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "n"(OFF));
#endif
  return r;
}
DD_DEV void wait_lds() {
#if __HIP_DEVICE_COMPILE__
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#endif
}
template <typename T>
DD_DEV void after_wait(T &x) {
#if __HIP_DEVICE_COMPILE__
  asm volatile("" : "+v"(x));
#endif
}
template <int N>
DD_DEV void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
#if __HIP_DEVICE_COMPILE__
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
#endif
}

// Combine the waves of a workgroup and write the split's result: the
// normalised output (one split) or the partial and its base-2 log-sum-exp.
// `o` is this lane's O^T slice (head lane % 16, dims 16 md + 4 (lane / 16)
// + i; for fp32 pages dims MD (4 (lane / 16) + i) + md, MD = D / 16),
// `m_run` / `lsum` its head's running max and (lane-partial) sum.
// `s_o` must hold NW * 16 * (D + 4) floats and be free (no loads in flight).
template <int DT, int D, int NW>
DD_DEV void stream_epilogue(const DecodeParams &p, float (*s_ml)[2][16], float *s_o, const f32x4 (&o)[D / 16],
                            float m_run, float lsum, int w, int lane, int b, long head0, int G, int split) {
  constexpr int MD = D / 16;
  constexpr int DP = D + 4;
  const int n16 = lane & 15;
  const int kg = lane >> 4;
  lsum = xor32_sum(xor16_sum(lsum));
  if (lane < 16) {
    s_ml[w][0][lane] = m_run;
    s_ml[w][1][lane] = lsum;
  }
  __syncthreads();
  float mm = s_ml[0][0][n16];
#pragma unroll
  for (int ww = 1; ww < NW; ++ww) mm = fmaxf(mm, s_ml[ww][0][n16]);
  const float fac = m_run == kNegInf ? 0.f : fast_exp2(m_run - mm);
  if (n16 < G) {
    if constexpr (DT == DD_F32 && MD % 4 == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int q = 0; q < MD / 4; ++q)
          *(f32x4 *)&s_o[(w * 16 + n16) * DP + MD * (4 * kg + i) + 4 * q] =
              f32x4{o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]} * fac;
    } else if constexpr (DT == DD_F32) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int md = 0; md < MD; ++md) s_o[(w * 16 + n16) * DP + MD * (4 * kg + i) + md] = o[md][i] * fac;
    } else {
#pragma unroll
      for (int md = 0; md < MD; ++md) *(f32x4 *)&s_o[(w * 16 + n16) * DP + 16 * md + 4 * kg] = o[md] * fac;
    }
  }
  __syncthreads();

  const int DR = p.DR;   // the head size (<= D): row stride of the output and partials
  for (int idx = threadIdx.x; idx < G * DR; idx += 64 * NW) {
    const int h = idx / DR;
    const int d = idx - h * DR;
    float m2 = s_ml[0][0][h];
    for (int ww = 1; ww < NW; ++ww) m2 = fmaxf(m2, s_ml[ww][0][h]);
    float l = 0.f, acc = 0.f;
    for (int ww = 0; ww < NW; ++ww) {
      const float mw = s_ml[ww][0][h];
      if (mw != kNegInf) l += s_ml[ww][1][h] * fast_exp2(mw - m2);
      acc += s_o[(ww * 16 + h) * DP + d];
    }
    const long bh = head0 + h;
    if (p.splits == 1) {
      if (p.sinks) {
        const float sk = p.sinks[bh - (long)b * p.H] * kLog2e;
        const float m3 = fmaxf(m2, sk);
        const float f = fast_exp2(m2 - m3);
        l = l * f + fast_exp2(sk - m3);
        acc *= f;
      }
      store_as<DT>(p.out, bh * DR + d, acc / l);
    } else {
      p.part[(bh * p.splits + split) * DR + d] = acc / l;
      if (d == 0) p.lse[bh * p.splits + split] = m2 + log2f(l);
    }
  }
}

template <int DT, int D, int NB, int NW>
__global__ __launch_bounds__(64 * NW) void stream_kernel(DecodeParams p) {
  // The host pass only needs the launch stub; the body is device code.
#if __HIP_DEVICE_COMPILE__
  constexpr bool F32 = DT == DD_F32;
  constexpr int ROWB = (F32 ? 4 : 2) * D;  // bytes per token row
  // LDS row stride: head sizes that are not powers of two (96) have rows of
  // a chunk count no XOR swizzle tiles, so their rows get a 16-byte pad
  // (stride 13 chunks: the 16-row K reads hit distinct banks); the DMA lanes
  // that land on a pad, or past the 16 rows, read out of the resource's range
  // and write zeros.
  constexpr bool PADR = (D & (D - 1)) != 0;
  constexpr int RSB = PADR ? ROWB + 16 : ROWB;
  constexpr int SPR = RSB / 16;      // 16-byte LDS slots per row
  constexpr int PAGEB = PADR ? (16 * RSB + 1023) / 1024 * 1024 : 16 * ROWB;  // one 16-token chunk of K (or V)
  constexpr int IPP = PAGEB / 1024;  // DMA instructions per chunk and plane
  constexpr int STAGE = 2 * PAGEB;
  constexpr int CPR = ROWB / 16;     // 16-byte chunks per row
  constexpr int NC = ROWB / 64;      // 16-byte K (and Q) operand reads per lane
  constexpr int MD = D / 16;         // O^T row tiles
  constexpr int DP = D + 4;          // padded row of the cross-wave buffer
  static_assert(IPP >= 1 && 2 * IPP * NB < 64 && NB <= 4, "vmcnt range, unrolled steps");
  static_assert((NB - 1) * STAGE + PAGEB < 65536, "ds offset range");
  // The ring's LDS also holds the epilogue's cross-wave buffer.
  constexpr int RING = NW * NB * STAGE > NW * 16 * DP * 4 ? NW * NB * STAGE : NW * 16 * DP * 4;

  __shared__ __align__(1024) char s_ring[RING];
  __shared__ float s_ml[NW][2][16];

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int n16 = lane & 15;  // head column (S^T, P^T, O^T) / token row (K operand)
  const int kg = lane >> 4;

  // Workgroup (split, sequence, KV head, head group): with more than 16
  // query heads per KV head, gsub workgroups of up to 16 heads each.
  const int wg = blockIdx.x;
  const int per_b = p.KH * p.gsub;
  const int nbkh = p.B * per_b;
  const int split = wg / nbkh;
  const int bkh = wg - split * nbkh;
  const int b = bkh / per_b;
  const int vk = bkh - b * per_b;
  const int kh = vk / p.gsub;
  const int gofs = 16 * (vk - kh * p.gsub);   // first head of this workgroup within the group
  const int G = p.gsub > 1 ? min(16, p.G - gofs) : p.G;   // heads of this workgroup

  const long pos64 = p.pos[b];
  const int row = p.slots ? (int)p.slots[b] : 0;
  const int t_hi = pos64 + 1 < p.ctx_limit ? (int)pos64 + 1 : p.ctx_limit;
  int t_lo = 0;
  if (p.window > 0 && pos64 - p.window + 1 > 0) t_lo = (int)(pos64 - p.window + 1);
  int s_lo = split * p.split_tokens;
  int s_hi = s_lo + p.split_tokens;
  if (s_hi > t_hi) s_hi = t_hi;
  if (s_lo < t_lo) s_lo = t_lo;
  if (s_lo >= s_hi) return;  // empty split: the merge never reads it
  const int pg_first = s_lo >> 4;
  const int pg_last = (s_hi - 1) >> 4;
  const long head0 = (long)b * p.H + (long)kh * p.G + gofs;
  const bool col_on = n16 < G;

  // Q^T operand: lane (head n16, dims 8kg + 32c ..+8); fp32: dims
  // (D/4) kg + 4c ..+4, one v_mfma_f32_16x16x4_f32 per dim of the four.
  // The head size DR may be below the layout's D (by 16, for head sizes that
  // are odd multiples of 16): rows are DR elements long in memory, and the
  // dims DR .. D-1 are zero queries, zero K/V in LDS and never stored.
  const int DR = p.DR;
  const int ROWG = (F32 ? 4 : 2) * DR;   // bytes per token row in memory
  u32x4 qa[NC];
  if constexpr (F32) {
    const float *qf = (const float *)p.q;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qa[c] = col_on && (D / 4) * kg + 4 * c < DR ? *(const u32x4 *)(qf + (head0 + n16) * DR + (D / 4) * kg + 4 * c)
                                                  : u32x4{0, 0, 0, 0};
  } else {
    const unsigned short *qb = (const unsigned short *)p.q;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qa[c] = col_on && 8 * kg + 32 * c < DR ? *(const u32x4 *)(qb + (head0 + n16) * DR + 8 * kg + 32 * c)
                                             : u32x4{0, 0, 0, 0};
  }
  float slope = (p.alibi && col_on) ? p.alibi[(long)kh * p.G + gofs + n16] * kLog2e : 0.f;

  // Per-lane LDS byte offsets (loop invariant).
  const unsigned wbase = (unsigned)(size_t)(lds_void *)s_ring + (unsigned)(w * NB * STAGE);
  unsigned dma_off[IPP];
#pragma unroll
  for (int j = 0; j < IPP; ++j) {
    const int e = 64 * j + lane;
    if constexpr (PADR) {
      const int r = e / SPR, c = e % SPR;
      dma_off[j] = r < 16 && 16 * c < ROWG ? (unsigned)(r * ROWG + 16 * c) : 0x40000000u;
    } else {
      const int r = e / CPR, c = (e % CPR) ^ stream_swz_of<DT, D>(r);
      dma_off[j] = 16 * c < ROWG ? (unsigned)(r * ROWG + 16 * c) : 0x40000000u;
    }
  }
  unsigned k_addr[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
    k_addr[c] = wbase + n16 * RSB + 16 * ((F32 ? (D / 16) * kg + c : 4 * c + kg) ^ stream_swz_of<DT, D>(n16));
  // V^T operand.  16-bit: transposing reads (lane: 4 keys of one dim per
  // tile).  fp32: O^T tile md, row m holds dim MD m + md, so that lane
  // (kg, n16) reads the MD contiguous dims MD n16 .. of key 4 kg + e
  // (MD / 4 reads of 16 bytes per key, address index e (MD / 4) + q).
  constexpr bool V8 = F32 && MD % 4 != 0;   // fp32 V read 8 bytes at a time (D = 96)
  unsigned v_addr[V8 ? 2 * MD : MD];
  if constexpr (V8) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int q = 0; q < MD / 2; ++q) {
        const int r = 4 * kg + e;
        v_addr[e * (MD / 2) + q] = wbase + PAGEB + r * RSB + 4 * (MD * n16 + 2 * q);
      }
  } else if constexpr (F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int q = 0; q < MD / 4; ++q) {
        const int r = 4 * kg + e;
        v_addr[e * (MD / 4) + q] =
            wbase + PAGEB + r * RSB + 16 * (((MD / 4) * n16 + q) ^ stream_swz_of<DT, D>(r));
      }
  } else {
    const int a = lane & 15;
    const int r = 4 * kg + (a >> 2);
    const int q = a & 3;
#pragma unroll
    for (int md = 0; md < MD; ++md)
      v_addr[md] = wbase + PAGEB + r * RSB + 16 * ((2 * md + (q >> 1)) ^ stream_swz_of<DT, D>(r)) + 8 * (q & 1);
  }

  // This wave's chunks: first + i * NW, i < n.
  const int first = pg_first + w;
  const int n = first <= pg_last ? (pg_last - first) / NW + 1 : 0;

  const char *kplane = (const char *)p.k;
  const char *vplane = (const char *)p.v;
  const __attribute__((address_space(4))) int32_t *tab = (const __attribute__((address_space(4))) int32_t *)p.table;
  // Buffer resources of chunk i of this wave (K, V).  Chunks past the wave's
  // last one get an empty resource (no memory traffic): every iteration then
  // has the same loads in flight and waits for a constant count.
  struct ChunkRsrc {
    __amdgpu_buffer_rsrc_t k, v;
  };
  auto chunk_rsrc = [&](int i) __attribute__((always_inline)) -> ChunkRsrc {
    const int pg = first + i * NW;
    long base;  // element offset of the chunk's first row, -1 when unmapped
    if (i >= n) {
      base = -1;
    } else if (p.paged) {
      base = -1;
      if (row >= 0 && row < p.table_rows) {
        const int entry = pg >> p.chunk_shift;
        const long phys = tab[(long)row * p.table_w + entry];
        if (phys >= 0 && phys < p.capacity)
          base = ((phys * p.KH + kh) * (long)p.page + ((pg - (entry << p.chunk_shift)) << 4)) * (long)DR;
      }
    } else {
      base = (row >= 0 && row < p.capacity) ? (((long)row * p.KH + kh) * (long)p.page + (long)pg * 16) * (long)DR : -1;
    }
    base = (long)uniform_ptr((const char *)base);
    const int live = base < 0 ? 0 : max(0, min(16, s_hi - pg * 16));
    const long off = base < 0 ? 0 : (F32 ? 4 : 2) * base;
    const int bytes = uniform(live * ROWG);
    return ChunkRsrc{
        __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr(kplane + off), (short)0, bytes, kRawBufferWord3),
        __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr(vplane + off), (short)0, bytes, kRawBufferWord3)};
  };
  // Chunk i straight into LDS `stage` (direct-to-LDS loads).
  auto issue = [&](int i, int stage) __attribute__((always_inline)) {
    const ChunkRsrc r = chunk_rsrc(i);
    char *dst = s_ring + (w * NB + stage) * STAGE;
#pragma unroll
    for (int j = 0; j < IPP; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r.k, (lds_void *)(dst + 1024 * j), 16, dma_off[j], 0, 0,
                                               kStreamLoadAux);
#pragma unroll
    for (int j = 0; j < IPP; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(r.v, (lds_void *)(dst + PAGEB + 1024 * j), 16, dma_off[j], 0, 0,
                                               kStreamLoadAux);
  };

  f32x4 o[MD];
#pragma unroll
  for (int md = 0; md < MD; ++md) o[md] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;  // running max of this lane's head (log2 domain)
  float lsum = 0.f;       // this lane's share of the running denominator

  auto consume = [&](int i, auto stage_tag) __attribute__((always_inline)) {
    constexpr int SOFF = decltype(stage_tag)::value * STAGE;
    const int t0 = (first + i * NW) * 16;
    u32x4 ka[NC];
    u32x2 va[F32 ? 1 : MD];
    u32x4 vf[F32 && !V8 ? MD : 1];
    u32x2 vh[V8 ? 2 * MD : 1];
#pragma unroll
    for (int c = 0; c < NC; ++c) ka[c] = lds_read_b128<SOFF>(k_addr[c]);
    if constexpr (V8) {
#pragma unroll
      for (int j = 0; j < 2 * MD; ++j) vh[j] = lds_read_b64<SOFF>(v_addr[j]);
    } else {
#pragma unroll
      for (int md = 0; md < MD; ++md) {
        if constexpr (F32) {
          vf[md] = lds_read_b128<SOFF>(v_addr[md]);
        } else {
          va[md] = lds_read_tr16<SOFF>(v_addr[md]);
        }
      }
    }
    wait_lds();
#pragma unroll
    for (int c = 0; c < NC; ++c) after_wait(ka[c]);
    if constexpr (V8) {
#pragma unroll
      for (int j = 0; j < 2 * MD; ++j) after_wait(vh[j]);
    } else {
#pragma unroll
      for (int md = 0; md < MD; ++md) {
        if constexpr (F32) {
          after_wait(vf[md]);
        } else {
          after_wait(va[md]);
        }
      }
    }
    // The stage is in registers now: refill it with chunk i + NB.
    issue(i + NB, decltype(stage_tag)::value);

    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (F32) {
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          s = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(ka[c][q]), __uint_as_float(qa[c][q]), s, 0, 0,
                                                   0);
    } else {
#pragma unroll
      for (int c = 0; c < NC; ++c) s = mfma16x16x32<DT>(ka[c], qa[c], s);
    }

    // logits of tokens t0 + 4kg + i for head n16
    float x[4];
    float mx = kNegInf;
    float rb[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.rel) {  // workgroup-uniform: no per-lane branch in the common path
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = t0 + 4 * kg + e;
        const long dist = pos64 - t > 0 ? pos64 - t : 0;
        rb[e] = p.rel[((long)kh * p.G + gofs + (col_on ? n16 : 0)) * p.rel_buckets +
                      rel_bucket((int)dist, p.rel_buckets, p.rel_denom)] * kLog2e;
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + 4 * kg + e;
      const float v = s[e] * p.scale_log2 + slope * (float)t + rb[e];
      x[e] = (t >= s_lo && t < s_hi) ? v : kNegInf;
      mx = fmaxf(mx, x[e]);
    }
    mx = xor32_max(xor16_max(mx));
    const bool up = mx > m_run + kStreamSlack;
    if (__builtin_amdgcn_ballot_w64(up)) {
      const float mn = up ? mx : m_run;
      const float alpha = up ? (m_run == kNegInf ? 0.f : fast_exp2(m_run - mn)) : 1.f;
      m_run = mn;
      lsum *= alpha;
#pragma unroll
      for (int md = 0; md < MD; ++md) o[md] *= alpha;
    }
    const float mu = m_run == kNegInf ? 0.f : m_run;
    float pr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      pr[e] = fast_exp2(x[e] - mu);
      lsum += pr[e];
    }
    if constexpr (F32) {
      // P^T stays fp32: key 4kg + e is k-index kg of the e-th MFMA of a tile.
      if (t0 < s_lo) {   // expired keys' V must not reach the MFMA (0 * NaN)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (t0 + 4 * kg + e < s_lo) {
            if constexpr (V8) {
#pragma unroll
              for (int q = 0; q < MD / 2; ++q) vh[e * (MD / 2) + q] = u32x2{0, 0};
            } else {
#pragma unroll
              for (int q = 0; q < MD / 4; ++q) vf[e * (MD / 4) + q] = u32x4{0, 0, 0, 0};
            }
          }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int md = 0; md < MD; ++md)
          o[md] = __builtin_amdgcn_mfma_f32_16x16x4f32(
              __uint_as_float(V8 ? vh[e * (MD / 2) + md / 2][md % 2] : vf[V8 ? 0 : e * (MD / 4) + md / 4][md % 4]),
              pr[e], o[md], 0, 0, 0);
    } else {
      // P^T in two 16-bit parts (high, and the residual): the P.V product
      // then carries the fp32 probabilities to ~2^-17, as the reference's fp32
      // weighted sum does, instead of the 2^-9 of one bf16 rounding.
      const u32x2 pb = {pack_pair<DT>(pr[0], pr[1]), pack_pair<DT>(pr[2], pr[3])};
      u32x2 pl;
      {
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned wd = pb[e >> 1];
          const unsigned short hb = (unsigned short)((e & 1) ? (wd >> 16) : (wd & 0xffffu));
          r[e] = pr[e] - (DT == DD_BF16 ? __uint_as_float((unsigned)hb << 16) : half_bits_to_float(hb));
        }
        pl = u32x2{pack_pair<DT>(r[0], r[1]), pack_pair<DT>(r[2], r[3])};
      }

      // Rows before the window start inside this chunk hold expired keys:
      // their V must not reach the MFMA (0 * NaN).
      if (t0 < s_lo) {
        const int r0 = 4 * kg;
#pragma unroll
        for (int md = 0; md < MD; ++md) {
          unsigned lo = va[md][0], hi = va[md][1];
          if (t0 + r0 + 0 < s_lo) lo &= 0xffff0000u;
          if (t0 + r0 + 1 < s_lo) lo &= 0x0000ffffu;
          if (t0 + r0 + 2 < s_lo) hi &= 0xffff0000u;
          if (t0 + r0 + 3 < s_lo) hi &= 0x0000ffffu;
          va[md] = u32x2{lo, hi};
        }
      }
#pragma unroll
      for (int md = 0; md < MD; ++md) o[md] = mfma16x16x16<DT>(va[md], pl, mfma16x16x16<DT>(va[md], pb, o[md]));
    }
  };

  // Prologue: NB chunks in flight, then the query operand (loaded before
  // them) is made visibly complete, so the loop carries no pending load the
  // compiler would wait for.
#pragma unroll
  for (int u = 0; u < NB; ++u) issue(u, u);
#pragma unroll
  for (int c = 0; c < NC; ++c) after_wait(qa[c]);
  after_wait(slope);
  // Chunk i: NB - 1 younger chunks (2 IPP loads each) stay in flight.  Full
  // groups of NB chunks run without guards and the last n % NB after the
  // loop, so that the loop body has one path and the accumulators keep
  // their registers across iterations.
  auto step = [&](int i, auto u_tag) __attribute__((always_inline)) {
    wait_vm<2 * IPP * (NB - 1)>();
    consume(i, u_tag);
  };
  int i0 = 0;
  for (; i0 + NB <= n; i0 += NB)
    static_for<NB>([&](auto u) __attribute__((always_inline)) { step(i0 + decltype(u)::value, u); });
  static_for<NB - 1>([&](auto u) __attribute__((always_inline)) {
    if (i0 + decltype(u)::value < n) step(i0 + decltype(u)::value, u);
  });
  wait_vm<0>();  // the trailing (empty) loads, before the ring is reused

  stream_epilogue<DT, D, NW>(p, s_ml, (float *)s_ring, o, m_run, lsum, w, lane, b, head0, G, split);
#endif  // __HIP_DEVICE_COMPILE__
}

template <int DT, int D, int NB, int NW>
int launch_stream(const DecodeParams &p, hipStream_t stream, int phase) {
  const long grid = (long)p.B * p.KH * p.gsub * p.splits;
  if (grid <= 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EINVAL;
  if (phase & 1) {
    hipLaunchKernelGGL((stream_kernel<DT, D, NB, NW>), dim3((unsigned)grid), dim3(64 * NW), 0, stream, p);
    DD_LAUNCH_CHECK();
  }
  if ((phase & 2) && p.splits > 1) {
    hipLaunchKernelGGL((merge_kernel<DT>), dim3((unsigned)((long)p.B * p.H)), dim3(p.DR < 256 ? p.DR : 256), 0,
                       stream, p, p.DR);
    DD_LAUNCH_CHECK();
  }
  return DD_OK;
}


// ---- int8 pages ------------------------------------------------------------
//
// Q8 pages (kv_quant.py:23-76 format: int8 rows + one fp16 scale per token,
// KV head and `group` channels; NG = D / group scales per row, NG = 1 or
// D / 32).  Same schedule as stream_kernel, but a wave consumes two 16-token
// chunks (32 keys) at a time, so that P.V is one v_mfma_f32_16x16x32 per 16
// dims: V^T comes from transposing byte reads (ds_read_b64_tr_b8), each lane
// receiving 8 keys of one dim, widened exactly to bf16/f16 in registers;
// K rows are read 8 bytes per lane and widened the same way.  Scales ride in
// the same stage: K scales multiply the logits, V scales the probabilities.
//
// Stage layout: K rows of both chunks (32 x D bytes), V rows (32 x D), then
// K scales and V scales of both chunks (4 x 32 NG bytes, room for NG = D/32).
// Row R = 16 chunk + r stores its 8-byte column c at c ^ i8_swz(R): with it
// the K reads (16 rows, 2 columns per half-wave) and the transposing V reads
// (8 rows x 2 columns per half-wave) hit 32 distinct 8-byte bank slots.
template <int D>
DD_DEV constexpr int i8_swz(int R) {
  const int hi = ((R >> 3) ^ (R >> 4)) & 1;
  if constexpr (D == 64) {
    return (((R >> 2) & 1) | (hi << 1)) << 1;
  } else if constexpr (D == 128) {
    return (((R >> 1) & 1) | (((R >> 2) & 1) << 1) | (hi << 2)) << 1;
  } else {
    return ((R & 1) | (((R >> 1) & 1) << 1) | (((R >> 2) & 1) << 2) | (hi << 3)) << 1;
  }
}

// int8 -> fp16 for the matrix cores: byte b (two's complement) becomes the
// fp16 number 1152 + b, exactly: b ^ 0x80 = b + 128 in [0, 255] is the low
// mantissa byte of an fp16 whose high byte is 0x64 (1024 + mantissa).  One
// XOR per 4 bytes and one byte permute per 2.
constexpr float kI8Offset = 1152.f;
DD_DEV u32x4 widen_i8x8_off(u32x2 w) {
  const unsigned a = w[0] ^ 0x80808080u, b = w[1] ^ 0x80808080u;
  constexpr unsigned kHi = 0x64646464u;
  // v_perm_b32(src0, src1, sel): bytes 0-3 of src1, 4-7 of src0
  return u32x4{__builtin_amdgcn_perm(a, kHi, 0x00050004u), __builtin_amdgcn_perm(a, kHi, 0x00070006u),
               __builtin_amdgcn_perm(b, kHi, 0x00050004u), __builtin_amdgcn_perm(b, kHi, 0x00070006u)};
}
DD_DEV unsigned cvt_pk_f16(float a, float b) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2_t{a, b}, f16x2_t));
}
// acc + lo(a) * lo(b) + hi(a) * hi(b) on fp16 pairs, fp32 accumulate
DD_DEV float dot2_f16(unsigned a, unsigned b, float acc) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), acc, false);
}

template <int QT, int D, int NG, int NB, int NW>
__global__ __launch_bounds__(64 * NW) void stream_i8_kernel(DecodeParams p) {
#if __HIP_DEVICE_COMPILE__
  constexpr int ROWB = D;               // bytes per token row
  constexpr int CHB = 16 * ROWB;        // one 16-token chunk of K (or V)
  constexpr int KOFF = 0, VOFF = 2 * CHB, SOFF0 = 4 * CHB;
  constexpr int SCB = 32 * NG;          // scale bytes of one chunk (16 tokens x NG x 2)
  constexpr int STAGE = 4 * CHB + 4 * D;  // scale room for NG up to D / 32
  constexpr int IPC = CHB / 1024;       // 16-byte DMA instructions per chunk
  constexpr int LPP = 4 * IPC + 4;      // loads per pair of chunks
  constexpr int CPR16 = ROWB / 16;
  constexpr int NC = D / 32;
  constexpr int MD = D / 16;
  constexpr int DP = D + 4;
  static_assert(IPC >= 1 && LPP * NB < 64 && NB >= 2 && NB <= 4, "vmcnt range, unrolled steps");
  static_assert(NG == 1 || NG == NC, "one scale per row or per 32 channels");
  static_assert((NB - 1) * STAGE + SOFF0 + 4 * SCB < 65536, "ds offset range");
  static_assert(NW * 16 * DP * 4 <= NW * NB * STAGE, "epilogue buffer fits the ring");

  __shared__ __align__(1024) char s_ring[NW * NB * STAGE];
  __shared__ float s_ml[NW][2][16];

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int n16 = lane & 15;
  const int kg = lane >> 4;

  // Workgroup (split, sequence, KV head, head group): with more than 16
  // query heads per KV head, gsub workgroups of up to 16 heads each.
  const int per_b = p.KH * p.gsub;
  const int nbkh = p.B * per_b;
  const int wg = xcd_remap(p, blockIdx.x, nbkh);
  const int split = wg / nbkh;
  const int bkh = wg - split * nbkh;
  const int b = bkh / per_b;
  const int vk = bkh - b * per_b;
  const int kh = vk / p.gsub;
  const int gofs = 16 * (vk - kh * p.gsub);   // first head of this workgroup within the group
  const int G = p.gsub > 1 ? min(16, p.G - gofs) : p.G;   // heads of this workgroup

  const long pos64 = p.pos[b];
  const int row = p.slots ? (int)p.slots[b] : 0;
  const int t_hi = pos64 + 1 < p.ctx_limit ? (int)pos64 + 1 : p.ctx_limit;
  int t_lo = 0;
  if (p.window > 0 && pos64 - p.window + 1 > 0) t_lo = (int)(pos64 - p.window + 1);
  int s_lo = split * p.split_tokens;
  int s_hi = s_lo + p.split_tokens;
  if (s_hi > t_hi) s_hi = t_hi;
  if (s_lo < t_lo) s_lo = t_lo;
  if (s_lo >= s_hi) return;
  const int pg_first = s_lo >> 4;
  const int pg_last = (s_hi - 1) >> 4;
  const long head0 = (long)b * p.H + (long)kh * p.G + gofs;
  const bool col_on = n16 < G;

  // The head size DR may be below the layout's D (one scale per row only):
  // rows are DR bytes in memory, the layout's dims DR .. D-1 are zero
  // queries and zero bytes in LDS, and they are never stored.
  const int DR = p.DR;
  u32x4 qa[NC];
  {
    const unsigned short *qb = (const unsigned short *)p.q;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qa[c] = col_on && 8 * kg + 32 * c < DR ? *(const u32x4 *)(qb + (head0 + n16) * DR + 8 * kg + 32 * c)
                                             : u32x4{0, 0, 0, 0};
  }
  float slope = (p.alibi && col_on) ? p.alibi[(long)kh * p.G + gofs + n16] * kLog2e : 0.f;

  const unsigned wbase = (unsigned)(size_t)(lds_void *)s_ring + (unsigned)(w * NB * STAGE);
  // K operand: row n16 of chunk ch, 8-byte column 4c + kg.
  unsigned k_addr[2][NC];
#pragma unroll
  for (int ch = 0; ch < 2; ++ch)
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int R = 16 * ch + n16;
      k_addr[ch][c] = wbase + KOFF + R * ROWB + 8 * ((4 * c + kg) ^ i8_swz<D>(R));
    }
  // V^T operand: lane a of group kg addresses key slot j = a / 2 (chunk j / 4,
  // row 4 kg + j % 4) and the 8 dims 16 md + 8 (a % 2).
  unsigned v_addr[MD];
  {
    const int a = lane & 15;
    const int j = a >> 1;
    const int R = 16 * (j >> 2) + 4 * kg + (j & 3);
#pragma unroll
    for (int md = 0; md < MD; ++md) v_addr[md] = wbase + VOFF + R * ROWB + 8 * ((2 * md + (a & 1)) ^ i8_swz<D>(R));
  }
  // Scales of this lane's keys (rows 4kg .. 4kg+3 of each chunk).
  const unsigned sc_addr = wbase + SOFF0 + 2 * (4 * kg * NG);

  const int first = w;  // pair index; chunks pg_first + 2 pair, +1
  const int npairs_all = (pg_last - pg_first) / 2 + 1;
  const int n = first < npairs_all ? (npairs_all - 1 - first) / NW + 1 : 0;

  const char *kplane = (const char *)p.k;
  const char *vplane = (const char *)p.v;
  const char *ksplane = (const char *)p.ks;
  const char *vsplane = (const char *)p.vs;
  const __attribute__((address_space(4))) int32_t *tab = (const __attribute__((address_space(4))) int32_t *)p.table;

  // Element (= byte) offset of a chunk's first row, -1 when unmapped or dead.
  auto chunk_row0 = [&](int pg, bool live_pair) __attribute__((always_inline)) -> long {
    long base = -1;
    if (!live_pair || pg > pg_last) return -1;
    if (p.paged) {
      if (row >= 0 && row < p.table_rows) {
        const int entry = pg >> p.chunk_shift;
        const long phys = tab[(long)row * p.table_w + entry];
        if (phys >= 0 && phys < p.capacity)
          base = ((phys * p.KH + kh) * (long)p.page + ((pg - (entry << p.chunk_shift)) << 4));
      }
    } else if (row >= 0 && row < p.capacity) {
      base = ((long)row * p.KH + kh) * (long)p.page + (long)pg * 16;
    }
    return base;
  };
  auto issue = [&](int i, int stage) __attribute__((always_inline)) {
    const int pair = first + i * NW;
    char *dst = s_ring + (w * NB + stage) * STAGE;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      const int pg = pg_first + 2 * pair + ch;
      long base = chunk_row0(pg, i < n);
      base = (long)uniform_ptr((const char *)base);
      const int live = base < 0 ? 0 : max(0, min(16, s_hi - pg * 16));
      const long rb = base < 0 ? 0 : base;  // token-row index
      const int bytes = uniform(live * DR);
      const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
          (void *)uniform_ptr(kplane + rb * DR), (short)0, bytes, kRawBufferWord3);
      const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
          (void *)uniform_ptr(vplane + rb * DR), (short)0, bytes, kRawBufferWord3);
      const int sbytes = uniform(base < 0 ? 0 : SCB);
      const __amdgpu_buffer_rsrc_t rks = __builtin_amdgcn_make_buffer_rsrc(
          (void *)uniform_ptr(ksplane + rb * 2 * NG), (short)0, sbytes, kRawBufferWord3);
      const __amdgpu_buffer_rsrc_t rvs = __builtin_amdgcn_make_buffer_rsrc(
          (void *)uniform_ptr(vsplane + rb * 2 * NG), (short)0, sbytes, kRawBufferWord3);
#pragma unroll
      for (int j = 0; j < IPC; ++j) {
        const int e = 64 * j + lane;
        const int r = e / CPR16;
        const int src16 = (e % CPR16) ^ (i8_swz<D>(16 * ch + r) >> 1);
        const unsigned off = 16 * src16 < DR ? (unsigned)(r * DR + 16 * src16) : 0x40000000u;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void *)(dst + KOFF + ch * CHB + 1024 * j), 16, off, 0,
                                                 0, kStreamLoadAux);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void *)(dst + VOFF + ch * CHB + 1024 * j), 16, off, 0,
                                                 0, kStreamLoadAux);
      }
      // SCB bytes each: only the first SCB / 4 lanes take part (an inactive
      // lane writes nothing), so neighbouring scale blocks stay intact.
      if (4 * lane < SCB) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rks, (lds_void *)(dst + SOFF0 + ch * SCB), 4, 4 * lane, 0, 0,
                                                 kStreamLoadAux);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rvs, (lds_void *)(dst + SOFF0 + 2 * SCB + ch * SCB), 4, 4 * lane,
                                                 0, 0, kStreamLoadAux);
      }
    }
  };

  // Everything enters the matrix cores as fp16 (see the int8 section note):
  // K and V bytes as exact fp16 values b + 1152, the query scaled by a power
  // of two 2^-qe (chosen per head so that its largest component is about
  // 2^14: no fp16 overflow, nothing relevant in subnormals) and rounded to
  // fp16 -- exact for bf16 queries, whose 8-bit significands fit -- and the
  // probabilities p * v_scale as fp16.  The 1152 offsets come out of S^T
  // through the column sums of Q (qoff) and out of O^T through the column
  // sums of the fp16 P^T operands (psum); 2^qe goes back into the logit scale.
  float qf[NC][8];
  float qmax = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    after_wait(qa[c]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      qf[c][2 * j] = QT == DD_BF16 ? bf16_lo(qa[c][j]) : f16_lo(qa[c][j]);
      qf[c][2 * j + 1] = QT == DD_BF16 ? bf16_hi(qa[c][j]) : f16_hi(qa[c][j]);
      qmax = fmaxf(qmax, fmaxf(__builtin_fabsf(qf[c][2 * j]), __builtin_fabsf(qf[c][2 * j + 1])));
    }
  }
  qmax = xor32_max(xor16_max(qmax));   // over the head's D components
  const int qe = qmax > 0.f && __builtin_isfinite(qmax) ? __builtin_amdgcn_frexp_expf(qmax) - 15 : 0;
  const float lscale = __builtin_ldexpf(p.scale_log2, qe);   // logit scale of the scaled query
  u32x4 qh[NC];
  float qoff[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      qh[c][j] = cvt_pk_f16(__builtin_ldexpf(qf[c][2 * j], -qe), __builtin_ldexpf(qf[c][2 * j + 1], -qe));
    float qs = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) qs = dot2_f16(qh[c][j], 0x3C003C00u, qs);
    qoff[c] = kI8Offset * xor32_sum(xor16_sum(qs));   // column n16's sum over the 32 dims of chunk c
  }

  // NG == 1: the S^T accumulator starts at minus the query's offset sum, so
  // the MFMAs leave q.k itself
  float qo_all = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) qo_all += qoff[c];
  const f32x4 s_init = {-qo_all, -qo_all, -qo_all, -qo_all};

  f32x4 o[MD];
#pragma unroll
  for (int md = 0; md < MD; ++md) o[md] = f32x4{0.f, 0.f, 0.f, 0.f};
  // running max of logit + exponent of the V scale (+ kExpBias)
  constexpr float kExpBias = NG == 1 ? 14.f : 0.f;
  float m_run = kNegInf;
  float lsum = 0.f;        // sum of exp2(logit - m_run)
  float psum[NG];          // sums of the fp16 P^T operands (this lane's keys)
#pragma unroll
  for (int g = 0; g < NG; ++g) psum[g] = 0.f;

  auto consume = [&](int i, auto stage_tag) __attribute__((always_inline)) {
    constexpr int SO = decltype(stage_tag)::value * STAGE;
    const int t0 = (pg_first + 2 * (first + i * NW)) * 16;  // first key of the pair
    u32x2 k8[2][NC];
    u32x2 v8[MD];
    u32x2 ks8[2][NG], vs8[2][NG];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int c = 0; c < NC; ++c) k8[ch][c] = lds_read_b64<SO>(k_addr[ch][c]);
#pragma unroll
    for (int md = 0; md < MD; ++md) v8[md] = lds_read_tr8<SO>(v_addr[md]);
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        ks8[ch][g] = lds_read_b64<SO>(sc_addr + ch * SCB + 8 * g);
        vs8[ch][g] = lds_read_b64<SO>(sc_addr + 2 * SCB + ch * SCB + 8 * g);
      }
    wait_lds();
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
      for (int c = 0; c < NC; ++c) after_wait(k8[ch][c]);
#pragma unroll
      for (int g = 0; g < NG; ++g) {
        after_wait(ks8[ch][g]);
        after_wait(vs8[ch][g]);
      }
    }
#pragma unroll
    for (int md = 0; md < MD; ++md) after_wait(v8[md]);
    issue(i + NB, decltype(stage_tag)::value);

    // scale of key 4kg + e of chunk ch, channel group g (fp16 at index e NG + g)
    auto scale_half = [&](const u32x2 (&sc)[2][NG], int ch, int e, int g) __attribute__((always_inline)) {
      const int idx = e * NG + g;
      const unsigned wd = sc[ch][idx >> 2][(idx >> 1) & 1];
      return __builtin_bit_cast(f16x2, wd)[idx & 1];
    };
    auto scale_of = [&](const u32x2 (&sc)[2][NG], int ch, int e, int g) __attribute__((always_inline)) {
      return (float)scale_half(sc, ch, e, g);
    };
    // x * scale in one mixed-precision FMA (the fp16 scale is read in place)
    auto times_scale = [&](float x, const u32x2 (&sc)[2][NG], int ch, int e, int g) __attribute__((always_inline)) {
      return __builtin_fmaf(x, (float)scale_half(sc, ch, e, g), 0.f);
    };
    // Biased exponent E of a V scale, from its fp16 bits: a normal scale
    // lies in [2^(E-15), 2^(E-14)), so E - 14 bounds its frexp exponent
    // (zero and subnormal scales get the bound -14).  The 14 is left in y
    // and the running max (kExpBias) and taken out of the offset once.
    auto scale_exp = [&](const u32x2 (&sc)[2][NG], int ch, int e) __attribute__((always_inline)) {
      const int idx = e * NG;
      const unsigned wd = sc[ch][idx >> 2][(idx >> 1) & 1];
      return (float)__builtin_amdgcn_ubfe(wd, (idx & 1) ? 26u : 10u, 5u);
    };
    // The common case -- every key of the pair inside [s_lo, s_hi), no ALiBi,
    // no relative bias -- runs a copy of the step without masks or bias terms.
    auto body = [&](auto fast_tag) __attribute__((always_inline)) {
    constexpr bool FAST = decltype(fast_tag)::value;
    // One scale per row and every key live: the logit is kept as
    // x = q.k * k_scale and the logit scale folded into the FMAs that use it.
    constexpr bool FOLD = FAST && NG == 1;
    const float xmul = FOLD ? lscale : 1.f;
    // logits x * xmul = key t0 + 16 ch + 4 kg + e for head n16; y adds the
    // exponent of the key's largest V scale (the quantity the running max
    // tracks)
    float x[2][4], y[2][4];
    bool lv[2][4];                        // key inside [s_lo, s_hi)
    float mx = kNegInf;
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      f32x4 sacc = {0.f, 0.f, 0.f, 0.f};
      if constexpr (NG == 1) {
        sacc = s_init;
#pragma unroll
        for (int c = 0; c < NC; ++c) sacc = mfma16x16x32<DD_F16>(widen_i8x8_off(k8[ch][c]), qh[c], sacc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sacc[e] = times_scale(sacc[e], ks8, ch, e, 0);
          if constexpr (!FOLD) sacc[e] *= lscale;
        }
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const f32x4 part = mfma16x16x32<DD_F16>(widen_i8x8_off(k8[ch][c]), qh[c], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int e = 0; e < 4; ++e) sacc[e] += scale_of(ks8, ch, e, c) * (part[e] - qoff[c]);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) sacc[e] *= lscale;
      }
      float rb[4] = {0.f, 0.f, 0.f, 0.f};
      if (!FAST && p.rel) {  // workgroup-uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int t = t0 + 16 * ch + 4 * kg + e;
          const long dist = pos64 - t > 0 ? pos64 - t : 0;
          rb[e] = p.rel[((long)kh * p.G + gofs + (col_on ? n16 : 0)) * p.rel_buckets +
                        rel_bucket((int)dist, p.rel_buckets, p.rel_denom)] * kLog2e;
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = t0 + 16 * ch + 4 * kg + e;
        const bool live = FAST || (t >= s_lo && t < s_hi);
        const float v = FAST ? sacc[e] : sacc[e] + slope * (float)t + rb[e];
        // Exponent of the key's largest V scale; dead keys' scales may be
        // garbage: they enter P as 0.
        float ex = 0.f;
        if constexpr (NG == 1) {
          ex = live ? scale_exp(vs8, ch, e) : 0.f;
        } else {
          // From the fp16 bits: scales are >= 0, so the largest bit pattern
          // is the largest scale, and a normal one with biased exponent E
          // lies in [2^(E-15), 2^(E-14)) (frexp's exponent E - 14).  The
          // scales are re-read from vs8 where P is formed, not held here.
          unsigned mh = 0;
#pragma unroll
          for (int m = 0; m < NG / 2; ++m) {
            const int k = (e * NG) / 2 + m;
            const unsigned wd = vs8[ch][k >> 1][k & 1];
            mh = max(mh, max(wd & 0xffffu, wd >> 16));
          }
          ex = live && mh ? (float)((int)((mh >> 10) & 31u) - 14) : 0.f;   // (kExpBias 0)
        }
        lv[ch][e] = live;
        x[ch][e] = live ? v : kNegInf;
        y[ch][e] = live ? __builtin_fmaf(v, xmul, ex) : kNegInf;
        mx = fmaxf(mx, y[ch][e]);
      }
    }
    mx = xor32_max(xor16_max(mx));
    const bool up = mx > m_run + kStreamSlack;
    if (__builtin_amdgcn_ballot_w64(up)) {
      const float mn = up ? mx : m_run;
      const float alpha = up ? (m_run == kNegInf ? 0.f : fast_exp2(m_run - mn)) : 1.f;
      m_run = mn;
      lsum *= alpha;
#pragma unroll
      for (int g = 0; g < NG; ++g) psum[g] *= alpha;
#pragma unroll
      for (int md = 0; md < MD; ++md) o[md] *= alpha;
    }
    const float mu = m_run == kNegInf ? 0.f : m_run - kExpBias;
    // p = exp2(x - mu) <= 2^(8 - exponent of the key's V scale), so every
    // p * v_scale <= 2^8 fits fp16; dead keys have p = 0.
    float pr[2][4];
#pragma unroll
    for (int ch = 0; ch < 2; ++ch)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pr[ch][e] = fast_exp2(__builtin_fmaf(x[ch][e], xmul, -mu));
        lsum += pr[ch][e];
      }
    // P^T operand per V scale group: slot j < 4 is key 4kg + j of chunk 0,
    // slot j >= 4 key 4kg + j - 4 of chunk 1.
    u32x4 pb[NG];
#pragma unroll
    for (int g = 0; g < NG; ++g) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int ch = j >> 1, e = 2 * (j & 1);
        // (a dead key's scale may be garbage; its p is 0)
        const float p0 = lv[ch][e] ? times_scale(pr[ch][e], vs8, ch, e, g) : 0.f;
        const float p1 = lv[ch][e + 1] ? times_scale(pr[ch][e + 1], vs8, ch, e + 1, g) : 0.f;
        pb[g][j] = cvt_pk_f16(p0, p1);
        psum[g] = dot2_f16(pb[g][j], 0x3C003C00u, psum[g]);
      }
    }
#pragma unroll
    for (int md = 0; md < MD; ++md) {
      const int g = NG == 1 ? 0 : (16 * md) / 32;
      o[md] = mfma16x16x32<DD_F16>(widen_i8x8_off(v8[md]), pb[g], o[md]);
    }
    };
    if (t0 >= s_lo && t0 + 32 <= s_hi && !p.alibi && !p.rel) {
      body(std::true_type{});
    } else {
      body(std::false_type{});
    }
  };

#pragma unroll
  for (int u = 0; u < NB; ++u) issue(u, u);
  after_wait(slope);
  // Full groups of NB pairs run without guards and the last n % NB after
  // the loop (see stream_kernel).
  auto step = [&](int i, auto u_tag) __attribute__((always_inline)) {
    wait_vm<LPP * (NB - 1)>();
    consume(i, u_tag);
  };
  int i0 = 0;
  for (; i0 + NB <= n; i0 += NB)
    static_for<NB>([&](auto u) __attribute__((always_inline)) { step(i0 + decltype(u)::value, u); });
  static_for<NB - 1>([&](auto u) __attribute__((always_inline)) {
    if (i0 + decltype(u)::value < n) step(i0 + decltype(u)::value, u);
  });
  wait_vm<0>();

  // remove the V offsets: O^T row d of head n16 holds 1152 * (sum of that
  // head's fp16 P over all keys, V group of d) too
#pragma unroll
  for (int g = 0; g < NG; ++g) psum[g] = kI8Offset * xor32_sum(xor16_sum(psum[g]));
#pragma unroll
  for (int md = 0; md < MD; ++md) o[md] -= psum[NG == 1 ? 0 : (16 * md) / 32];

  stream_epilogue<QT, D, NW>(p, s_ml, (float *)s_ring, o, m_run - kExpBias, lsum, w, lane, b, head0, G, split);
#endif  // __HIP_DEVICE_COMPILE__
}

template <int QT, int D, int NG, int NB, int NW>
int launch_stream_i8(const DecodeParams &p_in, hipStream_t stream, int phase) {
  DecodeParams p = p_in;
  const long grid = (long)p.B * p.KH * p.gsub * p.splits;
  if (grid <= 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EINVAL;
  // KV heads per 128-byte line of scales (the line holds whole blocks of
  // page * NG fp16 scales when that block is at most 64 bytes)
  const int block_bytes = p.page * NG * 2;
  p.xcd_units = 1;
  if (p.gsub == 1 && block_bytes <= 64) {
    const int u = 128 / block_bytes;
    if (p.KH % u == 0) p.xcd_units = u;
  }
  if (phase & 1) {
    hipLaunchKernelGGL((stream_i8_kernel<QT, D, NG, NB, NW>), dim3((unsigned)grid), dim3(64 * NW), 0, stream, p);
    DD_LAUNCH_CHECK();
  }
  if ((phase & 2) && p.splits > 1) {
    hipLaunchKernelGGL((merge_kernel<QT>), dim3((unsigned)((long)p.B * p.H)), dim3(p.DR < 256 ? p.DR : 256), 0,
                       stream, p, p.DR);
    DD_LAUNCH_CHECK();
  }
  return DD_OK;
}

}  // namespace dd_decode
