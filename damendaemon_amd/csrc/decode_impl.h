// Ragged paged / slotted split-KV decode attention for gfx950.
//
// Replaces the reference's Triton `_attention` + `_merge` pair
// (damendaemon/kernels.py:134-210) behind the same semantics:
//   * one query row per sequence; keys 0..pos (optionally a trailing window),
//     addressed through page_table[slot, t / page_size] (kernels.py:151-154)
//     or a contiguous slot (kernels.py:155-157);
//   * logits = q.k * scale (+ ALiBi slope * t, + T5 relative bias),
//     fp32 softmax, fp32 accumulation; optional sink logits enlarge the
//     denominator once (kernels.py:168-176, 198-206);
//   * long contexts are split; splits are combined by log-sum-exp.
//
// The streamed kernels of decode_stream.h take every 16-bit and fp32 case,
// int8 pages with one scale per row at every head size and int8 pages with
// group-32 scales at 64, 128 and 256; decode_kernel below, the general
// kernel, serves the remaining int8 cases.
//
// General kernel (not a translation of the Triton kernel):
//   * one workgroup = one (sequence, KV head, split); its 4 wavefronts take
//     interleaved 16-token pages, so every K/V byte is read once for the
//     whole GQA group (the reference re-reads K/V per query head);
//   * q.k for a 16-token page is a 16x16x32 MFMA (bf16/f16; int8 pages are
//     widened exactly in registers), rows = the group's query heads,
//     columns = the page's tokens;
//   * p.v runs on the VALU from 16-byte coalesced loads, each lane owning a
//     fixed 16-byte slice of the head dimension;
//   * every wavefront keeps its own online softmax; the four are merged in
//     LDS at the end of the split, and splits by a second small kernel.
#pragma once
#include <type_traits>

#include "common.h"

namespace dd_decode {

struct DecodeParams {
  const void *q;
  const void *k;
  const void *v;
  const unsigned short *ks;
  const unsigned short *vs;
  const int64_t *pos;
  const int64_t *slots;
  const int32_t *table;
  void *out;
  float *part;
  float *lse;
  const float *alibi;
  const float *rel;
  const float *sinks;
  long capacity;  // pages (paged) or slots (slotted); guards addressing
  int B, H, KH, G;
  int DR;         // head size: row length of Q, K, V, the output and the partials
  int gsub;       // workgroups per (sequence, KV head): query heads in groups of <= 16
  int table_w, table_rows;
  int page;       // page_size (paged) or context (slotted)
  int ctx_limit;  // table_w * page (paged) or context (slotted)
  int window;
  int splits, split_tokens;
  int group, ngroups;
  int rel_buckets;
  float rel_denom;
  float scale_log2;
  int paged;
  int chunk_shift;  // log2(page / 16) for paged caches
  int xcd_units;   // int8 pages: KV heads whose scale blocks share one 128-byte line (1 = no remap)
};

// Workgroup id -> logical (split, sequence, KV head) index for the int8
// kernel.  Workgroup w runs on XCD w % 8, and each XCD has its own L2.  The
// fp16 scale block of one (page, KV head) is page * groups * 2 bytes (32 B
// for 16-token pages with one scale per row), so xcd_units consecutive KV
// heads share each 128-byte line: blocks of 8 * xcd_units workgroups are
// permuted so that those heads run on one XCD and the line is fetched
// once, not once per XCD.  The ordering of splits is kept.
DD_DEV int xcd_remap(const DecodeParams &p, int wg, int nbkh) {
  const int u = p.xcd_units;
  if (u <= 1) return wg;
  const int split = wg / nbkh;
  int inner = wg - split * nbkh;
  const int blk = 8 * u;
  if (inner < (nbkh / blk) * blk) {
    const int base = inner / blk;
    const int rem = inner - base * blk;
    inner = (base * 8 + (rem & 7)) * u + (rem >> 3);
  }
  return split * nbkh + inner;
}

constexpr int kWaves = 4;
#ifndef DD_DECODE_PD
#define DD_DECODE_PD 1
#endif
#ifndef DD_DECODE_PD_I8
#define DD_DECODE_PD_I8 2
#endif
constexpr float kNegInf = -__builtin_inff();

// Element offset of the first token of 16-token chunk `pg` of (row, kh), or
// -1 when the chunk is not addressable (unallocated page-table entry).
DD_DEV long chunk_base(const DecodeParams &p, int row, int kh, int pg, int D) {
  if (p.paged) {
    if (row < 0 || row >= p.table_rows) return -1;
    const int entry = pg >> p.chunk_shift;
    const int within = (pg - (entry << p.chunk_shift)) * 16;
    const long phys = p.table[(long)row * p.table_w + entry];
    if (phys < 0 || phys >= p.capacity) return -1;
    return ((phys * p.KH + kh) * (long)p.page + within) * (long)D;
  }
  if (row < 0 || row >= p.capacity) return -1;
  return (((long)row * p.KH + kh) * (long)p.page + (long)pg * 16) * (long)D;
}

// 2^x on the hardware exp unit (inputs here are <= 0 or -inf; results that
// would be denormal only weight negligible terms).
DD_DEV float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Convert 8 signed bytes to 8 exact bf16 / f16 MFMA operands.
template <int QT>
DD_DEV u32x4 widen_i8x8(u32x2 w) {
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const unsigned word = w[j >> 1];
    const int a = (int)(signed char)(word >> (16 * (j & 1)));
    const int b = (int)(signed char)(word >> (16 * (j & 1) + 8));
    if constexpr (QT == DD_BF16) {
      r[j] = (__float_as_uint((float)a) >> 16) | (__float_as_uint((float)b) & 0xffff0000u);
    } else {
      r[j] = (unsigned)float_to_f16_bits((float)a) | ((unsigned)float_to_f16_bits((float)b) << 16);
    }
  }
  return r;
}

template <int QT>
DD_DEV f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (QT == DD_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// Decode 16 bytes of V (one lane's slice of one token) into VE floats.
template <int KVT, int VE>
DD_DEV void widen_v(const u32x4 &w, float (&x)[VE]) {
  if constexpr (KVT == DD_F32) {
#pragma unroll
    for (int e = 0; e < 4; ++e) x[e] = __uint_as_float(w[e]);
  } else if constexpr (KVT == DD_BF16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf16_lo(w[e]);
      x[2 * e + 1] = bf16_hi(w[e]);
    }
  } else if constexpr (KVT == DD_F16) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = f16_lo(w[e]);
      x[2 * e + 1] = f16_hi(w[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) x[e] = (float)(int)(signed char)(w[e >> 2] >> (8 * (e & 3)));
  }
}

// T5 relative-position bucket, restating kernels.py:162-167.
DD_DEV int rel_bucket(int distance, int buckets, float denom) {
  const int exact = buckets / 2;
  if (distance < exact) return distance;
  const int d = distance > exact ? distance : exact;
  const int large = exact + (int)(logf((float)d / (float)exact) / denom * (float)(buckets - exact));
  return large < buckets - 1 ? large : buckets - 1;
}

#ifdef DD_DECODE_WAVES_PER_EU
#define DD_DECODE_ATTR __attribute__((amdgpu_waves_per_eu(DD_DECODE_WAVES_PER_EU)))
#else
#define DD_DECODE_ATTR
#endif

template <int KVT, int QT, int D, int GB>
__global__ __launch_bounds__(256) DD_DECODE_ATTR void decode_kernel(DecodeParams p) {
  constexpr bool kMfma = KVT != DD_F32;
  constexpr int VE = KVT == DD_F32 ? 4 : (KVT == DD_I8 ? 16 : 8);  // V elems per 16 B
  constexpr int LPT = D / VE;                                       // lanes per V token
  constexpr int TPI = 64 / LPT;                                     // tokens per V load
  constexpr int NIT = (16 + TPI - 1) / TPI;                         // V loads per page
  constexpr int NC = D / 32;                                        // MFMA k-chunks
  constexpr int NC4 = D / 16;                                       // fp32 k-chunks
  constexpr int KB = KVT == DD_F32 ? 4 : (KVT == DD_I8 ? 1 : 2);    // bytes per element
  constexpr int PD = KVT == DD_I8 ? DD_DECODE_PD_I8 : DD_DECODE_PD;  // pages in flight per wave
  // The real head size DR (a multiple of 8, of 16 for int8; at most D) sets every row
  // stride; the dims DR .. D-1 of the layout hold zero queries (so the K
  // bytes read for them, a clamped copy of the row's first dims, add
  // nothing) and V columns that are never stored.
  const int DR = p.DR;

  __shared__ float s_p[kWaves][16][GB];       // per-wave page probabilities
  __shared__ float s_o[GB][D];                // cross-wave output accumulator
  __shared__ float s_ml[kWaves][2][GB];       // per-wave running max / sum
  __shared__ float s_q[kMfma ? 1 : GB][kMfma ? 1 : D];  // fp32 query (VALU q.k)

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int r = lane >> 4;
  const int tl = lane & 15;

  // Split-major order: every sequence's first split is dispatched before any
  // second split, so full-length splits run first and the short (or empty)
  // final splits fill the tail of the launch.  With more than 16 query heads
  // per KV head, (sequence, KV head) is covered by gsub workgroups of up to
  // 16 heads each.
  const int wg = blockIdx.x;
  const int per_b = p.KH * p.gsub;
  const int nbkh = p.B * per_b;
  const int split = wg / nbkh;
  const int bkh = wg - split * nbkh;
  const int b = bkh / per_b;
  const int vk = bkh - b * per_b;
  const int kh = vk / p.gsub;
  const int sub = vk - kh * p.gsub;
  const int G = p.gsub > 1 ? min(GB, p.G - sub * GB) : p.G;

  const long pos64 = p.pos[b];
  const int row = p.slots ? (int)p.slots[b] : 0;
  int t_hi = pos64 + 1 < p.ctx_limit ? (int)pos64 + 1 : p.ctx_limit;
  int t_lo = 0;
  if (p.window > 0 && pos64 - p.window + 1 > 0) t_lo = (int)(pos64 - p.window + 1);
  int s_lo = split * p.split_tokens;
  int s_hi = s_lo + p.split_tokens;
  if (s_hi > t_hi) s_hi = t_hi;
  if (s_lo < t_lo) s_lo = t_lo;
  if (s_lo >= s_hi) return;  // empty split: the merge never reads it

  const int pg_first = s_lo >> 4;
  const int pg_last = (s_hi - 1) >> 4;
  const long head0 = (long)b * p.H + (long)kh * p.G + (long)sub * GB;

  // ---- query operand ----------------------------------------------------
  u32x4 qa[kMfma ? NC : 1];
  if constexpr (kMfma) {
    const unsigned short *qb = (const unsigned short *)p.q;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      if (tl < G && 8 * r + 32 * c < DR) {
        qa[c] = *(const u32x4 *)(qb + (head0 + tl) * DR + 8 * r + 32 * c);
      } else {
        qa[c] = u32x4{0, 0, 0, 0};
      }
    }
  } else {
    for (int i = threadIdx.x; i < G * D; i += 256) {
      const int d = i % D;
      s_q[i / D][d] = d < DR ? load_as<QT>(p.q, (head0 + i / D) * DR + d) : 0.f;
    }
    __syncthreads();
  }

  // ---- per-wave online softmax state ------------------------------------
  float m_run[GB];
  float acc[GB][VE];
  float lsum[4];
#pragma unroll
  for (int h = 0; h < GB; ++h) {
    m_run[h] = kNegInf;
#pragma unroll
    for (int e = 0; e < VE; ++e) acc[h][e] = 0.f;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) lsum[i] = 0.f;

  const char *kbytes = (const char *)p.k;
  const char *vbytes = (const char *)p.v;
  const int vtok_lane = lane / LPT;        // token within a V load
  const int vdim = VE * (lane % LPT);      // first dim of this lane's V slice
  const int vdim_ld = vdim < DR ? vdim : 0;  // (a lane past DR reads the row's first dims)
  const bool v_lane_on = lane < LPT * TPI;

  // Registers of one page: raw K (MFMA layout), raw V (VALU layout) and,
  // for int8 pages, the per-token scales.  The next page is loaded into a
  // second set while the current one is consumed.
  struct PageRegs {
    long base;
    u32x4 k[kMfma ? NC : NC4];
    u32x2 k8[KVT == DD_I8 ? NC : 1];
    u32x4 v[NIT];
    float ks[KVT == DD_I8 ? NC : 1];
    float vs[KVT == DD_I8 ? NIT : 1];
  };
  // All loads are unconditional: invalid or missing tokens read a clamped,
  // always-mapped row (page 0 when the table entry is unallocated, the last
  // row of the slot for a slotted cache).  Their logits are masked to -inf
  // and their V rows are zeroed before use.
  constexpr bool kAllLanes = LPT * TPI == 64 && NIT * TPI == 16;
  // Per-lane byte offsets inside a 16-token chunk are loop invariant; the
  // chunk base is wave-uniform, so each load is SGPR base + 32-bit offset.
  auto load_page = [&](int pg, PageRegs &R) {
    const long base = chunk_base(p, row, kh, pg, DR);
    R.base = base;
    const long sb = base < 0 ? 0 : base;
    const int lim = p.paged ? 15 : min(15, p.page - 1 - pg * 16);
    const unsigned krow = (unsigned)min(tl, lim);
    const char *kb = kbytes + KB * sb;  // wave-uniform
    const char *vb = vbytes + KB * sb;
    if constexpr (KVT == DD_I8) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d0 = 8 * r + 32 * c < DR ? 8 * r + 32 * c : 0;
        R.k8[c] = __builtin_nontemporal_load((const u32x2 *)(kb + (krow * DR + d0)));
      }
      const unsigned short *ksc = p.ks + (sb / DR) * p.ngroups;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        R.ks[c] = (32 * c < DR && (c == 0 || p.group != DR)) ? half_bits_to_float(ksc[krow * p.ngroups + (32 * c) / p.group])
                                                             : 0.f;
      }
    } else if constexpr (kMfma) {
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int d0 = 8 * r + 32 * c < DR ? 8 * r + 32 * c : 0;
        R.k[c] = __builtin_nontemporal_load((const u32x4 *)(kb + 2u * (krow * DR + d0)));
      }
    } else {
#pragma unroll
      for (int c = 0; c < NC4; ++c) {
        const int d0 = 4 * r + 16 * c < DR ? 4 * r + 16 * c : 0;
        R.k[c] = __builtin_nontemporal_load((const u32x4 *)(kb + 4u * (krow * DR + d0)));
      }
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const unsigned vrow = (unsigned)min(it * TPI + vtok_lane, lim);
      R.v[it] = __builtin_nontemporal_load((const u32x4 *)(vb + KB * (vrow * DR + vdim_ld)));
      if constexpr (KVT == DD_I8) R.vs[it] = half_bits_to_float(p.vs[(sb / DR) * p.ngroups + vrow * p.ngroups + vdim_ld / p.group]);
    }
  };

  // Consume one page: logits, online softmax, p.v.
  auto consume = [&](int pg, PageRegs &cur) {
    const long base = cur.base;
    const int t0 = pg * 16;
    const int tk = t0 + tl;
    const bool kval = base >= 0 && tk >= s_lo && tk < s_hi;
    if (!kAllLanes || base < 0 || t0 < s_lo || t0 + 16 > s_hi) {
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int tv = it * TPI + vtok_lane;
        const bool vv = v_lane_on && tv < 16 && base >= 0 && t0 + tv >= s_lo && t0 + tv < s_hi;
        if (!vv) cur.v[it] = u32x4{0, 0, 0, 0};
        if constexpr (KVT == DD_I8) cur.vs[it] = vv ? cur.vs[it] : 0.f;
      }
    }
    if constexpr (KVT == DD_I8) {
#pragma unroll
      for (int c = 0; c < NC; ++c) cur.ks[c] = kval ? cur.ks[c] : 0.f;
    }

    // -- logits: lane holds token tl for heads 4r+i --
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
    if constexpr (KVT == DD_I8) {
      if (p.group == DR) {
#pragma unroll
        for (int c = 0; c < NC; ++c) s = mfma16x16x32<QT>(qa[c], widen_i8x8<QT>(cur.k8[c]), s);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] *= cur.ks[0];
      } else {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const f32x4 part = mfma16x16x32<QT>(qa[c], widen_i8x8<QT>(cur.k8[c]),
                                              f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int i = 0; i < 4; ++i) s[i] += cur.ks[c] * part[i];
        }
      }
    } else if constexpr (kMfma) {
#pragma unroll
      for (int c = 0; c < NC; ++c) s = mfma16x16x32<QT>(qa[c], cur.k[c], s);
    } else {
      float part[GB];
#pragma unroll
      for (int h = 0; h < GB; ++h) part[h] = 0.f;
#pragma unroll
      for (int c = 0; c < NC4; ++c) {
#pragma unroll
        for (int h = 0; h < GB; ++h) {
          const float *qrow = &s_q[h < G ? h : 0][4 * r + 16 * c];
          part[h] += qrow[0] * __uint_as_float(cur.k[c][0]) + qrow[1] * __uint_as_float(cur.k[c][1]) +
                     qrow[2] * __uint_as_float(cur.k[c][2]) + qrow[3] * __uint_as_float(cur.k[c][3]);
        }
      }
#pragma unroll
      for (int h = 0; h < GB; ++h) {
        part[h] += shfl(part[h], lane ^ 16);
        part[h] += shfl(part[h], lane ^ 32);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float x = 0.f;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          if (4 * rr + i < GB && r == rr) x = part[4 * rr + i];
        }
        s[i] = x;
      }
    }

#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int hg = 4 * r + i;  // head within the group
      float x = s[i] * p.scale_log2;
      if (p.alibi && hg < G) x += p.alibi[head0 - (long)b * p.H + hg] * kLog2e * (float)tk;
      if (p.rel && hg < G) {
        const long dist = pos64 - tk > 0 ? pos64 - tk : 0;
        const int bucket = rel_bucket((int)dist, p.rel_buckets, p.rel_denom);
        x += p.rel[(head0 - (long)b * p.H + hg) * p.rel_buckets + bucket] * kLog2e;
      }
      s[i] = kval ? x : kNegInf;
    }

    // -- page maxima per head, broadcast as wave-uniform values --
    float rmax[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rmax[i] = row16_max(s[i]);
    float m_use[GB], alpha[GB];
    bool rescale = false;
#pragma unroll
    for (int h = 0; h < GB; ++h) {
      const float mb = read_lane(rmax[h & 3], 16 * ((h >> 2) & 3));
      const float mn = fmaxf(m_run[h], mb);
      alpha[h] = mn == kNegInf ? 1.f : fast_exp2(m_run[h] - mn);
      m_use[h] = mn == kNegInf ? 0.f : mn;
      rescale |= alpha[h] != 1.f;
      m_run[h] = mn;
    }
    if (rescale) {
#pragma unroll
      for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[h][e] *= alpha[h];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float a = alpha[i < GB ? i : 0];
#pragma unroll
        for (int rr = 1; rr < 4; ++rr) {
          if (4 * rr + i < GB && r == rr) a = alpha[4 * rr + i];
        }
        lsum[i] *= a;
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mm = m_use[i < GB ? i : 0];
#pragma unroll
      for (int rr = 1; rr < 4; ++rr) {
        if (4 * rr + i < GB && r == rr) mm = m_use[4 * rr + i];
      }
      const float pr = fast_exp2(s[i] - mm);
      lsum[i] += pr;
      const int hg = 4 * r + i;
      if (hg < G && hg < GB) s_p[w][tl][hg] = pr;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    // -- p.v --
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      int tv = it * TPI + vtok_lane;
      tv = tv < 16 ? tv : 15;
      float pv[GB];
#pragma unroll
      for (int h = 0; h < GB; ++h) pv[h] = s_p[w][tv][h];
      if constexpr (KVT == DD_I8) {
#pragma unroll
        for (int h = 0; h < GB; ++h) pv[h] *= cur.vs[it];
      }
      float x[VE];
      widen_v<KVT, VE>(cur.v[it], x);
#pragma unroll
      for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[h][e] += pv[h] * x[e];
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  // Register ring: this wave's page i is pg_first + w + i*kWaves and lives in
  // register set i % PD; PD pages are in flight while one is consumed.  The
  // loop is unrolled by PD so every set has static register names.
  const int first = pg_first + w;
  const int n_pages = first <= pg_last ? (pg_last - first) / kWaves + 1 : 0;
  PageRegs ring[PD];
#pragma unroll
  for (int u = 0; u < PD; ++u) {
    if (u < n_pages) load_page(first + u * kWaves, ring[u]);
  }
  for (int i = 0; i < n_pages; i += PD) {
#pragma unroll
    for (int u = 0; u < PD; ++u) {
      if (i + u < n_pages) {
        consume(first + (i + u) * kWaves, ring[u]);
        if (i + u + PD < n_pages) load_page(first + (i + u + PD) * kWaves, ring[u]);
      }
    }
  }

  // ---- reduce inside the wave ---------------------------------------------
  float lw[GB];
  {
    float rs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) rs[i] = row16_sum(lsum[i]);
#pragma unroll
    for (int h = 0; h < GB; ++h) lw[h] = read_lane(rs[h & 3], 16 * ((h >> 2) & 3));
  }
  if constexpr ((TPI & (TPI - 1)) == 0 && (LPT & (LPT - 1)) == 0) {
#pragma unroll
    for (int off = LPT; off < LPT * TPI; off <<= 1) {
#pragma unroll
      for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int e = 0; e < VE; ++e) acc[h][e] += shfl(acc[h][e], lane ^ off);
      }
    }
  } else {
    float tot[GB][VE];
#pragma unroll
    for (int h = 0; h < GB; ++h) {
#pragma unroll
      for (int e = 0; e < VE; ++e) tot[h][e] = acc[h][e];
    }
#pragma unroll
    for (int g = 1; g < TPI; ++g) {
      const int src = (lane + g * LPT) & 63;
#pragma unroll
      for (int h = 0; h < GB; ++h) {
#pragma unroll
        for (int e = 0; e < VE; ++e) tot[h][e] += shfl(acc[h][e], src);
      }
    }
#pragma unroll
    for (int h = 0; h < GB; ++h) {
#pragma unroll
      for (int e = 0; e < VE; ++e) acc[h][e] = tot[h][e];
    }
  }

  // ---- merge the four wavefronts in LDS ------------------------------------
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < GB; ++h) {
      s_ml[w][0][h] = m_run[h];
      s_ml[w][1][h] = lw[h];
    }
  }
  __syncthreads();
  float mtot[GB], fac[GB];
#pragma unroll
  for (int h = 0; h < GB; ++h) {
    float mm = s_ml[0][0][h];
#pragma unroll
    for (int ww = 1; ww < kWaves; ++ww) mm = fmaxf(mm, s_ml[ww][0][h]);
    mtot[h] = mm;
    fac[h] = m_run[h] == kNegInf ? 0.f : fast_exp2(m_run[h] - mm);
  }
#pragma unroll
  for (int ww = 0; ww < kWaves; ++ww) {
    if (w == ww && lane < LPT) {
#pragma unroll
      for (int h = 0; h < GB; ++h) {
        if (h < G) {
#pragma unroll
          for (int e = 0; e < VE; ++e) {
            const float val = acc[h][e] * fac[h];
            s_o[h][vdim + e] = ww == 0 ? val : s_o[h][vdim + e] + val;
          }
        }
      }
    }
    __syncthreads();
  }

  for (int i = threadIdx.x; i < G * DR; i += 256) {
    const int h = i / DR;
    const int d = i - h * DR;
    float mm = s_ml[0][0][h];
    for (int ww = 1; ww < kWaves; ++ww) mm = fmaxf(mm, s_ml[ww][0][h]);
    float l = 0.f;
    for (int ww = 0; ww < kWaves; ++ww) {
      const float mw = s_ml[ww][0][h];
      if (mw != kNegInf) l += s_ml[ww][1][h] * fast_exp2(mw - mm);
    }
    float o = s_o[h][d];
    const long bh = head0 + h;
    if (p.splits == 1) {
      if (p.sinks) {
        const float sk = p.sinks[bh - (long)b * p.H] * kLog2e;
        const float m2 = fmaxf(mm, sk);
        const float f = fast_exp2(mm - m2);
        l = l * f + fast_exp2(sk - m2);
        o *= f;
      }
      store_as<QT>(p.out, bh * DR + d, o / l);
    } else {
      p.part[(bh * p.splits + split) * DR + d] = o / l;
      if (d == 0) p.lse[bh * p.splits + split] = mm + log2f(l);
    }
  }
  (void)mtot;
}

// Log-sum-exp combine of the split partials (restates kernels.py:191-210,
// in base-2).  One workgroup per (sequence, head); only the splits that
// overlap the sequence's live keys are read.
template <int QT>
__global__ __launch_bounds__(256) void merge_kernel(DecodeParams p, int D) {
  const long bh = blockIdx.x;
  const int b = (int)(bh / p.H);
  const int h = (int)(bh % p.H);
  const long pos = p.pos[b];
  long t_hi = pos + 1;
  if (t_hi > p.ctx_limit) t_hi = p.ctx_limit;
  long t_lo = 0;
  if (p.window > 0 && pos - p.window + 1 > 0) t_lo = pos - p.window + 1;
  const int s0 = (int)(t_lo / p.split_tokens);
  const int s1 = t_hi > t_lo ? (int)((t_hi - 1) / p.split_tokens) : s0 - 1;
  const float *lse = p.lse + bh * p.splits;
  const float sk = p.sinks ? p.sinks[h] * kLog2e : -__builtin_inff();
  // One online pass: kBatch splits' log-sum-exps and partials are loaded
  // together (all in flight), then folded into a running max, denominator
  // and sum, so a step of at most kBatch splits waits for one memory latency
  // after the position.
  constexpr int kBatch = 8;
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float mm = sk;                        // running max (the sink included)
    float den = p.sinks ? 1.f : 0.f;      // exp2(sink - mm)
    float o = 0.f;
    for (int s = s0; s <= s1; s += kBatch) {
      float v[kBatch], l[kBatch];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const bool ok = s + j <= s1;
        v[j] = ok ? p.part[(bh * p.splits + s + j) * D + d] : 0.f;
        l[j] = ok ? lse[s + j] : -__builtin_inff();
      }
      float nm = mm;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) nm = fmaxf(nm, l[j]);
      const float base = nm == -__builtin_inff() ? 0.f : nm;
      const float a = fast_exp2(mm - base);   // 0 while mm is -inf
      den *= a;
      o *= a;
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const float wgt = fast_exp2(l[j] - base);
        den += wgt;
        o += wgt * v[j];
      }
      mm = nm;
    }
    store_as<QT>(p.out, bh * D + d, o / den);
  }
}

// phase bit 1: split kernel; bit 2: merge kernel (only when splits > 1).
template <int KVT, int QT, int D, int GB>
int launch_decode(const DecodeParams &p, hipStream_t stream, int phase) {
  const long grid = (long)p.B * p.KH * p.gsub * p.splits;
  if (grid <= 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EINVAL;
  if (phase & 1) {
    hipLaunchKernelGGL((decode_kernel<KVT, QT, D, GB>), dim3((unsigned)grid), dim3(256), 0, stream, p);
    DD_LAUNCH_CHECK();
  }
  if ((phase & 2) && p.splits > 1) {
    hipLaunchKernelGGL((merge_kernel<QT>), dim3((unsigned)((long)p.B * p.H)), dim3(p.DR < 256 ? p.DR : 256), 0,
                       stream, p, p.DR);
    DD_LAUNCH_CHECK();
  }
  return DD_OK;
}

template <int KVT, int QT, int D>
int dispatch_g(const DecodeParams &p, hipStream_t s, int phase) {
  if (p.G <= 1) return launch_decode<KVT, QT, D, 1>(p, s, phase);
  if (p.G <= 2) return launch_decode<KVT, QT, D, 2>(p, s, phase);
  if (p.G <= 4) return launch_decode<KVT, QT, D, 4>(p, s, phase);
  if (p.G <= 8) return launch_decode<KVT, QT, D, 8>(p, s, phase);
  if (p.G <= 16) return launch_decode<KVT, QT, D, 16>(p, s, phase);
  DecodeParams wide = p;
  wide.gsub = (p.G + 15) / 16;
  return launch_decode<KVT, QT, D, 16>(wide, s, phase);
}

}  // namespace dd_decode

#include "decode_stream.h"

namespace dd_decode {

#ifndef DD_DECODE_STREAM
#define DD_DECODE_STREAM 1
#endif

// Instantiated once per dtype pair in decode_<dtype>.hip.  bf16 / f16 / fp32
// pages at every head size up to 256 that is a multiple of 8 (in the
// smallest streamed layout that holds it), int8 pages with one scale per row
// at every head size that is a multiple of 16 (the same way) and int8 pages
// with group-32 scales at D = 64, 128, 256 take the streamed kernels
// (decode_stream.h), any number of query heads per KV head; the other int8
// groupings take decode_kernel.
// LDS layout of the streamed 16-bit / fp32 kernels for head size D: the
// smallest of 64, 96, 128, 160, 192, 224, 256 that holds it (D a multiple of
// 8; the layout's extra dims are zeros), or 0.
inline int stream_layout(int D) {
  if (D <= 0 || D % 8 || D > 256) return 0;
  return D <= 64 ? 64 : (D + 31) / 32 * 32;
}

template <int KVT, int QT>
int dispatch_d(const DecodeParams &p0, int D, hipStream_t s, int phase) {
  // streamed kernels: more than 16 query heads per KV head run as gsub
  // workgroups of up to 16 heads (each reads the KV head's keys)
  DecodeParams p = p0;
  p.gsub = (p.G + 15) / 16;
  if constexpr (DD_DECODE_STREAM && KVT == QT && (KVT == DD_BF16 || KVT == DD_F16)) {
    {
      switch (stream_layout(D)) {
        case 64: return launch_stream<KVT, 64, DD_STREAM_NB64, DD_STREAM_NW64>(p, s, phase);
        case 96: return launch_stream<KVT, 96, DD_STREAM_NB96, DD_STREAM_NW96>(p, s, phase);
        case 128: return launch_stream<KVT, 128, DD_STREAM_NB128, DD_STREAM_NW128>(p, s, phase);
        case 160: return launch_stream<KVT, 160, DD_STREAM_NB_MID, DD_STREAM_NW_MID>(p, s, phase);
        case 192: return launch_stream<KVT, 192, DD_STREAM_NB_MID, DD_STREAM_NW_MID>(p, s, phase);
        case 224: return launch_stream<KVT, 224, DD_STREAM_NB_MID, DD_STREAM_NW_MID>(p, s, phase);
        case 256: return launch_stream<KVT, 256, DD_STREAM_NB256, DD_STREAM_NW256>(p, s, phase);
        default: break;
      }
    }
  }
  if constexpr (DD_DECODE_STREAM && KVT == DD_F32 && QT == DD_F32) {
    {
      switch (stream_layout(D)) {
        case 64: return launch_stream<DD_F32, 64, DD_STREAM_NB_F32, DD_STREAM_NW_F32>(p, s, phase);
        case 96: return launch_stream<DD_F32, 96, DD_STREAM_NB_F32, DD_STREAM_NW_F32_96>(p, s, phase);
        case 128: return launch_stream<DD_F32, 128, DD_STREAM_NB_F32, DD_STREAM_NW_F32>(p, s, phase);
        case 160: return launch_stream<DD_F32, 160, DD_STREAM_NB_F32_256, DD_STREAM_NW_F32_256>(p, s, phase);
        case 192: return launch_stream<DD_F32, 192, DD_STREAM_NB_F32_256, DD_STREAM_NW_F32_256>(p, s, phase);
        case 224: return launch_stream<DD_F32, 224, DD_STREAM_NB_F32_256, DD_STREAM_NW_F32_256>(p, s, phase);
        case 256: return launch_stream<DD_F32, 256, DD_STREAM_NB_F32_256, DD_STREAM_NW_F32_256>(p, s, phase);
        default: break;
      }
    }
  }
  if constexpr (DD_DECODE_STREAM && KVT == DD_I8 && (QT == DD_BF16 || QT == DD_F16)) {
    {
      if (p.group == D && D % 16 == 0) {
        // one scale per row: the smallest of the 64 / 128 / 256 layouts
        // that holds the head size (its extra dims zeros)
        switch (D <= 64 ? 64 : D <= 128 ? 128 : D <= 256 ? 256 : 0) {
          case 64: return launch_stream_i8<QT, 64, 1, DD_STREAM_I8_NB64, DD_STREAM_I8_NW64>(p, s, phase);
          case 128: return launch_stream_i8<QT, 128, 1, DD_STREAM_I8_NB128, DD_STREAM_I8_NW128>(p, s, phase);
          case 256: return launch_stream_i8<QT, 256, 1, DD_STREAM_I8_NB256, DD_STREAM_I8_NW256>(p, s, phase);
          default: break;
        }
      } else if (p.group == 32) {
        switch (D) {
          case 64: return launch_stream_i8<QT, 64, 2, DD_STREAM_I8_NB64, DD_STREAM_I8_NW64>(p, s, phase);
          case 128: return launch_stream_i8<QT, 128, 4, DD_STREAM_NB128G, DD_STREAM_I8_NW128>(p, s, phase);
          case 256: return launch_stream_i8<QT, 256, 8, DD_STREAM_I8_NB256, DD_STREAM_I8_NW256>(p, s, phase);
          default: break;
        }
      }
    }
  }
  // the general kernel: the smallest layout of 64, 96, 128, 256 dims that
  // holds the head size (a multiple of 8, of 16 for int8 pages: whole
  // 16-byte loads)
  if (D <= 0 || D % (KVT == DD_I8 ? 16 : 8) || D > 256) return DD_EUNSUPPORTED;
  if (D <= 64) return dispatch_g<KVT, QT, 64>(p0, s, phase);
  if (D <= 96) return dispatch_g<KVT, QT, 96>(p0, s, phase);
  if (D <= 128) return dispatch_g<KVT, QT, 128>(p0, s, phase);
  return dispatch_g<KVT, QT, 256>(p0, s, phase);
}

}  // namespace dd_decode

