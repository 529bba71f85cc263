// Streamed split-KV decode for bf16 / f16 KV pages (gfx950), D in {64,128,256}.
//
// Same contract as decode_kernel (the reference's `_attention`,
// damendaemon/kernels.py:134-187): one query row per sequence, keys
// [t_lo, pos] read through the page table, fp32 softmax, optional ALiBi,
// T5 relative bias, window and sinks; split partials are combined by
// merge_kernel.
//
// Memory path.  Each of the four waves of a workgroup (sequence, KV head,
// split) owns every fourth 16-token chunk and a private ring of NB LDS
// stages.  A chunk's K and V rows are copied HBM -> LDS by direct-to-LDS
// buffer loads (no VGPRs held while in flight), marked nontemporal because
// every KV byte is read exactly once per step.  A stage is refilled as soon
// as its chunk has been read into registers, so NB chunks per wave are in
// flight while one is computed.  A chunk's buffer resource covers only its
// live rows, so rows past the split or the context, and chunks whose page is
// unallocated, land as zeros.
//
// Math.  S^T = K Q^T with v_mfma_f32_16x16x32 (rows = the chunk's 16
// tokens, columns = the GQA group's heads); the accumulator already has the
// register layout of the P^T operand of O^T += V^T P^T, which runs on
// v_mfma_f32_16x16x16 with V^T read from LDS by transposing reads
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

namespace dd_decode {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

#ifndef DD_STREAM_NB128
#define DD_STREAM_NB128 2
#endif
#ifndef DD_STREAM_NB64
#define DD_STREAM_NB64 4
#endif
#ifndef DD_STREAM_NB256
#define DD_STREAM_NB256 2
#endif
#ifndef DD_STREAM_NW64
#define DD_STREAM_NW64 4
#endif
#ifndef DD_STREAM_NW128
#define DD_STREAM_NW128 4
#endif
#ifndef DD_STREAM_NW256
#define DD_STREAM_NW256 2
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

template <int DT, int D, int NB, int NW>
__global__ __launch_bounds__(64 * NW) void stream_kernel(DecodeParams p) {
  // The host pass only needs the launch stub; the body is device code.
#if __HIP_DEVICE_COMPILE__
  constexpr int ROWB = 2 * D;        // bytes per token row
  constexpr int PAGEB = 16 * ROWB;   // one 16-token chunk of K (or V)
  constexpr int IPP = PAGEB / 1024;  // DMA instructions per chunk and plane
  constexpr int STAGE = 2 * PAGEB;
  constexpr int CPR = ROWB / 16;     // 16-byte chunks per row
  constexpr int NC = D / 32;         // S^T k-chunks
  constexpr int MD = D / 16;         // O^T row tiles
  constexpr int DP = D + 4;          // padded row of the cross-wave buffer
  static_assert(IPP >= 1 && 2 * IPP * NB < 64 && NB <= 4, "vmcnt range, unrolled steps");
  static_assert((NB - 1) * STAGE + PAGEB < 65536, "ds offset range");
  static_assert(NW * 16 * DP * 4 <= NW * NB * STAGE, "epilogue buffer fits the ring");

  __shared__ __align__(1024) char s_ring[NW * NB * STAGE];
  __shared__ float s_ml[NW][2][16];

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int n16 = lane & 15;  // head column (S^T, P^T, O^T) / token row (K operand)
  const int kg = lane >> 4;
  const int G = p.G;

  const int wg = blockIdx.x;
  const int nbkh = p.B * p.KH;
  const int split = wg / nbkh;
  const int bkh = wg - split * nbkh;
  const int b = bkh / p.KH;
  const int kh = bkh - b * p.KH;

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
  const long head0 = (long)b * p.H + (long)kh * G;
  const bool col_on = n16 < G;

  // Q^T operand: lane (head n16, dims 8kg + 32c ..+8).
  u32x4 qa[NC];
  {
    const unsigned short *qb = (const unsigned short *)p.q;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      qa[c] = col_on ? *(const u32x4 *)(qb + (head0 + n16) * D + 8 * kg + 32 * c) : u32x4{0, 0, 0, 0};
  }
  float slope = (p.alibi && col_on) ? p.alibi[(long)kh * G + n16] * kLog2e : 0.f;

  // Per-lane LDS byte offsets (loop invariant).
  const unsigned wbase = (unsigned)(size_t)(lds_void *)s_ring + (unsigned)(w * NB * STAGE);
  unsigned dma_off[IPP];
#pragma unroll
  for (int j = 0; j < IPP; ++j) {
    const int e = 64 * j + lane;
    const int r = e / CPR;
    dma_off[j] = (unsigned)(r * ROWB + 16 * ((e % CPR) ^ stream_swz<D>(r)));
  }
  unsigned k_addr[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) k_addr[c] = wbase + n16 * ROWB + 16 * ((4 * c + kg) ^ stream_swz<D>(n16));
  unsigned v_addr[MD];
  {
    const int a = lane & 15;
    const int r = 4 * kg + (a >> 2);
    const int q = a & 3;
#pragma unroll
    for (int md = 0; md < MD; ++md)
      v_addr[md] = wbase + PAGEB + r * ROWB + 16 * ((2 * md + (q >> 1)) ^ stream_swz<D>(r)) + 8 * (q & 1);
  }

  // This wave's chunks: first + i * NW, i < n.
  const int first = pg_first + w;
  const int n = first <= pg_last ? (pg_last - first) / NW + 1 : 0;

  const char *kplane = (const char *)p.k;
  const char *vplane = (const char *)p.v;
  const __attribute__((address_space(4))) int32_t *tab = (const __attribute__((address_space(4))) int32_t *)p.table;
  // Chunk i of this wave into `stage`.  Chunks past the wave's last one are
  // issued too, with an empty resource (no memory traffic): every iteration
  // then has the same loads in flight and waits for a constant count.
  auto issue = [&](int i, int stage) __attribute__((always_inline)) {
    const int pg = first + i * NW;
    long base;  // element offset of the chunk's first row, -1 when unmapped
    if (i >= n) {
#ifdef DD_STREAM_NODUMMY
      return;
#endif
      base = -1;
    } else if (p.paged) {
      base = -1;
      if (row >= 0 && row < p.table_rows) {
        const int entry = pg >> p.chunk_shift;
        const long phys = tab[(long)row * p.table_w + entry];
        if (phys >= 0 && phys < p.capacity)
          base = ((phys * p.KH + kh) * (long)p.page + ((pg - (entry << p.chunk_shift)) << 4)) * (long)D;
      }
    } else {
      base = (row >= 0 && row < p.capacity) ? (((long)row * p.KH + kh) * (long)p.page + (long)pg * 16) * (long)D : -1;
    }
    base = (long)uniform_ptr((const char *)base);
    const int live = base < 0 ? 0 : max(0, min(16, s_hi - pg * 16));
    const long off = base < 0 ? 0 : 2 * base;
    const int bytes = uniform(live * ROWB);
    const __amdgpu_buffer_rsrc_t rk =
        __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr(kplane + off), (short)0, bytes, kRawBufferWord3);
    const __amdgpu_buffer_rsrc_t rv =
        __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr(vplane + off), (short)0, bytes, kRawBufferWord3);
    char *dst = s_ring + (w * NB + stage) * STAGE;
#pragma unroll
    for (int j = 0; j < IPP; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_void *)(dst + 1024 * j), 16, dma_off[j], 0, 0,
                                               kStreamLoadAux);
#pragma unroll
    for (int j = 0; j < IPP; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (lds_void *)(dst + PAGEB + 1024 * j), 16, dma_off[j], 0, 0,
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
    u32x2 va[MD];
#pragma unroll
    for (int c = 0; c < NC; ++c) ka[c] = lds_read_b128<SOFF>(k_addr[c]);
#pragma unroll
    for (int md = 0; md < MD; ++md) va[md] = lds_read_tr16<SOFF>(v_addr[md]);
    wait_lds();
#pragma unroll
    for (int c = 0; c < NC; ++c) after_wait(ka[c]);
#pragma unroll
    for (int md = 0; md < MD; ++md) after_wait(va[md]);
    // The stage is in registers now: refill it with chunk i + NB.
    issue(i + NB, decltype(stage_tag)::value);
#ifdef DD_STREAM_NOMATH
    {
      unsigned x = 0;
      for (int c = 0; c < NC; ++c) x ^= ka[c][0] ^ ka[c][3];
      for (int md = 0; md < MD; ++md) x ^= va[md][0] ^ va[md][1];
      lsum += (float)(x & 1);
      return;
    }
#endif

    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NC; ++c) s = mfma16x16x32<DT>(ka[c], qa[c], s);

    // logits of tokens t0 + 4kg + i for head n16
    float x[4];
    float mx = kNegInf;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int t = t0 + 4 * kg + e;
      float v = s[e] * p.scale_log2 + slope * (float)t;
      if (p.rel && col_on) {
        const long dist = pos64 - t > 0 ? pos64 - t : 0;
        v += p.rel[((long)kh * G + n16) * p.rel_buckets + rel_bucket((int)dist, p.rel_buckets, p.rel_denom)] *
             kLog2e;
      }
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
    const u32x2 pb = {pack_pair<DT>(pr[0], pr[1]), pack_pair<DT>(pr[2], pr[3])};

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
    for (int md = 0; md < MD; ++md) o[md] = mfma16x16x16<DT>(va[md], pb, o[md]);
  };

  // Prologue: NB chunks in flight, then the query operand (loaded before
  // them) is made visibly complete, so the loop carries no pending load the
  // compiler would wait for.
#pragma unroll
  for (int u = 0; u < NB; ++u) issue(u, u);
#pragma unroll
  for (int c = 0; c < NC; ++c) after_wait(qa[c]);
  after_wait(slope);
  // Chunk i: NB - 1 younger chunks (2 IPP loads each) stay in flight.
  for (int i0 = 0; i0 < n; i0 += NB) {
#define DD_STREAM_STEP(U)                                                  \
    if constexpr (U < NB) {                                                \
      const int i = i0 + U;                                                \
      if (i < n) {                                                         \
        wait_vm<2 * IPP * (NB - 1)>();                                     \
        consume(i, std::integral_constant<int, (U < NB ? U : 0)>{});       \
      }                                                                    \
    }
    DD_STREAM_STEP(0)
    DD_STREAM_STEP(1)
    DD_STREAM_STEP(2)
    DD_STREAM_STEP(3)
#undef DD_STREAM_STEP
  }
  wait_vm<0>();  // the trailing (empty) loads, before the ring is reused
#ifdef DD_STREAM_NOEPI
  if (lsum == 12345.f) ((float *)p.out)[0] = lsum;
  return;
#endif

  // ---- combine the four waves ---------------------------------------------
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
  float *s_o = (float *)s_ring;
  if (col_on) {
#pragma unroll
    for (int md = 0; md < MD; ++md)
      *(f32x4 *)&s_o[(w * 16 + n16) * DP + 16 * md + 4 * kg] = o[md] * fac;
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < G * D; idx += 64 * NW) {
    const int h = idx / D;
    const int d = idx - h * D;
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
      store_as<DT>(p.out, bh * D + d, acc / l);
    } else {
      p.part[(bh * p.splits + split) * D + d] = acc / l;
      if (d == 0) p.lse[bh * p.splits + split] = m2 + log2f(l);
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

template <int DT, int D, int NB, int NW>
int launch_stream(const DecodeParams &p, hipStream_t stream, int phase) {
  const long grid = (long)p.B * p.KH * p.splits;
  if (grid <= 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EINVAL;
  if (phase & 1) {
    hipLaunchKernelGGL((stream_kernel<DT, D, NB, NW>), dim3((unsigned)grid), dim3(64 * NW), 0, stream, p);
    DD_LAUNCH_CHECK();
  }
  if ((phase & 2) && p.splits > 1) {
    hipLaunchKernelGGL((merge_kernel<DT>), dim3((unsigned)((long)p.B * p.H)), dim3(D < 256 ? D : 256), 0, stream,
                       p, D);
    DD_LAUNCH_CHECK();
  }
  return DD_OK;
}

}  // namespace dd_decode
