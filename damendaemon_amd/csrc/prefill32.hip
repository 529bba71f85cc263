// Chunked-prefill attention for head sizes 64 and 128 on 32x32x16 MFMAs
// (gfx950); semantics as in prefill.hip (damendaemon/paged.py:97-111 with
// qwen2.py:754-770): query row j of segment i attends keys 0 .. start_i + j
// of its slot (and > position - window), GQA head h reads KV head h / G,
// softmax(q.k * scale) . v accumulated in fp32.
//
// Work split.  A workgroup of four waves owns 128 (query row, head) columns
// of one (segment, KV head), 32 per wave; keys stream in 32-key tiles (two
// 16-token chunks).  Two workgroups share a CU (56-72 KiB of LDS and <= 256
// registers per wave each), so each SIMD runs two independent waves whose
// matrix-core and vector-ALU work interleave; a single wave per SIMD was
// measured to serialise its MFMAs and FMAs.  Per tile and wave:
//   S^T = K Q^T       v_mfma_f32_32x32x16 (bf16 or fp16), 32 keys x 32
//                     columns, K from LDS, Q^T held in AGPRs;
//   online softmax    on the accumulator (lane l holds column l%32 and 16 of
//                     the 32 keys, lane l^32 the other 16: one permlane step);
//   O^T += V^T P^T    v_mfma_f32_32x32x16_f16 whose P^T operand is a slice of
//                     the S^T accumulator (keys contracted in the
//                     accumulator's own order, V^T read in that order by
//                     transposing LDS reads); O^T held in AGPRs.
// Probabilities enter P.V rounded to fp16 (11-bit significand, 8x finer
// than bf16): that is the arithmetic of the reference's own fp16 SDPA, and
// its error stays an order of magnitude inside the 2e-3 bound where one bf16
// rounding does not.  bf16 V tiles are converted to fp16 in LDS once per
// workgroup (exact for every bf16 value inside fp16's range, as an fp16 KV
// cache would store it); the softmax denominators come from an all-ones
// V^T MFMA over the same fp16 P, so numerator and denominator agree.
//
// Memory path.  K and V tiles rotate through four LDS slots; tile t+3 is
// loaded (direct-to-LDS buffer loads, one 16-token chunk of K or V per
// wave) while tile t is computed, and tile t+1 is converted.  A chunk's
// buffer resource covers only its live rows; the conversion writes zeros
// for rows that are not live.
//
// LDS (per slot, blocks of 1 KiB = one DMA instruction, reads lane-contiguous):
//   K block (chunk pc, dims 32dq..): DMA lane l holds
//     K[16pc + l%16][32dq + 16(l/32) + 8((l/16)%2) ..+8]
//   so the A operand of S^T for dims 16cc.. is read by lane l at block
//   ((l/16)%2, cc/2) offset 16(l%16) + 256(l/32) + 512(cc%2).
//   V block (chunk pc, dims 32md..): two 512-byte halves r; lane L of half r
//   holds 8 bytes V[8r + 4(L/32) + (L%16)/4][32md + 16((L/16)%2) + 4(L%4) ..+4]
//   which is what one ds_read_b64_tr_b16 wants to hand lane L dims
//   32md + L%32 of keys 8r + 4(L/32) + 0..3.
#include "prefill_common.h"

namespace dd_prefill {
namespace {

constexpr int kTab32 = 4096;

// The kernel's MFMAs are inline assembly so that Q^T and O^T stay in AGPRs
// (legal MFMA B / accumulator operands on gfx950) and the S^T accumulators
// the softmax reads stay in VGPRs, and so that the instruction order is the
// source order: the kernel interleaves its softmax with its MFMAs by hand.
// Hazards the assembler leaves to software: a B operand written by a VALU
// op needs two wait states before an MFMA reads it (the s_nop 1 of the P.V
// forms); a VALU read of an MFMA result needs 18 after a 32x32x16 MFMA
// (mfma_fence, used before the reads that could come that early).
template <int DT>
DD_DEV void mfma_s_first(f32x16 &acc, const u32x4 &k, const u32x4 &q) {
  if constexpr (DT == DD_BF16) {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(acc) : "v"(k), "a"(q));
  } else {
    asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, 0" : "=&v"(acc) : "v"(k), "a"(q));
  }
}
template <int DT>
DD_DEV void mfma_s(f32x16 &acc, const u32x4 &k, const u32x4 &q) {
  if constexpr (DT == DD_BF16) {
    asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(k), "a"(q));
  } else {
    asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(acc) : "v"(k), "a"(q));
  }
}
// O^T += V^T P^T: P^T and V^T are fp16 for both page dtypes (bf16 V^T is
// converted exactly in LDS first)
DD_DEV void mfma_o(f32x16 &acc, const u32x4 &v, const u32x4 &p) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(v), "v"(p));
}
DD_DEV void mfma_fence_v(f32x16 &x) { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+v"(x)); }
DD_DEV void mfma_fence_a(f32x16 &x) { asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 4" : "+a"(x)); }
DD_DEV void pin_a(u32x4 &x) { asm volatile("" : "+a"(x)); }

// LDS reads in inline assembly (immediate offsets, no compiler-inserted
// waits): the ring slots are chosen at run time, and a compiler-visible read
// of a slot would make the compiler wait for every direct-to-LDS load in
// flight.  Each read's consumer waits with lgkm_wait(n), n = reads issued
// after it (LDS reads complete in order).
typedef __attribute__((address_space(3))) char lds_char;
DD_DEV unsigned lds_addr(const char *p) { return (unsigned)(uintptr_t)(const lds_char *)p; }
DD_DEV u32x4 lds_read128(unsigned addr, int off) {
  u32x4 r;

  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off) : "memory");
  return r;
}
DD_DEV u32x2 lds_read_tr16(unsigned addr, int off) {
  u32x2 r;

  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off) : "memory");
  return r;
}
DD_DEV void lds_write128(unsigned addr, int off, u32x4 x) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(x), "i"(off) : "memory");
}
DD_DEV void lgkm_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
template <typename T>
DD_DEV void lgkm_wait(T &x, int n) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(n < 15 ? n : 15));
}

// s_waitcnt immediate for vmcnt(n) with no wait on the exp / lgkm counters
constexpr unsigned vmcnt_imm(int n) { return (unsigned)((n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8)); }

template <int DT, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void prefill32_kernel(PrefillParams p) {
  constexpr int NW = 4;
  constexpr int KT = 32;                // keys per tile: two 16-token chunks
  constexpr int NCC = D / 16;           // k-steps of S^T
  constexpr int MD = D / 32;            // 32-dim blocks of O^T
  constexpr int DQ = D / 32;            // 32-dim blocks of a K / V chunk
  constexpr int COLS = 32 * NW;
  constexpr int NT = 64 * NW;
  constexpr int PLANE = 2 * DQ * 1024;  // one tile of K (or V)
#ifndef DD_PF32_NB
#define DD_PF32_NB 4
#endif
  constexpr int NB = DD_PF32_NB;        // ring depth: tiles t+1 .. t+NB-1 load while tile t is computed
  constexpr int IPW = DQ;               // DMA instructions per wave per tile (one chunk of K or V)

  // K and V rings: tile t lives in slot (t - first) % NB.
  __shared__ __align__(1024) char s_kring[NB * PLANE];
  __shared__ __align__(1024) char s_vring[NB * PLANE];
  __shared__ int s_tab[kTab32];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int l32 = lane & 31;
  const int h2 = lane >> 5;             // which 16 of a column's 32 keys

  int grp, qt;
  if (p.plan) {
    const int item = p.plan[blockIdx.x];
    if (item < 0) return;
    grp = item / p.max_tiles;
    qt = item - grp * p.max_tiles;
  } else {
    const int xcd = blockIdx.x & 7;
    const int j = blockIdx.x >> 3;
    grp = xcd + 8 * (j / p.max_tiles);
    qt = p.max_tiles - 1 - j % p.max_tiles;
  }
  if (grp >= p.n * p.KH) return;
  const int seg = grp / p.KH;
  const int kh = grp - seg * p.KH;
  const long tok0 = p.cu[seg];
  const int len = (int)(p.cu[seg + 1] - tok0);
  const int G = p.G;
  const int rows = COLS / G;
  const int r0 = qt * rows;
  if (r0 >= len) return;
  const int context = (int)p.ctx[seg];
  const int start = context - len;
  const long slot = p.slots[seg];
  const int rows_here = min(rows, len - r0);

  const int k_hi = start + r0 + rows_here;  // exclusive
  int k_lo = 0;
  if (p.window > 0) k_lo = max(0, start + r0 - p.window + 1);
  const int kt_first = k_lo / KT;
  const int kt_last = (k_hi - 1) / KT;

  const int e_first = (kt_first * KT) >> p.page_shift;
  const int e_count = ((((kt_last + 1) * KT) - 1) >> p.page_shift) - e_first + 1;
  const bool slot_ok = slot >= 0 && slot < p.table_rows;
  auto table_entry = [&](int e) {
    const int phys = (slot_ok && e < p.table_w) ? p.table[slot * p.table_w + e] : -1;
    return (phys >= 0 && phys < p.capacity) ? phys : -1;
  };
  for (int i = tid; i < e_count && i < kTab32; i += NT) s_tab[i] = table_entry(e_first + i);

  // ---- query column and Q^T operands (B of S^T: lane = column + 32 * dim-half) ----
  const int col = w * 32 + l32;
  const int qr = col / G;
  const int gh = col - qr * G;
  const bool colok = qr < rows_here;
  const int qpos = start + r0 + (colok ? qr : 0);
  u32x4 qb[NCC];
  {
    const long row = (tok0 + r0 + (colok ? qr : 0)) * p.H + (long)kh * G + gh;
    const unsigned short *qsrc = (const unsigned short *)p.q;
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      qb[cc] = colok ? *(const u32x4 *)(qsrc + row * D + 16 * cc + 8 * h2) ^ p.q_sign : u32x4{0, 0, 0, 0};
      pin_a(qb[cc]);
    }
  }

  f32x16 o[MD];
#pragma unroll
  for (int md = 0; md < MD; ++md) o[md] = f32x16{};
  float m_run = kNegInf;
  // softmax denominators on the matrix cores: an all-ones V^T operand makes
  // every accumulator row the column sum of exactly the fp16 P that P.V uses
  f32x16 lacc = f32x16{};
  const u32x4 ones = {0x3C003C00u, 0x3C003C00u, 0x3C003C00u, 0x3C003C00u};
  __syncthreads();  // s_tab

  // ---- loads: wave w fetches chunk w%2 of the K (w < 2) or V (w >= 2) tile ----
  auto table_at = [&](int e) -> int {   // validated physical page of page-table entry e (wave-uniform)
    const int i = e - e_first;
    return i < kTab32 ? s_tab[i] : (i < e_count ? table_entry(e) : -1);
  };
  const bool loads_v = w >= 2;
  const int my_chunk = w & 1;
  unsigned dma_lane;
  if (!loads_v) {
    dma_lane = 2u * ((lane & 15) * D + 16 * (lane >> 5) + 8 * ((lane >> 4) & 1));
  } else {
    const int vm = lane & 31;
    const int v_key = 8 * (lane >> 5) + 4 * (vm >> 4) + ((vm & 7) >> 1);
    dma_lane = 2u * (v_key * D + 16 * ((vm >> 3) & 1) + 8 * (vm & 1));
  }
  const char *plane = loads_v ? (const char *)p.v : (const char *)p.k;
  char *ring = loads_v ? s_vring : s_kring;
  // The buffer resource covers only the chunk's live rows (0 bytes past the
  // context or for an unallocated page), so dead rows land as zeros.
  auto issue = [&](int kt) __attribute__((always_inline)) {
    const int key0 = kt * KT + 16 * my_chunk;
    const int phys = uniform(table_at(key0 >> p.page_shift));
    const int live = phys < 0 ? 0 : min(16, context - key0);
    const long base = phys < 0 ? 0 : ((((long)phys * p.KH + kh) << p.page_shift) | (key0 & (p.page - 1))) * (long)D;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        (void *)uniform_ptr(plane + 2 * base), (short)0, uniform(live > 0 ? live * D * 2 : 0), kBufferWord3);
    char *dst = ring + ((kt - kt_first) % NB) * PLANE + my_chunk * DQ * 1024;
#pragma unroll
    for (int j = 0; j < IPW; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)(dst + j * 1024), 16, dma_lane, 64 * j, 0, 0);
  };
  // Wait until only this wave's loads of the `younger` most recently issued
  // tiles may be in flight, then barrier.
  auto sync = [&](int younger) __attribute__((always_inline)) {
    if (younger >= 2) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * IPW));
    } else if (younger == 1) {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(IPW));
    } else {
      __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    }
    __syncthreads();
  };
  // bf16 pages: this thread's share of V tile kt converted to fp16 in place
  // (exact for every bf16 value in fp16's range, as an fp16 KV cache would
  // hold it; the P.V MFMAs then run on fp16 V^T and fp16 P^T)
  // Rows that are not live (past the context, or behind an unallocated
  // page-table entry) are written as zeros: the direct-to-LDS loads leave
  // them untouched, and a stale fp16 row read again as bf16 could be inf.
  auto convert_v = [&](int kt) __attribute__((always_inline)) {
    if constexpr (DT == DD_BF16) {
      constexpr int N16 = PLANE / NT / 16;
      const unsigned off = (unsigned)tid * (PLANE / NT);
      const unsigned base = lds_addr(s_vring) + (unsigned)(((kt - kt_first) % NB) * PLANE) + off;
      u32x4 x[N16];
#pragma unroll
      for (int j = 0; j < N16; ++j) x[j] = lds_read128(base, 16 * j);
      // 16-byte piece j is DMA lane m of block (chunk pc, dims 32md..): its key
      const int pc = (int)(off >> 10) / DQ;
      const int key0 = kt * KT + 16 * pc;
      const int phys = table_at(key0 >> p.page_shift);
      const int live = phys < 0 ? 0 : min(16, context - key0);
      lgkm_wait(x[N16 - 1], 0);
#pragma unroll
      for (int j = 0; j < N16; ++j) {
        const int m = (int)(((off + 16 * j) & 1023) >> 4);
        const int vm2 = m & 31;
        const int key = 8 * (m >> 5) + 4 * (vm2 >> 4) + ((vm2 & 7) >> 1);
        u32x4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const f32x2 f = {__uint_as_float(x[j][i] << 16), __uint_as_float(x[j][i] & 0xffff0000u)};
          y[i] = __builtin_bit_cast(unsigned, __builtin_convertvector(f, f16x2));
        }
        if (key >= live) y = u32x4{0, 0, 0, 0};
        lds_write128(base, 16 * j, y);
      }
      lgkm_drain();   // the writes land before the next barrier
    }
  };

  // ---- one tile ----
  const unsigned k_rd = lds_addr(s_kring) + 16u * (lane & 15) + 256u * h2 + 1024u * DQ * ((lane >> 4) & 1);
  const unsigned v_rd = lds_addr(s_vring) + 8u * lane;
  const float sc = p.scale_log2;
  const float slack = kMaxSlack / sc;
  auto tile = [&](int kt) __attribute__((always_inline)) {
    const unsigned slot_off = (unsigned)(((kt - kt_first) % NB) * PLANE);
    const unsigned kb = k_rd + slot_off, vb = v_rd + slot_off;
    // S^T = K Q^T (32 keys x 32 columns); K operands read four ahead, V^T
    // operands (both 16-key chunks) during the S chain
    constexpr int KR = 4;
    u32x4 kop[KR], va[2][MD];
    f32x16 s;
#pragma unroll
    for (int cc = 0; cc < KR; ++cc) kop[cc] = lds_read128(kb, (cc / 2) * 1024 + 512 * (cc & 1));
#pragma unroll
    for (int cc = 0; cc < NCC; ++cc) {
      // kop[cc] is the cc-th read; KR - 1 later ones are in flight while
      // cc + KR < NCC, fewer at the end
      lgkm_wait(kop[cc % KR], min(KR - 1, NCC - 1 - cc));
      if (cc == 0) {
        mfma_s_first<DT>(s, kop[0], qb[0]);
      } else {
        mfma_s<DT>(s, kop[cc % KR], qb[cc]);
      }
      if (cc + KR < NCC) kop[cc % KR] = lds_read128(kb, ((cc + KR) / 2) * 1024 + 512 * ((cc + KR) & 1));
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int md = 0; md < MD; ++md) {
        const u32x2 lo = lds_read_tr16(vb, (j * DQ + md) * 1024);
        const u32x2 hi = lds_read_tr16(vb, (j * DQ + md) * 1024 + 512);
        va[j][md] = u32x4{lo[0], lo[1], hi[0], hi[1]};
      }
    }
    mfma_fence_v(s);
    // mask: keys past a column's diagonal or before its window; key of
    // accumulator register r is kt*32 + 8(r/4) + 4h2 + r%4
    const int kbase = kt * KT;
    if (!(kbase + KT - 1 <= start + r0 && (p.window == 0 || kbase >= start + r0 + rows_here - p.window))) {
      const int lo = p.window > 0 ? qpos - p.window + 1 : -1;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = kbase + 8 * (r >> 2) + 4 * h2 + (r & 3);
        s[r] = ((key <= qpos) & (key >= lo)) ? s[r] : kNegInf;
      }
    }
    // online softmax: the running max moves only when the tile's max exceeds
    // it by more than kMaxSlack (exp2 domain)
    float mx = fmaxf(s[0], s[1]);
#pragma unroll
    for (int r = 2; r < 16; r += 2) mx = fmaxf(fmaxf(mx, s[r]), s[r + 1]);   // v_max3
    mx = xor32_max(mx);
    const bool up = mx > m_run + slack;   // m_run = -inf moves to any finite max
    const float mn = up ? mx : m_run;
    const float mu = mn == kNegInf ? 0.f : mn * sc;
    const float alpha = up ? __builtin_amdgcn_exp2f(m_run * sc - mu) : 1.f;
    m_run = mn;
    float e[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], sc, -mu));
    u32x4 pp[2];   // P^T of the two 16-key chunks, fp16
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const f32x4 x0 = {e[8 * j + 0], e[8 * j + 1], e[8 * j + 2], e[8 * j + 3]};
      const f32x4 x1 = {e[8 * j + 4], e[8 * j + 5], e[8 * j + 6], e[8 * j + 7]};
      pp[j] = pack8<DD_F16>(x0, x1);
    }
    if (__builtin_amdgcn_ballot_w64(up)) {
#pragma unroll
      for (int md = 0; md < MD; ++md) {
        mfma_fence_a(o[md]);
        o[md] *= alpha;
      }
      mfma_fence_a(lacc);
      lacc *= alpha;
    }
    lgkm_wait(va[1][MD - 1], 0);
    // O^T += V^T P^T
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int md = 0; md < MD; ++md) mfma_o(o[md], va[j][md], pp[j]);
      mfma_o(lacc, ones, pp[j]);
    }
  };

  // ---- schedule: tile t+2 is loaded while tile t is computed ----
  // Step kt: wait for tile kt+1 and barrier (tile kt's fp16 V^T, converted
  // in step kt-1, is visible; every wave is done with tile kt-1); load tile
  // kt+3 into the slot of tile kt-1; convert V of tile kt+1; compute tile kt.
  static_assert(NB == 4, "the schedule keeps tiles kt+1 .. kt+3 in flight");
#pragma unroll
  for (int i = 0; i < NB - 1; ++i) {
    if (kt_first + i <= kt_last) issue(kt_first + i);
  }
  sync(min(2, kt_last - kt_first));
  convert_v(kt_first);
  for (int kt = kt_first; kt <= kt_last; ++kt) {
    sync(kt + 1 <= kt_last ? min(1, kt_last - kt - 1) : 0);
    if (kt + 3 <= kt_last) issue(kt + 3);
    if (kt + 1 <= kt_last) convert_v(kt + 1);
    tile(kt);
  }

  // ---- normalise and store: lane holds dims 32md + 8(r/4) + 4h2 + r%4 of its column ----
  mfma_fence_a(lacc);
  const float l = lacc[0];
  if (!colok) return;
  const float inv = 1.f / l;
  const long orow = ((tok0 + r0 + qr) * p.H + (long)kh * G + gh) * D;
  unsigned short *dst = (unsigned short *)p.out;
#pragma unroll
  for (int md = 0; md < MD; ++md) {
    mfma_fence_a(o[md]);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x16 &x = o[md];
      const u32x2 pk = {pack2<DT>(x[4 * q4 + 0] * inv, x[4 * q4 + 1] * inv),
                        pack2<DT>(x[4 * q4 + 2] * inv, x[4 * q4 + 3] * inv)};
      *(u32x2 *)(dst + orow + 32 * md + 8 * q4 + 4 * h2) = pk;
    }
  }
}

template <int DT, int D>
int launch32(PrefillParams p, int max_len, int plan_len, hipStream_t s) {
  constexpr int COLS = 128;
  if (COLS / p.G < 1) return DD_EUNSUPPORTED;
  p.max_tiles = (int)dd_cdiv(max_len, COLS / p.G);
  const long grid = p.plan ? (long)plan_len : 8L * dd_cdiv((long)p.n * p.KH, 8) * p.max_tiles;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill32_kernel<DT, D>), dim3((unsigned)grid), dim3(256), 0, s, p);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

}  // namespace

int prefill32_dispatch(const PrefillParams &p, int dtype, int dim, int max_len, int plan_len, hipStream_t s) {
  if (dtype == DD_BF16) {
    if (dim == 64) return launch32<DD_BF16, 64>(p, max_len, plan_len, s);
    if (dim == 128) return launch32<DD_BF16, 128>(p, max_len, plan_len, s);
  } else if (dtype == DD_F16) {
    if (dim == 64) return launch32<DD_F16, 64>(p, max_len, plan_len, s);
    if (dim == 128) return launch32<DD_F16, 128>(p, max_len, plan_len, s);
  }
  return DD_EUNSUPPORTED;
}

}  // namespace dd_prefill
