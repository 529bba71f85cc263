// Chunked-prefill attention for head sizes 48 to 256 in steps of 16 (gfx950;
// 16 and 32 excepted), bf16 or fp16 pages, in four LDS layouts: 64 (48, 64),
// 128 (80-128), 160 (144, 160) and 256 (176-256); below a layout's size the
// missing dims are zeros in LDS that no MFMA reads.  Semantics as in prefill.hip (damendaemon/paged.py:97-111 with
// qwen2.py:754-770): query row j of segment i attends keys 0 .. start_i + j
// of its slot (and > position - window), GQA head h reads KV head h / G,
// softmax(q.k * scale) . v accumulated in fp32.
//
// Work split.  A workgroup of eight waves (two per SIMD, one workgroup per
// CU) owns 256 (query row, head) columns of one (segment, KV head), 32 per
// wave; keys stream in 64-key tiles (four 16-token chunks; 128-key tiles in
// the 64 layout, whose rows are half as long).  Per 64 keys and (D = 128)
// wave the matrix cores do 16 MFMAs of S^T = K Q^T and 16 of O^T += V^T P^T
// (v_mfma_f32_32x32x16), 1024 cycles; the softmax is ~100 VALU operations.
// The 160 layout has the same split with three K slots instead of four
// (its 20 KiB tiles).  The 256 layout: four waves (one per SIMD, each with
// the SIMD's whole register file: its O^T alone is 128 registers) own 128
// columns, and keys stream in 32-key tiles, so that the same K and V rings
// fit the LDS.
//
// Step structure.  Step t of a wave issues the MFMAs of S(t+1) = K(t+1) Q^T
// and O += V(t)^T P(t) back to back, then the vector work of tile t+1:
// mask, exponentials into the fp16 P^T operands, row sums, and the in-place
// fp16 conversion of V(t+1); one barrier per step.  The exponentials use
// the column's running offset without a max over the tile; only a tile
// that pushes a probability past fp16's range (or a column's first tile)
// takes the max and moves the offset.  The two
// waves of a SIMD drift apart within a step, so one's vector work fills the
// other's matrix-core phase (measured: interleaving the two inside a wave
// by hand was slower).
//
// Precision.  The probabilities enter P.V as fp16 (11-bit significand; one
// bf16 rounding, 2^-9 relative, is 8x coarser and puts short-context rows
// several 1e-3 off).  bf16 V is converted to fp16 in LDS: exact for every
// bf16 value of magnitude in [2^-14, 65504]; smaller ones round to fp16
// subnormals (absolute error <= 2^-25), larger ones become infinite.  So
// that no result depends on that, each work item checks its output at the
// end: a column whose largest |O| is not finite or is below 2^-12 (where an
// absolute 2^-25 could exceed 2^-13 of the row) flags the item in p.flags,
// and the caller's next launch recomputes the flagged items in fp32
// arithmetic (prefill_f32.hip, 16-bit values widened exactly).  N(0,1)-like
// data never takes that path.  The softmax denominators are summed
// (v_dot2_f32_f16, fp32 accumulate) from exactly the fp16 P that the P.V
// product uses.
//
// Memory path (per tile, 4 chunks of 16 tokens, 8 in the 64 layout, 2 in the 256 layout;
// larger pages are read 16 rows at a time).  K and V both arrive by
// direct-to-LDS buffer loads of 1 KiB per wave instruction, two (D = 64
// and 128), three (the 160 layout, one of them empty for half of the
// waves) or four (the 256 layout) per wave and operand, issued NKS
// steps ahead into rings of NKS (K) and NKS + 1 (V) tile slots.
// Every load goes through a buffer resource that covers only the chunk's
// live rows: rows past the context and chunks without an allocated page
// read as zeros.
//
// LDS layouts (lane-contiguous for every read):
//   K block (chunk pc, dims 32dq..+32), 1 KiB: DMA lane m holds
//     K[16pc + m%16][32dq + 8(m/16) ..+8]; the S^T A operand (32 keys of
//     block kb, dims 16cc..) of lane l sits in block (2kb + (l%32)/16, cc/2)
//     at 16(l%16) + 256(l/32) + 512(cc%2).
//   V region (kb, j2, md, half), 512 B (two of them, half 0 and 1, form the
//   1 KiB block that one direct-to-LDS load fills): lane L's 8 bytes are
//     V[32kb + 16j2 + 8half + 4(L/32) + (L%16)/4][32md + 16((L/16)%2) + 4(L%4) ..+4]
//     (fp16), what one ds_read_b64_tr_b16 hands lane L as dim 32md + L%32
//     of four keys; the keys follow the S^T accumulator's own order, so the
//     P^T operand is a slice of the accumulator.
#include "prefill_common.h"

#include <type_traits>

namespace dd_prefill {
namespace {

// Four K and five V slots with 3,584 staged page-table entries fit the
// 160 KiB of LDS (D = 128); measured 1 % faster on C4 than three K slots.
#ifndef DD_PF_NKS
#define DD_PF_NKS 4
#endif
#ifndef DD_PF_RING
#define DD_PF_RING 8
#endif
#ifndef DD_PF_TAB
#define DD_PF_TAB 3584
#endif
constexpr int kNKS = DD_PF_NKS;    // K tile slots: K(kt+NKS) and V(kt+NKS) are issued at step kt
constexpr int kTabP = DD_PF_TAB;   // page-table entries staged in LDS per work item
   // page-table entries staged in LDS per work item

typedef __attribute__((address_space(3))) char lds_char;
DD_DEV unsigned lds_addr(const void *p) { return (unsigned)(uintptr_t)(const lds_char *)p; }

// LDS reads and writes in inline assembly: the compiler cannot relate them
// to the direct-to-LDS loads in flight and would otherwise wait for all of
// them.  A read's consumer waits with lgkm_wait(x, n), n = LDS operations
// issued after it (they complete in order).
DD_DEV u32x4 lds_read128(unsigned addr, int off) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off) : "memory");
  return r;
}
DD_DEV u32x2 lds_read_tr(unsigned addr, int off) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(off) : "memory");
  return r;
}
DD_DEV void lds_write128(unsigned addr, int off, u32x4 x) {
  asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(x), "i"(off) : "memory");
}
// Every register an awaited read writes must be an operand of its wait:
// otherwise the compiler may read that register before the wait.
template <typename T>
DD_DEV void lgkm_wait(T &x, int n) {
  asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(x) : "i"(n < 15 ? n : 15));
}
template <typename T>
DD_DEV void lgkm_wait(T &x, T &y, int n) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(x), "+v"(y) : "i"(n < 15 ? n : 15));
}
DD_DEV void lgkm_drain() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }
DD_DEV void barrier() { asm volatile("s_barrier" ::: "memory"); }
// s_waitcnt vmcnt(n), no wait on the other counters
template <int N>
DD_DEV void vm_wait() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int DT>
DD_DEV f32x16 mfma_s(u32x4 k, u32x4 q, f32x16 c) {
  if constexpr (DT == DD_BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, k), __builtin_bit_cast(bf16x8, q), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, k), __builtin_bit_cast(f16x8, q), c, 0,
                                                  0, 0);
  }
}
DD_DEV f32x16 mfma_o(u32x4 v, u32x4 p, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, v), __builtin_bit_cast(f16x8, p), c, 0, 0,
                                                0);
}

DD_DEV unsigned cvt_pk_f16(float a, float b) {
  return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{a, b}, f16x2));
}
// 8 bf16 -> 8 fp16 (exact in fp16's normal range)
DD_DEV u32x4 bf16x8_to_f16x8(u32x4 x) {
  u32x4 y;
#pragma unroll
  for (int i = 0; i < 4; ++i) y[i] = cvt_pk_f16(__uint_as_float(x[i] << 16), __uint_as_float(x[i] & 0xffff0000u));
  return y;
}

// Waves per workgroup and keys per tile of a layout.  The 256 layout has one
// wave per SIMD (its 32 columns' O^T alone is 128 registers; the wave gets
// the SIMD's whole register file) and 32-key tiles (so the rings still fit
// the LDS); the 64 layout 128-key tiles (16 KiB, as the 128 layout's: half
// the steps, barriers and page lookups per key; 7 % faster on the C4 shape).
template <int D>
constexpr int pipe_waves() { return D == 256 ? 4 : 8; }
template <int D>
constexpr int pipe_keys() { return D == 256 ? 32 : D == 64 ? 128 : 64; }
// K tile slots of a layout: three in the 160 layout, whose 20 KiB tiles
// leave room for no more (3 K + 4 V slots + the staged table: 155 KiB).
template <int D>
constexpr int pipe_nks() { return D == 160 ? 3 : kNKS; }
// LDS operands in flight in the matrix-core phase (fewer in the 160 layout,
// whose Q and O^T registers leave less room)
#ifndef DD_PF_RING160
#define DD_PF_RING160 4
#endif
template <int D>
constexpr int pipe_ring() { return D == 160 ? DD_PF_RING160 : DD_PF_RING; }

// D is the LDS layout's head size (64, 128, 160 or 256); DR <= D the real one (a
// multiple of 16 above D / 2): rows are DR elements long in memory, the
// layout's dims DR .. D-1 are loaded as zeros and skipped by the MFMAs.
template <int DT, int D, int DR>
__global__ __launch_bounds__(64 * pipe_waves<D>()) __attribute__((amdgpu_waves_per_eu(pipe_waves<D>() / 4)))
void prefill_pipe_kernel(PrefillParams p) {
  static_assert(D == 64 || D == 128 || D == 160 || D == 256, "layouts for head sizes 64, 128, 160 and 256");
  static_assert(DR % 16 == 0 && DR <= D && 2 * DR > D, "real head size");
  constexpr int NCCR = DR / 16;         // k-steps of S^T over the real dims
  constexpr int MDR = (DR + 31) / 32;   // 32-dim blocks of O^T holding real dims
  constexpr int NW = pipe_waves<D>();
  constexpr int NT = 64 * NW;
  constexpr int KT = pipe_keys<D>();    // keys per tile
  constexpr int NSB = KT / 32;          // 32-key blocks of S^T per tile
  constexpr int MD = D / 32;            // 32-dim blocks of O^T
  constexpr int DQ = D / 32;            // 1 KiB K blocks per 16-key chunk
  constexpr int COLS = 32 * NW;
  constexpr int PLANE = KT * D * 2;     // bytes of one K or V tile
  constexpr int NKS = pipe_nks<D>();    // K tile slots
  constexpr int NVS = NKS + 1;          // V tile slots: V(kt) is read while V(kt+1) is converted
  constexpr int NBLK = (KT / 16) * DQ;  // 1 KiB blocks of a K (or V) tile
  // The 160 layout's 20 blocks (5 per chunk) go to the 8 waves as 3 + 2 per
  // chunk: a wave with two issues a third load that reads nothing (offset
  // past its resource) into a scratch block, so that every wave issues the
  // same number of loads and every wait count stays static.
  constexpr bool SPLIT = NBLK % NW != 0;
  constexpr int IPW = (NBLK + NW - 1) / NW;  // K DMA instructions per wave per tile
  static_assert(IPW >= 1 && IPW <= 4, "one to four 1 KiB blocks per wave and operand");
  static_assert(SPLIT ? (DQ == 5 && NW == 2 * (KT / 16) && IPW == 3) : DQ % IPW == 0,
                "a wave's blocks lie in one chunk");
  constexpr int VJ = (PLANE + 16 * NT - 1) / (16 * NT);  // 16-byte pieces per thread of a V tile
  constexpr bool VJ_PART = PLANE % (16 * NT) != 0;       // the last piece: the first threads only
  // loads issued after V(kt+2) that may still be in flight when this wave's
  // K(kt+2) and V(kt+2) must have landed (end of step kt): the K/V loads of
  // the NKS-2 later steps
  constexpr int VMW = (NKS - 2) * 2 * IPW;
  static_assert(NKS >= 3, "K/V tiles are issued at least three steps ahead");

  // K ring, then V ring (the output tile reuses both once the last step is done)
  __shared__ __align__(1024) char s_kv[(NKS + NVS) * PLANE];
  __shared__ __align__(1024) char s_dummy[SPLIT ? 1024 : 16];   // target of the loads that read nothing
  char *const s_k = s_kv;
  char *const s_v = s_kv + NKS * PLANE;
  __shared__ int s_tab[kTabP];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int l32 = lane & 31;
  const int h2 = lane >> 5;

  __shared__ int s_flag;   // some column of this item needs the exact re-run
  // A workgroup runs the plan's items for it one after another (one
  // workgroup per CU: no dispatch gap between them, and the next item's
  // plan entry is known before the current one ends).
  const int rounds = prefill_rounds(p);
  for (int round = 0; round < rounds; ++round) {
  PrefillItem it;
  if (!prefill_item(p, it, round)) break;
  if (round > 0) {
    // every wave has read its previous output tile out of the V ring
    lgkm_drain();
    barrier();
  }
  const int grp = it.grp, qt = it.qt, seg = it.seg;
  const int kh = grp - seg * p.KH;
  const long tok0 = it.tok0;
  const int len = it.len;
  const int G = p.G;
  const int rows = COLS / G;
  const int r0 = qt * rows;
  if (r0 >= len) continue;
  const int start = it.start;
  const int context = start + len;
  const long slot = it.slot;
  const int rows_here = min(rows, len - r0);

  const int k_hi = start + r0 + rows_here;  // exclusive
  const int k_lo = p.window > 0 ? max(0, start + r0 - p.window + 1) : 0;
  const int kt_first = k_lo / KT;
  const int kt_last = (k_hi - 1) / KT;

  // page-table entries of the 16-key chunks this item visits
  const int e_first = (kt_first * KT) >> p.page_shift;
  const int e_count = (((kt_last + 1) * KT - 1) >> p.page_shift) - e_first + 1;
  const bool slot_ok = slot >= 0 && slot < p.table_rows;
  auto table_entry = [&](int e) {
    const int phys = (slot_ok && e < p.table_w) ? p.table[slot * p.table_w + e] : -1;
    return (phys >= 0 && phys < p.capacity) ? phys : -1;
  };
  // The same lookup without a branch: every lane loads (through a buffer
  // resource over the table, so that an index past it reads 0 instead of
  // faulting) and the result is selected afterwards.  In the prologue this
  // keeps all of the loads in flight at once; behind a divergent branch the
  // compiler waits for each one before the next.
  const __amdgpu_buffer_rsrc_t tab_rsrc = __builtin_amdgcn_make_buffer_rsrc(
      (void *)p.table, (short)0, (int)min(0x7fffffffL, (long)p.table_rows * p.table_w * 4), kBufferWord3);
  auto table_entry_nb = [&](int e, bool want) __attribute__((always_inline)) {
    const bool ok = want && slot_ok && e < p.table_w;
    const long idx = ok ? slot * p.table_w + e : 0;
    const int v = __builtin_amdgcn_raw_buffer_load_b32(tab_rsrc, (int)(4 * idx), 0, 0);
    return (ok && v >= 0 && v < p.capacity) ? v : -1;
  };
  auto table_at = [&](int e) -> int {   // wave-uniform
    const int i = e - e_first;
    return i < kTabP ? s_tab[i] : table_entry(e);
  };

  // ---- this lane's query column; Q^T operands (B of S^T) ----
  const int col = w * 32 + l32;
  const int qr = col / G;
  const int gh = col - qr * G;
  const bool colok = qr < rows_here;
  const int qpos = start + r0 + (colok ? qr : 0);
  u32x4 qb[NCCR];  // loaded in the prologue

  // ---- loads ----
  // K: wave w fills blocks kb0 .. kb0 + nblk - 1 of a tile (block b: chunk
  // b / DQ, dims 32 (b % DQ)..)
  const int k_chunk = SPLIT ? w >> 1 : w * IPW / DQ;
  const int kq0 = SPLIT ? 3 * (w & 1) : w * IPW % DQ;   // first block within the chunk
  const int kb0 = k_chunk * DQ + kq0;
  const int nblk = SPLIT ? ((w & 1) ? DQ - 3 : 3) : IPW;
  // lanes whose 8 dims lie past the real head size load nothing (an offset
  // past every buffer resource reads as zero)
  // (the per-block offsets are held as scalars, not an array a lambda captures)
  auto k_off = [&](int j) {
    const int d0 = 32 * (kq0 + j) + 8 * (lane >> 4);
    return d0 < DR && j < nblk ? 2u * ((lane & 15) * DR + d0) : 0x80000000u;
  };
  constexpr bool DMA_IMM = DR == D && !SPLIT;   // block j at immediate offset 64 j of one lane offset
  const unsigned k_dma0 = k_off(0), k_dma1 = DMA_IMM || IPW < 2 ? 0u : k_off(1),
                 k_dma2 = DMA_IMM || IPW < 3 ? 0u : k_off(2), k_dma3 = DMA_IMM || IPW < 4 ? 0u : k_off(3);
  // LDS destination of load j within a tile slot (a scratch block for a load
  // that reads nothing)
  auto dma_dst = [&](char *slot, int j) __attribute__((always_inline)) -> char * {
    if constexpr (SPLIT) return j < nblk ? slot + (kb0 + j) * 1024 : s_dummy;
    return slot + (kb0 + j) * 1024;
  };
  // Page of one 16-key chunk of tile kt (-1: none, or past the last tile).
  // The lookups for a step's loads are read from LDS during the previous
  // step, so that no step starts by waiting for one.
  auto lookup = [&](int kt, int chunk) __attribute__((always_inline)) -> int {
    return kt <= kt_last ? table_at((kt * KT + 16 * chunk) >> p.page_shift) : -1;
  };
  // Buffer resource of the chunk's live rows; tiles past the last one load
  // nothing (zero-size resource): loads are issued unconditionally so that
  // every wait count is static.
  auto chunk_rsrc = [&](const void *plane, int kt, int chunk, int phys_in) __attribute__((always_inline)) {
    const int key0 = kt * KT + 16 * chunk;
    const int phys = uniform(phys_in);
    const int live = phys < 0 ? 0 : min(16, context - key0);
    const long base =
        phys < 0 ? 0 : ((((long)phys * p.KH + kh) << p.page_shift) | (key0 & (p.page - 1))) * (long)DR;
    return __builtin_amdgcn_make_buffer_rsrc((void *)uniform_ptr((const char *)plane + 2 * base), (short)0,
                                             uniform(live > 0 ? live * DR * 2 : 0), kBufferWord3);
  };
  auto issue_k = [&](int kt, int phys) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(p.k, kt, k_chunk, phys);
    char *slot = s_k + ((kt - kt_first) % NKS) * PLANE;
#pragma unroll
    for (int j = 0; j < IPW; ++j)
      if constexpr (DMA_IMM)   // block j is 32 dims (64 bytes) further along the row
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)dma_dst(slot, j), 16, k_dma0, 64 * j, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void *)dma_dst(slot, j), 16, j == 0 ? k_dma0 : j == 1 ? k_dma1 : j == 2 ? k_dma2 : k_dma3, 0, 0,
            0);
  };
  // V: blocks (chunk, md) of 1 KiB, the same chunk as K; DMA lane m of block
  // (c, md) brings the 16 bytes V[16c + 8(m/32) + 4((m%32)/16) + ((m%32)/2)%4]
  // [8q8 ..+8], q8 = 4md + 2(((m%32)/8)%2) + m%2: the two 8-byte pieces that
  // the transposing read of region (c, md, half m/32) hands lanes 2(m%32)
  // and 2(m%32)+1.  bf16 tiles are converted to fp16 in place afterwards.
  auto v_off = [&](int j) {
    const int m = lane & 31;
    const int key = 8 * (lane >> 5) + 4 * (m >> 4) + ((m >> 1) & 3);
    const int q8 = 4 * (kq0 + j) + 2 * ((m >> 3) & 1) + (m & 1);
    return 8 * q8 < DR && j < nblk ? (unsigned)(key * DR * 2 + 16 * q8) : 0x80000000u;
  };
  const unsigned v_dma0 = v_off(0), v_dma1 = DMA_IMM || IPW < 2 ? 0u : v_off(1),
                 v_dma2 = DMA_IMM || IPW < 3 ? 0u : v_off(2), v_dma3 = DMA_IMM || IPW < 4 ? 0u : v_off(3);
  auto issue_v = [&](int kt, int phys) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t rs = chunk_rsrc(p.v, kt, k_chunk, phys);
    char *slot = s_v + ((kt - kt_first) % NVS) * PLANE;
#pragma unroll
    for (int j = 0; j < IPW; ++j)
      if constexpr (DMA_IMM)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void *)dma_dst(slot, j), 16, v_dma0, 64 * j, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void *)dma_dst(slot, j), 16, j == 0 ? v_dma0 : j == 1 ? v_dma1 : j == 2 ? v_dma2 : v_dma3, 0, 0,
            0);
  };
  const unsigned v_base = lds_addr(s_v);
  // bf16 V tile kt -> fp16 in place (16 contiguous bytes per lane), in two
  // halves: the reads, and after other work the conversion and writes
  auto convert_v_read = [&](int kt, u32x4 (&x)[VJ]) __attribute__((always_inline)) {
    if constexpr (DT == DD_BF16) {
      const unsigned base = v_base + ((kt - kt_first) % NVS) * PLANE + 16u * tid;
#pragma unroll
      for (int j = 0; j < VJ; ++j)
        if (!VJ_PART || j + 1 < VJ || 16 * (tid + j * NT) < PLANE) x[j] = lds_read128(base, j * 16 * NT);
    }
  };
  auto convert_v_write = [&](int kt, u32x4 (&x)[VJ]) __attribute__((always_inline)) {
    if constexpr (DT == DD_BF16) {
      const unsigned base = v_base + ((kt - kt_first) % NVS) * PLANE + 16u * tid;
#pragma unroll
      for (int j = 0; j < VJ; ++j) lgkm_wait(x[j], 0);
#pragma unroll
      for (int j = 0; j < VJ; ++j)
        if (!VJ_PART || j + 1 < VJ || 16 * (tid + j * NT) < PLANE) lds_write128(base, j * 16 * NT, bf16x8_to_f16x8(x[j]));
    }
  };
  auto convert_v = [&](int kt) __attribute__((always_inline)) {
    u32x4 x[VJ];
    convert_v_read(kt, x);
    convert_v_write(kt, x);
  };

  // ---- S^T of one tile: two 32-key blocks ----
  const unsigned k_rd = lds_addr(s_k) + 1024u * DQ * ((lane >> 4) & 1) + 16u * (lane & 15) + 256u * h2;
  auto compute_s = [&](int kt, f32x16 (&s)[NSB]) __attribute__((always_inline)) {
    const unsigned kb_addr = k_rd + (unsigned)(((kt - kt_first) % NKS) * PLANE);
    // operand i = (cc, b) = (i / NSB, i % NSB); R reads in flight
    constexpr int N = NSB * NCCR, R = 4;
    auto rd = [&](int i) __attribute__((always_inline)) {
      const int cc = i / NSB, b = i % NSB;
      return lds_read128(kb_addr, (2 * b * DQ + cc / 2) * 1024 + 512 * (cc & 1));
    };
    u32x4 kop[R];
#pragma unroll
    for (int i = 0; i < R; ++i) kop[i] = rd(i);
#pragma unroll
    for (int i = 0; i < N; ++i) {
      const int cc = i / NSB, b = i % NSB;
      lgkm_wait(kop[i % R], min(R - 1, N - 1 - i));
      s[b] = mfma_s<DT>(kop[i % R], qb[cc], cc == 0 ? f32x16{} : s[b]);
      if (i + R < N) kop[i % R] = rd(i + R);
    }
  };
  f32x16 o[MDR];
#pragma unroll
  for (int md = 0; md < MDR; ++md) o[md] = f32x16{};
  float m_run = kNegInf;
  float l_part = 0.f;   // this lane's share of the column's denominator

  const float sc = p.scale_log2;
  const float slack = kMaxSlack / sc;
  const unsigned v_rd = v_base + 8u * lane;

  // ---- softmax pieces ----
  // Bookkeeping of tile kt from its column max: the exponent offset mu; O
  // and l are rescaled when the running max moves.
  auto softmax_begin = [&](float mx) __attribute__((always_inline)) -> float {
    const bool up = mx > m_run + slack;   // m_run = -inf moves to any finite max
    const float mn = up ? mx : m_run;
    const float mu = mn == kNegInf ? 0.f : mn * sc;
    const float alpha = up ? __builtin_amdgcn_exp2f(m_run * sc - mu) : 1.f;
    m_run = mn;
    if (__builtin_amdgcn_ballot_w64(up)) {
#pragma unroll
      for (int md = 0; md < MDR; ++md) o[md] *= alpha;
      l_part *= alpha;
    }
    return mu;
  };
  // Probabilities 2i, 2i+1 of this lane (i < 8 NSB: block i / 8, registers
  // 2 (i % 8) ..+2) into the fp16 P^T operands, and into the row sum.
  auto softmax_pair = [&](f32x16 (&s)[NSB], int i, float mu, u32x4 (&pp)[NSB][2], float &lsum)
      __attribute__((always_inline)) {
    const int b = i >> 3, r = 2 * (i & 7);
    const float e0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][r], sc, -mu));
    const float e1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[b][r + 1], sc, -mu));
    const unsigned h = cvt_pk_f16(e0, e1);
    pp[b][(i & 7) >> 2][i & 3] = h;
    lsum = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, h), f16x2{(_Float16)1.f, (_Float16)1.f}, lsum, false);
  };
  // mask of tile kt (keys past a column's diagonal or before its window);
  // key of register r of block b is kt*KT + 32b + 8(r/4) + 4h2 + r%4
  auto mask = [&](int kt, f32x16 (&s)[NSB]) __attribute__((always_inline)) {
    const int kbase = kt * KT;
    if (!(kbase + KT - 1 <= start + r0 && (p.window == 0 || kbase >= start + r0 + rows_here - p.window))) {
      const int lo = p.window > 0 ? qpos - p.window + 1 : -1;
#pragma unroll
      for (int b = 0; b < NSB; ++b) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = kbase + 32 * b + 8 * (r >> 2) + 4 * h2 + (r & 3);
          s[b][r] = ((key <= qpos) & (key >= lo)) ? s[b][r] : kNegInf;
        }
      }
    }
  };
  // partial column max over registers 4i .. 4i+3 of both blocks
  auto max_part = [&](f32x16 (&s)[NSB], int i, float &mx) __attribute__((always_inline)) {
#pragma unroll
    for (int b = 0; b < NSB; ++b) mx = fmaxf(fmaxf(mx, s[b][4 * i]), s[b][4 * i + 1]);
#pragma unroll
    for (int b = 0; b < NSB; ++b) mx = fmaxf(fmaxf(mx, s[b][4 * i + 2]), s[b][4 * i + 3]);
  };

  // ---- matrix-core phase of step kt: S(kt+1) = K(kt+1) Q^T (when there is
  // a tile kt+1), then O += V(kt)^T P(kt).  One stream of LDS operands: K
  // operands (one ds_read_b128 each), then V^T operands (two transposing
  // reads each), R operands in flight.  The step's loads are issued after
  // the first MFMAs, so that any wait for the memory pipeline overlaps them.
  auto mfma_phase = [&](auto has_next_c, int kt, f32x16 (&s)[NSB], const u32x4 (&pp)[NSB][2], auto &&loads)
      __attribute__((always_inline)) {
    constexpr bool HN = decltype(has_next_c)::value;
    constexpr int NS = HN ? NSB * NCCR : 0, NV = 2 * NSB * MDR, N = NS + NV, R = pipe_ring<D>();
    const unsigned kb_addr = k_rd + (unsigned)(((kt + 1 - kt_first) % NKS) * PLANE);
    const unsigned vb = v_rd + (unsigned)(((kt - kt_first) % NVS) * PLANE);
    // operand i < NS: one K read; else two transposing reads
    u32x4 kop[R];
    u32x2 lo[R], hi[R];
    auto rd = [&](int i) __attribute__((always_inline)) {
      if (i < NS) {
        const int cc = i / NSB, b = i % NSB;
        kop[i % R] = lds_read128(kb_addr, (2 * b * DQ + cc / 2) * 1024 + 512 * (cc & 1));
      } else {
        const int j = i - NS, blk = (j / MDR) * MD + j % MDR;   // (key block, dim block)
        lo[i % R] = lds_read_tr(vb, 2 * blk * 512);
        hi[i % R] = lds_read_tr(vb, 2 * blk * 512 + 512);
      }
    };
    // LDS instructions issued after operand i while it is awaited
    auto after = [](int i) constexpr {
      int n = 0;
      for (int j = i + 1; j < i + R && j < N; ++j) n += j < NS ? 1 : 2;
      return n;
    };
#pragma unroll
    for (int i = 0; i < R; ++i) rd(i);
    if constexpr (!HN) loads();
#pragma unroll
    for (int i = 0; i < N; ++i) {
      if (i < NS) {
        const int cc = i / NSB, b = i % NSB;
        lgkm_wait(kop[i % R], after(i));
        s[b] = mfma_s<DT>(kop[i % R], qb[cc], cc == 0 ? f32x16{} : s[b]);
      } else {
        const int j = i - NS, md = j % MDR, bj = j / MDR;
        lgkm_wait(lo[i % R], hi[i % R], after(i));
        const u32x4 op = {lo[i % R][0], lo[i % R][1], hi[i % R][0], hi[i % R][1]};
        o[md] = mfma_o(op, pp[bj >> 1][bj & 1], o[md]);
      }
      if (i + R < N) rd(i + R);
      if (HN && i == 1) loads();
    }
  };

  // ---- vector phase of step kt: P(kt+1) from S(kt+1); V(kt+1) to fp16 in
  // its LDS slot; the page number of the next step's loads.  The LDS reads
  // go first and the LDS writes mid-way, so that their latencies overlap
  // the softmax.
  // The exponentials are taken against the column's current offset without
  // a max over the tile: while no score exceeds the running max by 16 (in
  // the exp2 domain) every probability is a finite fp16 value and nothing
  // moves.  A column without a running max yet (offset -inf) or a
  // probability past fp16's range shows up as a non-finite row sum; then
  // the wave redoes the tile with the tile's max (moving the offset and
  // rescaling O and l as usual) ----
  auto valu_phase = [&](int kt, f32x16 (&s)[NSB], u32x4 (&pp)[NSB][2], int &pk)
      __attribute__((always_inline)) {
    u32x4 x[VJ];
    convert_v_read(kt + 1, x);
    pk = lookup(kt + NKS + 1, k_chunk);
    mask(kt + 1, s);
    const float mu0 = m_run * sc;
    float lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 4 * NSB; ++i) softmax_pair(s, i, mu0, pp, lsum);
    // V(kt+1) of every wave landed before the previous barrier
    convert_v_write(kt + 1, x);
#pragma unroll
    for (int i = 4 * NSB; i < 8 * NSB; ++i) softmax_pair(s, i, mu0, pp, lsum);
    if (__builtin_amdgcn_ballot_w64(!(lsum <= 3.0e38f))) {
      float m = kNegInf;
#pragma unroll
      for (int i = 0; i < 4; ++i) max_part(s, i, m);
      const float mu = softmax_begin(xor32_max(m));
      lsum = 0.f;
#pragma unroll
      for (int i = 0; i < 8 * NSB; ++i) softmax_pair(s, i, mu, pp, lsum);
    }
    l_part += lsum;
    // this wave's K(kt+2) and V(kt+2) land before the next barrier
    vm_wait<VMW>();
  };

  // ---- prologue: K and V of tiles f .. f+NKS-1 in flight, V(f) in fp16, P(f) ----
  f32x16 s[NSB];
  u32x4 pp[NSB][2];   // P(kt) as fp16 P^T operands
  // All the prologue's loads go out together, each without a branch (see
  // table_entry_nb): the first tiles' page numbers, then the item's
  // page-table entries for the LDS copy and Q; then, once the page numbers
  // are in, the first tiles' K/V loads.  The LDS writes of the entries wait
  // for them alone (loads complete in order), not for the tiles.
  int first_ph[NKS];
#pragma unroll
  for (int i = 0; i < NKS; ++i)
    first_ph[i] = table_entry_nb(((kt_first + i) * KT + 16 * k_chunk) >> p.page_shift, kt_first + i <= kt_last);
  constexpr int kTabPer = (kTabP + NT - 1) / NT;
  int tab_v[kTabPer];
#pragma unroll
  for (int j = 0; j < kTabPer; ++j) {
    const int i = tid + NT * j;
    tab_v[j] = table_entry_nb(e_first + i, i < e_count && i < kTabP);
  }
  {
    const long row = (tok0 + r0 + (colok ? qr : 0)) * p.H + (long)kh * G + gh;
    const unsigned short *qsrc = (const unsigned short *)p.q + row * DR + 8 * h2;
#pragma unroll
    for (int cc = 0; cc < NCCR; ++cc) {
      const u32x4 x = *(const u32x4 *)(qsrc + 16 * cc);   // row clamped into the segment
      // (a mask the compiler cannot see through: every lane loads, so the
      // loads are not put behind a branch and waited for one by one)
      unsigned m = colok ? ~0u : 0u;
      asm volatile("" : "+v"(m));
      qb[cc] = (x ^ p.q_sign) & m;
    }
  }
#pragma unroll
  for (int i = 0; i < NKS; ++i) {
    issue_k(kt_first + i, first_ph[i]);
    issue_v(kt_first + i, first_ph[i]);
  }
#pragma unroll
  for (int j = 0; j < kTabPer; ++j) {
    const int i = tid + NT * j;
    if (i < e_count && i < kTabP) s_tab[i] = tab_v[j];
  }
  if (tid == 0) s_flag = 0;
  // s_tab and s_flag for every wave; no wait for the tiles in flight (a
  // __syncthreads would wait for every load)
  lgkm_drain();
  barrier();
  int pk = lookup(kt_first + NKS, k_chunk);
  vm_wait<VMW>();   // K and V of tiles f and f+1 have landed
  barrier();        // ... for every wave
  convert_v(kt_first);
  lgkm_drain();
  barrier();
  compute_s(kt_first, s);
  {
    mask(kt_first, s);
    float m = kNegInf;
#pragma unroll
    for (int i = 0; i < 4; ++i) max_part(s, i, m);
    const float mu = softmax_begin(xor32_max(m));
    float lsum = 0.f;
#pragma unroll
    for (int i = 0; i < 8 * NSB; ++i) softmax_pair(s, i, mu, pp, lsum);
    l_part += lsum;
  }
  barrier();   // every wave has read K(kt_first) before step kt_first reloads its slot

  // ---- steady state ----
  // Step kt: K(kt+NKS) into the slot of K(kt) and V(kt+NKS) into the slot of
  // V(kt-1) (zero-size past the last tile, so that every wait count is
  // static); S(kt+1) and O += V(kt) P(kt) on the matrix cores; P(kt+1) and
  // V(kt+1) to fp16 on the vector ALU; barrier.
  // (the last step, which has no tile kt+1, is peeled off so that the loop
  // body has one path and the O accumulators keep their registers)
  for (int kt = kt_first; kt < kt_last; ++kt) {
    // this step's page number, read from LDS during the previous step, into
    // a scalar register now (no LDS operation of this wave is in flight)
    int pku = uniform(pk);
    asm volatile("" : "+s"(pku));
    mfma_phase(std::true_type{}, kt, s, pp, [&]() __attribute__((always_inline)) {
      issue_k(kt + NKS, pku);
      issue_v(kt + NKS, pku);
    });
    valu_phase(kt, s, pp, pk);
    lgkm_drain();
    barrier();
  }
  mfma_phase(std::false_type{}, kt_last, s, pp, [] {});
  vm_wait<0>();   // no load outlives the workgroup

  // ---- normalise and store: lane holds dims 32md + 8(r/4) + 4h2 + r%4 of its column ----
  const float l = xor32_sum(l_part);
  if constexpr (DT == DD_BF16) {
    if (p.flags) {
      // largest |O| of the column (as bits: infinities and NaNs compare
      // above every finite value), relative to the denominator
      unsigned mb = 0;
#pragma unroll
      for (int md = 0; md < MDR; ++md) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mb = max(mb, __float_as_uint(o[md][r]) & 0x7fffffffu);
      }
      mb = max(mb, (unsigned)__shfl_xor((int)mb, 32));
      const float top = __uint_as_float(mb) / l;
      const bool redo = colok && !(top >= 0x1p-12f && top <= 3.0e38f);
      if (__builtin_amdgcn_ballot_w64(redo) && lane == 0) s_flag = 1;
      __syncthreads();
      if (tid == 0) p.flags[(long)grp * p.max_tiles + qt] = s_flag;
      // the group's first item also clears the flags of the tiles past the
      // segment, so that every flag of a group with work is defined
      if (qt == 0)
        for (int t = (len + rows - 1) / rows + tid; t < p.max_tiles; t += NT) p.flags[(long)grp * p.max_tiles + t] = 0;
    }
  }
  // The output goes through LDS so that every store writes whole 16-byte
  // pieces of contiguous (query row, head) rows: stored straight from the
  // O^T registers, each 8-byte store instruction would touch 32 rows.  Each
  // wave writes its 32 normalised columns as rows (padded by 16 bytes) into
  // the V ring (the 160 layout: from the start of the K ring on), free once
  // every wave has finished its last P.V reads and its loads -- the
  // zero-size trailing ones included -- have landed.
  lgkm_drain();
  barrier();
  constexpr int ORS = 2 * DR + 16;      // LDS row stride of the output tile
  static_assert(NW * 32 * ORS <= (NKS + NVS) * PLANE, "output tile fits the K and V rings");
  char *otile = (NW * 32 * ORS <= NVS * PLANE ? s_v : s_kv) + w * 32 * ORS;
  if (colok) {
    const float inv = 1.f / l;
#pragma unroll
    for (int md = 0; md < MDR; ++md) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        if (DR < D && 32 * md + 8 * q4 + 4 * h2 >= DR) continue;
        const f32x16 &x = o[md];
        const u32x2 pk = {pack2<DT>(x[4 * q4 + 0] * inv, x[4 * q4 + 1] * inv),
                          pack2<DT>(x[4 * q4 + 2] * inv, x[4 * q4 + 3] * inv)};
        *(u32x2 *)(otile + l32 * ORS + 2 * (32 * md + 8 * q4 + 4 * h2)) = pk;
      }
    }
  }
  // (the wave reads back only what it wrote: LDS operations of one wave
  // complete in order)
  constexpr int PR = DR / 8;            // 16-byte pieces per row
  unsigned short *dst = (unsigned short *)p.out;
#pragma unroll
  for (int e0 = 0; e0 < 32 * PR; e0 += 64) {
    const int e = e0 + lane;
    const int c = e / PR, k = e - (e / PR) * PR;
    const int cq = (w * 32 + c) / G;
    if (e < 32 * PR && cq < rows_here) {
      const int cg = w * 32 + c - cq * G;
      const u32x4 x = *(const u32x4 *)(otile + c * ORS + 16 * k);
      *(u32x4 *)(dst + ((tok0 + r0 + cq) * p.H + (long)kh * G + cg) * DR + 8 * k) = x;
    }
  }
  }
}

template <int DT, int D, int DR = D>
int launch_pipe(PrefillParams p, int max_len, int plan_len, hipStream_t s) {
  constexpr int COLS = 32 * pipe_waves<D>();
  if (COLS / p.G < 1) return DD_EUNSUPPORTED;
  p.max_tiles = (int)dd_cdiv(max_len, COLS / p.G);
  const long grid = p.plan ? (long)plan_len : 8L * dd_cdiv((long)p.n * p.KH, 8) * p.max_tiles;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_pipe_kernel<DT, D, DR>), dim3((unsigned)grid), dim3(64 * pipe_waves<D>()), 0, s, p);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

template <int DT>
int pipe_dims(const PrefillParams &p, int dim, int max_len, int plan_len, hipStream_t s) {
  switch (dim) {
    case 48: return launch_pipe<DT, 64, 48>(p, max_len, plan_len, s);
    case 64: return launch_pipe<DT, 64>(p, max_len, plan_len, s);
    case 80: return launch_pipe<DT, 128, 80>(p, max_len, plan_len, s);
    case 96: return launch_pipe<DT, 128, 96>(p, max_len, plan_len, s);
    case 112: return launch_pipe<DT, 128, 112>(p, max_len, plan_len, s);
    case 128: return launch_pipe<DT, 128>(p, max_len, plan_len, s);
    case 144: return launch_pipe<DT, 160, 144>(p, max_len, plan_len, s);
    case 160: return launch_pipe<DT, 160>(p, max_len, plan_len, s);
    case 176: return launch_pipe<DT, 256, 176>(p, max_len, plan_len, s);
    case 192: return launch_pipe<DT, 256, 192>(p, max_len, plan_len, s);
    case 208: return launch_pipe<DT, 256, 208>(p, max_len, plan_len, s);
    case 224: return launch_pipe<DT, 256, 224>(p, max_len, plan_len, s);
    case 240: return launch_pipe<DT, 256, 240>(p, max_len, plan_len, s);
    case 256: return launch_pipe<DT, 256>(p, max_len, plan_len, s);
    default: return DD_EUNSUPPORTED;
  }
}

}  // namespace

int prefill_pipe_dispatch(const PrefillParams &p, int dtype, int dim, int max_len, int plan_len, hipStream_t s) {
  if (dtype == DD_BF16) return pipe_dims<DD_BF16>(p, dim, max_len, plan_len, s);
  if (dtype == DD_F16) return pipe_dims<DD_F16>(p, dim, max_len, plan_len, s);
  return DD_EUNSUPPORTED;
}

}  // namespace dd_prefill
