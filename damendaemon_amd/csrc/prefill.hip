// Chunked-prefill attention over the paged KV cache, bf16 / fp16 MFMA (gfx950).
//
// Semantics (damendaemon/paged.py:97-111 with qwen2.py:754-770 and
// device.py:65-80): segment i holds len_i query tokens appended after
// start_i cached tokens of slot_i; query row j (position start_i + j) attends
// the keys 0 .. start_i + j of that slot (lower-right causal), and with a
// window only keys > position - window; GQA head h reads KV head h / G;
// softmax(q.k * scale) . v in fp32.  The K/V of the chunk itself must already
// be in the pages (dd_store_kv_pages / dd_rope_batch), exactly as the
// reference gathers start+len tokens with copy_pages before its SDPA.
//
// This file holds the C entry point, the host-side workgroup plan, and the
// 16x16x32 MFMA kernel used for head sizes 144-240 (prefill_pipe.hip takes
// 48-128 and 256, prefill_f32.hip / prefill_generic.hip fp32 pages and the
// other head sizes).
//
// MI355X design of the 16x16x32 kernel:
//   * a workgroup owns one KV head and 16*NQ*NW (query row, head) columns of
//     one segment (all G query heads of a KV head share every K/V byte);
//   * keys stream in 64-key tiles (four 16-token pages): K and V rows are
//     staged row-major in LDS (16-byte conflict-free writes); the V^T MFMA
//     operand comes from two transposing LDS reads (ds_read_b64_tr_b16,
//     which hands each 16-lane group a 4-key x 16-dim block transposed);
//     the next tile's global loads are in flight while the current tile is
//     computed;
//   * S^T = K Q^T and O^T = V^T P^T with v_mfma_f32_16x16x32: in this
//     orientation the probabilities leave the S^T accumulators already in
//     the register layout of the P^T operand (keys are contracted in a fixed
//     permuted order that V^T is read in), and every lane owns one query
//     column, so the online-softmax state needs no cross-lane shuffles
//     beyond two xor-steps;
//   * P^T enters the P.V product as two 16-bit operands, its rounded high
//     part and the rounded residual, so the probabilities keep ~17 bits as
//     in the reference's fp32 softmax (one bf16 rounding, 2^-9 relative,
//     puts short-context rows several 1e-3 off);
//   * the softmax denominators come from the matrix cores too: extra MFMAs
//     of the same two P^T operands with an all-ones V^T yield the column
//     sums of exactly the P the P.V product uses.
#include "prefill_common.h"
#include "prefill_generic.h"

#include <algorithm>
#include <climits>
#include <functional>
#include <type_traits>
#include <vector>

#ifndef DD_PREFILL_NW
#define DD_PREFILL_NW 8
#endif
#ifndef DD_PREFILL_NBUF
#define DD_PREFILL_NBUF 3
#endif
// K/V tiles in flight: a tile is issued NBUF - 1 steps before it is used.
constexpr int NBUF = DD_PREFILL_NBUF;

using namespace dd_prefill;

namespace {

// LDS layout of a key tile: 1 KiB blocks, each holding exactly the data one
// wave instruction consumes, in lane order (lane l at byte 16*l or 8*l), so
// every LDS access is lane offset + immediate and conflict-free.
//   K block (mt, cc): lane l's 16 bytes = K[key 16mt + l%16][dims 8(l/16) + 32cc ..+8),
//     the A operand of the S^T MFMA for key tile mt and dim chunk cc.
//   V block pair (c2, h, mp): two 512-byte halves md = 2mp, 2mp+1; lane L of
//     a half reads 8 bytes at 8*L: V[key 32c2 + 16h + 4(L/16) + (L%16)/4]
//     [dims 16md + 4(L%4) ..+4) -- the addresses one transposing read wants.
// The direct-to-LDS loads fill these blocks: DMA lane l of a V block pair
// covers read lanes 2(l%32), 2(l%32)+1 of half l/32 (16 contiguous bytes).
//
// Schedule.  K and V tiles rotate through three LDS buffers each.  Step t
// issues the loads of tile t+2 into the buffers of tile t-1 (every wave left
// them at the previous barrier), computes S(t) = K(t) Q^T, the online
// softmax and O += V(t)^T P(t)^T, then waits for its own loads of tile t+1
// and meets the other waves at a barrier: a tile's loads have about two
// steps to land.  The two waves that share a SIMD overlap one's MFMAs with
// the other's softmax.
// Keys past the context and chunks without an allocated page are loaded as
// zeros: every chunk load goes through a buffer resource whose size covers
// only the chunk's live rows (out-of-range buffer loads return 0).

// D is the LDS layout's head size; DR <= D the real one (a multiple of 16
// above D / 2): rows are DR elements long in memory, the layout's dims DR ..
// D-1 are loaded as zeros (DMA lanes past DR read out of the resource's
// range) and the MFMAs skip the k-chunks and O^T tiles that hold only them.
template <int DT, int D, int NQ, int KT, int NW, int DR = D>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(NW / 4))) void prefill_kernel(PrefillParams p) {
  static_assert(DR % 16 == 0 && DR <= D && 2 * DR > D, "real head size");
  constexpr int NC = D / 32;           // k-chunks of q.k (layout)
  constexpr int NCR = (DR + 31) / 32;  // k-chunks holding real dims
  constexpr int MD = D / 16;           // O^T row tiles (layout)
  constexpr int MDR = DR / 16;         // O^T row tiles of real dims
  constexpr int MT = KT / 16;          // 16-key chunks per tile
  constexpr int C2 = KT / 32;          // 32-key MFMA k-steps of P.V per tile
  constexpr int COLS = 16 * NQ * NW;   // (query row, head) columns per workgroup
  constexpr int NT = 64 * NW;          // threads
  constexpr int KBLK = MT * NC;        // K blocks per tile
  constexpr int VBLK = C2 * 2 * (MD / 2);  // V block pairs per tile
  constexpr int PLANE = KBLK * 1024;
  static_assert(KBLK == VBLK && KBLK % NW == 0, "every wave issues whole blocks");
  constexpr int IPW = KBLK / NW;       // DMA instructions per wave per plane
  static_assert(NC % IPW == 0 && MD / 2 == NC, "a wave's blocks share one 16-key chunk");
  static_assert(2 * (NBUF - 2) * IPW < 16, "vmcnt immediate");

  // Six distinct buffers (three K, three V).  Every direct-to-LDS load and
  // every LDS read below names one of them at compile time (the tile loop is
  // unrolled by three), so the compiler can tell that reads of one buffer do
  // not wait for loads still landing in another.
  __shared__ __align__(1024) char s_v0[PLANE], s_v1[PLANE], s_v2[PLANE];  // lowest addresses: read most
  __shared__ __align__(1024) char s_v3[NBUF > 3 ? PLANE : 16];
  __shared__ __align__(16) char s_k0[PLANE], s_k1[PLANE], s_k2[PLANE];
  __shared__ __align__(16) char s_k3[NBUF > 3 ? PLANE : 16];
  __shared__ int s_tab[kTabCache];                   // page-table window of this slot

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int g4 = lane >> 4;
  const int l16 = lane & 15;

  // Without a plan: consecutive workgroups go to the 8 XCDs round-robin,
  // each XCD with its own L2; every query tile of one (segment, KV head)
  // group is sent to the same XCD, longest first.  With a plan
  // (dd_prefill_plan) the host has chosen and balanced this order.
  PrefillItem it;
  if (!prefill_item(p, it)) return;
  const int grp = it.grp, qt = it.qt, seg = it.seg;
  const int kh = grp - seg * p.KH;
  const long tok0 = it.tok0;
  const int len = it.len;
  const int G = p.G;
  const int rows = COLS / G;
  const int r0 = qt * rows;
  if (r0 >= len) return;
  const int start = it.start;
  const int context = start + len;
  const long slot = it.slot;
  const int rows_here = min(rows, len - r0);

  const int k_hi = start + r0 + rows_here;   // exclusive
  int k_lo = 0;
  if (p.window > 0) k_lo = max(0, start + r0 - p.window + 1);
  const int kt_first = k_lo / KT;
  const int kt_last = (k_hi - 1) / KT;

  // The page-table entries of the key range are staged in LDS once, already
  // validated (-1 for an unallocated entry or one outside the cache), so no
  // global page-table load or bounds test sits on a tile's critical path.
  // Entries past the first kTabCache of a very long history are read from
  // the table itself when their tile comes up.
  const int e_first = (kt_first * KT) >> p.page_shift;
  const int e_count = ((((kt_last + 1) * KT) - 1) >> p.page_shift) - e_first + 1;
  const bool slot_ok = slot >= 0 && slot < p.table_rows;
  auto table_entry = [&](int e) {
    const int phys = (slot_ok && e < p.table_w) ? p.table[slot * p.table_w + e] : -1;
    return (phys >= 0 && phys < p.capacity) ? phys : -1;
  };
  for (int i = tid; i < e_count && i < kTabCache; i += NT) s_tab[i] = table_entry(e_first + i);

  // ---- per-lane query columns and Q^T operands ----
  int qpos[NQ];
  bool colok[NQ];
  u32x4 qb[NQ][NCR];
  const unsigned short *qsrc = (const unsigned short *)p.q;
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    const int c = w * 16 * NQ + nq * 16 + l16;
    const int r = c / G;
    const int gh = c - r * G;
    colok[nq] = r < rows_here;
    qpos[nq] = start + r0 + (colok[nq] ? r : 0);
    const long row = (tok0 + r0 + (colok[nq] ? r : 0)) * p.H + (long)kh * G + gh;
#pragma unroll
    for (int cc = 0; cc < NCR; ++cc) {
      const bool live = colok[nq] && 32 * cc + 8 * g4 < DR;
      qb[nq][cc] = live ? *(const u32x4 *)(qsrc + row * DR + 8 * g4 + 32 * cc) ^ p.q_sign : u32x4{0, 0, 0, 0};
    }
  }

  f32x4 o[MDR][NQ];
  float m_run[NQ], alpha[NQ];
  // Row sums of P on the matrix cores: an all-ones V^T operand turns every
  // accumulator row into sum_k P[k][column] (no VALU adds, no lane reduction).
  f32x4 lacc[NQ];
  const unsigned one2 = DT == DD_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const u32x4 ones = {one2, one2, one2, one2};
  bool grew = false;
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    m_run[nq] = kNegInf;
    lacc[nq] = f32x4{0.f, 0.f, 0.f, 0.f};
    alpha[nq] = 1.f;
#pragma unroll
    for (int md = 0; md < MDR; ++md) o[md][nq] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();  // s_tab

  // ---- loads ----
  // A window of 64 consecutive staged page-table entries, one per lane, that
  // starts at the first entry of tile kt; it covers tiles kt and kt+1 (a tile
  // spans at most KT/16 <= 4 entries), so a tile's entries are read with
  // v_readlane instead of a dependent LDS round trip each.
  auto read_window = [&](int kt) -> int {
    const int i = ((kt * KT) >> p.page_shift) - e_first + lane;
    if (i < kTabCache) return s_tab[i];
    return i < e_count ? table_entry(e_first + i) : -1;
  };
  const int my_chunk = (w * IPW) / NC;   // every K and V block this wave loads lies in it
  const unsigned k_lane = 2u * (l16 * D + 8 * g4);             // K block, + 64cc bytes
  // (DR < D: a lane offset per block, past every resource for dims >= DR;
  // a wave loads at most two blocks per plane then)
  auto k_off = [&](int j) {
    const int d0 = 32 * ((w * IPW + j) % NC) + 8 * g4;
    return d0 < DR ? 2u * (l16 * DR + d0) : 0x80000000u;
  };
  const unsigned k_dma0 = DR < D ? k_off(0) : 0u, k_dma1 = DR < D && IPW > 1 ? k_off(1) : 0u;
  const int vq = lane & 31;                                     // V: read-lane pair
  const int v_key = 4 * (vq >> 3) + ((vq & 7) >> 1);           // key within the 16-key half
  const unsigned v_lane = 2u * (v_key * D + 16 * (lane >> 5) + 8 * (vq & 1));  // + 64mp bytes
  auto v_off = [&](int j) {
    const int d0 = 32 * ((w * IPW + j) % (MD / 2)) + 16 * (lane >> 5) + 8 * (vq & 1);
    return d0 < DR ? 2u * (v_key * DR + d0) : 0x80000000u;
  };
  const unsigned v_dma0 = DR < D ? v_off(0) : 0u, v_dma1 = DR < D && IPW > 1 ? v_off(1) : 0u;
  static_assert(DR == D || IPW <= 2, "per-block lane offsets held as two scalars");
  // Buffer resource over this wave's chunk of tile kt in `plane` (K or V
  // pages): its size is the chunk's live rows, 0 past the context or for an
  // unallocated page.  `win` is the window that starts at tile wkt.  Each
  // load adds a lane offset (row * 2D + column bytes) and a scalar column
  // offset; the column part stays below one 2D-byte row, so a lane's load is
  // zero exactly when its row is not live.
  auto chunk_rsrc = [&](const void *plane, int win, int wkt, int kt) __attribute__((always_inline)) __attribute__((always_inline)) {
    const int key0 = (kt * MT + my_chunk) * 16;
    const int rel = (key0 >> p.page_shift) - ((wkt * KT) >> p.page_shift);
    const int phys = __builtin_amdgcn_readlane(win, rel);
    const int live = phys < 0 ? 0 : min(16, context - key0);
    const long base = phys < 0 ? 0 : ((((long)phys * p.KH + kh) << p.page_shift) | (key0 & (p.page - 1))) * (long)DR;
    // the resource must sit in SGPRs: make its wave-uniformity explicit
    const char *addr = uniform_ptr((const char *)plane + 2 * base);
    return __builtin_amdgcn_make_buffer_rsrc((void *)addr, (short)0, uniform(live > 0 ? live * DR * 2 : 0),
                                             kBufferWord3);
  };
  auto issue_k = [&](int win, int wkt, int kt, char *buf) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = chunk_rsrc(p.k, win, wkt, kt);
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int blk = w * IPW + j;       // K block (mt, cc)
      if constexpr (DR == D)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(buf + blk * 1024), 16, k_lane, 64 * (blk % NC), 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(buf + blk * 1024), 16, j == 0 ? k_dma0 : k_dma1, 0, 0,
                                                 0);
    }
  };
  auto issue_v = [&](int win, int wkt, int kt, char *buf) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t r = chunk_rsrc(p.v, win, wkt, kt);
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int blk = w * IPW + j;       // V block pair (hc, mp)
      if constexpr (DR == D)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(buf + blk * 1024), 16, v_lane,
                                                 64 * (blk % (MD / 2)), 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void *)(buf + blk * 1024), 16, j == 0 ? v_dma0 : v_dma1, 0, 0,
                                                 0);
    }
  };
  // Wait for every load of this wave except the `recent` issued last, then
  // barrier: all waves' older loads are visible and all waves have left the
  // phase before.
  // Wait until only this wave's loads of the `younger` most recently issued
  // tiles may still be in flight, then barrier: all waves' older loads are
  // visible and all waves have left the phase before.
  auto sync = [&](int younger) __attribute__((always_inline)) {
    if (NBUF > 3 && younger >= 2) {
      __builtin_amdgcn_s_waitcnt((NBUF > 3 ? 4 * IPW : 0) | (0x7 << 4) | (0xF << 8));
    } else if (younger >= 1) {
      __builtin_amdgcn_s_waitcnt((2 * IPW) | (0x7 << 4) | (0xF << 8));
    } else {
      __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xF << 8));
    }
    __syncthreads();
  };

  // ---- S^T = K Q^T: lane holds keys 16mt + 4g4 + i for column l16 ----
  // Dim chunk outer, key chunk inner: consecutive MFMAs accumulate into
  // different registers, and the K operands of chunk cc+1 are read from LDS
  // while the MFMAs of chunk cc run.
  f32x4 s[MT][NQ];
  auto compute_s = [&](const char *kt_lds) __attribute__((always_inline)) {
#pragma unroll
    for (int cc = 0; cc < NCR; ++cc) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 a = *(const u32x4 *)(kt_lds + (mt * NC + cc) * 1024 + 16 * lane);
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq)
          s[mt][nq] = mfma<DT>(a, qb[nq][cc], cc == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : s[mt][nq]);
      }
    }
  };

  // ---- O^T += V^T P^T : keys contracted in the order of the S^T layout ----
  // k-slot 8*g4 + j of a 32-key chunk c2 is key 32c2 + 4g4 + j (j < 4) or
  // 32c2 + 16 + 4g4 + (j - 4): exactly the keys this lane's S^T registers
  // of chunks 2c2 and 2c2+1 hold, and the keys the two transposing reads
  // below return for rows 32c2 + 4g4 + (l16/4) and 16 further on.
  u32x4 pb[C2][NQ], pl[C2][NQ];  // P^T high parts and residuals
  auto compute_pv = [&](const char *vt_lds) __attribute__((always_inline)) {
    // O is rescaled only when some column's running max moved in the
    // softmax that produced P (rare after the first tile); wave-uniform.
    if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) {
#pragma unroll
        for (int md = 0; md < MDR; ++md) o[md][nq] *= alpha[nq];
        lacc[nq] *= alpha[nq];
      }
    }
#pragma unroll
    for (int c2 = 0; c2 < C2; ++c2) {
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) lacc[nq] = mfma<DT>(ones, pl[c2][nq], mfma<DT>(ones, pb[c2][nq], lacc[nq]));
    }
    // V^T operand of (md, c2): half h of key chunk c2 lives in block pair
    // (2c2 + h, md/2); the operand of the next md is read while the MFMAs of
    // this one run.
    auto vop = [&](int md, int c2) {
      const char *blk0 = vt_lds + ((2 * c2) * (MD / 2) + md / 2) * 1024 + (md & 1) * 512 + 8 * lane;
      const u32x2 lo = read_tr16((const unsigned short *)blk0);
      const u32x2 hi = read_tr16((const unsigned short *)(blk0 + (MD / 2) * 1024));
      return u32x4{lo[0], lo[1], hi[0], hi[1]};
    };
    u32x4 va[C2], vnx[C2];
#pragma unroll
    for (int c2 = 0; c2 < C2; ++c2) va[c2] = vop(0, c2);
#pragma unroll
    for (int md = 0; md < MDR; ++md) {
      if (md + 1 < MDR) {
#pragma unroll
        for (int c2 = 0; c2 < C2; ++c2) vnx[c2] = vop(md + 1, c2);
      }
#pragma unroll
      for (int c2 = 0; c2 < C2; ++c2) {
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq) o[md][nq] = mfma<DT>(va[c2], pl[c2][nq], mfma<DT>(va[c2], pb[c2][nq], o[md][nq]));
      }
      if (md + 1 < MDR) {
#pragma unroll
        for (int c2 = 0; c2 < C2; ++c2) va[c2] = vnx[c2];
      }
    }
  };

  // ---- mask + online softmax of S(kt) into P(kt) ----
  // A tile below every column's diagonal (and inside every window) needs no
  // mask; the test is workgroup-uniform.  Columns past the segment keep
  // finite logits and are never stored.  The running max is kept on raw
  // logits (the kernel's scale is positive: a negative one negates q) and only moved when a tile's max exceeds it by more
  // than kMaxSlack in the exp2 domain.
  const float sc = p.scale_log2;
  const float slack = kMaxSlack / sc;
  auto tile_full = [&](int kt) __attribute__((always_inline)) {
    const int kbase = kt * KT;
    return kbase + KT - 1 <= start + r0 && (p.window == 0 || kbase >= start + r0 + rows_here - p.window);
  };
  // Logits of keys past a column's diagonal or before its window become
  // -inf; applied (rarely) to a tile's S right after it is computed, so the
  // softmax itself is straight-line code.
  auto mask_s = [&](int kt) __attribute__((always_inline)) {
    const int kbase = kt * KT;
#pragma unroll
    for (int nq = 0; nq < NQ; ++nq) {
      const int lo = p.window > 0 ? qpos[nq] - p.window + 1 : -1;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kbase + 16 * mt + 4 * g4 + i;
          const bool ok = (key <= qpos[nq]) & (key >= lo);
          s[mt][nq][i] = ok ? s[mt][nq][i] : kNegInf;
        }
      }
    }
  };
  auto softmax = [&]() __attribute__((always_inline)) {
    grew = false;
#pragma unroll
    for (int nq = 0; nq < NQ; ++nq) {
      float mx = kNegInf;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nq][i]);
      }
      // max over the four lanes of this column (l16, +16, +32, +48)
      mx = xor32_max(xor16_max(mx));
      const bool up = mx > m_run[nq] + slack;  // m_run = -inf moves to any finite max
      grew |= up;
      const float mn = up ? mx : m_run[nq];
      const float mu = mn == kNegInf ? 0.f : mn * sc;
      alpha[nq] = up ? __builtin_amdgcn_exp2f(m_run[nq] * sc - mu) : 1.f;
      m_run[nq] = mn;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mt][nq][i], sc, -mu));
          s[mt][nq][i] = e;
        }
      }
    }
#pragma unroll
    for (int c2 = 0; c2 < C2; ++c2) {
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) {
        pb[c2][nq] = pack8<DT>(s[2 * c2][nq], s[2 * c2 + 1][nq]);
        pl[c2][nq] = residual8<DT>(s[2 * c2][nq], s[2 * c2 + 1][nq], pb[c2][nq]);
      }
    }
  };

  // Step kt: issue K and V of tile kt+NBUF-1 into the buffers tile kt-1 used
  // (every wave left tile kt-1 at the previous barrier); S(kt), mask if the
  // tile needs it, softmax, O += V(kt)^T P(kt)^T; then wait for this wave's
  // loads of tile kt+1 and barrier.  Tile t lives in buffer (t - first) %
  // NBUF.  `win` holds the page-table window of tile kt+NBUF-1 on entry.
  int win;
  auto step = [&](int kt, const char *kc, const char *vc, char *kw, char *vw) __attribute__((always_inline)) {
    if (kt + NBUF - 1 <= kt_last) {
      issue_k(win, kt + NBUF - 1, kt + NBUF - 1, kw);
      issue_v(win, kt + NBUF - 1, kt + NBUF - 1, vw);
    }
    win = read_window(kt + NBUF);
    compute_s(kc);
    if (!tile_full(kt)) mask_s(kt);
    softmax();
    compute_pv(vc);
    sync(min(NBUF - 2, kt_last - kt - 1));
  };

  // Prologue: tiles first .. first+NBUF-2.
  win = read_window(kt_first);
  issue_k(win, kt_first, kt_first, s_k0);
  issue_v(win, kt_first, kt_first, s_v0);
  if (kt_first + 1 <= kt_last) {
    issue_k(win, kt_first, kt_first + 1, s_k1);
    issue_v(win, kt_first, kt_first + 1, s_v1);
  }
  if (NBUF > 3 && kt_first + 2 <= kt_last) {
    win = read_window(kt_first + 2);
    issue_k(win, kt_first + 2, kt_first + 2, s_k2);
    issue_v(win, kt_first + 2, kt_first + 2, s_v2);
  }
  sync(min(NBUF - 2, kt_last - kt_first));
  win = read_window(kt_first + NBUF - 1);
  for (int kt = kt_first; kt <= kt_last; kt += NBUF) {
    if constexpr (NBUF == 3) {
      step(kt, s_k0, s_v0, s_k2, s_v2);
      if (kt + 1 <= kt_last) step(kt + 1, s_k1, s_v1, s_k0, s_v0);
      if (kt + 2 <= kt_last) step(kt + 2, s_k2, s_v2, s_k1, s_v1);
    } else {
      step(kt, s_k0, s_v0, s_k3, s_v3);
      if (kt + 1 <= kt_last) step(kt + 1, s_k1, s_v1, s_k0, s_v0);
      if (kt + 2 <= kt_last) step(kt + 2, s_k2, s_v2, s_k1, s_v1);
      if (kt + 3 <= kt_last) step(kt + 3, s_k3, s_v3, s_k2, s_v2);
    }
  }

  // ---- normalise and store: lane holds dims 16md + 4g4 + i of its column ----
  unsigned short *dst = (unsigned short *)p.out;
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    const float l = lacc[nq][0];
    if (!colok[nq]) continue;
    const float inv = 1.f / l;
    const int c = w * 16 * NQ + nq * 16 + l16;
    const int r = c / G;
    const int gh = c - r * G;
    const long row = (tok0 + r0 + r) * p.H + (long)kh * G + gh;
#pragma unroll
    for (int md = 0; md < MDR; ++md) {
      const u32x2 pk = {pack2<DT>(o[md][nq][0] * inv, o[md][nq][1] * inv),
                        pack2<DT>(o[md][nq][2] * inv, o[md][nq][3] * inv)};
      *(u32x2 *)(dst + row * DR + 16 * md + 4 * g4) = pk;
    }
  }
}

template <int DT, int D, int NQ, int KT, int NW, int DR = D>
int launch(PrefillParams p, int max_len, int plan_len, hipStream_t s) {
  if (16 * NQ * NW / p.G < 1) return DD_EUNSUPPORTED;
  p.max_tiles = (int)dd_cdiv(max_len, (16 * NQ * NW) / p.G);
  const long grid = p.plan ? (long)plan_len : 8L * dd_cdiv((long)p.n * p.KH, 8) * p.max_tiles;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_kernel<DT, D, NQ, KT, NW, DR>), dim3((unsigned)grid), dim3(64 * NW), 0, s, p);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

// Tile geometry per head dim: (query row, head) columns per workgroup and
// keys per tile.  The kernel instantiations below and the host-side plan
// both read it from here.
struct Geometry {
  int cols, kt;
};
constexpr Geometry kGeom64{256, 64};   // prefill_pipe_kernel: 8 waves x 32 columns, 64-key tiles
constexpr Geometry kGeom128{256, 64};
// 256 layout: prefill_pipe_kernel at D 256 (4 waves x 32 columns, 32-key
// tiles) and prefill_kernel at D 144-240 (DD_PREFILL_NW waves x 16 columns)
constexpr Geometry kGeom256{128, 32};
static_assert(16 * DD_PREFILL_NW == kGeom256.cols, "both 256-layout kernels take 128 columns");

// Head sizes prefill_pipe_kernel takes (48 in its 64 layout, 80-112 in its
// 128 layout, 256).
static bool pipe_dim(int D) {
  return D == 48 || D == 64 || D == 80 || D == 96 || D == 112 || D == 128 || D == 256;
}
// Head sizes prefill_kernel takes in its 256 layout (256 itself: the pipe kernel).
static bool wide_dim(int D) { return D > 128 && D <= 256 && D % 16 == 0; }

static bool geometry(int D, Geometry *g) {
  switch (D) {
    case 48:
    case 64: *g = kGeom64; return true;
    case 80:
    case 96:
    case 112:
    case 128: *g = kGeom128; return true;
    default:
      if (wide_dim(D)) {
        *g = kGeom256;
        return true;
      }
      return false;
  }
}

template <int DT>
int dispatch(const PrefillParams &p, int D, int max_len, int plan_len, hipStream_t s) {
  if (pipe_dim(D)) return prefill_pipe_dispatch(p, DT, D, max_len, plan_len, s);
  constexpr int KT = kGeom256.kt, NW = DD_PREFILL_NW;
  switch (D) {
    case 144: return launch<DT, 256, 1, KT, NW, 144>(p, max_len, plan_len, s);
    case 160: return launch<DT, 256, 1, KT, NW, 160>(p, max_len, plan_len, s);
    case 176: return launch<DT, 256, 1, KT, NW, 176>(p, max_len, plan_len, s);
    case 192: return launch<DT, 256, 1, KT, NW, 192>(p, max_len, plan_len, s);
    case 208: return launch<DT, 256, 1, KT, NW, 208>(p, max_len, plan_len, s);
    case 224: return launch<DT, 256, 1, KT, NW, 224>(p, max_len, plan_len, s);
    case 240: return launch<DT, 256, 1, KT, NW, 240>(p, max_len, plan_len, s);
    default: return DD_EUNSUPPORTED;
  }
}

}  // namespace

// phase bit 1: the attention kernel; bit 2: the exact re-run of the items
// the bf16 kernel flagged (nothing to do for other calls).
static int prefill_entry(int phase, const void *q, const void *k, const void *v, int dtype,
                         const int64_t *cu_seqlens, const int64_t *context_lens, const int64_t *slots, int n,
                         int max_len, int max_context, const int32_t *page_table, int table_rows, int table_width,
                         int heads, int kv_heads, int dim, int page_size, int64_t capacity, int window, float scale,
                         const int32_t *plan, int plan_len, int32_t *flags, void *out, void *stream) {
  if (phase < 1 || phase > 3) return DD_EINVAL;
  if (!q || !k || !v || !cu_seqlens || !context_lens || !slots || !page_table || !out || n < 0 || max_len < 0 ||
      heads <= 0 || kv_heads <= 0 || heads % kv_heads || page_size <= 0 || capacity <= 0 || table_width <= 0)
    return DD_EINVAL;
  (void)max_context;  // any history length: page-table entries past the LDS cache come from global memory
  if (plan && plan_len <= 0) return DD_EINVAL;
  if (!__builtin_isfinite(scale)) return DD_EINVAL;
  const int needs_flags = dd_prefill_flag_count(n, max_len, heads, kv_heads, dim, dtype);
  if (needs_flags < 0) return -needs_flags;
  if (needs_flags > 0 && scale != 0.f && !flags) return DD_EINVAL;
  if (n == 0 || max_len == 0) return DD_OK;
  PrefillParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.cu = cu_seqlens;
  p.ctx = context_lens;
  p.slots = slots;
  p.table = page_table;
  p.plan = plan;
  p.out = out;
  p.capacity = capacity;
  p.n = n;
  p.H = heads;
  p.KH = kv_heads;
  p.G = heads / kv_heads;
  p.page = page_size;
  p.page_shift = 0;
  while ((1 << p.page_shift) < page_size) ++p.page_shift;
  if ((1 << p.page_shift) != page_size || page_size < 16) return DD_EUNSUPPORTED;
  p.table_w = table_width;
  p.table_rows = table_rows;
  p.window = window > 0 ? window : 0;
  hipStream_t s = (hipStream_t)stream;
  Geometry geom;
  // fp32 pages, head sizes without a 16-bit MFMA kernel and scale 0 (every
  // logit 0: uniform weights over the allowed keys, as SDPA gives; the
  // 16-bit kernels take |scale| as a log2 step): fp32 arithmetic on the
  // matrix cores (head sizes in steps of 16), else the vector-ALU kernel (no
  // plan).  The same arguments serve the exact re-run of flagged bf16 items.
  PrefillGenericArgs a{};
  {
    a.q = q;
    a.k = k;
    a.v = v;
    a.cu = cu_seqlens;
    a.ctx = context_lens;
    a.slots = slots;
    a.table = page_table;
    a.out = out;
    a.capacity = capacity;
    a.n = n;
    a.max_len = max_len;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.dim = dim;
    a.page = page_size;
    a.page_shift = p.page_shift;
    a.table_w = table_width;
    a.table_rows = table_rows;
    a.window = p.window;
    a.scale_log2 = scale * kLog2e;
  }
  auto exact = [&](const PrefillGenericArgs &args) {
    const int rc = dd_prefill_f32(args, dtype, s);
    return rc != DD_EUNSUPPORTED ? rc : dd_prefill_generic(args, dtype, s);
  };
  // (and more query heads per KV head than one 16-bit work item has columns)
  if (dtype == DD_F32 || !geometry(dim, &geom) || geom.cols < heads / kv_heads || scale == 0.f)
    return (phase & 1) ? exact(a) : DD_OK;
  p.scale_log2 = __builtin_fabsf(scale) * kLog2e;
  p.q_sign = scale < 0.f ? 0x80008000u : 0u;
  p.flags = needs_flags > 0 ? flags : nullptr;
  int rc = DD_OK;
  if (phase & 1) {
    rc = DD_EUNSUPPORTED;
    if (dtype == DD_BF16) rc = dispatch<DD_BF16>(p, dim, max_len, plan_len, s);
    if (dtype == DD_F16) rc = dispatch<DD_F16>(p, dim, max_len, plan_len, s);
  }
  if (rc != DD_OK || !p.flags || !(phase & 2)) return rc;
  // the items the bf16 kernel flagged, again in fp32 arithmetic
  a.flags = flags;
  a.flag_rows = geom.cols / p.G;
  a.flag_tiles = (int)dd_cdiv(max_len, a.flag_rows);
  return exact(a);
}

extern "C" int dd_prefill_attention(const void *q, const void *k, const void *v, int dtype, const int64_t *cu_seqlens,
                                    const int64_t *context_lens, const int64_t *slots, int n, int max_len,
                                    int max_context, const int32_t *page_table, int table_rows, int table_width,
                                    int heads, int kv_heads, int dim, int page_size, int64_t capacity, int window,
                                    float scale, const int32_t *plan, int plan_len, int32_t *flags, void *out,
                                    void *stream) {
  return prefill_entry(3, q, k, v, dtype, cu_seqlens, context_lens, slots, n, max_len, max_context, page_table,
                       table_rows, table_width, heads, kv_heads, dim, page_size, capacity, window, scale, plan,
                       plan_len, flags, out, stream);
}

extern "C" int dd_prefill_attention_phase(const void *q, const void *k, const void *v, int dtype,
                                          const int64_t *cu_seqlens, const int64_t *context_lens,
                                          const int64_t *slots, int n, int max_len, int max_context,
                                          const int32_t *page_table, int table_rows, int table_width, int heads,
                                          int kv_heads, int dim, int page_size, int64_t capacity, int window,
                                          float scale, const int32_t *plan, int plan_len, int32_t *flags, void *out,
                                          int phase, void *stream) {
  return prefill_entry(phase, q, k, v, dtype, cu_seqlens, context_lens, slots, n, max_len, max_context, page_table,
                       table_rows, table_width, heads, kv_heads, dim, page_size, capacity, window, scale, plan,
                       plan_len, flags, out, stream);
}

extern "C" int dd_prefill_flag_count(int n, int max_len, int heads, int kv_heads, int dim, int dtype) {
  if (n < 0 || max_len < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads) return -DD_EINVAL;
  // only bf16 pages at the head sizes of prefill_pipe_kernel convert V to fp16
  Geometry g;
  if (dtype != DD_BF16 || !pipe_dim(dim) || !geometry(dim, &g)) return 0;
  const int rows = g.cols / (heads / kv_heads);
  if (rows < 1) return 0;   // more heads per KV head than one item holds: the exact kernel takes the call
  const long count = (long)n * kv_heads * dd_cdiv(max_len, rows);
  return count > 0x7fffffffL ? -DD_EUNSUPPORTED : (int)count;
}

extern "C" int dd_prefill_geometry(int dim, int *columns, int *keys_per_tile) {
  Geometry g;
  if (!columns || !keys_per_tile) return DD_EINVAL;
  if (!geometry(dim, &g)) return DD_EUNSUPPORTED;
  *columns = g.cols;
  *keys_per_tile = g.kt;
  return DD_OK;
}

// Workgroup order for dd_prefill_attention, computed on the host from the
// host copy of the segment lengths and starts.  A work item is one
// (segment, KV head, query tile); its cost is the number of key tiles it
// visits plus a fixed start-up charge.  Groups (segment, KV head) are spread
// over the 8 XCDs longest-processing-time first, so that every query tile of
// a group shares one XCD's L2; within an XCD the items run longest first.
// Workgroup b is dispatched to XCD b % 8, so entry 8 j + x is the j-th item
// of XCD x (item -1 pads the shorter XCD lists).  An entry is kPlanInts
// ints: the item, then its segment's token offset, length, start and slot.
extern "C" int dd_prefill_plan(const int64_t *lengths, const int64_t *starts, const int64_t *slots, int n,
                               int heads, int kv_heads, int dim, int window, int workgroups, int32_t *plan,
                               int capacity) {
  if (!lengths || !starts || !slots || n < 0 || heads <= 0 || kv_heads <= 0 || heads % kv_heads || capacity < 0)
    return -DD_EINVAL;
  Geometry g;
  if (!geometry(dim, &g)) return -DD_EUNSUPPORTED;
  const int G = heads / kv_heads;
  const int rows = g.cols / G;
  if (rows < 1) return -DD_EUNSUPPORTED;
  long max_len = 0;
  std::vector<long> tok0(n + 1, 0);
  for (int i = 0; i < n; ++i) {
    if (lengths[i] < 0 || starts[i] < 0 || lengths[i] + starts[i] > 0x7fffffffL || slots[i] < INT32_MIN ||
        slots[i] > INT32_MAX)
      return -DD_EINVAL;
    max_len = std::max<long>(max_len, lengths[i]);
    tok0[i + 1] = tok0[i] + lengths[i];
  }
  if (tok0[n] > 0x7fffffffL) return -DD_EUNSUPPORTED;
  const long max_tiles = dd_cdiv(max_len, rows);
  if ((long)n * kv_heads * std::max<long>(max_tiles, 1) > 0x7fffffffL) return -DD_EUNSUPPORTED;
  constexpr long kStartup = 2;  // charge of a workgroup's prologue and epilogue, in key tiles
  auto item_cost = [&](int seg, long qt) {
    const long r0 = qt * rows;
    const long here = std::min<long>(rows, lengths[seg] - r0);
    const long k_hi = starts[seg] + r0 + here;
    const long k_lo = window > 0 ? std::max<long>(0, starts[seg] + r0 - window + 1) : 0;
    return (k_hi - 1) / g.kt - k_lo / g.kt + 1 + kStartup;
  };
  // groups, heaviest first, each to the least-loaded XCD
  std::vector<std::pair<long, int>> groups;  // (-cost, group)
  for (int seg = 0; seg < n; ++seg) {
    const long tiles = dd_cdiv(lengths[seg], rows);
    long cost = 0;
    for (long qt = 0; qt < tiles; ++qt) cost += item_cost(seg, qt);
    if (tiles == 0) continue;
    for (int kh = 0; kh < kv_heads; ++kh) groups.push_back({-cost, seg * kv_heads + kh});
  }
  std::sort(groups.begin(), groups.end());
  constexpr int kXcds = 8;
  long load[kXcds] = {};
  std::vector<std::vector<std::pair<long, int>>> lists(kXcds);  // (-cost, item)
  for (const auto &gr : groups) {
    const int x = (int)(std::min_element(load, load + kXcds) - load);
    load[x] -= gr.first;
    const int seg = gr.second / kv_heads;
    const long tiles = dd_cdiv(lengths[seg], rows);
    for (long qt = 0; qt < tiles; ++qt)
      lists[x].push_back({-item_cost(seg, qt), (int)(gr.second * max_tiles + qt)});
  }
  size_t longest = 0;
  for (auto &l : lists) {
    std::stable_sort(l.begin(), l.end());
    longest = std::max(longest, l.size());
  }
  // Workgroup b runs on XCD b % 8.  Without a workgroup count: one item per
  // workgroup, item j of XCD x in workgroup 8 j + x (the hardware hands the
  // next workgroup to whichever CU frees first).  With one (at most one per
  // CU, so that all of them run at once): the items of XCD x go, longest
  // first, each to the least-loaded of that XCD's workgroups, which run them
  // in that order -- round r of workgroup b is entry r * G + b.
  long grid = (long)kXcds * (long)longest, rounds = 1;
  std::vector<std::vector<int>> per_wg;  // items of each workgroup (persistent form)
  if (workgroups >= kXcds && (long)workgroups / kXcds < (long)longest) {
    grid = (workgroups / kXcds) * kXcds;
    const long per_xcd = grid / kXcds;
    per_wg.assign(grid, {});
    for (int x = 0; x < kXcds; ++x) {
      std::vector<std::pair<long, long>> bins;  // (load, wg)
      for (long i = 0; i < per_xcd; ++i) bins.push_back({0, kXcds * i + x});
      std::make_heap(bins.begin(), bins.end(), std::greater<>());
      for (const auto &cw : lists[x]) {
        std::pop_heap(bins.begin(), bins.end(), std::greater<>());
        bins.back().first -= cw.first;   // cw.first is -cost
        per_wg[bins.back().second].push_back(cw.second);
        std::push_heap(bins.begin(), bins.end(), std::greater<>());
      }
    }
    rounds = 0;
    for (const auto &l : per_wg) rounds = std::max<long>(rounds, (long)l.size());
  }
  const long need = grid * rounds;
  if (need > 0x7fffffffL) return -DD_EUNSUPPORTED;
  if (!plan || capacity < need) return (int)need;
  auto item_of = [&](long r, long b) -> int {
    if (!per_wg.empty()) return r < (long)per_wg[b].size() ? per_wg[b][r] : -1;
    const long j = b / kXcds, x = b % kXcds;   // one round
    return j < (long)lists[x].size() ? lists[x][j].second : -1;
  };
  for (long r = 0; r < rounds; ++r)
    for (long b = 0; b < grid; ++b) {
      int32_t *e = plan + (long)kPlanInts * (r * grid + b);
      for (int k = 0; k < kPlanInts; ++k) e[k] = 0;
      e[5] = (int32_t)rounds;
      const int item = item_of(r, b);
      e[0] = item;
      if (item < 0) continue;
      const int seg = (int)(item / max_tiles) / kv_heads;
      e[1] = (int32_t)tok0[seg];
      e[2] = (int32_t)lengths[seg];
      e[3] = (int32_t)starts[seg];
      e[4] = (int32_t)slots[seg];
    }
  return (int)need;
}
