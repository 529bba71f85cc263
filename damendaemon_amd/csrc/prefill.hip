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
// MI355X design:
//   * a workgroup owns one KV head and 64*NQ (query row, head) columns of
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
//     beyond two xor-steps.
#include "common.h"

#ifndef DD_PREFILL_PIPE_S
#define DD_PREFILL_PIPE_S 0
#endif
// Compute S of tile kt+1 during the softmax of tile kt (needs a second S
// register set; only worth it when it does not push the kernel into spills).
constexpr bool kPipeS = DD_PREFILL_PIPE_S;
#ifndef DD_PREFILL_NW
#define DD_PREFILL_NW 8
#endif
#ifndef DD_PREFILL_NQ128
#define DD_PREFILL_NQ128 2
#endif

namespace {

constexpr float kNegInf = -__builtin_inff();
constexpr int kTabCache = 8192;  // page-table entries staged in LDS (128K keys at page 16)

struct PrefillParams {
  const void *q;       // (T, H, D)
  const void *k;       // (capacity, KH, page, D)
  const void *v;
  const int64_t *cu;   // (n+1) cu_seqlens of the packed tokens
  const int64_t *ctx;  // (n) start + len
  const int64_t *slots;
  const int32_t *table;
  void *out;           // (T, H, D)
  long capacity;
  int n, max_tiles;
  int H, KH, G;
  int page, page_shift;
  int table_w, table_rows;
  int window;
  float scale_log2;
};

template <int DT>
DD_DEV f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (DT == DD_BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Transposing LDS read (ds_read_b64_tr_b16): within each 16-lane group,
// lane i receives element i%4 of the 8-byte chunks addressed by lanes
// i/4, 4 + i/4, 8 + i/4 and 12 + i/4.
DD_DEV u32x2 read_tr16(const unsigned short *p) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (lds_s16x4 *)(__attribute__((address_space(3))) char *)(p));
  return __builtin_bit_cast(u32x2, v);
}

// Eight fp32 probabilities -> one 8 x 16-bit MFMA operand (RNE).
template <int DT>
DD_DEV u32x4 pack8(f32x4 x0, f32x4 x1) {
  u32x4 r;
  if constexpr (DT == DD_BF16) {
    r[0] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x0[0], x0[1]}, bf16x2));
    r[1] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x0[2], x0[3]}, bf16x2));
    r[2] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x1[0], x1[1]}, bf16x2));
    r[3] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x1[2], x1[3]}, bf16x2));
  } else {
    r[0] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x0[0], x0[1]}, f16x2));
    r[1] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x0[2], x0[3]}, f16x2));
    r[2] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x1[0], x1[1]}, f16x2));
    r[3] = __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2{x1[2], x1[3]}, f16x2));
  }
  return r;
}

template <int DT>
DD_DEV unsigned pack2(float a, float b) {
  if constexpr (DT == DD_BF16) {
    return (unsigned)float_to_bf16_bits(a) | ((unsigned)float_to_bf16_bits(b) << 16);
  } else {
    return (unsigned)float_to_f16_bits(a) | ((unsigned)float_to_f16_bits(b) << 16);
  }
}

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
#ifndef DD_PREFILL_WAVES
#define DD_PREFILL_WAVES 2
#endif

template <int DT, int D, int NQ, int KT, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(DD_PREFILL_WAVES))) void prefill_kernel(PrefillParams p) {
  constexpr int NC = D / 32;           // k-chunks of q.k
  constexpr int MD = D / 16;           // O^T row tiles
  constexpr int COLS = 16 * NQ * NW;   // (query row, head) columns per workgroup
  constexpr int NT = 64 * NW;          // threads
  constexpr int KBLK = (KT / 16) * NC;         // K blocks per tile
  constexpr int VBLK = (KT / 32) * 2 * (MD / 2);  // V block pairs per tile
  constexpr int PLANE = KBLK * 1024;
  static_assert(KBLK == VBLK && KBLK % NW == 0, "every wave issues whole blocks");
  constexpr int IPW = KBLK / NW;       // DMA instructions per wave per plane

  // Four distinct buffers (K and V, double-buffered).  Every direct-to-LDS
  // load and every LDS read below names one of them at compile time (the
  // tile loop is unrolled by two), so the compiler can tell that reads of
  // one buffer do not wait for loads still landing in another.
  __shared__ __align__(16) char s_k0[PLANE], s_k1[PLANE], s_v0[PLANE], s_v1[PLANE];
  __shared__ int s_tab[kTabCache];                   // page-table window of this slot

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int g4 = lane >> 4;
  const int l16 = lane & 15;

  // XCD-aware order.  Consecutive workgroups go to the 8 XCDs round-robin,
  // each XCD with its own L2; every query tile of one (segment, KV head)
  // group is sent to the same XCD, back to back, so they share its K/V
  // tiles in that L2.  Within a group the longest-running tiles go first.
  const int xcd = blockIdx.x & 7;
  const int j = blockIdx.x >> 3;
  const int grp = xcd + 8 * (j / p.max_tiles);
  if (grp >= p.n * p.KH) return;
  const int qt = p.max_tiles - 1 - j % p.max_tiles;
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

  const int k_hi = start + r0 + rows_here;   // exclusive
  int k_lo = 0;
  if (p.window > 0) k_lo = max(0, start + r0 - p.window + 1);
  const int kt_first = k_lo / KT;
  const int kt_last = (k_hi - 1) / KT;

  // The page-table entries of the whole key range are staged in LDS once, so
  // no scalar page-table load sits on the critical path of a tile's loads.
  const int e_first = (kt_first * KT) >> p.page_shift;
  const int e_count = ((((kt_last + 1) * KT) - 1) >> p.page_shift) - e_first + 1;
  {
    const bool slot_ok = slot >= 0 && slot < p.table_rows;
    for (int i = tid; i < e_count; i += NT) {
      const int e = e_first + i;
      s_tab[i] = (slot_ok && e < p.table_w && i < kTabCache) ? p.table[slot * p.table_w + e] : -1;
    }
  }
  __syncthreads();

  // ---- per-lane query columns and Q^T operands ----
  int qpos[NQ];
  bool colok[NQ];
  u32x4 qb[NQ][NC];
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
    for (int cc = 0; cc < NC; ++cc) {
      qb[nq][cc] = colok[nq] ? *(const u32x4 *)(qsrc + row * D + 8 * g4 + 32 * cc) : u32x4{0, 0, 0, 0};
    }
  }

  f32x4 o[MD][NQ];
  float m_run[NQ], l_run[NQ];
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    m_run[nq] = kNegInf;
    l_run[nq] = 0.f;
#pragma unroll
    for (int md = 0; md < MD; ++md) o[md][nq] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  const char *kbytes = (const char *)p.k;
  const char *vbytes = (const char *)p.v;
  // Element offset of the first row of 16-key chunk `ci`, or -1 when the
  // chunk is past the context or not backed by an allocated page.
  auto chunk_base = [&](int ci) -> long {
    const int key0 = ci * 16;
    if (key0 >= context) return -1;
    const int entry = key0 >> p.page_shift;
    // contexts longer than kTabCache pages are rejected by the host
    const long phys = entry - e_first < kTabCache ? uniform(s_tab[entry - e_first]) : -1;
    if (phys < 0 || phys >= p.capacity) return -1;
    return (((phys * p.KH + kh) << p.page_shift) | (key0 & (p.page - 1))) * (long)D;
  };
  // every key of tile kt live and backed by a page
  auto whole = [&](int kt) {
    if ((kt + 1) * KT > context) return false;
#pragma unroll
    for (int j = 0; j < KT / 16; ++j) {
      if (chunk_base(kt * (KT / 16) + j) < 0) return false;
    }
    return true;
  };
  // Loop-invariant per-lane byte offsets inside a 16-key chunk; each load
  // address is a wave-uniform chunk base (SGPRs) plus one of these, so no
  // 64-bit per-lane address has to stay live (or spill) across the loop.
  const unsigned k_lane = 2u * (l16 * D + 8 * g4);             // K block, + 64cc bytes
  const int vq = lane & 31;                                     // V: read-lane pair
  const int v_key = 4 * (vq >> 3) + ((vq & 7) >> 1);           // key within the 16-key half
  const unsigned v_lane = 2u * (v_key * D + 16 * (lane >> 5) + 8 * (vq & 1));  // + 64mp bytes
  auto issue_k = [&](int kt, char *buf) {
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int blk = w * IPW + j;                 // K block (mt, cc)
      const int mt = blk / NC, cc = blk - mt * NC;
      const long kb = chunk_base(kt * (KT / 16) + mt);
      const char *src = uniform_ptr(kbytes + 2 * ((kb < 0 ? 0 : kb) + 32 * cc)) + k_lane;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                       (__attribute__((address_space(3))) void *)(buf + blk * 1024), 16,
                                       0, 0);
    }
  };
  auto issue_v = [&](int kt, char *buf) {
#pragma unroll
    for (int j = 0; j < IPW; ++j) {
      const int blk = w * IPW + j;                 // V block pair (c2, h, mp), hc = 2*c2 + h
      const int hc = blk / (MD / 2), mp = blk - hc * (MD / 2);
      const long vb = chunk_base(kt * (KT / 16) + hc);
      const char *src = uniform_ptr(vbytes + 2 * ((vb < 0 ? 0 : vb) + 32 * mp)) + v_lane;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void *)src,
                                       (__attribute__((address_space(3))) void *)(buf + blk * 1024), 16,
                                       0, 0);
    }
  };
  // Dead keys of a partial tile: zero their V bytes so 0 * garbage cannot
  // reach the P.V product (their logits are masked to -inf as well).
  auto zero_dead = [&](int kt, char *vbuf) {
    for (int i = tid; i < VBLK * 64; i += NT) {
      const int blk = i >> 6, l = i & 63;
      const int hc = blk / (MD / 2);
      const int q = l & 31;
      const int key = kt * KT + 16 * hc + 4 * (q >> 3) + ((q & 7) >> 1);
      if (key >= context || chunk_base(key >> 4) < 0)
        *(u32x4 *)(vbuf + blk * 1024 + 16 * l) = u32x4{0, 0, 0, 0};
    }
  };
  auto tile_ready = [&]() {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  // S^T = K Q^T for tile kt: lane holds keys 16mt + 4g4 + i for column l16.
  // Dim chunk outer, key tile inner: consecutive MFMAs accumulate into
  // different registers, and the K operands of chunk cc+1 are read from LDS
  // while the MFMAs of chunk cc run.
  auto compute_s = [&](const char *kt_lds, f32x4 (&sv)[KT / 16][NQ]) {
    constexpr int MT = KT / 16;
    u32x4 a[MT], an[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      a[mt] = *(const u32x4 *)(kt_lds + (mt * NC + 0) * 1024 + 16 * lane);
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) sv[mt][nq] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int cc = 0; cc < NC; ++cc) {
      if (cc + 1 < NC) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) an[mt] = *(const u32x4 *)(kt_lds + (mt * NC + cc + 1) * 1024 + 16 * lane);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq) sv[mt][nq] = mfma<DT>(a[mt], qb[nq][cc], sv[mt][nq]);
      }
      if (cc + 1 < NC) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) a[mt] = an[mt];
      }
    }
  };

  f32x4 s_a[KT / 16][NQ], s_b[KT / 16][NQ];
  // One pipelined step for tile kt.  kc / vc: LDS buffers of K(kt) / V(kt);
  // kn / vn: the other pair (K(kt+1) already there, V(kt+1) to be loaded).
  auto step = [&](int kt, char *kc, char *vc, char *kn, char *vn, f32x4 (&s)[KT / 16][NQ],
                  f32x4 (&s_next)[KT / 16][NQ]) {
    if constexpr (kPipeS) {
      if (kt + 2 <= kt_last) issue_k(kt + 2, kc);
      if (kt + 1 <= kt_last) {
        issue_v(kt + 1, vn);
        compute_s(kn, s_next);
      }
    } else {
      if (kt + 1 <= kt_last) {
        issue_k(kt + 1, kn);
        issue_v(kt + 1, vn);
      }
      compute_s(kc, s);
    }
    const char *vt_lds = vc;

    // ---- mask, online softmax per column ----
    // A tile below every column's diagonal (and inside every window) needs
    // no mask; the test is workgroup-uniform.  Columns past the segment keep
    // finite logits and are never stored.  The running max is kept on raw
    // logits (scale > 0) and the scale is folded into the exp argument.
    const int kbase = kt * KT;
    const bool full = kbase + KT - 1 <= start + r0 &&
                      (p.window == 0 || kbase >= start + r0 + rows_here - p.window);
    const float sc = p.scale_log2;
    bool grew = false;
    float alpha[NQ];
#pragma unroll
    for (int nq = 0; nq < NQ; ++nq) {
      float mx = kNegInf;
      if (full) {
#pragma unroll
        for (int mt = 0; mt < KT / 16; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nq][i]);
        }
      } else {
        const int lo = p.window > 0 ? qpos[nq] - p.window + 1 : -1;
#pragma unroll
        for (int mt = 0; mt < KT / 16; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = kbase + 16 * mt + 4 * g4 + i;
            const bool ok = (key <= qpos[nq]) & (key >= lo);
            const float x = ok ? s[mt][nq][i] : kNegInf;
            s[mt][nq][i] = x;
            mx = fmaxf(mx, x);
          }
        }
      }
      mx = fmaxf(mx, shfl(mx, lane ^ 16));
      mx = fmaxf(mx, shfl(mx, lane ^ 32));
      const float mn = fmaxf(m_run[nq], mx);
      grew |= mn > m_run[nq];
      const float mu = mn == kNegInf ? 0.f : mn * sc;
      alpha[nq] = __builtin_amdgcn_exp2f(m_run[nq] * sc - mu);
      m_run[nq] = mn;
      float ls = 0.f;
#pragma unroll
      for (int mt = 0; mt < KT / 16; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[mt][nq][i], sc, -mu));
          s[mt][nq][i] = e;
          ls += e;
        }
      }
      l_run[nq] = l_run[nq] * alpha[nq] + ls;
    }
    // O is rescaled only when some column's running max grew in this tile
    // (after the first tiles this is rare); the test is wave-uniform.
    if (__builtin_amdgcn_ballot_w64(grew)) {
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) {
#pragma unroll
        for (int md = 0; md < MD; ++md) o[md][nq] *= alpha[nq];
      }
    }

    // ---- O^T += V^T P^T : keys contracted in the order of the S^T layout ----
    // k-slot 8*g4 + j of a 32-key chunk c2 is key 32c2 + 4g4 + j (j < 4) or
    // 32c2 + 16 + 4g4 + (j - 4): exactly the keys this lane's S^T registers
    // of tiles 2c2 and 2c2+1 hold, and the keys the two transposing reads
    // below return for rows 32c2 + 4g4 + (l16/4) and 16 further on.
    u32x4 pb[KT / 32][NQ];
#pragma unroll
    for (int c2 = 0; c2 < KT / 32; ++c2) {
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) pb[c2][nq] = pack8<DT>(s[2 * c2][nq], s[2 * c2 + 1][nq]);
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
    u32x4 va[KT / 32], vnx[KT / 32];
#pragma unroll
    for (int c2 = 0; c2 < KT / 32; ++c2) va[c2] = vop(0, c2);
#pragma unroll
    for (int md = 0; md < MD; ++md) {
      if (md + 1 < MD) {
#pragma unroll
        for (int c2 = 0; c2 < KT / 32; ++c2) vnx[c2] = vop(md + 1, c2);
      }
#pragma unroll
      for (int c2 = 0; c2 < KT / 32; ++c2) {
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq) o[md][nq] = mfma<DT>(va[c2], pb[c2][nq], o[md][nq]);
      }
      if (md + 1 < MD) {
#pragma unroll
        for (int c2 = 0; c2 < KT / 32; ++c2) va[c2] = vnx[c2];
      }
    }
    if (kt < kt_last) {
      tile_ready();  // K(kt+2) and V(kt+1) landed; every wave is done with kt
      if (!whole(kt + 1)) {
        zero_dead(kt + 1, vn);
        __syncthreads();
      }
    }
  };

  issue_k(kt_first, s_k0);
  if (kPipeS && kt_first < kt_last) issue_k(kt_first + 1, s_k1);
  issue_v(kt_first, s_v0);
  tile_ready();
  if (!whole(kt_first)) {
    zero_dead(kt_first, s_v0);
    __syncthreads();
  }
  if constexpr (kPipeS) compute_s(s_k0, s_a);
  for (int kt = kt_first; kt <= kt_last; kt += 2) {
    step(kt, s_k0, s_v0, s_k1, s_v1, s_a, s_b);
    if (kt + 1 <= kt_last) step(kt + 1, s_k1, s_v1, s_k0, s_v0, s_b, s_a);
  }

  // ---- normalise and store: lane holds dims 16md + 4g4 + i of its column ----
  unsigned short *dst = (unsigned short *)p.out;
#pragma unroll
  for (int nq = 0; nq < NQ; ++nq) {
    float l = l_run[nq];
    l += shfl(l, lane ^ 16);
    l += shfl(l, lane ^ 32);
    if (!colok[nq]) continue;
    const float inv = 1.f / l;
    const int c = w * 16 * NQ + nq * 16 + l16;
    const int r = c / G;
    const int gh = c - r * G;
    const long row = (tok0 + r0 + r) * p.H + (long)kh * G + gh;
#pragma unroll
    for (int md = 0; md < MD; ++md) {
      const u32x2 pk = {pack2<DT>(o[md][nq][0] * inv, o[md][nq][1] * inv),
                        pack2<DT>(o[md][nq][2] * inv, o[md][nq][3] * inv)};
      *(u32x2 *)(dst + row * D + 16 * md + 4 * g4) = pk;
    }
  }
}

template <int DT, int D, int NQ, int KT, int NW>
int launch(PrefillParams p, int max_len, hipStream_t s) {
  if (16 * NQ * NW / p.G < 1) return DD_EUNSUPPORTED;
  p.max_tiles = (int)dd_cdiv(max_len, (16 * NQ * NW) / p.G);
  const long grid = 8L * dd_cdiv((long)p.n * p.KH, 8) * p.max_tiles;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_kernel<DT, D, NQ, KT, NW>), dim3((unsigned)grid), dim3(64 * NW), 0, s, p);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

template <int DT>
int dispatch(const PrefillParams &p, int D, int max_len, hipStream_t s) {
  switch (D) {
    case 64: return launch<DT, 64, 2, 64, DD_PREFILL_NW>(p, max_len, s);
    case 128: return launch<DT, 128, DD_PREFILL_NQ128, 64, DD_PREFILL_NW>(p, max_len, s);
    case 256: return launch<DT, 256, 1, 32, 4>(p, max_len, s);
    default: return DD_EUNSUPPORTED;
  }
}

}  // namespace

extern "C" int dd_prefill_attention(const void *q, const void *k, const void *v, int dtype, const int64_t *cu_seqlens,
                                    const int64_t *context_lens, const int64_t *slots, int n, int max_len,
                                    int max_context,
                                    const int32_t *page_table, int table_rows, int table_width, int heads,
                                    int kv_heads, int dim, int page_size, int64_t capacity, int window, float scale,
                                    void *out, void *stream) {
  if (!q || !k || !v || !cu_seqlens || !context_lens || !slots || !page_table || !out || n < 0 || max_len < 0 ||
      heads <= 0 || kv_heads <= 0 || heads % kv_heads || page_size <= 0 || capacity <= 0 || table_width <= 0)
    return DD_EINVAL;
  if (heads / kv_heads > 16) return DD_EUNSUPPORTED;
  if ((long)max_context > (long)kTabCache * page_size) return DD_EUNSUPPORTED;
  if (n == 0 || max_len == 0) return DD_OK;
  PrefillParams p{};
  p.q = q;
  p.k = k;
  p.v = v;
  p.cu = cu_seqlens;
  p.ctx = context_lens;
  p.slots = slots;
  p.table = page_table;
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
  p.scale_log2 = scale * kLog2e;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == DD_BF16) return dispatch<DD_BF16>(p, dim, max_len, s);
  if (dtype == DD_F16) return dispatch<DD_F16>(p, dim, max_len, s);
  return DD_EUNSUPPORTED;
}
