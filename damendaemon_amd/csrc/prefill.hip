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

#include <cstdlib>

namespace {

constexpr int kKeys = 64;       // keys per tile
constexpr float kNegInf = -__builtin_inff();

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

template <int DT, int D, int NQ>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillParams p) {
  constexpr int NC = D / 32;         // k-chunks of q.k
  constexpr int MD = D / 16;         // O^T row tiles
  constexpr int KROW = D + 8;        // K row stride (elements) in LDS: 16 B pad
  constexpr int COLS = 64 * NQ;      // (query row, head) columns per workgroup
  constexpr int KCH = D / 8;         // 16-byte chunks per key row
  // V row stride: 32 B of pad puts the four rows of one transposing read
  // eight banks apart, so a 32-lane half-wave covers all 64 banks once.
  constexpr int VROW = D + 16;

  __shared__ __align__(16) unsigned short s_k[kKeys * KROW];
  __shared__ __align__(16) unsigned short s_v[kKeys * VROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int g4 = lane >> 4;
  const int l16 = lane & 15;

  const int kh = blockIdx.x % p.KH;
  const int rest = blockIdx.x / p.KH;
  const int seg = rest % p.n;
  const int qt = rest / p.n;
  const long tok0 = p.cu[seg];
  const int len = (int)(p.cu[seg + 1] - tok0);
  const int G = p.G;
  const int rows = COLS / G;                 // query rows per workgroup
  const int r0 = qt * rows;
  if (r0 >= len) return;
  const int context = (int)p.ctx[seg];
  const int start = context - len;
  const long slot = p.slots[seg];
  const int rows_here = min(rows, len - r0);

  // key range of the whole tile
  const int k_hi = start + r0 + rows_here;   // exclusive
  int k_lo = 0;
  if (p.window > 0) k_lo = max(0, start + r0 - p.window + 1);
  const int kt_first = k_lo / kKeys;
  const int kt_last = (k_hi - 1) / kKeys;

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

  // ---- global -> register staging of one key tile ----
  // K and V: 64 keys x KCH 16-byte chunks; thread t takes chunks t, t+256, ...
  constexpr int KLOADS = kKeys * KCH / 256;
  u32x4 kreg[KLOADS];
  u32x4 vreg[KLOADS];
  const char *kbytes = (const char *)p.k;
  const char *vbytes = (const char *)p.v;
  // Element offset of the first row of 16-key chunk `ci` of this slot and KV
  // head (page sizes are powers of two >= 16), or -1 when the chunk is not
  // backed by an allocated page.  All arguments are workgroup-uniform, so
  // the page-table reads are scalar loads.
  auto chunk_base = [&](int ci) -> long {
    const int key0 = ci * 16;
    if (key0 >= context) return -1;
    const int entry = key0 >> p.page_shift;
    if (slot < 0 || slot >= p.table_rows || entry >= p.table_w) return -1;
    const long phys = p.table[slot * p.table_w + entry];
    if (phys < 0 || phys >= p.capacity) return -1;
    return ((phys * p.KH + kh) << p.page_shift | (key0 & (p.page - 1))) * (long)D;
  };
  auto load_tile = [&](int kt) {
    long cb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) cb[j] = chunk_base(kt * 4 + j);
    // every key of the tile live and backed by a page (workgroup-uniform)
    const bool whole = (kt + 1) * kKeys <= context && cb[0] >= 0 && cb[1] >= 0 && cb[2] >= 0 && cb[3] >= 0;
#pragma unroll
    for (int j = 0; j < KLOADS; ++j) {
      const int idx = tid + 256 * j;
      const int key = idx / KCH;          // 0..63
      const int ch = idx - key * KCH;
      const long base = cb[key >> 4];
      const long off = (base < 0 ? 0 : base) + (long)(key & 15) * D + 8 * ch;
      kreg[j] = *(const u32x4 *)(kbytes + 2 * off);
    }
#pragma unroll
    for (int j = 0; j < KLOADS; ++j) {
      const int idx = tid + 256 * j;
      const int key = idx / KCH;
      const int ch = idx - key * KCH;
      const long base = cb[key >> 4];
      const long off = (base < 0 ? 0 : base) + (long)(key & 15) * D + 8 * ch;
      vreg[j] = *(const u32x4 *)(vbytes + 2 * off);
      if (!whole) {  // dead keys must not carry NaN into P.V
        const bool ok = (base >= 0) & (kt * kKeys + key < context);
        vreg[j] = ok ? vreg[j] : u32x4{0, 0, 0, 0};
      }
    }
  };

  auto store_tile = [&]() {
#pragma unroll
    for (int j = 0; j < KLOADS; ++j) {
      const int idx = tid + 256 * j;
      const int key = idx / KCH;
      const int ch = idx - key * KCH;
      *(u32x4 *)(s_k + key * KROW + 8 * ch) = kreg[j];
      *(u32x4 *)(s_v + key * VROW + 8 * ch) = vreg[j];
    }
  };

  if (kt_first <= kt_last) load_tile(kt_first);
  for (int kt = kt_first; kt <= kt_last; ++kt) {
    __syncthreads();
    store_tile();
    __syncthreads();
    if (kt + 1 <= kt_last) load_tile(kt + 1);

    // ---- S^T = K Q^T : lane holds keys 16mt + 4g4 + i for column l16 ----
    f32x4 s[4][NQ];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) s[mt][nq] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int cc = 0; cc < NC; ++cc) {
        const u32x4 a = *(const u32x4 *)(s_k + (16 * mt + l16) * KROW + 8 * g4 + 32 * cc);
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq) s[mt][nq] = mfma<DT>(a, qb[nq][cc], s[mt][nq]);
      }
    }
    // ---- mask, online softmax per column ----
    // A tile below every column's diagonal (and inside every window) needs
    // no mask; the test is workgroup-uniform.  Columns past the segment keep
    // finite logits and are never stored.  The running max is kept on raw
    // logits (scale > 0) and the scale is folded into the exp argument.
    const int kbase = kt * kKeys;
    const bool full = kbase + kKeys - 1 <= start + r0 &&
                      (p.window == 0 || kbase >= start + r0 + rows_here - p.window);
    const float sc = p.scale_log2;
    bool grew = false;
    float alpha[NQ];
#pragma unroll
    for (int nq = 0; nq < NQ; ++nq) {
      float mx = kNegInf;
      if (full) {
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][nq][i]);
        }
      } else {
        const int lo = p.window > 0 ? qpos[nq] - p.window + 1 : -1;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
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
      for (int mt = 0; mt < 4; ++mt) {
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
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      u32x4 pb[NQ];
#pragma unroll
      for (int nq = 0; nq < NQ; ++nq) pb[nq] = pack8<DT>(s[2 * c2][nq], s[2 * c2 + 1][nq]);
      const int vrow = 32 * c2 + 4 * g4 + (l16 >> 2);
#pragma unroll
      for (int md = 0; md < MD; ++md) {
        const unsigned short *at = s_v + vrow * VROW + 16 * md + 4 * (l16 & 3);
        const u32x2 lo = read_tr16(at);
        const u32x2 hi = read_tr16(at + 16 * VROW);
        const u32x4 a = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int nq = 0; nq < NQ; ++nq) o[md][nq] = mfma<DT>(a, pb[nq], o[md][nq]);
      }
    }
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

template <int DT, int D, int NQ>
int launch(const PrefillParams &p, hipStream_t s) {
  const long grid = (long)p.max_tiles * p.n * p.KH;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL || 64 * NQ / p.G < 1) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_kernel<DT, D, NQ>), dim3((unsigned)grid), dim3(256), 0, s, p);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

template <int DT>
int dispatch(PrefillParams p, int D, int max_len, hipStream_t s) {
  auto tiles = [&](int nq) { return (int)dd_cdiv(max_len, (64 * nq) / p.G); };
  switch (D) {
    case 64: p.max_tiles = tiles(2); return launch<DT, 64, 2>(p, s);
    case 128:
      if (getenv("DAMENDAEMON_AMD_PREFILL_NQ") && atoi(getenv("DAMENDAEMON_AMD_PREFILL_NQ")) == 1) {
        p.max_tiles = tiles(1);
        return launch<DT, 128, 1>(p, s);
      }
      p.max_tiles = tiles(2);
      return launch<DT, 128, 2>(p, s);
    case 256: p.max_tiles = tiles(1); return launch<DT, 256, 1>(p, s);
    default: return DD_EUNSUPPORTED;
  }
}

}  // namespace

extern "C" int dd_prefill_attention(const void *q, const void *k, const void *v, int dtype, const int64_t *cu_seqlens,
                                    const int64_t *context_lens, const int64_t *slots, int n, int max_len,
                                    const int32_t *page_table, int table_rows, int table_width, int heads,
                                    int kv_heads, int dim, int page_size, int64_t capacity, int window, float scale,
                                    void *out, void *stream) {
  if (!q || !k || !v || !cu_seqlens || !context_lens || !slots || !page_table || !out || n < 0 || max_len < 0 ||
      heads <= 0 || kv_heads <= 0 || heads % kv_heads || page_size <= 0 || capacity <= 0 || table_width <= 0)
    return DD_EINVAL;
  if (heads / kv_heads > 16) return DD_EUNSUPPORTED;
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
