// Chunked-prefill attention for the cases the MFMA kernel (prefill.hip) does
// not take: fp32 pages, and head sizes other than 64 / 128 / 256 (e.g. 96).
//
// Same semantics as prefill.hip (damendaemon/paged.py:97-111 with
// qwen2.py:754-770): query row j of segment i attends keys 0 .. start_i + j
// of its slot (and only keys > position - window), GQA head h reads KV head
// h / G, softmax(q.k * scale) . v with every product and sum in fp32.  The
// reference runs its paged prefill in compute_dtype, which is fp32 on some
// models (qwen2.py:403-409), with SDPA accepting any head size.
//
// Design: plain fp32 FMA on the vector ALUs (fp32 pages hold twice the bytes
// of the 16-bit ones and have no full-rate MFMA).  A workgroup owns one
// (segment, query head) and 64 query rows, one wave per 16 rows.  Per step a
// wave takes 64 keys, one per lane: the lane forms the 16 logits of its key
// against the wave's rows (q broadcast from LDS, K streamed in 16-byte or
// 8-byte loads), the online softmax reduces across the wave, and the P.V
// product runs with lanes over head dims (V rows read coalesced, the 64
// probabilities broadcast from LDS).  Keys outside the context or behind an
// unallocated page-table entry are never loaded; a zero probability never
// multiplies V, so NaN-filled unused pages cannot leak in.
#include "common.h"

#include "prefill_generic.h"

namespace {

constexpr int kRows = 16;      // query rows per wave
constexpr int kWaves = 4;
constexpr int kDMax = 256;
constexpr float kNegInf = -__builtin_inff();

DD_DEV float wave_max(float x) {
  x = row16_max(x);
  x = xor16_max(x);
  return xor32_max(x);
}
DD_DEV float wave_sum(float x) {
  x = row16_sum(x);
  x = xor16_sum(x);
  return xor32_sum(x);
}

template <int DT>
__global__ __launch_bounds__(64 * kWaves) void prefill_generic_kernel(PrefillGenericArgs p) {
  __shared__ float s_q[kWaves * kRows][kDMax];        // the workgroup's query rows, fp32
  __shared__ float s_p[kWaves][kRows][64];             // one step's probabilities per wave

  const int lane = threadIdx.x & 63;
  const int w = uniform(threadIdx.x >> 6);
  const int D = p.dim;
  const int G = p.heads / p.kv_heads;

  long blk = blockIdx.x;
  const int qt = (int)(blk % p.max_tiles);
  blk /= p.max_tiles;
  const int h = (int)(blk % p.heads);
  const int seg = (int)(blk / p.heads);
  const int kh = h / G;
  const long tok0 = p.cu[seg];
  const int len = (int)(p.cu[seg + 1] - tok0);
  const int r0 = qt * kWaves * kRows;
  if (r0 >= len) return;
  if (!rerun_wanted(p, seg * p.kv_heads + kh, r0, min(kWaves * kRows, len - r0))) return;
  const int context = (int)p.ctx[seg];
  const int start = context - len;
  const long slot = p.slots[seg];
  const bool slot_ok = slot >= 0 && slot < p.table_rows;

  // query rows of the workgroup, fp32 (rows past the segment read as 0)
  for (int i = threadIdx.x; i < kWaves * kRows * D; i += 64 * kWaves) {
    const int r = i / D, d = i - (i / D) * D;
    const int row = r0 + r;
    s_q[r][d] = row < len ? load_as<DT>(p.q, ((tok0 + row) * p.heads + h) * (long)D + d) : 0.f;
  }
  __syncthreads();

  const int wrow0 = r0 + w * kRows;                 // first row of this wave
  const int wrows = max(0, min(kRows, len - wrow0));
  if (wrows == 0) return;                           // no barrier follows
  const int qpos_hi = start + wrow0 + wrows - 1;    // the wave's last row position
  int k_lo = 0;
  if (p.window > 0) k_lo = max(0, start + wrow0 - p.window + 1);
  const int k_hi = qpos_hi + 1;                     // exclusive

  constexpr int NDL = kDMax / 64;                   // dims per lane in P.V
  float acc[kRows][NDL];
  float m_run[kRows], l_run[kRows];
#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    m_run[r] = kNegInf;
    l_run[r] = 0.f;
#pragma unroll
    for (int j = 0; j < NDL; ++j) acc[r][j] = 0.f;
  }

  // Element offset of token t of this slot in the (capacity, KH, page, D)
  // planes, or -1 when its page is unallocated / out of the pool.
  auto token_base = [&](int t) -> long {
    const int e = t >> p.page_shift;
    const int phys = (slot_ok && e < p.table_w) ? p.table[slot * p.table_w + e] : -1;
    if (phys < 0 || phys >= p.capacity) return -1;
    return (((long)phys * p.kv_heads + kh) * p.page + (t & (p.page - 1))) * (long)D;
  };

  for (int kb = k_lo - (k_lo & 63); kb < k_hi; kb += 64) {
    const int key = kb + lane;
    const long kbase = (key >= k_lo && key < k_hi) ? token_base(key) : -1;
    float s[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) s[r] = 0.f;
    if (kbase >= 0) {
      for (int d = 0; d < D; d += 4) {
        float kv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) kv[e] = load_as<DT>(p.k, kbase + d + e);
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
          const float *qr = &s_q[w * kRows + r][d];
          s[r] = __builtin_fmaf(qr[0], kv[0], s[r]);
          s[r] = __builtin_fmaf(qr[1], kv[1], s[r]);
          s[r] = __builtin_fmaf(qr[2], kv[2], s[r]);
          s[r] = __builtin_fmaf(qr[3], kv[3], s[r]);
        }
      }
    }
    // logits in the exp2 domain, masked per row
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      const int qpos = start + wrow0 + r;
      const bool ok = kbase >= 0 && r < wrows && key <= qpos && (p.window == 0 || key > qpos - p.window);
      const float x = ok ? s[r] * p.scale_log2 : kNegInf;
      const float mx = wave_max(x);
      const float mn = fmaxf(m_run[r], mx);
      const float alpha = mn == kNegInf ? 1.f : __builtin_amdgcn_exp2f(m_run[r] - mn);
      const float pr = ok ? __builtin_amdgcn_exp2f(x - mn) : 0.f;
      m_run[r] = mn;
      l_run[r] = l_run[r] * alpha + wave_sum(pr);
#pragma unroll
      for (int j = 0; j < NDL; ++j) acc[r][j] *= alpha;
      s_p[w][r][lane] = pr;
    }
    // P.V: lane owns dims lane + 64 j; keys one at a time, V rows coalesced
    const int kend = min(64, k_hi - kb);
    for (int jk = 0; jk < kend; ++jk) {
      const int kk = kb + jk;
      if (kk < k_lo) continue;
      const long vb = token_base(kk);   // wave-uniform
      if (vb < 0) continue;
      float v[NDL];
#pragma unroll
      for (int j = 0; j < NDL; ++j) {
        const int d = lane + 64 * j;
        v[j] = d < D ? load_as<DT>(p.v, vb + d) : 0.f;
      }
#pragma unroll
      for (int r = 0; r < kRows; ++r) {
        const float pr = s_p[w][r][jk];
        if (pr != 0.f) {
#pragma unroll
          for (int j = 0; j < NDL; ++j) acc[r][j] = __builtin_fmaf(pr, v[j], acc[r][j]);
        }
      }
    }
  }

#pragma unroll
  for (int r = 0; r < kRows; ++r) {
    if (r >= wrows) continue;
    const float inv = 1.f / l_run[r];
    const long orow = ((tok0 + wrow0 + r) * p.heads + h) * (long)D;
#pragma unroll
    for (int j = 0; j < NDL; ++j) {
      const int d = lane + 64 * j;
      if (d < D) store_as<DT>(p.out, orow + d, acc[r][j] * inv);
    }
  }
}

}  // namespace

int dd_prefill_generic(const PrefillGenericArgs &a, int dtype, hipStream_t stream) {
  if (a.dim <= 0 || a.dim > kDMax || a.dim % 4) return DD_EUNSUPPORTED;
  const long tiles = dd_cdiv(a.max_len, kWaves * kRows);
  const long grid = (long)a.n * a.heads * tiles;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  PrefillGenericArgs p = a;
  p.max_tiles = (int)tiles;
  switch (dtype) {
    case DD_F32:
      hipLaunchKernelGGL(prefill_generic_kernel<DD_F32>, dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, p);
      break;
    case DD_BF16:
      hipLaunchKernelGGL(prefill_generic_kernel<DD_BF16>, dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, p);
      break;
    case DD_F16:
      hipLaunchKernelGGL(prefill_generic_kernel<DD_F16>, dim3((unsigned)grid), dim3(64 * kWaves), 0, stream, p);
      break;
    default:
      return DD_EUNSUPPORTED;
  }
  DD_LAUNCH_CHECK();
  return DD_OK;
}
