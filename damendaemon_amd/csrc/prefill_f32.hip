// Chunked-prefill attention for fp32 pages on the matrix cores (gfx950),
// head sizes 64 and 128.
//
// Same semantics as the other prefill kernels (damendaemon/paged.py:97-111
// with qwen2.py:754-770, run in an fp32 compute_dtype, qwen2.py:403-409):
// query row j of segment i attends keys 0 .. start_i + j of its slot, and
// only keys > position - window when a window is set; GQA head h reads KV
// head h / G; softmax(q.k * scale) . v.
//
// Every product is exact fp32: Q, K, V and the probabilities enter
// v_mfma_f32_16x16x4_f32 unrounded, accumulation is fp32.
//
// Layout.  A workgroup of eight waves owns one (segment, KV head) and 128
// (query row, head) columns, a wave 16 of them with its Q in registers
// (lane (kg, n16): column n16, dims (D/4) kg ..+D/4).  Per step the
// workgroup stages a tile of kKT keys of K and V in LDS (plain 16-byte loads of
// the next tile are in flight while the current one is computed; double
// buffer, one barrier per step).  A wave forms S^T = K Q^T for its columns
// (16-key MFMA tiles, one MFMA per dim of the four each lane holds), the
// online softmax per column across the four lanes that hold it, and
// O^T += V^T P^T with key 4 kg + e of a 16-key tile as k-index kg of the
// e-th MFMA, so P^T is the softmax registers themselves.  O^T tile md row m
// holds dim (D/16) m + md, so a lane reads the D/16 contiguous dims of a V
// row in 16-byte pieces.  Rows are stored with their 16-byte chunks at
// position chunk ^ (row & 15), so the 16-row K operand reads hit distinct
// banks.  Keys past the context or behind an unallocated page-table entry
// are staged as zeros (a zero probability then never meets a NaN).
#include "common.h"

#include "prefill_generic.h"

namespace {

#ifndef DD_PF32_WAVES
#define DD_PF32_WAVES 8
#endif
constexpr int kWaves = DD_PF32_WAVES;
constexpr int kCols = 16 * kWaves;  // (query row, head) columns per workgroup
#ifndef DD_PF32_KT
#define DD_PF32_KT 32
#endif
constexpr int kKT = DD_PF32_KT;     // keys per tile
constexpr int kSub = kKT / 16;      // 16-key MFMA tiles per key tile
constexpr float kNegInf = -__builtin_inff();
constexpr float kSlack = 8.f;       // running-max slack (exp2 domain)

DD_DEV int chunk_swz(int r) { return r & 15; }

template <int D>
__global__ __launch_bounds__(64 * kWaves) void prefill_f32_kernel(PrefillGenericArgs p) {
#if __HIP_DEVICE_COMPILE__
  constexpr int ROWB = 4 * D;                      // bytes per key row
  constexpr int CPR = ROWB / 16;                   // 16-byte chunks per row
  constexpr int TILEB = kKT * ROWB;                // one tile of K (or V)
  constexpr int NC = D / 16;                       // 16-byte Q / K pieces per lane
  constexpr int MD = D / 16;                       // O^T row tiles
  constexpr int PCS = kKT * CPR / (64 * kWaves);   // 16-byte pieces per thread and plane
  static_assert(CPR >= 16 && CPR % 16 == 0 && PCS >= 1, "row geometry");

  __shared__ __align__(16) char s_kv[2][2][TILEB];  // [buffer][K, V]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int n16 = lane & 15;
  const int kg = lane >> 4;

  // ---- work item: later query tiles (more keys) first ----
  const int G = p.heads / p.kv_heads;
  const int rows = kCols / G;
  const int ngrp = p.n * p.kv_heads;
  const int qt = p.max_tiles - 1 - (int)(blockIdx.x / ngrp);
  const int grp = (int)(blockIdx.x % ngrp);
  const int seg = grp / p.kv_heads;
  const int kh = grp - seg * p.kv_heads;
  const long tok0 = p.cu[seg];
  const int len = (int)(p.cu[seg + 1] - tok0);
  const int r0 = qt * rows;
  if (r0 >= len) return;
  const int context = (int)p.ctx[seg];
  const int start = context - len;
  const long slot = p.slots[seg];
  const int rows_here = min(rows, len - r0);
  const int k_hi = start + r0 + rows_here;  // exclusive
  const int k_lo = p.window > 0 ? max(0, start + r0 - p.window + 1) : 0;
  const int t_first = k_lo / kKT;
  const int t_last = (k_hi - 1) / kKT;

  // ---- this lane's column and its Q^T operand ----
  const int col = w * 16 + n16;
  const int qr = col / G;
  const int gh = col - qr * G;
  const bool colok = qr < rows_here;
  const int qpos = start + r0 + qr;
  const long qrow = ((tok0 + r0 + (colok ? qr : 0)) * p.heads + (long)kh * G + gh) * D;
  u32x4 qa[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c)
    qa[c] = colok ? *(const u32x4 *)((const float *)p.q + qrow + (D / 4) * kg + 4 * c) : u32x4{0, 0, 0, 0};

  // ---- tile staging: thread piece e = tid + 64 kWaves j is row e / CPR, chunk e % CPR ----
  const bool slot_ok = slot >= 0 && slot < p.table_rows;
  auto fetch = [&](int t, u32x4 (&kr)[PCS], u32x4 (&vr)[PCS]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PCS; ++j) {
      const int e = tid + 64 * kWaves * j;
      const int key = t * kKT + e / CPR;
      const int c = e % CPR;
      long base = -1;
      if (slot_ok && key < context) {
        const int entry = key >> p.page_shift;
        const long phys = entry < p.table_w ? p.table[slot * p.table_w + entry] : -1;
        if (phys >= 0 && phys < p.capacity)
          base = (((phys * p.kv_heads + kh) << p.page_shift) + (key & (p.page - 1))) * (long)D + 4 * c;
      }
      kr[j] = base >= 0 ? *(const u32x4 *)((const float *)p.k + base) : u32x4{0, 0, 0, 0};
      vr[j] = base >= 0 ? *(const u32x4 *)((const float *)p.v + base) : u32x4{0, 0, 0, 0};
    }
  };
  auto stage = [&](int buf, const u32x4 (&kr)[PCS], const u32x4 (&vr)[PCS]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PCS; ++j) {
      const int e = tid + 64 * kWaves * j;
      const int r = e / CPR;
      const int off = r * ROWB + 16 * ((e % CPR) ^ chunk_swz(r));
      *(u32x4 *)(s_kv[buf][0] + off) = kr[j];
      *(u32x4 *)(s_kv[buf][1] + off) = vr[j];
    }
  };

  f32x4 o[MD];
#pragma unroll
  for (int md = 0; md < MD; ++md) o[md] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = kNegInf;  // running max of this lane's column (scaled, exp2 domain)
  float lsum = 0.f;       // this lane's share of the column's denominator

  auto compute = [&](int buf, int t) __attribute__((always_inline)) {
    const char *sk = s_kv[buf][0];
    const char *sv = s_kv[buf][1];
    float x[kSub][4];
    float mx = kNegInf;
#pragma unroll
    for (int h = 0; h < kSub; ++h) {
      const int r = 16 * h + n16;
      u32x4 ka[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) ka[c] = *(const u32x4 *)(sk + r * ROWB + 16 * (((D / 16) * kg + c) ^ chunk_swz(r)));
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          s = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(ka[c][q]), __uint_as_float(qa[c][q]), s, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = t * kKT + 16 * h + 4 * kg + i;
        const bool live = colok && key <= qpos && (p.window <= 0 || key > qpos - p.window);
        x[h][i] = live ? s[i] * p.scale_log2 : kNegInf;
        mx = fmaxf(mx, x[h][i]);
      }
    }
    mx = xor32_max(xor16_max(mx));
    const bool up = mx > m_run + kSlack;
    if (__builtin_amdgcn_ballot_w64(up)) {
      const float mn = up ? mx : m_run;
      const float alpha = up ? (m_run == kNegInf ? 0.f : __builtin_amdgcn_exp2f(m_run - mn)) : 1.f;
      m_run = mn;
      lsum *= alpha;
#pragma unroll
      for (int md = 0; md < MD; ++md) o[md] *= alpha;
    }
    const float mu = m_run == kNegInf ? 0.f : m_run;
#pragma unroll
    for (int h = 0; h < kSub; ++h) {
      float pr[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pr[i] = __builtin_amdgcn_exp2f(x[h][i] - mu);
        lsum += pr[i];
      }
      u32x4 vf[4][MD / 4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 16 * h + 4 * kg + e;
#pragma unroll
        for (int q = 0; q < MD / 4; ++q)
          vf[e][q] = *(const u32x4 *)(sv + r * ROWB + 16 * (((MD / 4) * n16 + q) ^ chunk_swz(r)));
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int md = 0; md < MD; ++md)
          o[md] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(vf[e][md / 4][md % 4]), pr[e], o[md], 0, 0, 0);
    }
  };

  {
    u32x4 kr[PCS], vr[PCS];
    fetch(t_first, kr, vr);
    stage(0, kr, vr);
  }
  __syncthreads();
  for (int t = t_first; t <= t_last; ++t) {
    const int buf = (t - t_first) & 1;
    u32x4 kr[PCS], vr[PCS];
    const bool more = t < t_last;
    if (more) fetch(t + 1, kr, vr);
    compute(buf, t);
    if (more) stage(buf ^ 1, kr, vr);
    __syncthreads();
  }

  // ---- normalise and store: lane holds dims (D/16) (4 kg + i) + md of its column ----
  const float l = xor32_sum(xor16_sum(lsum));
  if (!colok) return;
  const float inv = 1.f / l;
  float *dst = (float *)p.out + qrow;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int q = 0; q < MD / 4; ++q)
      *(f32x4 *)(dst + MD * (4 * kg + i) + 4 * q) =
          f32x4{o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]} * inv;
#endif  // __HIP_DEVICE_COMPILE__
}

template <int D>
int launch_f32(PrefillGenericArgs a, hipStream_t s) {
  const int G = a.heads / a.kv_heads;
  const int rows = kCols / G;
  a.max_tiles = (int)dd_cdiv(a.max_len, rows);
  const long grid = (long)a.max_tiles * a.n * a.kv_heads;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_f32_kernel<D>), dim3((unsigned)grid), dim3(64 * kWaves), 0, s, a);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

}  // namespace

// fp32 pages at D = 64 / 128 with at most 128 query heads per KV head; any
// other case returns DD_EUNSUPPORTED (the caller then uses the vector-ALU
// kernel).
int dd_prefill_f32(const PrefillGenericArgs &a, hipStream_t s) {
  if (a.kv_heads <= 0 || a.heads % a.kv_heads || a.heads / a.kv_heads > kCols) return DD_EUNSUPPORTED;
  switch (a.dim) {
    case 64: return launch_f32<64>(a, s);
    case 128: return launch_f32<128>(a, s);
    default: return DD_EUNSUPPORTED;
  }
}
