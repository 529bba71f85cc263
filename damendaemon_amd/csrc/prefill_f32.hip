// Chunked-prefill attention in fp32 arithmetic on the matrix cores (gfx950):
// fp32 pages at any head size that is a multiple of 16 up to 256, and
// bf16 / fp16 pages at the head sizes the 16-bit MFMA kernels are not built
// for (e.g. 80, 96, 160).
//
// Same semantics as the other prefill kernels (damendaemon/paged.py:97-111
// with qwen2.py:754-770; fp32 pages are the fp32 compute_dtype of
// qwen2.py:403-409, and SDPA accepts any head size): query row j of segment
// i attends keys 0 .. start_i + j of its slot, and only keys > position -
// window when a window is set; GQA head h reads KV head h / G;
// softmax(q.k * scale) . v.
//
// Every product is exact fp32: Q, K and V (16-bit values widened exactly
// when they are loaded) and the probabilities enter v_mfma_f32_16x16x4_f32
// unrounded, accumulation is fp32; 16-bit outputs are rounded once at the
// end.
//
// Layout.  A workgroup of W = 8 waves (two per SIMD; at most 204 VGPRs up to
// D = 256) owns one (segment, KV head) and 16 W (query row, head) columns, a
// wave 16 of them with its Q in registers (lane (kg, n16): column n16, dims
// (D/4) kg ..+D/4).  Per step the workgroup stages a 32-key tile of K and V
// in LDS as fp32 (plain loads of the next tile are in flight while the
// current one is computed; double buffer, one barrier per step).  A wave
// forms S^T = K Q^T for its columns (16-key MFMA tiles, one MFMA per dim of
// the four each lane holds per 16-byte piece), the online softmax per column
// across the four lanes that hold it, and O^T += V^T P^T with key 4 kg + e of
// a 16-key tile as k-index kg of the e-th MFMA, so P^T is the softmax
// registers themselves.  O^T tile md row m holds dim (D/16) m + md, so a lane
// reads the D/16 contiguous dims of a V row.  LDS rows are padded by 16 bytes,
// so the 16-row K operand reads hit distinct banks.  Keys past the context or
// behind an unallocated page-table entry are staged as zeros (a zero
// probability then never meets a NaN).
#include "common.h"

#include "prefill_generic.h"

namespace {

constexpr int kKT = 32;            // keys per tile
constexpr int kSub = kKT / 16;     // 16-key MFMA tiles per key tile
constexpr float kNegInf = -__builtin_inff();
constexpr float kSlack = 8.f;      // running-max slack (exp2 domain)

// Four elements of the given dtype at element index idx, widened to fp32.
template <int DT>
DD_DEV f32x4 load4(const void *base, long idx) {
  if constexpr (DT == DD_F32) {
    return *(const f32x4 *)((const float *)base + idx);
  } else {
    const u32x2 w = *(const u32x2 *)((const unsigned short *)base + idx);
    if constexpr (DT == DD_BF16) {
      return f32x4{bf16_lo(w[0]), __uint_as_float(w[0] & 0xffff0000u), bf16_lo(w[1]),
                   __uint_as_float(w[1] & 0xffff0000u)};
    } else {
      return f32x4{half_bits_to_float((unsigned short)(w[0] & 0xffffu)), half_bits_to_float((unsigned short)(w[0] >> 16)),
                   half_bits_to_float((unsigned short)(w[1] & 0xffffu)), half_bits_to_float((unsigned short)(w[1] >> 16))};
    }
  }
}

// One work item: query rows qt * rows .. of group grp = (segment, KV head).
template <int DT, int D, int W>
DD_DEV void f32_item(const PrefillGenericArgs &p, char (&s_kv)[2][2][kKT * (4 * D + 16)], int grp, int qt) {
  constexpr int NT = 64 * W;
  constexpr int COLS = 16 * W;                     // (query row, head) columns per workgroup
  constexpr int RS = 4 * D + 16;                   // LDS row stride (bytes, padded)
  constexpr int TILEB = kKT * RS;                  // one tile of K (or V)
  constexpr int NC = D / 16;                       // 4-dim Q / K pieces per lane
  constexpr int MD = D / 16;                       // O^T row tiles
  constexpr int PPR = D / 4;                       // 4-element pieces per key row
  constexpr int PCS = (kKT * PPR + NT - 1) / NT;   // pieces per thread and plane
  static_assert(D % 16 == 0 && D <= 256, "head size");


  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = uniform(tid >> 6);
  const int n16 = lane & 15;
  const int kg = lane >> 4;

  const int G = p.heads / p.kv_heads;
  const int rows = COLS / G;
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
  f32x4 qa[NC];
#pragma unroll
  for (int c = 0; c < NC; ++c) qa[c] = colok ? load4<DT>(p.q, qrow + (D / 4) * kg + 4 * c) : f32x4{0.f, 0.f, 0.f, 0.f};

  // ---- tile staging: thread piece e = tid + NT j is row e / PPR, dims 4 (e % PPR) ..+4 ----
  const bool slot_ok = slot >= 0 && slot < p.table_rows;
  auto fetch = [&](int t, f32x4 (&kr)[PCS], f32x4 (&vr)[PCS]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PCS; ++j) {
      const int e = tid + NT * j;
      const int key = t * kKT + e / PPR;
      long base = -1;
      if (e < kKT * PPR && slot_ok && key < context) {
        const int entry = key >> p.page_shift;
        const long phys = entry < p.table_w ? p.table[slot * p.table_w + entry] : -1;
        if (phys >= 0 && phys < p.capacity)
          base = (((phys * p.kv_heads + kh) << p.page_shift) + (key & (p.page - 1))) * (long)D + 4 * (e % PPR);
      }
      kr[j] = base >= 0 ? load4<DT>(p.k, base) : f32x4{0.f, 0.f, 0.f, 0.f};
      vr[j] = base >= 0 ? load4<DT>(p.v, base) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  };
  auto stage = [&](int buf, const f32x4 (&kr)[PCS], const f32x4 (&vr)[PCS]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < PCS; ++j) {
      const int e = tid + NT * j;
      if (e < kKT * PPR) {
        const int off = (e / PPR) * RS + 16 * (e % PPR);
        *(f32x4 *)(s_kv[buf][0] + off) = kr[j];
        *(f32x4 *)(s_kv[buf][1] + off) = vr[j];
      }
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
      const char *krow = sk + (16 * h + n16) * RS + D * kg;   // dims (D/4) kg ..
      f32x4 ka[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) ka[c] = *(const f32x4 *)(krow + 16 * c);
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int q = 0; q < 4; ++q) s = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[c][q], qa[c][q], s, 0, 0, 0);
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
      // V of key 16h + 4kg + e, dims MD n16 .. +MD (16-, 8- or 4-byte reads)
      float vf[4][MD];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float *vrow = (const float *)(sv + (16 * h + 4 * kg + e) * RS) + MD * n16;
        if constexpr (MD % 4 == 0) {
#pragma unroll
          for (int q = 0; q < MD / 4; ++q) {
            const f32x4 v4 = *(const f32x4 *)(vrow + 4 * q);
#pragma unroll
            for (int u = 0; u < 4; ++u) vf[e][4 * q + u] = v4[u];
          }
        } else if constexpr (MD % 2 == 0) {
#pragma unroll
          for (int q = 0; q < MD / 2; ++q) {
            const float2 v2 = *(const float2 *)(vrow + 2 * q);
            vf[e][2 * q] = v2.x;
            vf[e][2 * q + 1] = v2.y;
          }
        } else {
#pragma unroll
          for (int md = 0; md < MD; ++md) vf[e][md] = vrow[md];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int md = 0; md < MD; ++md) o[md] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[e][md], pr[e], o[md], 0, 0, 0);
    }
  };

  {
    f32x4 kr[PCS], vr[PCS];
    fetch(t_first, kr, vr);
    stage(0, kr, vr);
  }
  __syncthreads();
  for (int t = t_first; t <= t_last; ++t) {
    const int buf = (t - t_first) & 1;
    f32x4 kr[PCS], vr[PCS];
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
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const long d0 = qrow + MD * (4 * kg + i);
    if constexpr (DT == DD_F32 && MD % 4 == 0) {
#pragma unroll
      for (int q = 0; q < MD / 4; ++q)
        *(f32x4 *)((float *)p.out + d0 + 4 * q) =
            f32x4{o[4 * q][i], o[4 * q + 1][i], o[4 * q + 2][i], o[4 * q + 3][i]} * inv;
    } else {
#pragma unroll
      for (int md = 0; md < MD; ++md) store_as<DT>(p.out, d0 + md, o[md][i] * inv);
    }
  }
}

template <int DT, int D, int W>
__global__ __launch_bounds__(64 * W) void prefill_f32_kernel(PrefillGenericArgs p) {
#if __HIP_DEVICE_COMPILE__
  __shared__ __align__(16) char s_kv[2][2][kKT * (4 * D + 16)];  // [buffer][K, V], rows padded by 16 bytes
  const int G = p.heads / p.kv_heads;
  const int rows = 16 * W / G;
  if (!p.flags) {
    // one work item per workgroup, later query tiles (more keys) first
    const int ngrp = p.n * p.kv_heads;
    f32_item<DT, D, W>(p, s_kv, (int)(blockIdx.x % ngrp), p.max_tiles - 1 - (int)(blockIdx.x / ngrp));
    return;
  }
  // Re-run of the 16-bit kernel's flagged work items: workgroup b owns group
  // b and recomputes those of its query tiles that a flagged item covers.
  // Every flag of the group is defined (the 16-bit kernel zeroes those of
  // tiles past the segment), so the common case -- nothing flagged -- costs
  // one load per lane and no other memory access.
  const int grp = blockIdx.x;
  const int lane = threadIdx.x & 63;
  for (int f0 = 0; f0 < p.flag_tiles; f0 += 64) {
    const int f = f0 + lane;
    const unsigned long long hot =
        __builtin_amdgcn_ballot_w64(f < p.flag_tiles && p.flags[(long)grp * p.flag_tiles + f] != 0);
    if (!hot) continue;
    // query tiles of this kernel that overlap the flagged items f0 + bit
    for (int qt = (f0 * p.flag_rows) / rows; qt < p.max_tiles && qt * rows < (f0 + 64) * p.flag_rows; ++qt) {
      const int lo = qt * rows / p.flag_rows - f0, hi = ((qt + 1) * rows - 1) / p.flag_rows - f0;
      bool any = false;
      for (int b = lo < 0 ? 0 : lo; b <= hi && b < 64; ++b) any |= (hot >> b) & 1;
      if (!any) continue;
      __syncthreads();   // the previous item's LDS reads are done
      f32_item<DT, D, W>(p, s_kv, grp, qt);
    }
  }
#endif  // __HIP_DEVICE_COMPILE__
}

template <int DT, int D>
int launch_f32(PrefillGenericArgs a, hipStream_t s) {
  constexpr int W = 8;
  const int G = a.heads / a.kv_heads;
  if (G > 16 * W) return DD_EUNSUPPORTED;
  const int rows = 16 * W / G;
  a.max_tiles = (int)dd_cdiv(a.max_len, rows);
  const long grid = a.flags ? (long)a.n * a.kv_heads : (long)a.max_tiles * a.n * a.kv_heads;
  if (grid == 0) return DD_OK;
  if (grid > 0x7fffffffL) return DD_EUNSUPPORTED;
  hipLaunchKernelGGL((prefill_f32_kernel<DT, D, W>), dim3((unsigned)grid), dim3(64 * W), 0, s, a);
  DD_LAUNCH_CHECK();
  return DD_OK;
}

template <int DT>
int dispatch_f32(const PrefillGenericArgs &a, hipStream_t s) {
  switch (a.dim) {
    case 16: return launch_f32<DT, 16>(a, s);
    case 32: return launch_f32<DT, 32>(a, s);
    case 48: return launch_f32<DT, 48>(a, s);
    case 64: return launch_f32<DT, 64>(a, s);
    case 80: return launch_f32<DT, 80>(a, s);
    case 96: return launch_f32<DT, 96>(a, s);
    case 112: return launch_f32<DT, 112>(a, s);
    case 128: return launch_f32<DT, 128>(a, s);
    case 160: return launch_f32<DT, 160>(a, s);
    case 176: return launch_f32<DT, 176>(a, s);
    case 192: return launch_f32<DT, 192>(a, s);
    case 208: return launch_f32<DT, 208>(a, s);
    case 224: return launch_f32<DT, 224>(a, s);
    case 240: return launch_f32<DT, 240>(a, s);
    case 256: return launch_f32<DT, 256>(a, s);
    default: return DD_EUNSUPPORTED;
  }
}

}  // namespace

int dd_prefill_f32(const PrefillGenericArgs &a, int dtype, hipStream_t s) {
  if (a.kv_heads <= 0 || a.heads % a.kv_heads) return DD_EUNSUPPORTED;
  if (dtype == DD_F32) return dispatch_f32<DD_F32>(a, s);
  if (dtype == DD_BF16) return dispatch_f32<DD_BF16>(a, s);
  if (dtype == DD_F16) return dispatch_f32<DD_F16>(a, s);
  return DD_EUNSUPPORTED;
}
