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
// This file holds the C entry point and the host-side workgroup plan; the
// 16-bit MFMA kernel is in prefill_pipe.hip (head sizes 48-256), the fp32
// arithmetic and vector kernels for fp32 pages and the other head sizes in
// prefill_f32.hip and prefill_generic.hip.
#include "prefill_common.h"
#include "prefill_generic.h"

#include <algorithm>
#include <climits>
#include <functional>
#include <type_traits>
#include <vector>

using namespace dd_prefill;

namespace {

// Tile geometry per head dim: (query row, head) columns per workgroup and
// keys per tile, as the host-side plan and the flag workspace count them.
struct Geometry {
  int cols, kt;
};
// prefill_pipe_kernel's layouts: 8 waves x 32 columns and 64-key tiles for
// the 128 and 160 layouts (128-key tiles for the 64 layout), 4 waves x 32
// columns and 32-key tiles for the 256 layout (prefill_pipe.hip:
// pipe_waves, pipe_keys).
constexpr Geometry kGeom64{256, 128};
constexpr Geometry kGeom128{256, 64};
constexpr Geometry kGeom160{256, 64};
constexpr Geometry kGeom256{128, 32};

// Head sizes prefill_pipe_kernel takes: 48 in its 64 layout, 80-112 in its
// 128 layout, 144 in its 160 layout, 176-240 in its 256 layout.
static bool pipe_dim(int D) {
  return D == 48 || D == 64 || D == 80 || D == 96 || D == 112 || D == 128 || (D > 128 && D <= 256 && D % 16 == 0);
}

static bool geometry(int D, Geometry *g) {
  if (!pipe_dim(D)) return false;
  *g = D <= 64 ? kGeom64 : D <= 128 ? kGeom128 : D <= 160 ? kGeom160 : kGeom256;
  return true;
}

template <int DT>
int dispatch(const PrefillParams &p, int D, int max_len, int plan_len, hipStream_t s) {
  return pipe_dim(D) ? prefill_pipe_dispatch(p, DT, D, max_len, plan_len, s) : DD_EUNSUPPORTED;
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
