// Shared pieces of the chunked-prefill kernels (prefill.hip,
// prefill_pipe.hip): the launch parameters, the plan entry of a work item,
// 16-bit output packing and buffer-resource constants.
#pragma once

#include "common.h"

// The running max of a column is only moved when a tile's max exceeds it by
// more than 2^kMaxSlack in the exp2 domain: probabilities then stay <= 2^8
// (exact in fp32 sums and bf16/f16 operands), and O and l are rescaled a few
// times per column instead of on almost every tile.
constexpr float kMaxSlack = 8.f;

namespace dd_prefill {


constexpr float kNegInf = -__builtin_inff();

struct PrefillParams {
  const void *q;       // (T, H, D)
  const void *k;       // (capacity, KH, page, D)
  const void *v;
  const int64_t *cu;   // (n+1) cu_seqlens of the packed tokens
  const int64_t *ctx;  // (n) start + len
  const int64_t *slots;
  const int32_t *table;
  const int32_t *plan;  // optional: kPlanInts ints per workgroup (see PrefillItem), item -1 = none
  void *out;           // (T, H, D)
  long capacity;
  int n, max_tiles;
  int H, KH, G;
  int page, page_shift;
  int table_w, table_rows;
  int window;
  float scale_log2;     // |scale| * log2(e)
  unsigned q_sign;      // 0x80008000 when scale < 0: q enters negated (exact), so logits use |scale|
  int32_t *flags;       // bf16 pages, D 64/128: per work item, 1 = result must be recomputed exactly
};

// One work item of the prefill kernels: query tile qt of group grp =
// (segment seg, KV head).  A plan entry (dd_prefill_plan) carries the item
// and its segment's token offset, length, start and slot, so that a
// workgroup reads them with one load instead of a chain of two.
constexpr int kPlanInts = DD_PREFILL_PLAN_INTS;   // item, tok0, len, start, slot, rounds, 2 unused
struct PrefillItem {
  int grp, qt, seg, len, start;
  long tok0, slot;
};
// Work items per workgroup under a plan: the plan holds `rounds` entries per
// workgroup, round-major (entry round * gridDim.x + blockIdx.x); every entry
// stores the count (field 5).  1 without a plan.
DD_DEV int prefill_rounds(const PrefillParams &p) {
  return p.plan ? p.plan[(long)kPlanInts * blockIdx.x + 5] : 1;
}
// Item of round `round` of this workgroup; false: nothing to do
DD_DEV bool prefill_item(const PrefillParams &p, PrefillItem &it, int round = 0) {
  if (p.plan) {
    const int32_t *e = p.plan + (long)kPlanInts * ((long)round * gridDim.x + blockIdx.x);
    const int item = e[0];
    if (item < 0) return false;
    it.grp = item / p.max_tiles;
    it.qt = item - it.grp * p.max_tiles;
    it.seg = it.grp / p.KH;
    it.tok0 = e[1];
    it.len = e[2];
    it.start = e[3];
    it.slot = e[4];
    return it.grp < p.n * p.KH;
  }
  // Without a plan: consecutive workgroups go to the 8 XCDs round-robin,
  // each XCD with its own L2; every query tile of one (segment, KV head)
  // group is sent to the same XCD, longest first.
  const int xcd = blockIdx.x & 7;
  const int j = blockIdx.x >> 3;
  it.grp = xcd + 8 * (j / p.max_tiles);
  it.qt = p.max_tiles - 1 - j % p.max_tiles;
  if (it.grp >= p.n * p.KH) return false;
  it.seg = it.grp / p.KH;
  it.tok0 = p.cu[it.seg];
  it.len = (int)(p.cu[it.seg + 1] - it.tok0);
  it.start = (int)p.ctx[it.seg] - it.len;
  it.slot = p.slots[it.seg];
  return true;
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

template <int DT>
DD_DEV unsigned pack2(float a, float b) {
  if constexpr (DT == DD_BF16) {
    return (unsigned)float_to_bf16_bits(a) | ((unsigned)float_to_bf16_bits(b) << 16);
  } else {
    return (unsigned)float_to_f16_bits(a) | ((unsigned)float_to_f16_bits(b) << 16);
  }
}

// 32-bit word 3 of a raw (untyped) buffer resource.
constexpr int kBufferWord3 = 0x00020000;

typedef __attribute__((address_space(3))) void lds_void;

int prefill_pipe_dispatch(const PrefillParams &p, int dtype, int dim, int max_len, int plan_len, hipStream_t s);

}  // namespace dd_prefill
