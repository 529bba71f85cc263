/* A plain C caller of the library's host-side entry points: it is built
 * against include/damendaemon_amd.h only (no HIP, no torch) and checks the
 * version, the error names, the decode split policy and the prefill plan,
 * the way a non-Python host (cgo, JNI, N-API) would bind the C ABI. */
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "damendaemon_amd.h"

#define CHECK(cond)                                              \
  do {                                                           \
    if (!(cond)) {                                               \
      fprintf(stderr, "check failed line %d: %s\n", __LINE__, #cond); \
      return 1;                                                  \
    }                                                            \
  } while (0)

int main(void) {
  CHECK(dd_abi_version() == DD_ABI_VERSION);
  CHECK(dd_error_string(DD_OK) != NULL);
  CHECK(dd_error_string(DD_EINVAL) != NULL);

  int tokens = 0;
  const int splits = dd_decode_splits(8192, 512, &tokens);
  CHECK(splits >= 1 && tokens % 64 == 0 && splits * tokens >= 8192);
  CHECK(dd_decode_splits(0, 1, &tokens) < 0);
  CHECK(dd_decode_splits_for(8192, 256, 256, DD_BF16, &tokens) == 11 && tokens == 768);

  int cols = 0, kt = 0;
  CHECK(dd_prefill_geometry(128, &cols, &kt) == DD_OK && cols > 0 && kt > 0);
  CHECK(dd_prefill_geometry(100, &cols, &kt) == DD_EUNSUPPORTED);

  /* plan for 3 segments (two chunks and a short one) over 8 KV heads */
  const int64_t lengths[3] = {512, 300, 17};
  const int64_t starts[3] = {4000, 0, 900};
  const int64_t slots[3] = {5, 2, 7};
  const int need = dd_prefill_plan(lengths, starts, slots, 3, 32, 8, 128, 0, 0, NULL, 0);
  CHECK(need > 0 && need % 8 == 0);
  static int32_t entries[4096 * DD_PREFILL_PLAN_INTS];
  int32_t plan[4096];
  CHECK(need <= 4096);
  CHECK(dd_prefill_plan(lengths, starts, slots, 3, 32, 8, 128, 0, 0, entries, need) == need);
  for (int i = 0; i < need; ++i) {
    const int32_t *e = entries + (long)i * DD_PREFILL_PLAN_INTS;
    plan[i] = e[0];
    if (e[0] < 0) continue;
    const int seg = e[0] / ((512 + cols / 4 - 1) / (cols / 4)) / 8;
    CHECK(e[2] == lengths[seg] && e[3] == starts[seg] && e[4] == slots[seg]);
    CHECK(e[1] == (seg == 0 ? 0 : seg == 1 ? 512 : 812));
  }
  /* every (segment, KV head, query tile) item appears exactly once */
  const int rows = cols / 4;
  const int max_tiles = (512 + rows - 1) / rows;
  int seen[3 * 8 * 64];
  memset(seen, 0, sizeof(seen));
  int items = 0;
  for (int i = 0; i < need; ++i) {
    if (plan[i] < 0) continue;
    const int grp = plan[i] / max_tiles, qt = plan[i] % max_tiles;
    CHECK(grp < 24 && qt * rows < lengths[grp / 8]);
    CHECK(seen[plan[i]]++ == 0);
    ++items;
  }
  int expect = 0;
  for (int s = 0; s < 3; ++s) expect += 8 * (int)((lengths[s] + rows - 1) / rows);
  CHECK(items == expect);
  printf("ok: abi %d, decode splits %d x %d, prefill %d items in a plan of %d\n", dd_abi_version(), splits,
         tokens, items, need);
  return 0;
}
