// Host-side check of the workgroup -> (tile, head) mapping of attn_tiles.h
// (map_tile / tile_order) and of the launch-size guard grid_fits
// (tt_internal.h), built with hipcc for the host only by
// tests/test_tile_order.py; no GPU is used.  For every shape below the
// mapping must be a bijection from workgroup ids onto (tile, head) pairs,
// keep every head on XCD bh % 8 when the head count is a multiple of 8, and
// put the held-back cheap ranks after every heavy one on each XCD.  Exit
// status 0 = all checks passed.
#include <cstdio>
#include <vector>

#include "attn_tiles.h"

static int g_failures = 0;
#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      std::fprintf(stderr, "CHECK failed: %s: ", #cond);   \
      std::fprintf(stderr, __VA_ARGS__);                   \
      std::fprintf(stderr, "\n");                          \
      ++g_failures;                                        \
    }                                                      \
  } while (0)

static void check(int BH, int ntile, int target, int light_div, bool heavy_last) {
  const int order = tt::tile_order(BH, ntile, target, light_div);
  const int group = order & 0xffff, light = order >> 16;
  CHECK(light >= 0 && light <= ntile, "BH %d ntile %d light %d", BH, ntile, light);
  CHECK(light_div > 0 || light == 0, "BH %d ntile %d: light_div 0 holds ranks back", BH, ntile);
  const long n = (long)ntile * BH;
  std::vector<int> seen(n, 0);
  // last heavy position and first light position per XCD, in dispatch order
  std::vector<long> last_heavy(8, -1), first_light(8, n);
  for (long id = 0; id < n; ++id) {
    int tile = -1, bh = -1;
    tt::map_tile((int)id, ntile, BH, order, tile, bh, heavy_last);
    if (tile < 0 || tile >= ntile || bh < 0 || bh >= BH) {
      CHECK(false, "BH %d ntile %d id %ld -> tile %d head %d out of range", BH, ntile, id, tile, bh);
      continue;
    }
    ++seen[(long)bh * ntile + tile];
    if (BH % 8 == 0 && group > 0) {
      CHECK(bh % 8 == id % 8, "BH %d ntile %d id %ld -> head %d on another XCD", BH, ntile, id, bh);
      const int rank = heavy_last ? ntile - 1 - tile : tile;
      const int x = (int)(id % 8);
      if (rank < ntile - light) last_heavy[x] = id;
      else if (id < first_light[x]) first_light[x] = id;
    }
  }
  for (long i = 0; i < n; ++i)
    CHECK(seen[i] == 1, "BH %d ntile %d: pair (head %ld, tile %ld) mapped %d times", BH, ntile, i / ntile,
          i % ntile, seen[i]);
  for (int x = 0; x < 8; ++x)
    CHECK(last_heavy[x] < first_light[x], "BH %d ntile %d XCD %d: a cheap rank precedes a heavy one", BH, ntile, x);
}

int main() {
  const int heads[] = {1, 3, 7, 8, 12, 16, 24, 40, 64, 128, 256};
  const int tiles[] = {1, 2, 3, 7, 8, 9, 16, 31, 32, 33, 64, 129};
  const int targets[] = {32, 64, 96};
  for (int BH : heads)
    for (int nt : tiles)
      for (int tg : targets)
        for (int ld : {0, 1, 2, 4})
          for (int hl = 0; hl < 2; ++hl) check(BH, nt, tg, ld, hl != 0);
  // the held-back count saturates for very long heads
  {
    const int order = tt::tile_order(8, 70000, 64, 2);
    CHECK((order >> 16) == 0x7fff && (order & 0xffff) == 1, "order %#x", order);
    check(8, 70000, 64, 2, true);
  }
  // launch-size guard: at most 2^32 - 1 work-items per one-dimensional launch
  CHECK(tt::grid_fits(0, 256) && tt::grid_fits(1, 256), "small grids");
  CHECK(tt::grid_fits(16777215, 256) && !tt::grid_fits(16777216, 256), "256-thread limit");
  CHECK(tt::grid_fits(4194303, 1024) && !tt::grid_fits(4194304, 1024), "1024-thread limit");
  CHECK(tt::grid_fits(4294967295LL, 1) && !tt::grid_fits(4294967296LL, 1), "1-thread limit");
  CHECK(!tt::grid_fits(-1, 256) && !tt::grid_fits(int64_t(1) << 40, 64), "negative and huge grids");
  if (g_failures) {
    std::fprintf(stderr, "%d check(s) failed\n", g_failures);
    return 1;
  }
  std::printf("tile order checks passed\n");
  return 0;
}
