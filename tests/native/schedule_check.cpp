// Host check of the workgroup -> work-item order (cdna3-bench_amd/csrc/
// mxfp4_schedule.h).  Prints two counts of violations:
//   xcd_chunked_id is a permutation of [0, count) for count = 1 .. 5000;
//   tile_of covers every (tm, tn, split) exactly once for every grid with
//   tiles_m, tiles_n in 1 .. 40, splits in {1, 2, 3, 5}, group_m in {1, 4, 7},
//   and for the BASELINE grids (128 x 256 tiles).
#include <cstdio>
#include <vector>

#include "mxfp4_schedule.h"

using namespace mxfp4;

static long check_tiles(int tm, int tn, int splits, int group_m) {
  const int total = tm * tn * splits;
  std::vector<int> seen(total, 0);
  long bad = 0;
  for (int b = 0; b < total; ++b) {
    const TileCoord t = tile_of(b, tm, tn, splits, group_m);
    if (t.tm < 0 || t.tm >= tm || t.tn < 0 || t.tn >= tn || t.split < 0 || t.split >= splits) {
      ++bad;
      continue;
    }
    seen[(t.tm * tn + t.tn) * splits + t.split]++;
  }
  for (int v : seen) bad += v != 1;
  return bad;
}

int main() {
  long bad_xcd = 0;
  for (int count = 1; count <= 5000; ++count) {
    std::vector<int> seen(count, 0);
    for (int id = 0; id < count; ++id) {
      const int l = xcd_chunked_id(id, count);
      if (l < 0 || l >= count) {
        ++bad_xcd;
        continue;
      }
      seen[l]++;
    }
    for (int v : seen) bad_xcd += v != 1;
  }
  long bad_tiles = 0;
  const int splits_set[] = {1, 2, 3, 5}, group_set[] = {1, 4, 7};
  for (int tm = 1; tm <= 40; ++tm)
    for (int tn = 1; tn <= 40; ++tn)
      for (int s : splits_set)
        for (int g : group_set) bad_tiles += check_tiles(tm, tn, s, g);
  // dit_up, dit_down, 70B FFN M = 128 (split 2) / 8192, at 128 x 256 tiles
  bad_tiles += check_tiles(32, 48, 1, 4) + check_tiles(36, 12, 1, 4) + check_tiles(1, 112, 2, 4) +
               check_tiles(64, 112, 1, 4);
  std::printf("%ld %ld\n", bad_xcd, bad_tiles);
  return 0;
}
