// Workgroup -> work-item order of the tiled, GEMV and streaming kernels
// (host and device; the host side is what the CPU tests check).
//
// Replaces the reference's detect_num_xcds / remap_xcd (csrc/bf16_gemm.h:
// 156-175), which derives the XCD count as CUs / 38 (6 on MI355X, which has
// 8) and falls back to the linear order when the tile count is not a
// multiple of it.
#pragma once

#include "mxfp4_layout.h"

namespace mxfp4 {

constexpr int kNumXcds = 8;  // MI355X: 8 XCDs x 32 CUs

// Workgroups are dispatched round-robin over the XCDs (id % 8).  Renumber so
// each XCD owns one contiguous range of logical ids; a bijection on
// [0, count) for any count.  Neighbouring logical tiles then share an XCD's L2.
MXFP4_HD int xcd_chunked_id(int id, int count) {
  const int q = count / kNumXcds, r = count % kNumXcds;
  const int x = id % kNumXcds, local = id / kNumXcds;
  return x * q + (x < r ? x : r) + local;
}

struct TileCoord {
  int tm, tn, split;
};

// Tile (tm, tn) and K split of workgroup `block` for a tiles_m x tiles_n grid
// with `splits` K splits: XCD chunking, then groups of group_m M-tiles that
// sweep every N-tile (column-major inside a group, so the CTAs of one round
// on an XCD share A rows and B columns), the splits of one tile adjacent.
// A bijection of [0, tiles_m * tiles_n * splits) onto the (tile, split) set.
MXFP4_HD TileCoord tile_of(int block, int tiles_m, int tiles_n, int splits, int group_m) {
  const int total = tiles_m * tiles_n * splits;
  const int logical = xcd_chunked_id(block, total);
  const int tile = logical / splits;
  const int split = logical - tile * splits;
  const int group_size = group_m * tiles_n;
  const int group = tile / group_size;
  const int first_m = group * group_m;
  const int gm_rows = tiles_m - first_m < group_m ? tiles_m - first_m : group_m;
  const int in_group = tile - group * group_size;
  return TileCoord{first_m + in_group % gm_rows, in_group / gm_rows, split};
}

}  // namespace mxfp4
