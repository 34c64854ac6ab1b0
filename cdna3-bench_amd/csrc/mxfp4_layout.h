// Byte positions of the four weight layouts (host and device).
//
// Every layout stores the same bytes: packed byte kp of column n holds the
// E2M1 codes of K = 2kp (low nibble) and 2kp + 1, and scale byte g of column
// n scales K = 32g .. 32g + 31.  Only the positions differ:
//
//   KN  codes [K/2][N]                 scales [K/32][N]
//       (reference API, csrc/mxfp4_ext.cpp:21-24)
//   NK  codes [N][K/2]                 scales [N][K/32]
//   G   codes [N/128][K/8][128][4]     scales [N/128][K/32][128]
//       (strategy G prepack, python/mxfp4_cdna3/ref.py:85-101 with n_tile
//       128; consumer csrc/strategy_g_prepacked.cu:31-51,77-81)
//   P   codes [N/32][K/64][2][32][16]  scales [N/32][K/64][2][32]
//       (panels: the 1 KB block of 32 columns x 64 K is stored in the order
//       a wave reads it -- lane 32h + c holds the 16 bytes = 32 K of column c,
//       K 32h .. 32h + 31 of the block -- and the block's 64 scale bytes in the
//       same lane order)
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "../../include/mxfp4_mi355x.h"

#ifdef __HIPCC__
#define MXFP4_HD __host__ __device__ __forceinline__
#else
#define MXFP4_HD inline
#endif

namespace mxfp4 {

enum Layout : int {
  kLayoutKN = MXFP4_LAYOUT_KN,
  kLayoutNK = MXFP4_LAYOUT_NK,
  kLayoutG = MXFP4_LAYOUT_G,
  kLayoutP = MXFP4_LAYOUT_P,
};

constexpr int kGCols = 128;  // G: columns per block
constexpr int kPCols = 32;   // P: columns per panel
constexpr int kPK = 64;      // P: K per block

// Shape rules beyond K % 32 == 0.
MXFP4_HD bool layout_shape_ok(int layout, int64_t N, int64_t K) {
  switch (layout) {
    case kLayoutKN:
    case kLayoutNK:
      return true;
    case kLayoutG:
      return N % kGCols == 0;
    case kLayoutP:
      return N % kPCols == 0 && K % kPK == 0;
    default:
      return false;
  }
}

// Offset of packed byte kp (K pair) of column n.
template <int L>
MXFP4_HD size_t code_offset(size_t kp, size_t n, size_t K, size_t N) {
  if constexpr (L == kLayoutKN) {
    return kp * N + n;
  } else if constexpr (L == kLayoutNK) {
    return n * (K / 2) + kp;
  } else if constexpr (L == kLayoutG) {
    return ((n / kGCols) * (K / 8) + kp / 4) * (kGCols * 4) + (n % kGCols) * 4 + kp % 4;
  } else {
    return ((n / kPCols) * (K / kPK) + kp / 32) * 1024 + ((kp / 16) % 2) * 512 + (n % kPCols) * 16 +
           kp % 16;
  }
}

// Inverse of code_offset: (kp, n) of the byte at offset o.
template <int L>
MXFP4_HD void code_position(size_t o, size_t K, size_t N, size_t& kp, size_t& n) {
  if constexpr (L == kLayoutKN) {
    kp = o / N;
    n = o - kp * N;
  } else if constexpr (L == kLayoutNK) {
    n = o / (K / 2);
    kp = o - n * (K / 2);
  } else if constexpr (L == kLayoutG) {
    const size_t blk = o / (kGCols * 4), w = o % (kGCols * 4);
    const size_t nb = blk / (K / 8), chunk = blk - nb * (K / 8);
    kp = 4 * chunk + w % 4;
    n = nb * kGCols + w / 4;
  } else {
    const size_t blk = o / 1024, w = o % 1024;
    const size_t p = blk / (K / kPK), t = blk - p * (K / kPK);
    kp = 32 * t + 16 * (w / 512) + w % 16;
    n = p * kPCols + (w % 512) / 16;
  }
}

// Offset of scale byte g (K group) of column n.
template <int L>
MXFP4_HD size_t scale_offset(size_t g, size_t n, size_t K, size_t N) {
  if constexpr (L == kLayoutKN) {
    return g * N + n;
  } else if constexpr (L == kLayoutNK) {
    return n * (K / 32) + g;
  } else if constexpr (L == kLayoutG) {
    return ((n / kGCols) * (K / 32) + g) * kGCols + n % kGCols;
  } else {
    return ((n / kPCols) * (K / kPK) + g / 2) * 64 + (g % 2) * 32 + n % kPCols;
  }
}

template <int L>
MXFP4_HD void scale_position(size_t o, size_t K, size_t N, size_t& g, size_t& n) {
  if constexpr (L == kLayoutKN) {
    g = o / N;
    n = o - g * N;
  } else if constexpr (L == kLayoutNK) {
    n = o / (K / 32);
    g = o - n * (K / 32);
  } else if constexpr (L == kLayoutG) {
    const size_t blk = o / kGCols;
    const size_t nb = blk / (K / 32);
    g = blk - nb * (K / 32);
    n = nb * kGCols + o % kGCols;
  } else {
    const size_t blk = o / 64, w = o % 64;
    const size_t p = blk / (K / kPK), t = blk - p * (K / kPK);
    g = 2 * t + w / 32;
    n = p * kPCols + w % 32;
  }
}

}  // namespace mxfp4
