// Internal launch interface between the C-ABI (mxfp4_api.hip) and the kernel
// families.  Not installed; callers use include/mxfp4_mi355x.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "mxfp4_layout.h"

namespace mxfp4 {

// Fused epilogue of the GEMM kernels: v = act(acc + bias[col]) + residual[row][col].
struct Epilogue {
  const void* bias = nullptr;      // [N]
  const void* residual = nullptr;  // [M, N]
  int bias_bf16 = 0, res_bf16 = 0;
  int act = 0;                     // MXFP4_ACT_*
  int any = 0;                     // any term present (else the plain store)
  int res_vec = 0;                 // residual aligned for 4-element vector reads (8 B bf16, 16 B fp32)
};

// Tiled MFMA family (M > 32): BM x BN x 64 tiles, WM x WN waves, each wave
// owning RB 32-row blocks x 128 columns, bf16 MFMA 32x32x16.
struct TiledArgs {
  const uint16_t* A;
  const uint8_t* B;
  const uint8_t* S;
  void* C;
  int M, N, K;
  int out_bf16;
  int tiles_m, tiles_n;
  int group_m;          // tiles along M sharing one pass over N (L2 grouping)
  int ksteps;           // ceil(K / 64)
  int steps_per_split;  // K steps per split (last split may get fewer)
  int splits;
  float* partials;      // splits > 1: [tiles][splits][BM*BN]
  uint32_t* counters;   // splits > 1: [tiles], zero on entry, zero on exit

  Epilogue ep;
};

struct TiledShape {
  int wm, wn, rb;   // waves along M, waves along N, 32-row blocks per wave
  int wnc = 4;      // 32-column MFMA blocks per wave (pipelined kernel: 2 or 4)
  int stages = 3;   // pipelined kernel: LDS ring depth
  int bm() const { return wm * rb * 32; }
  int bn() const { return wn * 32 * wnc; }
  int threads() const { return wm * wn * 64; }
};

// Memory-bound family (M <= 32): bf16 MFMA 16x16x32 with M padded to 16/32.
struct GemvArgs {
  const uint16_t* A;
  const uint8_t* B;
  const uint8_t* S;
  void* C;
  int M, N, K;
  int out_bf16;
  int col_groups;       // ceil(N / columns per CTA)
  int steps;            // K steps (32 K for [K/2,N], 128 K for [N,K/2])
  int steps_per_split;
  int splits;
  float* partials;      // splits > 1: [col_groups][splits][rows*cols]
  uint32_t* counters;   // splits > 1: [col_groups]

  Epilogue ep;
};

struct GemvShape {
  int mt;    // 16-row MFMA tiles (1: M <= 16, 2: M <= 32)
  int cb;    // [K/2,N]: bytes per lane per K-pair row (4, 8, 16); [N,K/2]: 16-column blocks per wave
  int wpc;   // waves per CTA (all on the same columns, each a run of K steps)
  int u;     // K steps of loads issued before compute
  int cols() const { return 16 * cb; }
};

hipError_t launch_tiled(int layout, const TiledShape& shape, const TiledArgs& args,
                        hipStream_t stream);
bool tiled_shape_available(int layout, const TiledShape& shape);

// Three-stage pipelined variant of the tiled family (mxfp4_tiled_pipe.hip).
hipError_t launch_tiled_pipe(int layout, const TiledShape& shape, const TiledArgs& args,
                             hipStream_t stream);
bool tiled_pipe_shape_available(int layout, const TiledShape& shape);

// Hand-scheduled 256 x 256 x 64 kernel, 4 waves of 128 x 128 ([K/2,N], K % 64 == 0).
hipError_t launch_tiled_sched(int layout, const TiledShape& shape, const TiledArgs& args,
                              hipStream_t stream);
bool tiled_sched_available(int layout, const TiledShape& shape);
// [K/2,N] codes (and scales) within the scheduled kernel's 1 GiB descriptor range
bool tiled_sched_kn_fits(int64_t N, int64_t K);

hipError_t launch_gemv(int layout, const GemvShape& shape, const GemvArgs& args,
                       hipStream_t stream);
bool gemv_shape_available(int layout, const GemvShape& shape);

// Streaming family for M <= 32 and [N,K/2] or P weights (mxfp4_stream.hip).
// Split-K kernel: 32-column groups, K in `splits` ranges of waves * kw, one
// CTA per (group block, split) processing `splits` units; partials travel as
// tagged packets.  Whole-K kernel (nslot == 1, splits == 1): one CTA of
// K / kw waves per 32-column group.
struct StreamArgs {
  const uint16_t* A;
  const uint8_t* B;
  const uint8_t* S;
  void* C;
  int M, N, K;
  int out_bf16;
  int splits;           // ceil(K / (waves * 256)), <= smax
  int groups;           // ceil(N / 32): 32-column groups
  int ctas;             // ceil(groups / splits) * splits
  float* partials;      // splits > 1: [ctas][splits][16*mt*32] packets of 8 bytes, zero on entry/exit
  uint32_t* counters;   // splits > 1: [ctas], zero on entry, zero on exit
  int spin_limit;       // polls of the late unit before it falls back to counter arbitration

  Epilogue ep;
};

struct StreamShape {
  int mt;     // 16-row MFMA tiles (1: M <= 16, 2: M <= 32)
  int waves;  // compute waves per CTA (split = waves * kw K)
  int gcb;    // 16-column blocks per group (2)
  int nslot;  // LDS ring units per wave
  int smax;   // largest split count of this instantiation
  int kw;     // K per compute wave and unit (256 or 512)
  int direct = 0;    // 8 or 16: the decode kernel (mxfp4_decode.hip) for M <= direct
  int resident = 0;  // 1, 8 or 32: a resident kernel (mxfp4_decode.hip) for M <= resident
  int k_split() const { return waves * kw; }
  int tile() const { return 16 * mt * 16 * gcb; }
};

hipError_t launch_stream(int layout, const StreamShape& shape, const StreamArgs& args, hipStream_t stream);
bool stream_shape_available(const StreamShape& shape);

// Decode kernel (mxfp4_decode.hip): [N,K/2], M <= rows with rows = 16 (64
// columns x 4096 K per CTA) or 8 (32 columns x 8192 K per CTA), the CTA's
// activation slice resident in LDS; S = ceil(K / KR) <= 8 CTAs per column
// group, their tiles meeting as packets of decode_workspace bytes after the
// counters.
int64_t decode_splits(int rows, int64_t K);
size_t decode_workspace(int rows, int64_t N, int64_t K);
bool decode_shape_ok(int rows, int layout, int64_t M, int64_t N, int64_t K);
hipError_t launch_decode(int rows, int layout, const StreamArgs& args, hipStream_t stream);

// Resident kernels (mxfp4_decode.hip): [N,K/2], every weight load of a CTA
// issued at entry into VGPRs.  rows = 1 or 8 (M <= rows): one CTA of K / 512
// waves per 32 columns x the whole K (K % 512 == 0, K <= 8192), no split, no
// workspace.  rows = 16 or 32 (M <= rows): one CTA of 8 waves per 128
// columns x 2048 K, S = ceil(K / 2048) <= 8 CTAs per column group whose fp32 partials
// (resident_workspace bytes after the counters) the last arrival sums.
int64_t resident_splits(int rows, int64_t K);
size_t resident_workspace(int rows, int64_t N, int64_t K);
bool resident_shape_ok(int rows, int layout, int64_t M, int64_t N, int64_t K);
hipError_t launch_resident(int rows, int layout, const StreamArgs& args, hipStream_t stream);
// M = 1 form with whole 256-byte column segments per load and dot products
// instead of MFMAs (StreamShape::nslot = 1); shape rules of rows = 1.
hipError_t launch_resident_dot(int layout, const StreamArgs& args, hipStream_t stream);

// Any shape with K % 32 == 0; one thread per output, for shapes the fast
// families do not cover (N % 16 != 0, unaligned pointers).
hipError_t launch_generic(int layout, const uint16_t* A, const uint8_t* B, const uint8_t* S,
                          void* C, int out_bf16, int M, int N, int K, const Epilogue& ep,
                          hipStream_t stream);

// Dequantized [K, N] tile (bf16 or fp32) from either layout.
hipError_t launch_dequant(int layout, const uint8_t* B, const uint8_t* S, void* out,
                          int out_bf16, int K, int N, hipStream_t stream);

// Weights rewritten from one layout to another (codes and scales).
hipError_t launch_convert(int src_layout, int dst_layout, const uint8_t* B, const uint8_t* S,
                          uint8_t* B_out, uint8_t* S_out, size_t K, size_t N, hipStream_t stream);

// fp32 / bf16 weights (X [K,N] or [N,K]) -> MXFP4 codes and scales in b_layout.
hipError_t launch_quantize(const void* X, int x_bf16, int x_layout, uint8_t* B, uint8_t* S, int b_layout,
                           size_t K, size_t N, hipStream_t stream);

// [N,K/2] -> G (codes and scales), N % 128 == 0, B and B_out 16-byte
// aligned, S_out 4-byte aligned.
hipError_t launch_convert_nk_to_g(const uint8_t* B, const uint8_t* S, uint8_t* B_out, uint8_t* S_out, size_t K,
                                  size_t N, hipStream_t stream);

// C = 0 (K == 0).
hipError_t launch_zero_fill(void* C, size_t bytes, hipStream_t stream);

}  // namespace mxfp4
