// Tiled MFMA kernel family for M > 32 (MFMA-bound shapes).
//
// Replaces the reference's fused dequant-GEMM kernels (csrc/strategy_b..m*.cu,
// e.g. strategy_j_synthesis.cu:93-185) and their loaders
// (bf16_gemm.h:56-121, strategy_j_synthesis.cu:21-91).  Design:
//   * tile BM x BN x 64, WM x WN waves, a wave owns RB 32-row blocks x 128
//     columns and issues v_mfma_f32_32x32x16_bf16;
//   * A (bf16) and the raw FP4 bytes go global -> LDS with 16-byte
//     buffer_load ... lds (no VGPR staging), two LDS stages;
//   * the weights stay 4-bit in LDS; each wave converts its operand with
//     v_cvt_scalef32_pk_bf16_fp4 (scale applied exactly in the convert) right
//     before the MFMA, so no bf16 weight tile is ever written;
//   * E8M0 scales are read straight from global into registers one stage
//     ahead;
//   * split-K writes fp32 partials to a workspace and the last CTA of a tile
//     (device-scope counter) sums them in split order: deterministic.
//
// Operand layouts (v_mfma_f32_32x32x16_bf16, lane l, c = l % 32, h = l / 32):
//   A operand: row c, 8 K-consecutive bf16 (K half h);  B operand: column c,
//   the same 8 K positions;  D: column c, rows 8*(i/4) + 4*h + (i%4).
// The K order inside one MFMA only has to agree between A and B, which lets
// each layout pick the K assignment that makes its loads contiguous.
//
// [K/2, N] weights: a lane reads one word (4 columns) from each of 4 K-pair
// rows and feeds MFMA j with byte j of each word, so MFMA j covers columns
// 4c + j: four MFMAs span the wave's 128 columns and the epilogue writes 4
// adjacent columns per lane.
// [N, K/2] weights: a lane reads 16 bytes = 32 K of one column; MFMA s uses
// word s (K 32h + 8s .. +7) against the matching A chunk.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

constexpr int kBK = 64;

template <int LAYOUT, int WM, int WN, int RB>
struct TiledCfg {
  static constexpr int NWAVES = WM * WN;
  static constexpr int NT = NWAVES * 64;
  static constexpr int BM = WM * RB * 32;
  static constexpr int BN = WN * 128;
  static constexpr int A_BYTES = BM * 128;  // BM rows x 64 bf16
  static constexpr int B_BYTES = BN * 32;   // BN columns x 64 codes x 4 bit
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_INSTR = A_BYTES / 1024;  // one wave instruction moves 1 KB
  static constexpr int B_INSTR = B_BYTES / 1024;
  static constexpr int KN_CPR = BN / 16;  // 16-byte chunks per K-pair row ([K/2,N] tile)
};

// A tile: 128-byte rows of 8 chunks.  XOR swizzle so the 8 (or 16) lanes a
// ds_read_b128 serves per cycle hit distinct banks for 32 or 64 banks.
__device__ __forceinline__ int a_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// [K/2,N] B tile: rows r and r+4 are read by the two lane halves of one
// ds_read_b32; flip the upper half of the row for (r >> 2) odd.
template <int CPR>
__device__ __forceinline__ int kn_swz(int row) { return ((row >> 2) & 1) * (CPR / 2); }

// [N,K/2] B tile: 32-byte rows of 2 chunks; 8 lanes of one ds_read_b128 read
// rows 8a..8a+7, swap the chunks of rows with bit 2 set.
__device__ __forceinline__ int nk_swz(int row) { return (row >> 2) & 1; }

template <int LAYOUT, int WM, int WN, int RB>
__global__ void __launch_bounds__(WM* WN * 64, 1) tiled_kernel(TiledArgs p) {
  using Cfg = TiledCfg<LAYOUT, WM, WN, RB>;
  constexpr int NT = Cfg::NT, BM = Cfg::BM, BN = Cfg::BN, NWAVES = Cfg::NWAVES;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[2 * Cfg::STAGE];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int wm = wave / WN, wn = wave % WN;
  const int c = lane & 31, h = lane >> 5;

  // ---- tile / split assignment -------------------------------------------
  const TileCoord tc = tile_of((int)blockIdx.x, p.tiles_m, p.tiles_n, p.splits, p.group_m);
  const int tile = tc.tm * p.tiles_n + tc.tn;
  const int split = tc.split, tm = tc.tm, tn = tc.tn;
  const int m0 = tm * BM, n0 = tn * BN;

  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;
  const int s_begin = split * p.steps_per_split;
  const int s_end = min(p.ksteps, s_begin + p.steps_per_split);

  // ---- loaders -------------------------------------------------------------
  auto load_stage = [&](int buf, int step) __attribute__((always_inline)) {
    uint8_t* sA = smem + buf * Cfg::STAGE;
    uint8_t* sB = sA + Cfg::A_BYTES;
    const int k0 = step * kBK;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A + (size_t)m0 * K + k0);
#pragma unroll
    for (int i = wave; i < Cfg::A_INSTR; i += NWAVES) {
      const int row = i * 8 + (lane >> 3);
      const int lc = (lane & 7) ^ a_swz(row);
      const bool ok = (m0 + row < M) && (k0 + lc * 8 < K);
      buffer_load_lds16(ra, sA + i * 1024, ok ? (uint32_t)(row * K * 2 + lc * 16) : kOobOffset);
    }
    if constexpr (LAYOUT == kLayoutKN) {
      constexpr int CPR = Cfg::KN_CPR;
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + (size_t)(k0 >> 1) * N + n0);
#pragma unroll
      for (int i = wave; i < Cfg::B_INSTR; i += NWAVES) {
        const int q = i * 64 + lane;
        const int row = q / CPR;
        const int lc = (q % CPR) ^ kn_swz<CPR>(row);
        const bool ok = ((k0 >> 1) + row < Kh) && (n0 + lc * 16 < N);
        buffer_load_lds16(rb, sB + i * 1024, ok ? (uint32_t)(row * N + lc * 16) : kOobOffset);
      }
    } else {
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + (size_t)n0 * Kh + (k0 >> 1));
#pragma unroll
      for (int i = wave; i < Cfg::B_INSTR; i += NWAVES) {
        const int q = i * 64 + lane;
        const int row = q >> 1;
        const int lc = (q & 1) ^ nk_swz(row);
        const bool ok = (n0 + row < N) && ((k0 >> 1) + lc * 16 < Kh);
        buffer_load_lds16(rb, sB + i * 1024, ok ? (uint32_t)(row * Kh + lc * 16) : kOobOffset);
      }
    }
  };

  // Scales for one stage into registers: [K/32,N]: 2 words (4 columns, groups
  // g0, g0+1); [N,K/32]: 4 bytes (column block cb, group g0 + h).
  uint32_t sc_next[4] = {0u, 0u, 0u, 0u};
  auto load_scales = [&](int step) __attribute__((always_inline)) {
    const int g0 = step * 2;
    if constexpr (LAYOUT == kLayoutKN) {
      const int col = n0 + wn * 128 + 4 * c;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const bool ok = (g0 + g < G) && (col < N);
        sc_next[g] = ok ? *reinterpret_cast<const uint32_t*>(p.S + (size_t)(g0 + g) * N + col) : 0u;
      }
    } else {
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int col = n0 + wn * 128 + 32 * cb + c;
        const bool ok = (g0 + h < G) && (col < N);
        sc_next[cb] = ok ? (uint32_t)p.S[(size_t)col * G + g0 + h] : 0u;
      }
    }
  };

  f32x16 acc[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][j][e] = 0.f;

  auto compute_stage = [&](int buf, const uint32_t (&sc)[4]) __attribute__((always_inline)) {
    const uint8_t* sA = smem + buf * Cfg::STAGE;
    const uint8_t* sB = sA + Cfg::A_BYTES;
    if constexpr (LAYOUT == kLayoutKN) {
      constexpr int CPR = Cfg::KN_CPR;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const uint32_t sw = sc[ks >> 1];
        const float s0 = e8m0_to_f32(sw), s1 = e8m0_to_f32(sw >> 8);
        const float s2 = e8m0_to_f32(sw >> 16), s3 = e8m0_to_f32(sw >> 24);
        uint32_t raw[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = ks * 8 + h * 4 + i;
          const int lc = (wn * 128 + 4 * c) >> 4;
          const int pc = lc ^ kn_swz<CPR>(row);
          raw[i] = *reinterpret_cast<const uint32_t*>(sB + row * BN + pc * 16 + 4 * (c & 3));
        }
        bf16x8 a[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int row = wm * RB * 32 + rb * 32 + c;
          const int pc = (ks * 2 + h) ^ a_swz(row);
          a[rb] = *reinterpret_cast<const bf16x8*>(sA + row * 128 + pc * 16);
        }
        const bf16x8 b0 = operand_from_bytes<0>(raw[0], raw[1], raw[2], raw[3], s0);
        const bf16x8 b1 = operand_from_bytes<1>(raw[0], raw[1], raw[2], raw[3], s1);
        const bf16x8 b2 = operand_from_bytes<2>(raw[0], raw[1], raw[2], raw[3], s2);
        const bf16x8 b3 = operand_from_bytes<3>(raw[0], raw[1], raw[2], raw[3], s3);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          acc[rb][0] = mfma_32x32x16(a[rb], b0, acc[rb][0]);
          acc[rb][1] = mfma_32x32x16(a[rb], b1, acc[rb][1]);
          acc[rb][2] = mfma_32x32x16(a[rb], b2, acc[rb][2]);
          acc[rb][3] = mfma_32x32x16(a[rb], b3, acc[rb][3]);
        }
      }
    } else {
      u32x4 raw[4];
      float sf[4];
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int row = wn * 128 + cb * 32 + c;
        const int pc = h ^ nk_swz(row);
        raw[cb] = *reinterpret_cast<const u32x4*>(sB + row * 32 + pc * 16);
        sf[cb] = e8m0_to_f32(sc[cb]);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        bf16x8 a[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
          const int row = wm * RB * 32 + rb * 32 + c;
          const int pc = (h * 4 + s) ^ a_swz(row);
          a[rb] = *reinterpret_cast<const bf16x8*>(sA + row * 128 + pc * 16);
        }
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          const bf16x8 b = operand_from_word(raw[cb][s], sf[cb]);
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) acc[rb][cb] = mfma_32x32x16(a[rb], b, acc[rb][cb]);
        }
      }
    }
  };

  // ---- main loop: two LDS stages -------------------------------------------
  if (s_begin < s_end) {
    load_stage(0, s_begin);
    load_scales(s_begin);
    wait_vmcnt0();
    __syncthreads();
    for (int s = s_begin; s < s_end; ++s) {
      const int buf = (s - s_begin) & 1;
      uint32_t sc[4] = {sc_next[0], sc_next[1], sc_next[2], sc_next[3]};
      if (s + 1 < s_end) {
        load_stage(buf ^ 1, s + 1);
        load_scales(s + 1);
      }
      compute_stage(buf, sc);
      wait_vmcnt0();
      __syncthreads();
    }
  }

  // ---- split-K fix-up ------------------------------------------------------
  // Partial slot of (tile, split): [quad][thread] f32x4, written and read with
  // device-coherent (SC1) accesses; the last CTA of the tile sums the splits
  // in split order (deterministic).
  if (p.splits > 1) {
    constexpr int Q = RB * 16;  // f32x4 quads per thread
    constexpr uint32_t SLOT = (uint32_t)Q * NT * 16;  // bytes per split slot
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(reinterpret_cast<uint8_t*>(p.partials) + (size_t)tile * p.splits * SLOT);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 v = {acc[rb][j][q4 * 4 + 0], acc[rb][j][q4 * 4 + 1], acc[rb][j][q4 * 4 + 2],
                           acc[rb][j][q4 * 4 + 3]};
          const uint32_t off = split * SLOT + (uint32_t)(((rb * 4 + j) * 4 + q4) * NT + threadIdx.x) * 16;
          store_coherent(rp, off, v);
        }
    if (!splitk_arrive_last(p.counters + tile, (uint32_t)p.splits, &s_last)) return;
    splitk_sum<RB * 16>(rp, SLOT, p.splits, NT, [&](int i, f32x4 v) __attribute__((always_inline)) {
      const int rb = i / 16, j = (i / 4) % 4, q4 = i % 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[rb][j][q4 * 4 + e] = v[e];
    });
  }

  // ---- epilogue ------------------------------------------------------------
  // Plain and fused stores are separate loops, chosen once (see StoreKind).
  auto store = [&](auto fused, auto out) __attribute__((always_inline)) {
    constexpr bool kFused = decltype(fused)::value;
    const bool bf16 = decltype(out)::value == 2 ? p.out_bf16 != 0 : decltype(out)::value == 1;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int row = m0 + wm * RB * 32 + rb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
        if (row >= M) continue;
        if constexpr (LAYOUT == kLayoutKN) {
          const int col = n0 + wn * 128 + 4 * c;
          if (col >= N) continue;
          float v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j)
            v[j] = kFused ? epilogue_value(p.ep, acc[rb][j][i], row, col + j, N) : acc[rb][j][i];
          if (bf16) {
            u32x2 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.C) + (size_t)row * N + col) = w;
          } else {
            *reinterpret_cast<f32x4*>(static_cast<float*>(p.C) + (size_t)row * N + col) = f32x4{v[0], v[1], v[2], v[3]};
          }
        } else {
#pragma unroll
          for (int cb = 0; cb < 4; ++cb) {
            const int col = n0 + wn * 128 + 32 * cb + c;
            if (col >= N) continue;
            const float v = kFused ? epilogue_value(p.ep, acc[rb][cb][i], row, col, N) : acc[rb][cb][i];
            if (bf16)
              static_cast<uint16_t*>(p.C)[(size_t)row * N + col] = (uint16_t)bf16_bits_rne(v);
            else
              static_cast<float*>(p.C)[(size_t)row * N + col] = v;
          }
        }
      }
    }
  };
  if (p.ep.any)
    store(StoreKind<true>{}, OutKind<2>{});
  else if (p.out_bf16)
    store(StoreKind<false>{}, OutKind<1>{});
  else
    store(StoreKind<false>{}, OutKind<0>{});
}

template <int LAYOUT, int WM, int WN, int RB>
hipError_t launch_one(const TiledArgs& a, hipStream_t stream) {
  using Cfg = TiledCfg<LAYOUT, WM, WN, RB>;
  const int grid = a.tiles_m * a.tiles_n * a.splits;
  hipLaunchKernelGGL((tiled_kernel<LAYOUT, WM, WN, RB>), dim3(grid), dim3(Cfg::NT), 0, stream, a);
  return hipGetLastError();
}

template <int LAYOUT>
hipError_t dispatch_shape(const TiledShape& s, const TiledArgs& a, hipStream_t stream) {
  if (s.wm == 2 && s.wn == 2 && s.rb == 4) return launch_one<LAYOUT, 2, 2, 4>(a, stream);
  if (s.wm == 4 && s.wn == 2 && s.rb == 2) return launch_one<LAYOUT, 4, 2, 2>(a, stream);
  if (s.wm == 2 && s.wn == 2 && s.rb == 2) return launch_one<LAYOUT, 2, 2, 2>(a, stream);
  if (s.wm == 1 && s.wn == 2 && s.rb == 2) return launch_one<LAYOUT, 1, 2, 2>(a, stream);
  if (s.wm == 2 && s.wn == 1 && s.rb == 2) return launch_one<LAYOUT, 2, 1, 2>(a, stream);
  if (s.wm == 1 && s.wn == 2 && s.rb == 1) return launch_one<LAYOUT, 1, 2, 1>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool tiled_shape_available(int layout, const TiledShape& s) {
  (void)layout;
  return (s.wm == 2 && s.wn == 2 && s.rb == 4) || (s.wm == 4 && s.wn == 2 && s.rb == 2) ||
         (s.wm == 2 && s.wn == 2 && s.rb == 2) || (s.wm == 1 && s.wn == 2 && s.rb == 2) ||
         (s.wm == 2 && s.wn == 1 && s.rb == 2) || (s.wm == 1 && s.wn == 2 && s.rb == 1);
}

hipError_t launch_tiled(int layout, const TiledShape& shape, const TiledArgs& args,
                        hipStream_t stream) {
  if (layout == kLayoutKN) return dispatch_shape<kLayoutKN>(shape, args, stream);
  if (layout == kLayoutNK) return dispatch_shape<kLayoutNK>(shape, args, stream);
  return hipErrorInvalidValue;
}

}  // namespace mxfp4
