// Pipelined tiled MFMA kernel (M > 32): the production kernel of the tiled
// family.  Same operand layouts, loaders and split-K protocol as tiled_kernel
// (mxfp4_tiled.hip); the main loop differs:
//
//   * an NS-stage LDS ring: while stage t is consumed, stages t+1 .. t+NS-1
//     are resident or in flight (16-byte buffer_load ... lds);
//   * LDS operands are read one 16-K sub-step ahead into registers, so the
//     ds_read latency of sub-step s+1 hides under the MFMAs of sub-step s;
//   * one barrier per stage, placed before the last sub-step: it publishes
//     stage t+1 (every wave waited for its own loads with a counted vmcnt)
//     and retires stage t-1's buffer; the first operands of stage t+1 are
//     read while the last MFMAs of stage t drain;
//   * the per-lane LDS offsets (XOR swizzles included) are computed once; a
//     sub-step read is one add of the stage base plus immediate offsets.
//
// Wave tile: RB 32-row blocks x (32 * WNC) columns.  Every B element is
// converted once per wave that reads it, i.e. (BM / wave rows) times per
// tile: converts per MFMA = 128 / (32 * RB).  WNC = 4 with RB = 2 (4 x 2
// waves of 64 x 128) or WNC = 2 with RB = 4 (2 x 4 waves of 128 x 64).
//   [K/2,N] weights: a lane reads WNC bytes (WNC adjacent columns) of each of
//     4 K-pair rows; MFMA j uses byte j of each row word (WNC = 4) or bytes j,
//     j+2 of two packed row pairs (WNC = 2), so MFMA j covers columns
//     WNC*c + j and the epilogue writes WNC adjacent columns per lane.
//   [N,K/2] weights: a lane reads 16 bytes = 32 K of column block cb; word s
//     against the A chunk K 32h + 8s .. +7.
//   G (128-column prepack): the [K/2,N] lane map with words instead of bytes:
//     a stage of a 128-column block is 8 chunk rows x 512 bytes, contiguous
//     in HBM and in LDS; a lane reads the WNC adjacent words of its columns
//     in chunk 2ks + h (one 16- or 8-byte read) and MFMA j converts word j.
//     The MFMA operands equal the [K/2,N] kernel's exactly.
//   P (panels): the [N,K/2] lane map; a stage of a 32-column panel is one
//     1 KB block already in lane order, so the DMA and the LDS read are both
//     linear (no swizzle) and the MFMA operands equal the [N,K/2] kernel's.
//
// Reference counterpart: the K loop of strategy_j/strategy_m
// (csrc/strategy_j_synthesis.cu:120-170, csrc/strategy_m_asm.cu:131-185),
// which double-buffers a dequantized bf16 tile with a barrier per step.
//
// This header holds the kernel template and its shape dispatch; each weight
// layout is instantiated in its own translation unit
// (mxfp4_tiled_pipe_{kn,nk,g,p}.hip), so the 36 kernels compile in
// parallel, and mxfp4_tiled_pipe.hip holds the entry points.
#pragma once

#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

constexpr int kBK = 64;

__device__ __forceinline__ int a_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

template <int LAYOUT, int WM, int WN, int RB, int WNC>
struct PipeCfg {
  static constexpr int NWAVES = WM * WN;
  static constexpr int NT = NWAVES * 64;
  static constexpr int BM = WM * RB * 32;
  static constexpr int WCOLS = 32 * WNC;  // columns per wave
  static constexpr int BN = WN * WCOLS;
  static constexpr int A_BYTES = BM * 128;
  static constexpr int B_BYTES = BN * 32;
  // E8M0 scales of a stage also go through LDS: [K/2,N]: the stage's two K
  // group rows of BN bytes; [N,K/2]: per column the aligned dword holding its
  // two groups (needs K % 128 == 0).  One 64-lane x 4-byte DMA per wave.
  //   G, P: two groups per column as well, 256 bytes per 128 columns.
  static constexpr int SC_BYTES = LAYOUT == kLayoutNK ? 4 * BN : 2 * BN;
  static constexpr int SC_INSTR = SC_BYTES / 256;
  static constexpr int STAGE = A_BYTES + B_BYTES + SC_BYTES;
  static constexpr int A_INSTR = A_BYTES / 1024;
  static constexpr int B_INSTR = B_BYTES / 1024;
  static_assert(A_INSTR % NWAVES == 0 && B_INSTR % NWAVES == 0, "loads split evenly over waves");
  static constexpr int A_PER_WAVE = A_INSTR / NWAVES;
  static constexpr int B_PER_WAVE = B_INSTR / NWAVES;
  static_assert(SC_INSTR >= 1 && SC_INSTR <= NWAVES, "one scale DMA per wave");
  // LDS DMAs one wave issues per stage (A, B, one scale DMA).
  static constexpr int VM_PER_ITER = A_PER_WAVE + B_PER_WAVE + 1;
  static constexpr int KN_CPR = BN / 16;  // 16-byte chunks per K-pair row
  static_assert(LAYOUT != kLayoutG || (BN % kGCols == 0 && WCOLS <= kGCols), "G: whole 128-column blocks");
};

template <int LAYOUT, int RB, int WNC>
struct SubOps;  // operands of one 16-K sub-step

template <int RB, int WNC>
struct SubOps<kLayoutKN, RB, WNC> {
  bf16x8 a[RB];
  uint32_t raw[WNC == 4 ? 4 : 2];  // WNC=4: row words; WNC=2: packed row pairs (0,1), (2,3)
};

template <int RB, int WNC>
struct SubOps<kLayoutNK, RB, WNC> {
  bf16x8 a[RB];
};

template <int RB, int WNC>
struct SubOps<kLayoutG, RB, WNC> {
  bf16x8 a[RB];
  uint32_t raw[WNC];  // word of column WNC*c + j in chunk 2ks + h
};

template <int RB, int WNC>
struct SubOps<kLayoutP, RB, WNC> {
  bf16x8 a[RB];
};

// Layouts whose lanes follow the [K/2,N] map (WNC adjacent columns per lane)
// or the [N,K/2] map (one column per column block, 32 K per lane).
template <int L>
constexpr bool kColumnWords = L == kLayoutKN || L == kLayoutG;

template <int LAYOUT, int WM, int WN, int RB, int WNC, int NS>
__global__ void __launch_bounds__(WM* WN * 64, 1) tiled_pipe_kernel(TiledArgs p) {
  using Cfg = PipeCfg<LAYOUT, WM, WN, RB, WNC>;
  constexpr int NT = Cfg::NT, BM = Cfg::BM, BN = Cfg::BN, WCOLS = Cfg::WCOLS;
  static_assert(NS >= 3, "the barrier placement needs at least three stages");
  static_assert(WNC == 2 || WNC == 4, "wave column width");
  static_assert(NS * Cfg::STAGE + 256 <= 160 * 1024, "LDS ring exceeds 160 KB");
  // NS stages, then a 256-byte window that the scale DMAs of waves beyond
  // SC_INSTR fill (so every wave issues the same DMA count per stage).
  __shared__ __attribute__((aligned(1024))) uint8_t smem[NS * Cfg::STAGE + 256];
  int* s_last = reinterpret_cast<int*>(smem);  // split-K flag; the ring has drained by then

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int wm = wave / WN, wn = wave % WN;
  const int c = lane & 31, h = lane >> 5;

  const TileCoord tc = tile_of((int)blockIdx.x, p.tiles_m, p.tiles_n, p.splits, p.group_m);
  const int tile = tc.tm * p.tiles_n + tc.tn;
  const int split = tc.split, tm = tc.tm, tn = tc.tn;
  const int m0 = tm * BM, n0 = tn * BN;

  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;
  const int s_begin = split * p.steps_per_split;
  const int T = min(p.ksteps, s_begin + p.steps_per_split) - s_begin;

  // ---- global -> LDS ---------------------------------------------------------
  auto load_stage = [&](int buf, int step, bool live) __attribute__((always_inline)) {
    uint8_t* sA = smem + buf * Cfg::STAGE;
    uint8_t* sB = sA + Cfg::A_BYTES;
    const int k0 = step * kBK;
    const desc_t ra = make_desc(p.A + (size_t)m0 * K + k0);
#pragma unroll
    for (int ii = 0; ii < Cfg::A_PER_WAVE; ++ii) {
      const int i = wave * Cfg::A_PER_WAVE + ii;
      const int row = i * 8 + (lane >> 3);
      const int lc = (lane & 7) ^ a_swz(row);
      const bool ok = live && (m0 + row < M) && (k0 + lc * 8 < K);
      dma16(ra, sA + i * 1024, ok ? (uint32_t)(row * K * 2 + lc * 16) : kOobOffset);
    }
    if constexpr (LAYOUT == kLayoutKN) {
      constexpr int CPR = Cfg::KN_CPR;
      const desc_t rb = make_desc(p.B + (size_t)(k0 >> 1) * N + n0);
#pragma unroll
      for (int ii = 0; ii < Cfg::B_PER_WAVE; ++ii) {
        const int i = wave * Cfg::B_PER_WAVE + ii;
        const int q = i * 64 + lane;
        const int row = q / CPR;
        // rows with bit 2 set store their two row halves swapped
        const int lc = (q % CPR) ^ (((row >> 2) & 1) * (CPR / 2));
        const bool ok = live && ((k0 >> 1) + row < Kh) && (n0 + lc * 16 < N);
        dma16(rb, sB + i * 1024, ok ? (uint32_t)(row * N + lc * 16) : kOobOffset);
      }
    } else if constexpr (LAYOUT == kLayoutNK) {
      const desc_t rb = make_desc(p.B + (size_t)n0 * Kh + (k0 >> 1));
#pragma unroll
      for (int ii = 0; ii < Cfg::B_PER_WAVE; ++ii) {
        const int i = wave * Cfg::B_PER_WAVE + ii;
        const int q = i * 64 + lane;
        const int row = q >> 1;
        const int lc = (q & 1) ^ ((row >> 2) & 1);  // rows with bit 2 set swap their chunks
        const bool ok = live && (n0 + row < N) && ((k0 >> 1) + lc * 16 < Kh);
        dma16(rb, sB + i * 1024, ok ? (uint32_t)(row * Kh + lc * 16) : kOobOffset);
      }
    } else if constexpr (LAYOUT == kLayoutG) {
      // block nbl's stage: chunks k0/8 .. k0/8 + 7 x 128 columns x 4 bytes
      const uint32_t blk = (uint32_t)Kh * kGCols;  // bytes per 128-column block
      const desc_t rb = make_desc(p.B + (size_t)(n0 / kGCols) * blk + (size_t)step * 4096);
#pragma unroll
      for (int ii = 0; ii < Cfg::B_PER_WAVE; ++ii) {
        const int i = wave * Cfg::B_PER_WAVE + ii;
        const int byte = i * 1024 + 16 * lane;
        const int nbl = byte >> 12, w = byte & 4095;
        const bool ok = live && (n0 + nbl * kGCols < N) && (k0 + 8 * (w >> 9) < K);
        dma16(rb, sB + i * 1024, ok ? (uint32_t)(nbl * blk + w) : kOobOffset);
      }
    } else {
      // panel i's stage: one 1 KB block
      const uint32_t pan = (uint32_t)Kh * kPCols;  // bytes per panel
      const desc_t rb = make_desc(p.B + (size_t)(n0 / kPCols) * pan + (size_t)step * 1024);
#pragma unroll
      for (int ii = 0; ii < Cfg::B_PER_WAVE; ++ii) {
        const int i = wave * Cfg::B_PER_WAVE + ii;
        const bool ok = live && (n0 + i * kPCols < N) && (k0 < K);
        dma16(rb, sB + i * 1024, ok ? (uint32_t)(i * pan + 16 * lane) : kOobOffset);
      }
    }
    // scales: wave w < SC_INSTR loads bytes 256w .. 256w+255 of the stage's scale block
    const int g0 = step * 2;
    const bool sc_wave = wave < Cfg::SC_INSTR;
    uint8_t* sC = sB + Cfg::B_BYTES;
    if constexpr (LAYOUT == kLayoutKN) {
      const desc_t rs = make_desc(p.S + (size_t)g0 * N + n0);
      const int byte = 256 * wave + 4 * lane;
      const int row = byte / BN, col = byte % BN;
      const bool ok = live && sc_wave && (g0 + row < G) && (n0 + col < N);
      dma4(rs, sc_wave ? sC + 256 * wave : smem + NS * Cfg::STAGE, ok ? (uint32_t)(row * N + col) : kOobOffset);
    } else if constexpr (LAYOUT == kLayoutNK) {
      const desc_t rs = make_desc(p.S + (size_t)n0 * G + (g0 & ~3));
      const int n = 64 * wave + lane;
      const bool ok = live && sc_wave && (n0 + n < N) && (g0 < G);
      dma4(rs, sc_wave ? sC + 256 * wave : smem + NS * Cfg::STAGE, ok ? (uint32_t)(n * G) : kOobOffset);
    } else if constexpr (LAYOUT == kLayoutG) {
      // wave w: block w's groups g0, g0 + 1 (2 x 128 bytes) -> sC[w][2][128]
      const desc_t rs = make_desc(p.S + ((size_t)(n0 / kGCols) * G + g0) * kGCols);
      const int g = lane >> 5, ni = (4 * lane) & 127;
      const bool ok = live && sc_wave && (n0 + wave * kGCols < N) && (g0 + g < G);
      dma4(rs, sc_wave ? sC + 256 * wave : smem + NS * Cfg::STAGE,
           ok ? (uint32_t)(wave * G * kGCols + g * kGCols + ni) : kOobOffset);
    } else {
      // wave w: the stage's 64-byte blocks of panels 4w .. 4w + 3 -> sC[panel][64]
      const desc_t rs = make_desc(p.S + (size_t)(n0 / kPCols) * (K / kPK) * 64 + (size_t)step * 64);
      const int i = 4 * wave + (lane >> 4);
      const bool ok = live && sc_wave && (n0 + i * kPCols < N) && (k0 < K);
      dma4(rs, sc_wave ? sC + 256 * wave : smem + NS * Cfg::STAGE,
           ok ? (uint32_t)(i * (K / kPK) * 64 + 4 * (lane & 15)) : kOobOffset);
    }
  };

  // ---- per-lane LDS offsets (loop invariant) ---------------------------------
  // A: row wm*RB*32 + 32*rb + c; its swizzle ignores rb (bit 5).
  uint32_t a_off[4];
  {
    const int row = wm * RB * 32 + c;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int lc = kColumnWords<LAYOUT> ? ks * 2 + h : h * 4 + ks;
      a_off[ks] = (uint32_t)(row * 128 + ((lc ^ a_swz(row)) * 16));
    }
  }
  // B: [K/2,N] row ks*8 + 4h + i (its swizzle depends on h only);
  //    [N,K/2] row wn*WCOLS + 32*cb + c (its swizzle depends on c only).
  //    G: block col/128, chunk 2ks + h, word col%128 (col = wn*WCOLS + WNC*c);
  //    P: panel wn*WNC + cb, lane slot 32h + c.
  uint32_t b_off;
  if constexpr (LAYOUT == kLayoutKN) {
    constexpr int CPR = Cfg::KN_CPR;
    const int byte = wn * WCOLS + WNC * c;
    b_off = (uint32_t)(Cfg::A_BYTES + h * 4 * BN + (((byte >> 4) ^ (h * (CPR / 2))) * 16) + (byte & 15));
  } else if constexpr (LAYOUT == kLayoutNK) {
    b_off = (uint32_t)(Cfg::A_BYTES + (wn * WCOLS + c) * 32 + ((h ^ ((c >> 2) & 1)) * 16));
  } else if constexpr (LAYOUT == kLayoutG) {
    const int col = wn * WCOLS + WNC * c;
    b_off = (uint32_t)(Cfg::A_BYTES + (col >> 7) * 4096 + h * 512 + (col & 127) * 4);
  } else {
    b_off = (uint32_t)(Cfg::A_BYTES + wn * WNC * 1024 + (32 * h + c) * 16);
  }

  // ---- LDS -> registers ------------------------------------------------------
  using Ops = SubOps<LAYOUT, RB, WNC>;
  auto read_ops = [&](int buf, int ks, Ops& o) __attribute__((always_inline)) {
    const uint8_t* base = smem + buf * Cfg::STAGE;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
      o.a[rb] = *reinterpret_cast<const bf16x8*>(base + a_off[ks] + rb * 32 * 128);
    if constexpr (LAYOUT == kLayoutKN) {
      const uint8_t* pb = base + b_off + ks * 8 * BN;
      if constexpr (WNC == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) o.raw[i] = *reinterpret_cast<const uint32_t*>(pb + i * BN);
      } else {
        const uint32_t r0 = *reinterpret_cast<const uint16_t*>(pb);
        const uint32_t r1 = *reinterpret_cast<const uint16_t*>(pb + BN);
        const uint32_t r2 = *reinterpret_cast<const uint16_t*>(pb + 2 * BN);
        const uint32_t r3 = *reinterpret_cast<const uint16_t*>(pb + 3 * BN);
        o.raw[0] = r0 | (r1 << 16);
        o.raw[1] = r2 | (r3 << 16);
      }
    } else if constexpr (LAYOUT == kLayoutG) {
      const uint8_t* pb = base + b_off + ks * 1024;
      if constexpr (WNC == 4) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(pb);
#pragma unroll
        for (int j = 0; j < 4; ++j) o.raw[j] = v[j];
      } else {
        const u32x2 v = *reinterpret_cast<const u32x2*>(pb);
        o.raw[0] = v.x;
        o.raw[1] = v.y;
      }
    }
  };
  // [N,K/2], P: the column blocks' 16 bytes for the whole stage (column
  // blocks are 1 KB apart in both LDS images).
  auto read_braw = [&](int buf, u32x4 (&raw)[WNC]) __attribute__((always_inline)) {
    const uint8_t* base = smem + buf * Cfg::STAGE + b_off;
#pragma unroll
    for (int cb = 0; cb < WNC; ++cb) raw[cb] = *reinterpret_cast<const u32x4*>(base + cb * 1024);
  };

  f32x16 acc[RB][WNC];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < WNC; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][j][e] = 0.f;

  // cvt + MFMA for one sub-step; sc = the column scales of its K group.
  auto mma_kn = [&](const Ops& o, const float (&sc)[WNC]) __attribute__((always_inline)) {
    if constexpr (LAYOUT == kLayoutG) {
#pragma unroll
      for (int j = 0; j < WNC; ++j) {
        const bf16x8 b = operand_from_word(o.raw[j], sc[j]);
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) acc[rb][j] = mfma_32x32x16(o.a[rb], b, acc[rb][j]);
      }
    } else if constexpr (LAYOUT != kLayoutKN) {
      (void)o;
      (void)sc;
    } else if constexpr (WNC == 4) {
      const bf16x8 b0 = operand_from_bytes<0>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], sc[0]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][0] = mfma_32x32x16(o.a[rb], b0, acc[rb][0]);
      const bf16x8 b1 = operand_from_bytes<1>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], sc[1]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][1] = mfma_32x32x16(o.a[rb], b1, acc[rb][1]);
      const bf16x8 b2 = operand_from_bytes<2>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], sc[2]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][2] = mfma_32x32x16(o.a[rb], b2, acc[rb][2]);
      const bf16x8 b3 = operand_from_bytes<3>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], sc[3]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][3] = mfma_32x32x16(o.a[rb], b3, acc[rb][3]);
    } else {
      u32x4 v0, v1;
      v0.x = fp4x2_to_bf16x2<0>(o.raw[0], sc[0]);
      v0.y = fp4x2_to_bf16x2<2>(o.raw[0], sc[0]);
      v0.z = fp4x2_to_bf16x2<0>(o.raw[1], sc[0]);
      v0.w = fp4x2_to_bf16x2<2>(o.raw[1], sc[0]);
      const bf16x8 b0 = __builtin_bit_cast(bf16x8, v0);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][0] = mfma_32x32x16(o.a[rb], b0, acc[rb][0]);
      v1.x = fp4x2_to_bf16x2<1>(o.raw[0], sc[1]);
      v1.y = fp4x2_to_bf16x2<3>(o.raw[0], sc[1]);
      v1.z = fp4x2_to_bf16x2<1>(o.raw[1], sc[1]);
      v1.w = fp4x2_to_bf16x2<3>(o.raw[1], sc[1]);
      const bf16x8 b1 = __builtin_bit_cast(bf16x8, v1);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][1] = mfma_32x32x16(o.a[rb], b1, acc[rb][1]);
    }
  };
  auto mma_nk = [&](const Ops& o, const u32x4 (&raw)[WNC], const float (&sf)[WNC], int s) __attribute__((always_inline)) {
#pragma unroll
    for (int cb = 0; cb < WNC; ++cb) {
      const bf16x8 b = operand_from_word(raw[cb][s], sf[cb]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][cb] = mfma_32x32x16(o.a[rb], b, acc[rb][cb]);
    }
  };

  if (T > 0) {
    // Every iteration issues the same DMA sequence (stage t+NS-1; ranges past
    // the split masked to the OOB offset instead of skipped), so one counted
    // wait per iteration publishes the next stage and leaves NS-2 in flight.
#pragma unroll
    for (int st = 0; st < NS - 1; ++st) load_stage(st, s_begin + st, st < T);
    wait_vmcnt0();
    __syncthreads();
    Ops cur, nxt;
    u32x4 braw_cur[WNC], braw_nxt[WNC];
    read_ops(0, 0, cur);
    if constexpr (!kColumnWords<LAYOUT>) read_braw(0, braw_cur);

    for (int t = 0; t < T; ++t) {
      const int buf = t % NS;
      load_stage((t + NS - 1) % NS, s_begin + t + NS - 1, t + NS - 1 < T);
      // this stage's scales (published with its data)
      const uint8_t* sC = smem + buf * Cfg::STAGE + Cfg::A_BYTES + Cfg::B_BYTES;
      float sf[WNC];       // [N,K/2], P: per column block
      float skn[2][WNC];   // [K/2,N], G: per K group, per column of the lane
      if constexpr (LAYOUT == kLayoutNK) {
        const int shift = 8 * (((2 * (s_begin + t)) & 2) + h);
#pragma unroll
        for (int cb = 0; cb < WNC; ++cb)
          sf[cb] = e8m0_to_f32(*reinterpret_cast<const uint32_t*>(sC + 4 * (wn * WCOLS + 32 * cb + c)) >> shift);
      } else if constexpr (LAYOUT == kLayoutP) {
#pragma unroll
        for (int cb = 0; cb < WNC; ++cb) sf[cb] = e8m0_to_f32(sC[(wn * WNC + cb) * 64 + 32 * h + c]);
      } else {
        const int col = wn * WCOLS + WNC * c;
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const uint8_t* row = LAYOUT == kLayoutKN ? sC + g * BN + col
                                                   : sC + (col >> 7) * 256 + g * kGCols + (col & 127);
          const uint32_t w = WNC == 4 ? *reinterpret_cast<const uint32_t*>(row)
                                      : (uint32_t)*reinterpret_cast<const uint16_t*>(row);
#pragma unroll
          for (int j = 0; j < WNC; ++j) skn[g][j] = e8m0_to_f32(w >> (8 * j));
        }
      }
#pragma unroll
      for (int ks = 0; ks < 3; ++ks) {
        read_ops(buf, ks + 1, nxt);
        if constexpr (kColumnWords<LAYOUT>)
          mma_kn(cur, skn[ks >> 1]);
        else
          mma_nk(cur, braw_cur, sf, ks);
        cur = nxt;
      }
      // Publish stage t+1: this wave's DMAs for it were issued NS-2 iterations
      // ago; the ones issued since stay in flight.
      wait_vmcnt<(NS - 2) * Cfg::VM_PER_ITER>();
      __syncthreads();
      // Past the last step this reads a stage of OOB zeros; the values are unused.
      read_ops((t + 1) % NS, 0, nxt);
      if constexpr (!kColumnWords<LAYOUT>) read_braw((t + 1) % NS, braw_nxt);
      if constexpr (kColumnWords<LAYOUT>)
        mma_kn(cur, skn[1]);
      else
        mma_nk(cur, braw_cur, sf, 3);
      cur = nxt;
      if constexpr (!kColumnWords<LAYOUT>) {
#pragma unroll
        for (int cb = 0; cb < WNC; ++cb) braw_cur[cb] = braw_nxt[cb];
      }
    }
    // The masked DMAs of the last iterations still write the ring.
    wait_vmcnt0();
    __syncthreads();
  }

  // ---- split-K fix-up (same protocol as tiled_kernel) -------------------------
  if (p.splits > 1) {
    constexpr int Q = RB * WNC * 4;  // f32x4 quads per thread
    constexpr uint32_t SLOT = (uint32_t)Q * NT * 16;
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(reinterpret_cast<uint8_t*>(p.partials) + (size_t)tile * p.splits * SLOT);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < WNC; ++j)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const f32x4 v = {acc[rb][j][q4 * 4 + 0], acc[rb][j][q4 * 4 + 1], acc[rb][j][q4 * 4 + 2],
                           acc[rb][j][q4 * 4 + 3]};
          store_coherent(rp, split * SLOT + (uint32_t)(((rb * WNC + j) * 4 + q4) * NT + threadIdx.x) * 16, v);
        }
    if (!splitk_arrive_last(p.counters + tile, (uint32_t)p.splits, s_last)) return;
    splitk_sum<RB * WNC * 4>(rp, SLOT, p.splits, NT, [&](int i, f32x4 v) __attribute__((always_inline)) {
      const int rb = i / (WNC * 4), j = (i / 4) % WNC, q4 = i % 4;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[rb][j][q4 * 4 + e] = v[e];
    });
  }

  // ---- epilogue ----------------------------------------------------------------
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
        if constexpr (kColumnWords<LAYOUT>) {
          const int col = n0 + wn * WCOLS + WNC * c;
          if (col >= N) continue;
          float v[WNC];
#pragma unroll
          for (int j = 0; j < WNC; ++j)
            v[j] = kFused ? epilogue_value(p.ep, acc[rb][j][i], row, col + j, N) : acc[rb][j][i];
          if constexpr (WNC == 4) {
            if (bf16) {
              u32x2 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
              *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.C) + (size_t)row * N + col) = w;
            } else {
              *reinterpret_cast<f32x4*>(static_cast<float*>(p.C) + (size_t)row * N + col) = f32x4{v[0], v[1], v[2], v[3]};
            }
          } else {
            if (bf16) {
              *reinterpret_cast<uint32_t*>(static_cast<uint16_t*>(p.C) + (size_t)row * N + col) = pack_bf16x2(v[0], v[1]);
            } else {
              typedef float f32x2 __attribute__((ext_vector_type(2)));
              *reinterpret_cast<f32x2*>(static_cast<float*>(p.C) + (size_t)row * N + col) = f32x2{v[0], v[1]};
            }
          }
        } else {
#pragma unroll
          for (int cb = 0; cb < WNC; ++cb) {
            const int col = n0 + wn * WCOLS + 32 * cb + c;
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

template <int LAYOUT, int WM, int WN, int RB, int WNC, int NS>
hipError_t launch_one(const TiledArgs& a, hipStream_t stream) {
  using Cfg = PipeCfg<LAYOUT, WM, WN, RB, WNC>;
  const int grid = a.tiles_m * a.tiles_n * a.splits;
  hipLaunchKernelGGL((tiled_pipe_kernel<LAYOUT, WM, WN, RB, WNC, NS>), dim3(grid), dim3(Cfg::NT), 0,
                     stream, a);
  return hipGetLastError();
}

// (wm, wn, rb, wnc, stages) instantiated for both layouts.
#define MXFP4_PIPE_SHAPES(X) \
  X(4, 2, 2, 4, 3)           \
  X(2, 4, 4, 2, 3)           \
  X(2, 2, 2, 4, 3)           \
  X(2, 2, 2, 4, 4)           \
  X(2, 4, 2, 2, 4)           \
  X(1, 4, 4, 2, 4)           \
  X(2, 1, 2, 4, 4)

template <int LAYOUT>
hipError_t dispatch_shape(const TiledShape& s, const TiledArgs& a, hipStream_t stream) {
#define X(WM_, WN_, RB_, WNC_, NS_)                                                     \
  if (s.wm == WM_ && s.wn == WN_ && s.rb == RB_ && s.wnc == WNC_ && s.stages == NS_) \
    return launch_one<LAYOUT, WM_, WN_, RB_, WNC_, NS_>(a, stream);
  MXFP4_PIPE_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace

}  // namespace mxfp4
