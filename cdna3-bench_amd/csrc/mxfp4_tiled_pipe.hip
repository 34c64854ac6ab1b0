// Pipelined tiled MFMA kernel (M > 32): the production kernel of the tiled
// family.  Same tile geometry, operand layouts, loaders and split-K protocol
// as tiled_kernel (mxfp4_tiled.hip); the main loop differs:
//
//   * three LDS stages in a ring: while stage t is consumed, stage t+1 is
//     resident and stage t+2 is in flight (16-byte buffer_load ... lds);
//   * LDS operands are read one 16-K sub-step ahead into registers, so the
//     ds_read latency of sub-step s+1 hides under the MFMAs of sub-step s;
//   * one barrier per stage, placed before the last sub-step: it publishes
//     stage t+1 (every wave waited for its own loads with a counted vmcnt)
//     and retires stage t-1's buffer, and the first operands of stage t+1
//     are read while the last MFMAs of stage t drain -- no pipeline bubble at
//     the stage boundary.
//
// Reference counterpart: the K loop of strategy_j/strategy_m
// (csrc/strategy_j_synthesis.cu:120-170, csrc/strategy_m_asm.cu:131-185),
// which double-buffers a dequantized bf16 tile with a barrier per step.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

constexpr int kBK = 64;
constexpr int kStages = 3;

__device__ __forceinline__ int a_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }
template <int CPR>
__device__ __forceinline__ int kn_swz(int row) { return ((row >> 2) & 1) * (CPR / 2); }
__device__ __forceinline__ int nk_swz(int row) { return (row >> 2) & 1; }

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int LAYOUT, int WM, int WN, int RB>
struct PipeCfg {
  static constexpr int NWAVES = WM * WN;
  static constexpr int NT = NWAVES * 64;
  static constexpr int BM = WM * RB * 32;
  static constexpr int BN = WN * 128;
  static constexpr int A_BYTES = BM * 128;
  static constexpr int B_BYTES = BN * 32;
  static constexpr int STAGE = A_BYTES + B_BYTES;
  static constexpr int A_INSTR = A_BYTES / 1024;
  static constexpr int B_INSTR = B_BYTES / 1024;
  static_assert(A_INSTR % NWAVES == 0 && B_INSTR % NWAVES == 0, "loads split evenly over waves");
  static constexpr int A_PER_WAVE = A_INSTR / NWAVES;
  static constexpr int B_PER_WAVE = B_INSTR / NWAVES;
  static constexpr int SC_LOADS = LAYOUT == kLayoutKN ? 2 : 4;
  // VMEM instructions one wave issues per iteration (next-next stage + next scales).
  static constexpr int VM_PER_ITER = A_PER_WAVE + B_PER_WAVE + SC_LOADS;
  static constexpr int KN_CPR = BN / 16;
};

template <int LAYOUT, int RB>
struct SubOps;  // operands of one 16-K sub-step

template <int RB>
struct SubOps<kLayoutKN, RB> {
  bf16x8 a[RB];
  uint32_t raw[4];
};

template <int RB>
struct SubOps<kLayoutNK, RB> {
  bf16x8 a[RB];
};

template <int LAYOUT, int WM, int WN, int RB>
__global__ void __launch_bounds__(WM* WN * 64, 1) tiled_pipe_kernel(TiledArgs p) {
  using Cfg = PipeCfg<LAYOUT, WM, WN, RB>;
  constexpr int NT = Cfg::NT, BM = Cfg::BM, BN = Cfg::BN;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[kStages * Cfg::STAGE];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int wm = wave / WN, wn = wave % WN;
  const int c = lane & 31, h = lane >> 5;

  const int total = p.tiles_m * p.tiles_n * p.splits;
  const int logical = xcd_chunked_id((int)blockIdx.x, total);
  const int tile = logical / p.splits;
  const int split = logical - tile * p.splits;
  const int group_size = p.group_m * p.tiles_n;
  const int group = tile / group_size;
  const int first_m = group * p.group_m;
  const int gm_rows = min(p.tiles_m - first_m, p.group_m);
  const int in_group = tile - group * group_size;
  const int tm = first_m + in_group % gm_rows;
  const int tn = in_group / gm_rows;
  const int m0 = tm * BM, n0 = tn * BN;

  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;
  const int s_begin = split * p.steps_per_split;
  const int T = min(p.ksteps, s_begin + p.steps_per_split) - s_begin;

  // ---- global -> LDS ---------------------------------------------------------
  auto load_stage = [&](int buf, int step) {
    uint8_t* sA = smem + buf * Cfg::STAGE;
    uint8_t* sB = sA + Cfg::A_BYTES;
    const int k0 = step * kBK;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A + (size_t)m0 * K + k0);
#pragma unroll
    for (int ii = 0; ii < Cfg::A_PER_WAVE; ++ii) {
      const int i = wave * Cfg::A_PER_WAVE + ii;
      const int row = i * 8 + (lane >> 3);
      const int lc = (lane & 7) ^ a_swz(row);
      const bool ok = (m0 + row < M) && (k0 + lc * 8 < K);
      buffer_load_lds16(ra, sA + i * 1024, ok ? (uint32_t)(row * K * 2 + lc * 16) : kOobOffset);
    }
    if constexpr (LAYOUT == kLayoutKN) {
      constexpr int CPR = Cfg::KN_CPR;
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + (size_t)(k0 >> 1) * N + n0);
#pragma unroll
      for (int ii = 0; ii < Cfg::B_PER_WAVE; ++ii) {
        const int i = wave * Cfg::B_PER_WAVE + ii;
        const int q = i * 64 + lane;
        const int row = q / CPR;
        const int lc = (q % CPR) ^ kn_swz<CPR>(row);
        const bool ok = ((k0 >> 1) + row < Kh) && (n0 + lc * 16 < N);
        buffer_load_lds16(rb, sB + i * 1024, ok ? (uint32_t)(row * N + lc * 16) : kOobOffset);
      }
    } else {
      const __amdgpu_buffer_rsrc_t rb = make_rsrc(p.B + (size_t)n0 * Kh + (k0 >> 1));
#pragma unroll
      for (int ii = 0; ii < Cfg::B_PER_WAVE; ++ii) {
        const int i = wave * Cfg::B_PER_WAVE + ii;
        const int q = i * 64 + lane;
        const int row = q >> 1;
        const int lc = (q & 1) ^ nk_swz(row);
        const bool ok = (n0 + row < N) && ((k0 >> 1) + lc * 16 < Kh);
        buffer_load_lds16(rb, sB + i * 1024, ok ? (uint32_t)(row * Kh + lc * 16) : kOobOffset);
      }
    }
  };

  // Scales straight from global (L2-resident) one stage ahead.  Exactly
  // SC_LOADS VMEM instructions per call (masked lanes load nothing).
  auto load_scales = [&](uint32_t (&dst)[4], int step) {
    const int g0 = step * 2;
    if constexpr (LAYOUT == kLayoutKN) {
      const int col = n0 + wn * 128 + 4 * c;
      const bool cok = col < N;
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.S + (size_t)g0 * N + n0 + wn * 128);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const bool ok = cok && (g0 + g < G);
        dst[g] = __builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (uint32_t)(g * N + 4 * c) : kOobOffset, 0, 0);
      }
    } else {
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.S + (size_t)(n0 + wn * 128) * G + g0);
#pragma unroll
      for (int cb = 0; cb < 4; ++cb) {
        const int col = n0 + wn * 128 + 32 * cb + c;
        const bool ok = (g0 + h < G) && (col < N);
        dst[cb] = __builtin_amdgcn_raw_buffer_load_b8(
            rs, ok ? (uint32_t)((32 * cb + c) * G + h) : kOobOffset, 0, 0);
      }
    }
  };

  // ---- LDS -> registers ------------------------------------------------------
  using Ops = SubOps<LAYOUT, RB>;
  auto read_ops = [&](int buf, int ks, Ops& o) {
    const uint8_t* sA = smem + buf * Cfg::STAGE;
    const uint8_t* sB = sA + Cfg::A_BYTES;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = wm * RB * 32 + rb * 32 + c;
      const int lc = LAYOUT == kLayoutKN ? ks * 2 + h : h * 4 + ks;
      o.a[rb] = *reinterpret_cast<const bf16x8*>(sA + row * 128 + ((lc ^ a_swz(row)) * 16));
    }
    if constexpr (LAYOUT == kLayoutKN) {
      constexpr int CPR = Cfg::KN_CPR;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = ks * 8 + h * 4 + i;
        const int lc = (wn * 128 + 4 * c) >> 4;
        o.raw[i] = *reinterpret_cast<const uint32_t*>(sB + row * BN + (lc ^ kn_swz<CPR>(row)) * 16 + 4 * (c & 3));
      }
    }
  };
  // [N,K/2]: the 4 column blocks' 16 bytes for the whole stage.
  auto read_braw = [&](int buf, u32x4 (&raw)[4]) {
    const uint8_t* sB = smem + buf * Cfg::STAGE + Cfg::A_BYTES;
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const int row = wn * 128 + cb * 32 + c;
      raw[cb] = *reinterpret_cast<const u32x4*>(sB + row * 32 + ((h ^ nk_swz(row)) * 16));
    }
  };

  f32x16 acc[RB][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][j][e] = 0.f;

  // cvt + MFMA for one sub-step.
  auto mma_kn = [&](const SubOps<kLayoutKN, RB>& o, uint32_t sw) {
    const float s0 = e8m0_to_f32(sw), s1 = e8m0_to_f32(sw >> 8);
    const float s2 = e8m0_to_f32(sw >> 16), s3 = e8m0_to_f32(sw >> 24);
    const bf16x8 b0 = operand_from_bytes<0>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], s0);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb][0] = mfma_32x32x16(o.a[rb], b0, acc[rb][0]);
    const bf16x8 b1 = operand_from_bytes<1>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], s1);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb][1] = mfma_32x32x16(o.a[rb], b1, acc[rb][1]);
    const bf16x8 b2 = operand_from_bytes<2>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], s2);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb][2] = mfma_32x32x16(o.a[rb], b2, acc[rb][2]);
    const bf16x8 b3 = operand_from_bytes<3>(o.raw[0], o.raw[1], o.raw[2], o.raw[3], s3);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb][3] = mfma_32x32x16(o.a[rb], b3, acc[rb][3]);
  };
  auto mma_nk = [&](const SubOps<kLayoutNK, RB>& o, const u32x4 (&raw)[4], const float (&sf)[4], int s) {
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
      const bf16x8 b = operand_from_word(raw[cb][s], sf[cb]);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb][cb] = mfma_32x32x16(o.a[rb], b, acc[rb][cb]);
    }
  };

  if (T > 0) {
    // prologue: stages 0 and 1 in flight, scales of stage 0
    uint32_t sc_cur[4] = {0u, 0u, 0u, 0u}, sc_nxt[4] = {0u, 0u, 0u, 0u};
    load_stage(0, s_begin);
    if (T > 1) load_stage(1, s_begin + 1);
    load_scales(sc_cur, s_begin);
    wait_vmcnt0();
    __syncthreads();
    Ops cur, nxt;
    u32x4 braw_cur[4], braw_nxt[4];
    read_ops(0, 0, cur);
    if constexpr (LAYOUT == kLayoutNK) read_braw(0, braw_cur);

    for (int t = 0; t < T; ++t) {
      const int buf = t % kStages;
      const bool more2 = t + 2 < T, more1 = t + 1 < T;
      if (more2) load_stage((t + 2) % kStages, s_begin + t + 2);
      if (more1) load_scales(sc_nxt, s_begin + t + 1);
      float sf[4];
      if constexpr (LAYOUT == kLayoutNK) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) sf[cb] = e8m0_to_f32(sc_cur[cb]);
      }
#pragma unroll
      for (int ks = 0; ks < 3; ++ks) {
        read_ops(buf, ks + 1, nxt);
        if constexpr (LAYOUT == kLayoutKN)
          mma_kn(cur, sc_cur[ks >> 1]);
        else
          mma_nk(cur, braw_cur, sf, ks);
        cur = nxt;
      }
      // Publish stage t+1: this wave's loads for it were issued one iteration
      // earlier; only this iteration's VMEM may still be in flight.
      if (more2 && more1)
        wait_vmcnt<Cfg::VM_PER_ITER>();
      else
        wait_vmcnt0();
      __syncthreads();
      if (more1) {
        read_ops((t + 1) % kStages, 0, nxt);
        if constexpr (LAYOUT == kLayoutNK) read_braw((t + 1) % kStages, braw_nxt);
      }
      if constexpr (LAYOUT == kLayoutKN)
        mma_kn(cur, sc_cur[1]);
      else
        mma_nk(cur, braw_cur, sf, 3);
      cur = nxt;
      if constexpr (LAYOUT == kLayoutNK) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) braw_cur[cb] = braw_nxt[cb];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) sc_cur[i] = sc_nxt[i];
    }
  }

  // ---- split-K fix-up (as tiled_kernel) --------------------------------------
  if (p.splits > 1) {
    constexpr int Q = RB * 16;
    constexpr uint32_t SLOT = (uint32_t)Q * NT * 16;
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
          store_coherent(rp, split * SLOT + (uint32_t)(((rb * 4 + j) * 4 + q4) * NT + threadIdx.x) * 16, v);
        }
    if (!splitk_arrive_last(p.counters + tile, (uint32_t)p.splits, &s_last)) return;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const uint32_t off = (uint32_t)(((rb * 4 + j) * 4 + q4) * NT + threadIdx.x) * 16;
          f32x4 sum = load_coherent4(rp, off);
          for (int sp = 1; sp < p.splits; ++sp) sum += load_coherent4(rp, sp * SLOT + off);
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[rb][j][q4 * 4 + e] = sum[e];
        }
  }

  // ---- epilogue ----------------------------------------------------------------
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int row = m0 + wm * RB * 32 + rb * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
      if (row >= M) continue;
      if constexpr (LAYOUT == kLayoutKN) {
        const int col = n0 + wn * 128 + 4 * c;
        if (col >= N) continue;
        if (p.out_bf16) {
          u32x2 v = {pack_bf16x2(acc[rb][0][i], acc[rb][1][i]), pack_bf16x2(acc[rb][2][i], acc[rb][3][i])};
          *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.C) + (size_t)row * N + col) = v;
        } else {
          f32x4 v = {acc[rb][0][i], acc[rb][1][i], acc[rb][2][i], acc[rb][3][i]};
          *reinterpret_cast<f32x4*>(static_cast<float*>(p.C) + (size_t)row * N + col) = v;
        }
      } else {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
          const int col = n0 + wn * 128 + 32 * cb + c;
          if (col >= N) continue;
          if (p.out_bf16)
            static_cast<uint16_t*>(p.C)[(size_t)row * N + col] = (uint16_t)bf16_bits_rne(acc[rb][cb][i]);
          else
            static_cast<float*>(p.C)[(size_t)row * N + col] = acc[rb][cb][i];
        }
      }
    }
  }
}

template <int LAYOUT, int WM, int WN, int RB>
hipError_t launch_one(const TiledArgs& a, hipStream_t stream) {
  using Cfg = PipeCfg<LAYOUT, WM, WN, RB>;
  const int grid = a.tiles_m * a.tiles_n * a.splits;
  hipLaunchKernelGGL((tiled_pipe_kernel<LAYOUT, WM, WN, RB>), dim3(grid), dim3(Cfg::NT), 0, stream, a);
  return hipGetLastError();
}

template <int LAYOUT>
hipError_t dispatch_shape(const TiledShape& s, const TiledArgs& a, hipStream_t stream) {
  if (s.wm == 4 && s.wn == 2 && s.rb == 2) return launch_one<LAYOUT, 4, 2, 2>(a, stream);
  if (s.wm == 2 && s.wn == 2 && s.rb == 2) return launch_one<LAYOUT, 2, 2, 2>(a, stream);
  if (s.wm == 2 && s.wn == 2 && s.rb == 4) return launch_one<LAYOUT, 2, 2, 4>(a, stream);
  if (s.wm == 2 && s.wn == 1 && s.rb == 2) return launch_one<LAYOUT, 2, 1, 2>(a, stream);
  return hipErrorInvalidValue;
}

}  // namespace

bool tiled_pipe_shape_available(int layout, const TiledShape& s) {
  (void)layout;
  return (s.wm == 4 && s.wn == 2 && s.rb == 2) || (s.wm == 2 && s.wn == 2 && s.rb == 2) ||
         (s.wm == 2 && s.wn == 2 && s.rb == 4) || (s.wm == 2 && s.wn == 1 && s.rb == 2);
}

hipError_t launch_tiled_pipe(int layout, const TiledShape& shape, const TiledArgs& args,
                             hipStream_t stream) {
  if (layout == kLayoutKN) return dispatch_shape<kLayoutKN>(shape, args, stream);
  if (layout == kLayoutNK) return dispatch_shape<kLayoutNK>(shape, args, stream);
  return hipErrorInvalidValue;
}

}  // namespace mxfp4
