// Memory-bound kernel family for M <= 32 (decode / GEMV-like shapes).
//
// The reference has no kernel for these shapes: every launcher rejects
// M % 64 != 0 (csrc/common.h:80-99, strategy_b_lds_dequant.cu:65).  This
// family streams the 4-bit weights once from HBM with 16-byte loads and runs
// the products on v_mfma_f32_16x16x32_bf16 with the activation rows padded to
// 16 (MT = 1) or 32 (MT = 2): the MFMA work is free next to the HBM time.
//
// Lane l: c = l % 16, q = l / 16.  For the MFMA the A operand is row
// 16*mt + c with 8 K-consecutive values, the B operand is the weight column
// with the same 8 K positions, D lane l holds rows 4q..4q+3 of column c.
//
// [K/2, N] weights (step = 32 K = one scale group): lane loads CB bytes of
//   4 K-pair rows (4q .. 4q+3); byte j of those 4 loads is the B operand of
//   MFMA j, whose 16 lanes c cover columns c*CB + j.  The A operand of every
//   MFMA in the step is the same 16 bytes (K 8q .. 8q+7).
// [N, K/2] weights (step = 128 K): lane loads 16 bytes = 32 K of one column
//   (K group q of the step) for CB column blocks; word s of it against the A
//   chunk K 32q + 8s .. +7.
//
// A CTA of WPC waves covers one column group; waves interleave over the CTA's
// K steps, their partial tiles are summed in LDS in wave order, and with
// split-K the last CTA of a column group sums the split partials in split
// order (deterministic, device-scope counter, no atomics on data).
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

template <int LAYOUT, int MT, int CB, int WPC, int U>
struct GemvCfg {
  static constexpr int NT = WPC * 64;
  static constexpr int COLS = 16 * CB;
  static constexpr int ROWS = 16 * MT;
  static constexpr int TILE = ROWS * COLS;  // floats per CTA partial
  // The wave reduction runs over column chunks so its LDS stays <= 64 KB.
  static constexpr int CHUNKS = (WPC * TILE * 4 + 65535) / 65536;
  static constexpr int CCOLS = COLS / CHUNKS;
  static constexpr int CTILE = ROWS * CCOLS;
};

template <int LAYOUT, int MT, int CB>
struct GemvRegs;

template <int MT, int CB>
struct GemvRegs<kLayoutKN, MT, CB> {
  uint32_t raw[4][CB / 4];  // 4 K-pair rows x CB bytes
  uint32_t sw[CB / 4];      // CB scale bytes
  u32x4 a[MT];              // A operand (8 bf16) per row tile
};

template <int MT, int CB>
struct GemvRegs<kLayoutNK, MT, CB> {
  u32x4 raw[CB];     // 16 bytes (32 K) per column block
  uint32_t sb[CB];   // one scale byte per column block
  u32x4 a[MT][4];    // A operand per row tile and word s
};

template <int N_>
// Weight and scale words are read once per launch: non-temporal loads.
__device__ __forceinline__ void load_words(uint32_t (&dst)[N_], const uint8_t* src, bool ok) {
  if constexpr (N_ == 4) {
    u32x4 v = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src)) : u32x4{0u, 0u, 0u, 0u};
    dst[0] = v.x; dst[1] = v.y; dst[2] = v.z; dst[3] = v.w;
  } else if constexpr (N_ == 2) {
    u32x2 v = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src)) : u32x2{0u, 0u};
    dst[0] = v.x; dst[1] = v.y;
  } else {
    dst[0] = ok ? __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src)) : 0u;
  }
}

template <int LAYOUT, int MT, int CB, int WPC, int U>
__global__ void __launch_bounds__(WPC * 64, 1) gemv_kernel(GemvArgs p) {
  using Cfg = GemvCfg<LAYOUT, MT, CB, WPC, U>;
  constexpr int NT = Cfg::NT, COLS = Cfg::COLS, TILE = Cfg::TILE;
  constexpr int CHUNKS = Cfg::CHUNKS, CCOLS = Cfg::CCOLS, CTILE = Cfg::CTILE;
  __shared__ __attribute__((aligned(16))) float red[WPC * CTILE];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform (SGPR)
  const int c = lane & 15, q = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;

  const int total = p.col_groups * p.splits;
  const int logical = xcd_chunked_id((int)blockIdx.x, total);
  const int cg = logical / p.splits;
  const int split = logical - cg * p.splits;
  const int n0 = cg * COLS;
  const int s_begin = split * p.steps_per_split;
  const int s_end = min(p.steps, s_begin + p.steps_per_split);
  // Each wave owns a contiguous run of the CTA's K steps.
  const int per_wave = (s_end - s_begin + WPC - 1) / WPC;
  const int w_begin = s_begin + wave * per_wave;
  const int w_end = min(s_end, w_begin + per_wave);

  f32x4 acc[MT][CB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < CB; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  using Regs = GemvRegs<LAYOUT, MT, CB>;

  auto load = [&](Regs& r, int st, bool live) __attribute__((always_inline)) {
    if constexpr (LAYOUT == kLayoutKN) {
      const int col = n0 + c * CB;
      const bool cok = live && col < N;
      const uint8_t* bp = p.B + (size_t)(st * 16 + 4 * q) * N + col;
#pragma unroll
      for (int i = 0; i < 4; ++i) load_words(r.raw[i], bp + (size_t)i * N, cok);
      load_words(r.sw, p.S + (size_t)st * N + col, cok);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + c;
        r.a[mt] = (live && m < M) ? *reinterpret_cast<const u32x4*>(p.A + (size_t)m * K + st * 32 + 8 * q)
                                  : u32x4{0u, 0u, 0u, 0u};
      }
    } else {
      const int k0 = st * 128 + 32 * q;  // this lane's K group
      const bool kok = live && k0 < K;
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int col = n0 + cb * 16 + c;
        const bool ok = kok && col < N;
        r.raw[cb] = ok ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.B + (size_t)col * Kh + (k0 >> 1)))
                       : u32x4{0u, 0u, 0u, 0u};
        r.sb[cb] = ok ? (uint32_t)__builtin_nontemporal_load(p.S + (size_t)col * G + (k0 >> 5)) : 0u;
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = mt * 16 + c;
        const bool ok = kok && m < M;
        const uint16_t* ap = p.A + (size_t)m * K + k0;
#pragma unroll
        for (int s = 0; s < 4; ++s)
          r.a[mt][s] = ok ? *reinterpret_cast<const u32x4*>(ap + 8 * s) : u32x4{0u, 0u, 0u, 0u};
      }
    }
  };

  auto compute = [&](const Regs& r) __attribute__((always_inline)) {
    if constexpr (LAYOUT == kLayoutKN) {
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const float sc = e8m0_to_f32(r.sw[j >> 2] >> (8 * (j & 3)));
        const int w = j >> 2;
        bf16x8 b;
        switch (j & 3) {
          case 0: b = operand_from_bytes<0>(r.raw[0][w], r.raw[1][w], r.raw[2][w], r.raw[3][w], sc); break;
          case 1: b = operand_from_bytes<1>(r.raw[0][w], r.raw[1][w], r.raw[2][w], r.raw[3][w], sc); break;
          case 2: b = operand_from_bytes<2>(r.raw[0][w], r.raw[1][w], r.raw[2][w], r.raw[3][w], sc); break;
          default: b = operand_from_bytes<3>(r.raw[0][w], r.raw[1][w], r.raw[2][w], r.raw[3][w], sc); break;
        }
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt][j] = mfma_16x16x32(__builtin_bit_cast(bf16x8, r.a[mt]), b, acc[mt][j]);
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const bf16x8 b = operand_from_word(r.raw[cb][s], e8m0_to_f32(r.sb[cb]));
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            acc[mt][cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, r.a[mt][s]), b, acc[mt][cb]);
        }
      }
    }
  };

  // U steps of loads in flight before any compute.
  for (int st = w_begin; st < w_end; st += U) {
    Regs r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) load(r[u], st + u, st + u < w_end);
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (st + u < w_end) compute(r[u]);
  }

  // ---- CTA reduction over waves (LDS, wave order), CHUNKS column chunks ----
  constexpr int PER = (CTILE + NT - 1) / NT;  // elements per thread per chunk
  float v[CHUNKS][PER];
#pragma unroll
  for (int ch = 0; ch < CHUNKS; ++ch) {
    float* my = red + wave * CTILE;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < CB; ++j) {
        const int col = (LAYOUT == kLayoutKN) ? c * CB + j : j * 16 + c;
        if (col / CCOLS != ch) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) my[(mt * 16 + 4 * q + i) * CCOLS + col % CCOLS] = acc[mt][j][i];
      }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < PER; ++e) {
      const int idx = e * NT + threadIdx.x;
      float sum = 0.f;
      if (CTILE % NT == 0 || idx < CTILE) {
        sum = red[idx];
#pragma unroll
        for (int w = 1; w < WPC; ++w) sum += red[w * CTILE + idx];
      }
      v[ch][e] = sum;
    }
    __syncthreads();
  }

  // element (ch, e) <-> tile row / column
  auto row_of = [&](int e) __attribute__((always_inline)) { return (e * NT + (int)threadIdx.x) / CCOLS; };
  auto col_of = [&](int ch, int e) __attribute__((always_inline)) { return ch * CCOLS + (e * NT + (int)threadIdx.x) % CCOLS; };
  auto live = [&](int e) __attribute__((always_inline)) { return (CTILE % NT == 0 || e * NT + (int)threadIdx.x < CTILE); };

  if (p.splits > 1) {
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(p.partials + (size_t)cg * p.splits * TILE);
#pragma unroll
    for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
      for (int e = 0; e < PER; ++e)
        if (live(e) && row_of(e) < M)
          store_coherent(rp, (uint32_t)((split * TILE + row_of(e) * COLS + col_of(ch, e)) * 4), v[ch][e]);
    if (!splitk_arrive_last(p.counters + cg, (uint32_t)p.splits, &s_last)) return;
    // the splits in split order, every element of one split in flight at once
    // (a per-element loop waited for each load: splits x elements round trips)
    for (int sp = 0; sp < p.splits; ++sp) {
      float t[CHUNKS][PER];
#pragma unroll
      for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
        for (int e = 0; e < PER; ++e)
          t[ch][e] = live(e) && row_of(e) < M
                         ? load_coherent1(rp, (uint32_t)((sp * TILE + row_of(e) * COLS + col_of(ch, e)) * 4))
                         : 0.f;
#pragma unroll
      for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
        for (int e = 0; e < PER; ++e) v[ch][e] = sp == 0 ? t[ch][e] : v[ch][e] + t[ch][e];
    }
  }

  // plain and fused stores are separate loops, chosen once (see StoreKind)
  auto store = [&](auto fused, auto out) __attribute__((always_inline)) {
    constexpr bool kFused = decltype(fused)::value;
    const bool bf16 = decltype(out)::value == 2 ? p.out_bf16 != 0 : decltype(out)::value == 1;
#pragma unroll
    for (int ch = 0; ch < CHUNKS; ++ch)
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int row = row_of(e), col = n0 + col_of(ch, e);
        if (live(e) && row < M && col < N) {
          const float x = kFused ? epilogue_value(p.ep, v[ch][e], row, col, N) : v[ch][e];
          if (bf16)
            static_cast<uint16_t*>(p.C)[(size_t)row * N + col] = (uint16_t)bf16_bits_rne(x);
          else
            static_cast<float*>(p.C)[(size_t)row * N + col] = x;
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

template <int LAYOUT, int MT, int CB, int WPC, int U>
hipError_t launch_one(const GemvArgs& a, hipStream_t stream) {
  using Cfg = GemvCfg<LAYOUT, MT, CB, WPC, U>;
  static_assert(Cfg::COLS % Cfg::CHUNKS == 0, "column chunks must divide the tile");
  const int grid = a.col_groups * a.splits;
  hipLaunchKernelGGL((gemv_kernel<LAYOUT, MT, CB, WPC, U>), dim3(grid), dim3(Cfg::NT), 0, stream, a);
  return hipGetLastError();
}

// (MT, CB, WPC, U); index = plan variant.  [K/2,N] needs CB >= 4.
#define MXFP4_GEMV_SHAPES(X) \
  X(1, 8, 8, 4)              \
  X(1, 16, 8, 2)             \
  X(1, 8, 16, 2)             \
  X(1, 4, 16, 4)             \
  X(2, 8, 8, 2)              \
  X(2, 4, 16, 2)             \
  X(1, 2, 16, 4)             \
  X(2, 2, 16, 2)             \
  X(1, 4, 8, 4)              \
  X(1, 2, 8, 4)              \
  X(2, 4, 8, 2)              \
  X(1, 8, 4, 4)              \
  X(1, 2, 16, 2)             \
  X(1, 4, 16, 2)             \
  X(1, 8, 8, 2)

template <int LAYOUT>
hipError_t dispatch(const GemvShape& s, const GemvArgs& a, hipStream_t stream) {
#define X(MT_, CB_, WPC_, U_)                                   \
  if constexpr (LAYOUT == kLayoutNK || CB_ >= 4) {              \
    if (s.mt == MT_ && s.cb == CB_ && s.wpc == WPC_ && s.u == U_) \
      return launch_one<LAYOUT, MT_, CB_, WPC_, U_>(a, stream); \
  }
  MXFP4_GEMV_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace

bool gemv_shape_available(int layout, const GemvShape& s) {
  if (layout == kLayoutKN && s.cb == 2) return false;  // [K/2,N] needs >= 4 bytes per lane row
#define X(MT_, CB_, WPC_, U_) \
  if (s.mt == MT_ && s.cb == CB_ && s.wpc == WPC_ && s.u == U_) return true;
  MXFP4_GEMV_SHAPES(X)
#undef X
  return false;
}

hipError_t launch_gemv(int layout, const GemvShape& shape, const GemvArgs& args,
                       hipStream_t stream) {
  if (!gemv_shape_available(layout, shape)) return hipErrorInvalidValue;
  if (layout == kLayoutKN) return dispatch<kLayoutKN>(shape, args, stream);
  if (layout == kLayoutNK) return dispatch<kLayoutNK>(shape, args, stream);
  return hipErrorInvalidValue;
}

}  // namespace mxfp4
