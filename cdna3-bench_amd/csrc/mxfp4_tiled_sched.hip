// Hand-scheduled tiled MFMA kernel (M > 32; [K/2,N] or G weights with
// K % 64 == 0, [N,K/2] weights with K % 128 == 0): 128 x 256 x 64 tiles, 4
// waves of 64 x 128, two CTAs per CU.  The production kernel of the tiled
// family for these layouts; they differ only in the B / scale loaders, the B
// operand reads and the converts.
//
// Why it is built this way (measured on MI355X, dit_up 4096 x 12288 x 3072):
//  * v_mfma_f32_16x16x32_bf16 sustains 1.68 PF/s (one wave per SIMD) and
//    1.91 PF/s (two) on random bf16 operands, against 1.45 / 1.72 PF/s for
//    v_mfma_f32_32x32x16_bf16: the 16x16x32 form is the faster one on data
//    that toggles (both reach ~2.2-2.35 PF/s on constant operands).
//  * Two waves per SIMD from two independent CTAs: one CTA's barrier, LDS
//    latency and DMA issue overlap the other CTA's MFMAs (one 4-wave CTA per
//    CU spent ~40 % of every stage in such bubbles).
//  * The compiler's schedule issues LDS operand reads one or two MFMAs before
//    their use.  Here every LDS read, convert, MFMA, LDS DMA, wait and
//    barrier in the main loop is its own volatile asm statement, so their
//    order is exactly the program order and the compiler only allocates
//    registers; the waits are counted by hand (it cannot see the asm loads).
//
// Stage t (64 K) = sub-steps (t,0) and (t,1) of 32 K, 32 MFMAs each:
//   (t,0): LDS reads of (t,1)'s raw B words and A operands; 32 MFMAs with one
//          convert after each (see below); lgkmcnt waits.
//   (t,1): s_waitcnt vmcnt (this wave's DMAs of stage t+1) + s_barrier, which
//          publishes stage t+1 and retires stage t's ring slot (every read of
//          stage t was issued and waited for in (t,0)); LDS reads of
//          (t+1,0)'s operands and stage t+1's scales; the LDS DMAs of stage
//          t+3 into the retired slot, spread over the MFMAs; 32 MFMAs with
//          converts.
//   Three ring slots hold stages t+1 (published), t+2 (in flight) and t+3
//   (issued): a stage's loads get two stages of lead before their barrier.
// Converts: MFMA block cb = 0..7 of a sub-step (4 MFMAs, one per 16-row
// block) is followed by the four converts of B operand cb-2 of the NEXT
// sub-step (its register's last reader was block cb-2); blocks 0, 1 convert
// this sub-step's operands 6, 7.  Raw words are therefore read one sub-step
// ahead into a double buffer, A operands likewise.
//
// Stage in LDS ([K/2,N]: 24.25 KB, [N,K/2]: 25 KB):
//   A  [128 rows][128 B]; 16-byte chunk c of row r at c ^ (r & 7) ^ ((r >> 3) & 1)
//   B  [K/2,N]: [32 K-pair rows][256 B]; 16-byte chunk c of row R at
//      c ^ 4 * ((R >> 2) & 3)
//      [N,K/2]: the 16-byte halves (K 0..31, 32..63 of the stage) of the 256
//      columns; column 128w + 64g + 4c + j (c = 0..15) half h at byte
//      4096w + 2048g + 512j + 32c + 16(h ^ (c >> 3)) -- each DMA moves 32 whole
//      32-byte column segments, and the 16 columns of one operand read (fixed
//      g, j, h) fill the 16 16-byte bank slots
//      G: the tile's two 128-column blocks as stored, [block][8 chunks of 8 K]
//      [128 columns][4 B] (each DMA is 1 KB of contiguous HBM); the words of
//      columns 4c .. 4c+3 are one 16-byte read
//   S  [K/2,N] and G: [2 K groups][256 B] E8M0 scales of the stage's columns
//      [N,K/2]: [256 columns][4 B]: the column's scale dword of the stage pair
//      (K groups 4u .. 4u+3 for stages 2u, 2u+1); a stage uses bytes
//      2 (stage % 2) + 0, 1
// MFMA v_mfma_f32_16x16x32_bf16: lane l holds A row l % 16, K 8(l / 16) .. +7
// of the 32-K sub-step, and B column 4c + j of a 64-column group (c = l % 16,
// MFMA j of the group): [K/2,N] byte j of the four K-pair rows 4(l / 16) ..
// +3, [N,K/2] word l / 16 of the column's half, G the column's word of chunk
// 4 sub + l / 16; the result holds rows 4(l / 16) .. +3 of that column.
//
// Reference counterpart: the K loop of strategy_j / strategy_m
// (csrc/strategy_j_synthesis.cu:120-170, csrc/strategy_m_asm.cu:131-185).
#include <type_traits>

#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

constexpr int kBM = 128, kBN = 256, kBK = 64;
constexpr int kWaves = 4;                       // 2 x 2 (M x N)
constexpr int kThreads = kWaves * 64;
constexpr int kRB = 4, kCB = 8;                 // 16-row x 16-column MFMA blocks per wave (64 x 128)
constexpr int kABytes = kBM * kBK * 2;          // 16 KB
constexpr int kBBytes = kBN * kBK / 2;          // 8 KB
constexpr int kNS = 3;                          // LDS ring depth
constexpr int kADma = kABytes / 1024 / kWaves;  // 4 per wave per stage
constexpr int kBDma = kBBytes / 1024 / kWaves;  // 2
constexpr int kVmPerStage = kADma + kBDma + 1;  // + one scale DMA
static_assert(2 * kVmPerStage < 64, "vmcnt range");

// Per-layout LDS sizes: [K/2,N] and G stages hold 2 x 256 scale bytes (two
// of the four waves move them; the other two DMA into a spare 256-byte
// window), [N,K/2] stages 256 scale dwords (one DMA per wave).
template <int L>
struct SchedLds {
  static constexpr int kSBytes = L == kLayoutNK ? 4 * kBN : 2 * kBN;
  static constexpr int kStage = kABytes + kBBytes + kSBytes;
  static constexpr int kLds = kNS * kStage + (L == kLayoutNK ? 0 : 256);
  static_assert(kStage % 256 == 0, "slot offsets are ds_read2st64 immediates");
  static_assert(2 * kLds <= 160 * 1024, "two CTAs per CU");
};

__device__ __forceinline__ int a_swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

// ---- one instruction each; volatile keeps them in program order ------------
template <int OFF>
__device__ __forceinline__ bf16x8 lds_b128(uint32_t addr) {
  bf16x8 v;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(addr), "i"(OFF));
  return v;
}
template <int O0, int O1>
__device__ __forceinline__ u32x2 lds_2st64(uint32_t addr) {
  u32x2 v;
  asm volatile("ds_read2st64_b32 %0, %1 offset0:%2 offset1:%3" : "=v"(v) : "v"(addr), "i"(O0), "i"(O1));
  return v;
}
// Byte SEL of w (two E2M1 codes) -> two bf16 scaled by s (the E8M0 byte in
// the fp32 exponent field).
template <int SEL>
__device__ __forceinline__ uint32_t cvt_fp4(uint32_t w, float s) {
  uint32_t r;
  if constexpr (SEL == 0)
    asm volatile("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2" : "=v"(r) : "v"(w), "v"(s));
  else if constexpr (SEL == 1)
    asm volatile("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2 op_sel:[1,0,0]" : "=v"(r) : "v"(w), "v"(s));
  else if constexpr (SEL == 2)
    asm volatile("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2 op_sel:[0,1,0]" : "=v"(r) : "v"(w), "v"(s));
  else
    asm volatile("v_cvt_scalef32_pk_bf16_fp4 %0, %1, %2 op_sel:[1,1,0]" : "=v"(r) : "v"(w), "v"(s));
  return r;
}
__device__ __forceinline__ void mfma16(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
template <int N>
__device__ __forceinline__ void lgkm_wait() {
  asm volatile("s_waitcnt lgkmcnt(%0)" ::"i"(N));
}
// The same wait, redefining w and x: compiler-scheduled code that reads them
// (asm LDS reads' results) cannot move above it.
template <int N, typename T>
__device__ __forceinline__ void lgkm_wait(T& w, T& x) {
  asm volatile("s_waitcnt lgkmcnt(%2)" : "+v"(w), "+v"(x) : "i"(N));
}
template <int N>
__device__ __forceinline__ void vm_wait() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N));
}
__device__ __forceinline__ void barrier_asm() { asm volatile("s_barrier"); }
// 16 (4) bytes per lane, global (desc + voffset + soffset) -> LDS m0 + 16 (4) * lane.
// soff is wave-uniform; readfirstlane keeps it in an SGPR when the compiler
// cannot prove that.  The compiler may then write that SGPR with a VALU
// instruction (v_readfirstlane) right before the asm, and its hazard checks
// do not look inside inline asm: a VMEM instruction reading an SGPR that a
// VALU instruction wrote needs 5 wait states, hence the s_nop.
__device__ __forceinline__ void dma16s(const desc_t& d, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 4\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(d),
               "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4s(const desc_t& d, uint32_t lds, uint32_t voff, uint32_t soff) {
  asm volatile("s_nop 4\n\tbuffer_load_dword %0, %1, %2 offen lds" ::"v"(voff), "s"(d),
               "s"(__builtin_amdgcn_readfirstlane(soff)), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ float e8m0_byte(uint32_t w, int j) {
  return __builtin_bit_cast(float, ((w >> (8 * j)) & 0xFFu) << 23);
}

// kOut: 0 plain fp32 C, 1 plain bf16 C, 2 fused epilogue (either C type) with
// activation kAct (MXFP4_ACT_*).  One instantiation per store kind: with all
// three store loops in one kernel the register allocator spills accumulators
// before the branch, so even the plain stores went through scratch; and a
// fused loop with the activation chosen per element inlined all three
// activations 128 times (dit_up with bias + SiLU took 373 us against 240 us).
template <int L, int kOut, int kAct>
__global__ void __launch_bounds__(kThreads, 2) tiled_sched_kernel(TiledArgs p) {
  static_assert(L == kLayoutKN || L == kLayoutNK || L == kLayoutG, "layout");
  constexpr bool kKN = L == kLayoutKN, kG = L == kLayoutG;
  constexpr bool kScRows = !(L == kLayoutNK);  // scales in LDS as [2 K groups][256 columns]
  constexpr int kStage = SchedLds<L>::kStage;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[SchedLds<L>::kLds];
  const uint32_t lds0 = (uint32_t)(uintptr_t)smem;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int c = lane & 15, q = lane >> 4;

  const TileCoord tc = tile_of((int)blockIdx.x, p.tiles_m, p.tiles_n, p.splits, p.group_m);
  const int tile = tc.tm * p.tiles_n + tc.tn;
  const int split = tc.split, tm = tc.tm, tn = tc.tn;
  const int m0 = tm * kBM, n0 = tn * kBN;

  const int M = p.M, N = p.N, K = p.K;
  const int s_begin = split * p.steps_per_split;
  const int T = min(p.ksteps, s_begin + p.steps_per_split) - s_begin;

  // ---- loop-invariant DMA offsets (the K step goes in soffset) ---------------
  const desc_t dA = make_desc(p.A + (size_t)m0 * K);
  const int G = K / 32;
  // G: the tile's two 128-column blocks start at byte n0 * K/2 (codes) and
  // n0 * K/32 (scales), like [N,K/2]
  const desc_t dB = make_desc(kKN ? p.B + n0 : p.B + (size_t)n0 * (K / 2));
  const desc_t dS = make_desc(kKN ? p.S + n0 : p.S + (size_t)n0 * G);
  const desc_t dNull = make_desc(p.A, 0u);  // every lane out of range: writes zeros
  uint32_t va[kADma];                       // A: DMA i covers rows 8i .. 8i+7
#pragma unroll
  for (int ii = 0; ii < kADma; ++ii) {
    const int i = wave * kADma + ii;
    const int row = i * 8 + (lane >> 3);
    const int lc = (lane & 7) ^ a_swz(row);
    va[ii] = m0 + row < M ? (uint32_t)(row * K * 2 + lc * 16) : kOobOffset;
  }
  uint32_t vb[kBDma];
#pragma unroll
  for (int ii = 0; ii < kBDma; ++ii) {
    const int d = wave * kBDma + ii;
    if constexpr (kKN) {
      // DMA d covers K-pair rows 4d .. 4d+3
      const int qq = d * 64 + lane;
      const int row = qq >> 4;
      const int lc = (qq & 15) ^ (4 * ((row >> 2) & 3));
      vb[ii] = n0 + lc * 16 < N ? (uint32_t)(row * N + lc * 16) : kOobOffset;
    } else if constexpr (kG) {
      // DMA d covers 8-K chunks 2(d % 4), +1 of block d / 4: 1 KB contiguous,
      // landing as [block][8 chunks][128 columns][4 B]
      const int blk = d >> 2;
      vb[ii] = n0 + 128 * blk < N ? (uint32_t)((blk * (K / 8) + 2 * (d & 3)) * 512 + 16 * lane) : kOobOffset;
    } else {
      // DMA d = 4w + 2g + j/2 covers columns 128w + 64g + 4c + j (c = 0..15,
      // j = 2 (d % 2) + cl / 16) of lane pair cl = lane / 2; lane bit h' is
      // half h' ^ (c >> 3) of its column
      const int cl = lane >> 1, cc = cl & 15;
      const int col = 128 * (d >> 2) + 64 * ((d >> 1) & 1) + 4 * cc + 2 * (d & 1) + (cl >> 4);
      const int half = (lane & 1) ^ (cc >> 3);
      vb[ii] = n0 + col < N ? (uint32_t)(col * (K / 2) + 16 * half) : kOobOffset;
    }
  }
  // scales, [K/2,N]: waves 0, 1 move K group rows 0, 1 of the stage (256
  // columns each); waves 2, 3 issue the same DMA into a spare window so every
  // wave counts the same number of loads per stage.  [N,K/2]: wave w moves
  // the stage pair's dword of columns 64w .. 64w+63.
  // G: wave kg < 2 moves K group kg of both blocks (lane / 32 = block), into
  // the [K/2,N] arrangement.
  const bool sc_wave = !kScRows || wave < 2;
  uint32_t vs;
  if constexpr (kKN) {
    vs = sc_wave && n0 + 4 * lane < N ? (uint32_t)(wave * N + 4 * lane) : kOobOffset;
  } else if constexpr (kG) {
    const int blk = lane >> 5;
    vs = sc_wave && n0 + 128 * blk < N ? (uint32_t)((blk * G + wave) * 128 + 4 * (lane & 31)) : kOobOffset;
  } else {
    vs = n0 + 64 * wave + lane < N ? (uint32_t)((64 * wave + lane) * G) : kOobOffset;
  }
  const uint32_t sc_lds = sc_wave ? (uint32_t)(kABytes + kBBytes + 256 * wave) : 0u;

  auto issue_a = [&](int ii, int slot, int step, bool live) __attribute__((always_inline)) {
    dma16s(live ? dA : dNull, lds0 + slot * kStage + (wave * kADma + ii) * 1024, va[ii],
           (uint32_t)step * (kBK * 2));
  };
  auto issue_b = [&](int ii, int slot, int step, bool live) __attribute__((always_inline)) {
    dma16s(live ? dB : dNull, lds0 + slot * kStage + kABytes + (wave * kBDma + ii) * 1024, vb[ii],
           kKN ? (uint32_t)step * (kBK / 2) * (uint32_t)N
               : kG ? (uint32_t)step * 4096u : (uint32_t)step * (kBK / 2));
  };
  auto issue_s = [&](int slot, int step, bool live) __attribute__((always_inline)) {
    dma4s(live ? dS : dNull, sc_wave ? lds0 + slot * kStage + sc_lds : lds0 + kNS * kStage, vs,
          kKN ? (uint32_t)step * 2u * (uint32_t)N
              : kG ? (uint32_t)step * 256u : (uint32_t)(step >> 1) * 4u);
  };
  // DMA number d (0 .. kVmPerStage-1) of a stage
  auto issue_dma = [&](int d, int slot, int step, bool live) __attribute__((always_inline)) {
    if (d < kADma)
      issue_a(d, slot, step, live);
    else if (d < kADma + kBDma)
      issue_b(d - kADma, slot, step, live);
    else
      issue_s(slot, step, live);
  };

  // ---- loop-invariant LDS read offsets ---------------------------------------
  uint32_t a_off[2];  // per sub-step; 16-row blocks are +2048 (immediate)
  {
    const int row = wm * 64 + c;
#pragma unroll
    for (int sub = 0; sub < 2; ++sub) a_off[sub] = lds0 + (uint32_t)(row * 128 + (((sub * 4 + q) ^ a_swz(row)) * 16));
  }
  // B, [K/2,N]: K-pair row sub*16 + 4q + i, column byte wn*128 + 64g + 4c
  // (b_off[g]; the row swizzle depends on q only).  [N,K/2]: word q of half
  // `sub` of column wn*128 + 64g + 4c + j (b_off[sub]; g, j are immediates).
  uint32_t b_off[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if constexpr (kKN) {
      const int colb = wn * 128 + 64 * i + 4 * c;
      b_off[i] = lds0 + (uint32_t)(kABytes + 4 * q * kBN + (((colb >> 4) ^ (4 * q)) * 16) + (colb & 15));
    } else if constexpr (kG) {
      // chunk 4 sub + q of block wn, columns 4c .. 4c+3 (+ 64 g: immediate)
      b_off[i] = lds0 + (uint32_t)(kABytes + 4096 * wn + 512 * (4 * i + q) + 16 * c);
    } else {
      b_off[i] = lds0 + (uint32_t)(kABytes + 4096 * wn + 32 * c + 16 * (i ^ (c >> 3)) + 4 * q);
    }
  }
  // scales: [K/2,N] bytes of columns wn*128 + 4c .. +3 (+ 64 g), [N,K/2] their
  // dwords
  const uint32_t s_off = kScRows ? lds0 + (uint32_t)(kABytes + kBBytes + wn * 128 + 4 * c)
                                 : lds0 + (uint32_t)(kABytes + kBBytes + wn * 512 + 16 * c);
  using ScaleWords = std::conditional_t<kScRows, u32x2, u32x4>;

  f32x4 acc[kRB][kCB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) acc[rb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (T > 0) {
    bf16x8 a[2][kRB];    // A operands, double-buffered by sub-step
    uint32_t raw[2][8];  // raw B words (group g, row i at 4g + i), double-buffered
    bf16x8 b[kCB];       // converted B operands, block cb = 4g + j
    float sc[2][kCB];    // scales per K group of the stage and block

    // LDS reads of ring slot SL (a compile-time constant: every address is a
    // loop-invariant register plus an immediate offset; kStage is a multiple
    // of 256 B).  Raw word 4g + i: [K/2,N] K-pair row 4q + i of columns
    // 4c .. +3, [N,K/2] column 4c + i (both of group g).
    auto read_raw = [&](auto slot_c, int sub, uint32_t (&r)[8]) __attribute__((always_inline)) {
      constexpr int O = decltype(slot_c)::value * (kStage / 256);
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        u32x2 x, y;
        if constexpr (kG) {
          // chunk 4 sub + q (b_off[sub]): the words of columns 4c + j, j =
          // 0..3, are 16 contiguous bytes; group g is 256 B further
          const uint32_t base = b_off[sub];
          const u32x4 v = __builtin_bit_cast(u32x4, g == 0 ? lds_b128<O * 256>(base) : lds_b128<O * 256 + 256>(base));
          r[4 * g + 0] = v.x; r[4 * g + 1] = v.y; r[4 * g + 2] = v.z; r[4 * g + 3] = v.w;
          continue;
        } else if constexpr (kKN) {
          if (sub == 0) {
            x = lds_2st64<O + 0, O + 1>(b_off[g]);
            y = lds_2st64<O + 2, O + 3>(b_off[g]);
          } else {
            x = lds_2st64<O + 16, O + 17>(b_off[g]);
            y = lds_2st64<O + 18, O + 19>(b_off[g]);
          }
        } else {
          // columns j are 512 B apart, groups 2048 B
          const uint32_t base = b_off[sub];
          if (g == 0) {
            x = lds_2st64<O + 0, O + 2>(base);
            y = lds_2st64<O + 4, O + 6>(base);
          } else {
            x = lds_2st64<O + 8, O + 10>(base);
            y = lds_2st64<O + 12, O + 14>(base);
          }
        }
        r[4 * g + 0] = x.x; r[4 * g + 1] = x.y; r[4 * g + 2] = y.x; r[4 * g + 3] = y.y;
      }
    };
    auto read_a = [&](auto slot_c, int sub, bf16x8 (&o)[kRB]) __attribute__((always_inline)) {
      constexpr int O = decltype(slot_c)::value * kStage;
      const uint32_t addr = a_off[sub];
      o[0] = lds_b128<O + 0>(addr);
      o[1] = lds_b128<O + 2048>(addr);
      o[2] = lds_b128<O + 4096>(addr);
      o[3] = lds_b128<O + 6144>(addr);
    };
    // scale words of column group 0 (w) and 1 (x): [K/2,N] K group 0, 1;
    // [N,K/2] the dwords of columns 4c + j
    auto read_scales = [&](auto slot_c, ScaleWords& w, ScaleWords& x) __attribute__((always_inline)) {
      if constexpr (kScRows) {
        constexpr int O = decltype(slot_c)::value * (kStage / 256);
        w = lds_2st64<O, O + 1>(s_off);
        x = lds_2st64<O, O + 1>(s_off + 64);
      } else {
        constexpr int O = decltype(slot_c)::value * kStage;
        w = __builtin_bit_cast(u32x4, lds_b128<O>(s_off));
        x = __builtin_bit_cast(u32x4, lds_b128<O + 256>(s_off));
      }
    };
    // step: the absolute K step of the scales ([N,K/2]: its parity picks the
    // half of the stage pair's dword)
    auto scales_from = [&](ScaleWords w, ScaleWords x, int step) __attribute__((always_inline)) {
      if constexpr (kScRows) {
        (void)step;
#pragma unroll
        for (int kg = 0; kg < 2; ++kg)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            sc[kg][j] = e8m0_byte(kg ? w.y : w.x, j);
            sc[kg][4 + j] = e8m0_byte(kg ? x.y : x.x, j);
          }
      } else {
        const uint32_t sh = 16u * (uint32_t)(step & 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t h0 = w[j] >> sh, h1 = x[j] >> sh;
          sc[0][j] = e8m0_byte(h0, 0);
          sc[1][j] = e8m0_byte(h0, 1);
          sc[0][4 + j] = e8m0_byte(h1, 0);
          sc[1][4 + j] = e8m0_byte(h1, 1);
        }
      }
    };
    // the four converts of B operand cb (= 4g + j) from raw words r
    auto convert = [&](int cb, const uint32_t (&r)[8], float s) __attribute__((always_inline)) {
      const int g = cb >> 2, j = cb & 3;
      const uint32_t* w = r + 4 * g;
      u32x4 v;
      if constexpr (!kKN) {
        // one word: K pairs 4q .. 4q+3 of column 4c + j
        const uint32_t x = r[cb];
        v = u32x4{cvt_fp4<0>(x, s), cvt_fp4<1>(x, s), cvt_fp4<2>(x, s), cvt_fp4<3>(x, s)};
        b[cb] = __builtin_bit_cast(bf16x8, v);
        return;
      }
      switch (j) {
        case 0: v = u32x4{cvt_fp4<0>(w[0], s), cvt_fp4<0>(w[1], s), cvt_fp4<0>(w[2], s), cvt_fp4<0>(w[3], s)}; break;
        case 1: v = u32x4{cvt_fp4<1>(w[0], s), cvt_fp4<1>(w[1], s), cvt_fp4<1>(w[2], s), cvt_fp4<1>(w[3], s)}; break;
        case 2: v = u32x4{cvt_fp4<2>(w[0], s), cvt_fp4<2>(w[1], s), cvt_fp4<2>(w[2], s), cvt_fp4<2>(w[3], s)}; break;
        default: v = u32x4{cvt_fp4<3>(w[0], s), cvt_fp4<3>(w[1], s), cvt_fp4<3>(w[2], s), cvt_fp4<3>(w[3], s)}; break;
      }
      b[cb] = __builtin_bit_cast(bf16x8, v);
    };

    // ---- prologue: stages 0, 1, 2 in flight; operands of (0,0) ---------------
#pragma unroll
    for (int st = 0; st < kNS; ++st)
#pragma unroll
      for (int d = 0; d < kVmPerStage; ++d) issue_dma(d, st, s_begin + st, st < T);
    vm_wait<(kNS - 1) * kVmPerStage>();
    barrier_asm();
    {
      ScaleWords w, x;
      read_scales(std::integral_constant<int, 0>{}, w, x);
      read_raw(std::integral_constant<int, 0>{}, 0, raw[0]);
      read_a(std::integral_constant<int, 0>{}, 0, a[0]);
      lgkm_wait<0>(w, x);
      scales_from(w, x, s_begin);
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) convert(cb, raw[0], sc[0][cb]);
    }

    // Stage t in ring slot SL = t % kNS (the caller unrolls the slots).
    auto stage = [&](auto slot_c, int t) __attribute__((always_inline)) {
      constexpr int SL = decltype(slot_c)::value;
      using Next = std::integral_constant<int, (SL + 1) % kNS>;
      const int dstep = s_begin + t + kNS;  // stage t+3 goes into slot SL, retired by (t,1)'s barrier
      const bool dlive = t + kNS < T;
#pragma unroll
      for (int sub = 0; sub < 2; ++sub) {
        const int pc = sub, pn = sub ^ 1;  // raw / A buffers of this and the next sub-step
        ScaleWords w{}, x{};
        if (sub == 0) {
          read_raw(slot_c, 1, raw[pn]);
          read_a(slot_c, 1, a[pn]);
        } else {
          // publish stage t+1: this wave's DMAs for it are done (stage t+2's
          // are the ones in flight)
          vm_wait<kVmPerStage>();
          barrier_asm();
          read_scales(Next{}, w, x);
          read_raw(Next{}, 0, raw[pn]);
          read_a(Next{}, 0, a[pn]);
        }
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
#pragma unroll
          for (int rb = 0; rb < kRB; ++rb) {
            mfma16(acc[rb][cb], a[pc][rb], b[cb]);
            // stage t+3's DMAs, one after every fourth MFMA from block 1 on
            if (sub == 1 && rb == 3 && cb >= 1 && cb - 1 < kVmPerStage) issue_dma(cb - 1, SL, dstep, dlive);
          }
          // converts: blocks 0, 1 finish this sub-step's operands 6, 7 (K
          // group `sub`); blocks 2 .. 7 convert the next sub-step's operands
          // 0 .. 5 (K group 1 of this stage, or 0 of the next)
          if (cb == 1) {
            // the next sub-step's raw words (and stage t+1's scales) landed
            if (sub == 0) {
              lgkm_wait<kRB>();
              convert(7, raw[pc], sc[0][7]);
            } else {
              lgkm_wait<kRB>(w, x);
              convert(7, raw[pc], sc[1][7]);
              scales_from(w, x, s_begin + t + 1);  // stage t's scales are dead from here
            }
          } else if (cb == 0) {
            convert(6, raw[pc], sc[sub][6]);
          } else {
            convert(cb - 2, raw[pn], sc[sub == 0 ? 1 : 0][cb - 2]);
          }
        }
        lgkm_wait<0>();
      }
    };
    for (int t = 0; t < T; t += kNS) {
      stage(std::integral_constant<int, 0>{}, t);
      if (t + 1 >= T) break;
      stage(std::integral_constant<int, 1>{}, t + 1);
      if (t + 2 >= T) break;
      stage(std::integral_constant<int, 2>{}, t + 2);
    }
    static_assert(kNS == 3, "the stage loop unrolls three ring slots");
    // the DMAs of the stages past the end still write the ring; the MFMAs
    // must finish before the accumulators are read
    vm_wait<0>();
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");
    __syncthreads();
  }

  // Lane-derived values of the epilogue, recomputed here: nothing
  // lane-derived that only the epilogue reads stays live across the main loop
  // (which takes all 256 registers; the allocator spilled such values, and
  // the reloads waited for the C stores issued before them).  wave, wm, wn
  // are SGPRs.
  const int lane_e = fresh_lane();
  const int tid_e = wave * 64 + lane_e;
  const int ce = lane_e & 15, qe = lane_e >> 4;

  // ---- split-K fix-up (the pipelined kernel's protocol) ------------------------
  int* s_last = reinterpret_cast<int*>(smem);
  if (p.splits > 1) {
    constexpr int Q = kRB * kCB;  // f32x4 per thread
    constexpr uint32_t SLOT = (uint32_t)Q * kThreads * 16;
    const __amdgpu_buffer_rsrc_t rp =
        make_rsrc(reinterpret_cast<uint8_t*>(p.partials) + (size_t)tile * p.splits * SLOT);
#pragma unroll
    for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb)
        store_coherent(rp, split * SLOT + (uint32_t)((rb * kCB + cb) * kThreads + tid_e) * 16, acc[rb][cb]);
    if (!splitk_arrive_last(p.counters + tile, (uint32_t)p.splits, s_last, tid_e)) return;
    splitk_sum_tid<Q>(rp, SLOT, p.splits, kThreads, tid_e,
                      [&](int i, f32x4 v) __attribute__((always_inline)) { acc[i / kCB][i % kCB] = v; });
  }

  // ---- epilogue: 4 adjacent columns (blocks 4g .. 4g+3) per lane and row --------
  // Plain and fused stores are separate loops, chosen once (see StoreKind).
  // Fused: v = act(acc + bias[col]) + residual[row][col]; the lane's 8 bias
  // values are read once (-0.0f where there is no bias: x + -0 == x for
  // every x), the residual's 4 columns with one vector read when aligned.
  // N % 4 == 0 here, so the 4 columns of a group are all inside the row.
  auto store = [&](auto fused, auto out) __attribute__((always_inline)) {
    constexpr bool kFused = decltype(fused)::value;
    const bool bf16 = decltype(out)::value == 2 ? p.out_bf16 != 0 : decltype(out)::value == 1;
    float bias[2][4];
    if constexpr (kFused) {
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int col = n0 + wn * 128 + 64 * g + 4 * ce;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          bias[g][j] = -0.0f;
          if (p.ep.bias && col < N)
            bias[g][j] = p.ep.bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p.ep.bias)[col + j])
                                        : static_cast<const float*>(p.ep.bias)[col + j];
        }
      }
    }
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      const int col = n0 + wn * 128 + 64 * g + 4 * ce;
      if (col >= N) continue;
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = m0 + wm * 64 + rb * 16 + 4 * qe + i;
          if (row >= M) continue;
          float v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = acc[rb][4 * g + j][i];
          if constexpr (decltype(out)::value == 0) {
            // plain fp32 store: each element copied to a VGPR on its own
            // (packing the four AGPR elements straight into the store's
            // register quad went through scratch, four round trips per store)
#pragma unroll
            for (int j = 0; j < 4; ++j) asm("" : "+v"(v[j]));
          }
          if constexpr (kFused) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = activate_c<kAct>(v[j] + bias[g][j]);
            if (p.ep.residual) {
              const size_t o = (size_t)row * N + col;
              float r[4];
              if (p.ep.res_bf16) {
                const uint16_t* rp = static_cast<const uint16_t*>(p.ep.residual) + o;
                if (p.ep.res_vec) {
                  const u32x2 w = *reinterpret_cast<const u32x2*>(rp);
                  r[0] = __builtin_bit_cast(float, w.x << 16);
                  r[1] = __builtin_bit_cast(float, w.x & 0xFFFF0000u);
                  r[2] = __builtin_bit_cast(float, w.y << 16);
                  r[3] = __builtin_bit_cast(float, w.y & 0xFFFF0000u);
                } else {
#pragma unroll
                  for (int j = 0; j < 4; ++j) r[j] = bf16_to_f32(rp[j]);
                }
              } else {
                const float* rp = static_cast<const float*>(p.ep.residual) + o;
                if (p.ep.res_vec) {
                  const f32x4 w = *reinterpret_cast<const f32x4*>(rp);
                  r[0] = w.x; r[1] = w.y; r[2] = w.z; r[3] = w.w;
                } else {
#pragma unroll
                  for (int j = 0; j < 4; ++j) r[j] = rp[j];
                }
              }
#pragma unroll
              for (int j = 0; j < 4; ++j) v[j] += r[j];
            }
          }
          // C is not read again here: non-temporal stores (measured ~2 %
          // faster on dit_up, whose rounds end in a synchronized store burst)
          if (bf16) {
            const u32x2 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            __builtin_nontemporal_store(w, reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p.C) + (size_t)row * N + col));
          } else {
            __builtin_nontemporal_store(f32x4{v[0], v[1], v[2], v[3]},
                                        reinterpret_cast<f32x4*>(static_cast<float*>(p.C) + (size_t)row * N + col));
          }
        }
      }
    }
  };
  // Interior tiles with a plain bf16 C: one buffer store per lane, row and 4
  // columns, row offsets in the scalar offset, no bounds checks and no 64-bit
  // address arithmetic -- about half the epilogue's instructions, which run
  // once per tile from a cold instruction cache.
  if constexpr (kOut == 1) {
    if (m0 + kBM <= M && n0 + kBN <= N && N <= (1 << 22)) {
      constexpr int kNt = 2;  // non-temporal: C is not read again here
      const __amdgpu_buffer_rsrc_t rc =
          make_rsrc(static_cast<uint16_t*>(p.C) + ((size_t)(m0 + wm * 64) * N + n0 + wn * 128));
      const uint32_t voff = (uint32_t)(4 * qe * N + 4 * ce) * 2;
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t row = (uint32_t)((rb * 16 + i) * N) * 2;
#pragma unroll
          for (int g = 0; g < 2; ++g) {
            const u32x2 w = {pack_bf16x2(acc[rb][4 * g][i], acc[rb][4 * g + 1][i]),
                             pack_bf16x2(acc[rb][4 * g + 2][i], acc[rb][4 * g + 3][i])};
            __builtin_amdgcn_raw_buffer_store_b64(w, rc, voff, row + 128u * g, kNt);
          }
        }
      return;
    }
  }
  store(StoreKind<kOut == 2>{}, OutKind<kOut>{});
}

}  // namespace

bool tiled_sched_kn_fits(int64_t N, int64_t K) {
  // the largest offset from B + n0 is (K/2 - 1) * N + 255 (+ 16 for the
  // DMA's own bytes)
  return (K / 2) * N + 256 <= (int64_t)kNumRecords;
}

bool tiled_sched_available(int layout, const TiledShape& s) {
  return (layout == kLayoutKN || layout == kLayoutNK || layout == kLayoutG) && s.bm() == kBM && s.bn() == kBN &&
         s.wm * s.wn == kWaves && s.stages == kNS;
}

template <int L>
void launch_sched_layout(const TiledArgs& args, int grid, hipStream_t stream) {
  if (args.ep.any) {
    switch (args.ep.act) {
      case 1: hipLaunchKernelGGL((tiled_sched_kernel<L, 2, 1>), dim3(grid), dim3(kThreads), 0, stream, args); break;
      case 2: hipLaunchKernelGGL((tiled_sched_kernel<L, 2, 2>), dim3(grid), dim3(kThreads), 0, stream, args); break;
      case 3: hipLaunchKernelGGL((tiled_sched_kernel<L, 2, 3>), dim3(grid), dim3(kThreads), 0, stream, args); break;
      default: hipLaunchKernelGGL((tiled_sched_kernel<L, 2, 0>), dim3(grid), dim3(kThreads), 0, stream, args); break;
    }
  } else if (args.out_bf16) {
    hipLaunchKernelGGL((tiled_sched_kernel<L, 1, 0>), dim3(grid), dim3(kThreads), 0, stream, args);
  } else {
    hipLaunchKernelGGL((tiled_sched_kernel<L, 0, 0>), dim3(grid), dim3(kThreads), 0, stream, args);
  }
}

hipError_t launch_tiled_sched(int layout, const TiledShape& shape, const TiledArgs& args, hipStream_t stream) {
  // [N,K/2] reads each column's scales as aligned dwords of K-step pairs;
  // [K/2,N] and G move whole 64-K steps
  const int kmod = layout == kLayoutNK ? 2 * kBK : kBK;
  if (!tiled_sched_available(layout, shape) || args.K % kmod != 0) return hipErrorInvalidValue;
  // the store writes 4 adjacent columns per lane and row
  if (args.N % 4 != 0) return hipErrorInvalidValue;
  if (layout == kLayoutKN && !tiled_sched_kn_fits(args.N, args.K)) return hipErrorInvalidValue;
  const int grid = args.tiles_m * args.tiles_n * args.splits;
  if (layout == kLayoutKN)
    launch_sched_layout<kLayoutKN>(args, grid, stream);
  else if (layout == kLayoutNK)
    launch_sched_layout<kLayoutNK>(args, grid, stream);
  else
    launch_sched_layout<kLayoutG>(args, grid, stream);
  return hipGetLastError();
}

}  // namespace mxfp4
