// Streaming split-K kernel for M <= 32 with [N, K/2] or panel (P) weights
// (decode shapes).
//
// The reference has no kernel for these shapes (every launcher rejects
// M % 64 != 0, csrc/common.h:80-99).  Design points, all measured on MI355X:
//
// * Weights stream through LDS.  A wave's unit is 32 columns x KW K (KW = 256
//   or 512); each 16-byte-per-lane LDS DMA moves CPD whole column segments of
//   KW/2 bytes, so HBM sees full lines, and a chunk rotation (chunk_rot) makes
//   a 16-lane MFMA read of chunk j of columns 0..15 hit 16 distinct 16-byte
//   bank slots.  (Reading the MFMA layout straight from global -- 16 rows x
//   64 B per load -- ran ~25% slower in a streaming probe.)
// * Activations: each wave DMAs its 16 (or 32) rows x KW first and alone, then
//   keeps them in VGPRs for every unit.  K is split S ways (split r = the
//   waves' K ranges r*KR .. r*KR+KR-1), so the activation bytes read from L2
//   are S times fewer than with whole-K CTAs.
// * Scales: per unit each wave DMAs its share of the CTA's [32][KR/32] scale
//   block (4 bytes per lane); a barrier per unit publishes it.
// * Panel weights (P): a unit's 32 columns are one panel, so a wave's unit is
//   KW/64 consecutive 1 KB blocks already in MFMA lane order and the unit's
//   scales are KR consecutive bytes: every DMA reads 1 KB of contiguous HBM
//   and lands linearly in LDS, and the reads need no rotation.  The K order
//   per lane is the [N,K/2] one, so both give identical results.
// * Split-K without a serial tail.  CTA b = (jg, r) processes the S units
//   (group S*jg + (u + r) % S, split r), u = 0 .. S-1, so every column group
//   has exactly one unit at the last position u = S-1 (its "late" unit) and
//   S-1 "early" units finished by other CTAs before.  Early units publish
//   their partial tile as 8-byte packets (value, tag) with device-coherent
//   stores and move on -- no store completion wait.  The late unit polls the
//   packets (device-coherent loads see each packet atomically), adds its own
//   partial last (a fixed order: bit-reproducible), writes C and clears the
//   packets.  A per-group counter arbitrates the case where the late unit
//   gives up polling (a bounded spin: CTAs that are not co-resident must not
//   deadlock): then whoever arrives last reduces.
// * Compute waves issue their global->LDS loads as asm and count them (the
//   compiler would wait for vmcnt(0) before every LDS read); a separate
//   reducer wave owns every global store, counter and poll, so the compute
//   waves never wait for a store.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

template <int MT, int WAVES, int GCB, int NSLOT, int KW>
struct StreamCfg {
  static_assert(KW == 256 || KW == 512, "K per wave and unit");
  static constexpr int GC = 16 * GCB;         // columns per group
  static constexpr int ROWS = 16 * MT;
  static constexpr int KR = WAVES * KW;       // K per split
  static constexpr int STEPS = KW / 128;      // 4-MFMA steps per unit
  static constexpr int CH = KW / 32;          // 16-byte chunks per column per wave
  static constexpr int CPD = 2048 / KW;       // columns per weight DMA (whole segments)
  static constexpr int NI = 16 / CPD;         // weight DMAs per 16-column block
  static constexpr int SLOT = GC * KW / 2;    // weight bytes per wave per unit
  static constexpr int W_LOADS = SLOT / 1024; // 1 KB DMAs per wave per unit
  static constexpr int SC_COL = KR / 32;      // scale bytes per column per unit
  static constexpr int SC_UNIT = GC * SC_COL; // scale bytes per unit (all waves)
  static constexpr int SC_LOADS = SC_UNIT / WAVES / 256;  // 64 x 4-byte DMAs per wave per unit
  static constexpr int A_ROW = KW * 2;        // activation bytes per row per wave
  static constexpr int A_GCH = A_ROW / 16;    // 16-byte chunks per activation row
  static constexpr int A_BYTES = ROWS * A_ROW;
  static constexpr int A_LOADS = A_BYTES / 1024;
  static constexpr int A_SLOTS = (A_BYTES + SLOT - 1) / SLOT;
  static constexpr int VM_UNIT = W_LOADS + SC_LOADS;
  static constexpr int TILE = ROWS * GC;       // floats per unit partial
  static constexpr int NV = TILE / 256;        // reducer: f32x4 per lane
  static constexpr int RING = WAVES * NSLOT * SLOT;
  static constexpr int SCR = NSLOT * SC_UNIT;
  static constexpr int RED = WAVES * TILE * 4;  // one buffer: two barriers per unit
  static constexpr int LDS = RING + SCR + RED;
  static constexpr int NT = (WAVES + 1) * 64;
  static_assert(GCB == 2, "the column permutation and scale DMA assume 32-column groups");
  static_assert(SC_LOADS >= 1 && SC_UNIT == WAVES * 256 * SC_LOADS, "whole 64 x 4-byte scale DMAs per wave");
  static_assert(A_SLOTS <= NSLOT, "the activations are staged in the ring");
  static_assert(TILE % 256 == 0, "reducer lanes own 4 consecutive elements per vector");
  static_assert(NSLOT * VM_UNIT < 64 && A_LOADS < 64, "vmcnt range");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

// Weight DMA i of a 16-column block moves CPD whole column segments of KW/2
// bytes; column 16cb + CPD*i + rr's chunk j lands at 16-byte position
// (j + rot(i, rr)) % CH of row rr.  The rotation makes the 16 lanes that read
// chunk j of columns 0..15 hit 16 distinct 16-byte bank slots (and any 8
// consecutive lanes 8 distinct slots of 128 bytes).
template <int KW>
__device__ __forceinline__ int chunk_rot(int i, int rr) {
  return KW == 256 ? (rr ^ i) : (4 * i + rr);
}

template <int LAYOUT, int MT, int WAVES, int GCB, int NSLOT, int SMAX, int KW>
__global__ void __launch_bounds__((WAVES + 1) * 64, 1) stream_kernel(StreamArgs p) {
  static_assert(LAYOUT == kLayoutNK || LAYOUT == kLayoutP, "weight layout");
  using Cfg = StreamCfg<MT, WAVES, GCB, NSLOT, KW>;
  constexpr int STEPS = Cfg::STEPS, CH = Cfg::CH, CPD = Cfg::CPD, NI = Cfg::NI;
  constexpr int GC = Cfg::GC, TILE = Cfg::TILE, NV = Cfg::NV, SLOT = Cfg::SLOT;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::LDS];
  uint8_t* const ring = smem;
  uint8_t* const scr = smem + Cfg::RING;
  float* const red = reinterpret_cast<float*>(smem + Cfg::RING + Cfg::SCR);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int S = p.splits;
  const int r = (int)blockIdx.x % S;  // this CTA's K split
  const int jg = (int)blockIdx.x / S;
  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;
  auto group_of = [&](int u) __attribute__((always_inline)) { return jg * S + (u + r) % S; };

  // The compiler may lay the two roles out as sequential regions (the
  // reducer's exit falling into the compute region's guard); its wait
  // insertion would then carry the reducer's pending stores into the compute
  // loop and add a vmcnt wait per unit.  A full wait at each role's entry
  // (nothing is outstanding there) clears that state.
  if (wave < WAVES) {
    // ============================ compute wave ============================
    __builtin_amdgcn_s_waitcnt(0);
    const int c = lane & 15, q = lane >> 4;
    const int kw0 = r * Cfg::KR + wave * KW;  // this wave's K range
    const bool kok = kw0 < K;                  // K % 256 == 0: a wave range is all in or all out
    uint8_t* const wring = ring + wave * NSLOT * SLOT;

    // DMA of unit u (< S) into ring slot u % NSLOT (lanes past the last group /
    // column / K masked).  Units past S are not issued; the waits below count
    // exactly the units in flight.
    auto issue_unit = [&](int u) __attribute__((always_inline)) {
      const int sl = u % NSLOT;
      const int g = group_of(u);
      const bool live = g < p.groups;
      if constexpr (LAYOUT == kLayoutP) {
        // scales: the unit's KR/64 blocks of 64 bytes, consecutive
        const desc_t ds = make_desc(p.S + (size_t)g * (K / kPK) * 64 + (size_t)r * Cfg::KR);
#pragma unroll
        for (int k = 0; k < Cfg::SC_LOADS; ++k) {
          const int base = 256 * (Cfg::SC_LOADS * wave + k), byte = base + 4 * lane;
          const bool ok = live && r * Cfg::KR + 64 * (byte >> 6) < K;
          dma4_nt(ds, scr + sl * Cfg::SC_UNIT + base, ok ? (uint32_t)byte : kOobOffset);
        }
        // weights: this wave's KW/64 consecutive 1 KB blocks of panel g
        const desc_t d = make_desc(p.B + ((size_t)g * (K / kPK) + (kw0 >> 6)) * 1024);
#pragma unroll
        for (int i = 0; i < Cfg::W_LOADS; ++i)
          dma16_nt(d, wring + sl * SLOT + i * 1024, live && kok ? (uint32_t)(i * 1024 + 16 * lane) : kOobOffset);
        return;
      }
      // scales: the unit's [GC][KR/32] block, wave w moving bytes
      // [w*SC_UNIT/WAVES, ...) in 64-lane x 4-byte DMAs (4 groups per lane)
      {
        const desc_t d = make_desc(p.S + (size_t)g * GC * G);
#pragma unroll
        for (int k = 0; k < Cfg::SC_LOADS; ++k) {
          const int base = 256 * (Cfg::SC_LOADS * wave + k);
          const int byte = base + 4 * lane;
          const int col = byte / Cfg::SC_COL, b = byte % Cfg::SC_COL;
          const int gi = r * Cfg::SC_COL + b;
          const bool ok = live && g * GC + col < N && gi < G;
          dma4_nt(d, scr + sl * Cfg::SC_UNIT + base, ok ? (uint32_t)(col * G + gi) : kOobOffset);
        }
      }
      const desc_t d = make_desc(p.B + (size_t)g * GC * Kh);
      const int rr = lane / CH;  // column of this lane within the DMA
#pragma unroll
      for (int cb = 0; cb < GCB; ++cb)
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int col = 16 * cb + CPD * i + rr;
          const int j = ((lane % CH) - chunk_rot<KW>(i, rr)) & (CH - 1);
          const bool ok = live && kok && g * GC + col < N;
          dma16_nt(d, wring + sl * SLOT + (NI * cb + i) * 1024,
                ok ? (uint32_t)(col * Kh + (kw0 >> 1) + 16 * j) : kOobOffset);
        }
    };

    // ---- prologue: activations -> VGPRs (through the ring), then the units ----
    uint8_t* const abuf = wring;
    {
      const desc_t d = make_desc(p.A);
#pragma unroll
      for (int pa = 0; pa < Cfg::A_LOADS; ++pa) {
        // row m, its chunk gch at position (gch + m) % A_GCH (bank spread over rows)
        const int m = pa * (1024 / Cfg::A_ROW) + lane / Cfg::A_GCH;
        const int gch = ((lane % Cfg::A_GCH) - m) & (Cfg::A_GCH - 1);
        const bool ok = kok && m < M;
        dma16(d, abuf + pa * 1024, ok ? (uint32_t)(m * K * 2 + kw0 * 2 + 16 * gch) : kOobOffset);
      }
    }
    // The activations go first and alone: behind the weight DMAs of every CTA
    // they would land only after the memory system drained that flood, and
    // the units that reuse their slots would start that late.
    wait_vmcnt<0>();
    u32x4 a[MT][STEPS][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int t = 0; t < STEPS; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int m = 16 * mt + c;
          const int gch = 16 * t + 4 * q + s;  // K 128t + 32q + 8s of the wave's range
          a[mt][t][s] = *reinterpret_cast<const u32x4*>(abuf + m * Cfg::A_ROW +
                                                       16 * ((gch + m) & (Cfg::A_GCH - 1)));
        }
    wait_lgkm0();  // the activation slots are reused below
    // Issue schedule.  A ring of two units is staggered: unit u+1 is issued
    // once half of unit u's weights have landed, so every CTA's units arrive
    // roughly in order -- early units early, which is what lets the late
    // units find their partners' partials published.  (Issuing everything at
    // once interleaves all units in the memory system and makes every unit
    // complete near the end.)  Deeper rings issue NSLOT units up front.
    constexpr bool kStagger = NSLOT == 2;
    const int first = kStagger ? 1 : (S < NSLOT ? S : NSLOT);  // units issued by the prologue
    for (int u = 0; u < first; ++u) issue_unit(u);
    // unit 0's scales (every wave's share) before the first barrier: the
    // scale DMA is the first of its unit, followed by its weights and the
    // other units
    wait_vmcnt_rt(Cfg::W_LOADS + (first - 1) * Cfg::VM_UNIT);
    __syncthreads();

    const int i_c = c / CPD, rr_c = c % CPD;
    const int rot_c = chunk_rot<KW>(i_c, rr_c);
    for (int u = 0; u < S; ++u) {
      const int sl = u % NSLOT;
      // units issued after unit u: u+1 .. min(S, u+NSLOT)-1
      int after;  // units issued after unit u when its weights are waited for
      if constexpr (kStagger) {
        after = u + 1 < S ? 1 : 0;
        if (after) {
          wait_vmcnt<Cfg::W_LOADS / 2>();  // half of unit u's weights
          issue_unit(u + 1);
        }
      } else {
        after = (S < u + NSLOT ? S : u + NSLOT) - 1 - u;
      }
      wait_vmcnt_rt(after * Cfg::VM_UNIT);  // this wave's weights of unit u
      f32x4 acc[MT][GCB];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int cb = 0; cb < GCB; ++cb) acc[mt][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint8_t* ws = wring + sl * SLOT;
      const uint8_t* ss = scr + sl * Cfg::SC_UNIT;
#pragma unroll
      for (int cb = 0; cb < GCB; ++cb) {
        if constexpr (LAYOUT == kLayoutP) {
          // chunk j = 4t + q (K 32j of the wave's range): block j/2, lane slot
          // 32 (j % 2) + column; its scale at the same position of the block's
          // 64 scale bytes
#pragma unroll
          for (int t = 0; t < STEPS; ++t) {
            const int blk = 2 * t + (q >> 1), slot = 32 * (q & 1) + 16 * cb + c;
            const u32x4 wv = *reinterpret_cast<const u32x4*>(ws + blk * 1024 + slot * 16);
            const float sc = e8m0_to_f32(ss[((wave * KW) / kPK + blk) * 64 + slot]);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
              const bf16x8 b = operand_from_word(wv[s], sc);
#pragma unroll
              for (int mt = 0; mt < MT; ++mt)
                acc[mt][cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a[mt][t][s]), b, acc[mt][cb]);
            }
          }
          continue;
        }
        // this wave's KW/32 scale bytes of the column: byte j scales chunk j
        uint32_t scw[STEPS];
        if constexpr (STEPS == 2) {
          const u32x2 v2 = *reinterpret_cast<const u32x2*>(ss + (16 * cb + c) * Cfg::SC_COL + CH * wave);
          scw[0] = v2.x;
          scw[1] = v2.y;
        } else {
          const u32x4 v4 = *reinterpret_cast<const u32x4*>(ss + (16 * cb + c) * Cfg::SC_COL + CH * wave);
          scw[0] = v4.x;
          scw[1] = v4.y;
          scw[2] = v4.z;
          scw[3] = v4.w;
        }
#pragma unroll
        for (int t = 0; t < STEPS; ++t) {
          const int j = 4 * t + q;
          const u32x4 wv = *reinterpret_cast<const u32x4*>(
              ws + (NI * cb + i_c) * 1024 + rr_c * (KW / 2) + 16 * ((j + rot_c) & (CH - 1)));
          const float sc = e8m0_to_f32(scw[t] >> (8 * q));
#pragma unroll
          for (int s = 0; s < 4; ++s) {
            const bf16x8 b = operand_from_word(wv[s], sc);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              acc[mt][cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a[mt][t][s]), b, acc[mt][cb]);
          }
        }
      }
      // B'(u-1): the reducer has read the previous unit's tiles
      __syncthreads();
      float* my = red + wave * TILE;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int cb = 0; cb < GCB; ++cb)
#pragma unroll
          for (int i = 0; i < 4; ++i) my[(16 * mt + 4 * q + i) * GC + 16 * cb + c] = acc[mt][cb][i];
      // B(u): this unit's tiles, and the next unit's scales (all waves' shares)
      if (after > 0) wait_vmcnt_rt(Cfg::W_LOADS + (after - 1) * Cfg::VM_UNIT);
      __syncthreads();
      if (!kStagger && u + NSLOT < S) issue_unit(u + NSLOT);  // into the slot just consumed
    }
    return;
  }

  // ============================== reducer wave ==============================
  __builtin_amdgcn_s_waitcnt(0);
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(p.partials);
  uint32_t* const cnt = p.counters;
  const bool split = S > 1;
  auto packet_off = [&](int g, int rs, int v) __attribute__((always_inline)) {  // byte offset of element 4*lane + 256*v
    return (uint32_t)((((size_t)g * S + rs) * TILE + 4 * lane + 256 * v) * 8);
  };
  // The split of group g whose unit is its late unit: group t = g % S of a
  // block is processed last by the CTA with split (t + 1) % S.
  auto late_split = [&](int g) __attribute__((always_inline)) { return (g % S + 1) % S; };
  auto store_c = [&](int g, int v, f32x4 x) __attribute__((always_inline)) {
    const int e = 4 * lane + 256 * v;
    const int row = e / GC, col = g * GC + e % GC;
    if (row >= M) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (col + i >= N) break;
      const float y = p.ep.any ? epilogue_value(p.ep, x[i], row, col + i, N) : x[i];
      if (p.out_bf16)
        static_cast<uint16_t*>(p.C)[(size_t)row * N + col + i] = (uint16_t)bf16_bits_rne(y);
      else
        static_cast<float*>(p.C)[(size_t)row * N + col + i] = y;
    }
  };
  auto clear_packets = [&](int g, int rs) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, pr, packet_off(g, rs, v), 0, kCPolDevice);
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, pr, packet_off(g, rs, v) + 16, 0, kCPolDevice);
    }
  };
  // Sum of group g's published partials except split `skip` (-1: none), in
  // split order.  Polls PCH splits at a time until their tags are all in, at
  // most `limit` rounds per chunk (limit < 0: until they land -- only used when
  // every split has arrived, so their stores are in flight).  Returns false on
  // a timeout.
  constexpr int PCH = 4 / NV;  // splits per poll round: 8 VGPRs per split and row tile
  auto sum_packets = [&](int g, int skip, int limit, f32x4 (&tot)[NV]) __attribute__((always_inline)) -> bool {
    bool first = true;
    for (int base = 0; base < S; base += PCH) {
      u32x4 pk[PCH][NV][2];
      bool got = false;
      for (int it = 0; limit < 0 || it < limit; ++it) {
        bool ok = true;
#pragma unroll
        for (int ch = 0; ch < PCH; ++ch) {
          const int rs = base + ch;
          if (rs >= S || rs == skip) continue;
#pragma unroll
          for (int v = 0; v < NV; ++v) {
            pk[ch][v][0] = load_packets(pr, packet_off(g, rs, v));
            pk[ch][v][1] = load_packets(pr, packet_off(g, rs, v) + 16);
          }
        }
#pragma unroll
        for (int ch = 0; ch < PCH; ++ch) {
          const int rs = base + ch;
          if (rs >= S || rs == skip) continue;
#pragma unroll
          for (int v = 0; v < NV; ++v) ok = ok && tagged(pk[ch][v][0], pk[ch][v][1]);
        }
        if (__builtin_amdgcn_ballot_w64(ok) == ~0ull) {
          got = true;
          break;
        }
        if (limit < 0 && it > (1 << 20)) break;  // cannot happen: stores in flight always land
        __builtin_amdgcn_s_sleep(1);
      }
      if (!got) return false;
#pragma unroll
      for (int ch = 0; ch < PCH; ++ch) {
        const int rs = base + ch;
        if (rs >= S || rs == skip) continue;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          const f32x4 val = packet_values(pk[ch][v][0], pk[ch][v][1]);
          tot[v] = first ? val : tot[v] + val;
        }
        first = false;
      }
    }
    return true;
  };
  // Reduction by the last arriver (only when a late unit gave up polling):
  // the same order as the late unit's fast path -- the other splits in
  // split order, then the late split.
  // A poll that never completes (it cannot: every arrival follows its
  // packet stores) writes NaN rather than a partial sum.
  auto reduce_from_packets = [&](int g) __attribute__((always_inline)) {
    const int rl = late_split(g);
    f32x4 tot[NV], own[NV];
    bool ok_all = sum_packets(g, rl, -1, tot);
    {
      u32x4 x0[NV], x1[NV];
      bool landed = false;
      for (int it = 0; it <= (1 << 20); ++it) {
        bool ok = true;
#pragma unroll
        for (int v = 0; v < NV; ++v) {
          x0[v] = load_packets(pr, packet_off(g, rl, v));
          x1[v] = load_packets(pr, packet_off(g, rl, v) + 16);
          ok = ok && tagged(x0[v], x1[v]);
        }
        if (__builtin_amdgcn_ballot_w64(ok) == ~0ull) {
          landed = true;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      ok_all = ok_all && landed;
#pragma unroll
      for (int v = 0; v < NV; ++v) own[v] = packet_values(x0[v], x1[v]);
    }
    const float nan = __builtin_nanf("");
#pragma unroll
    for (int v = 0; v < NV; ++v)
      store_c(g, v, !ok_all ? f32x4{nan, nan, nan, nan} : S > 1 ? tot[v] + own[v] : own[v]);
    for (int rs = 0; rs < S; ++rs) clear_packets(g, rs);
    if (lane == 0) __hip_atomic_store(cnt + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto arrive = [&](int g) __attribute__((always_inline)) -> uint32_t {
    uint32_t prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(cnt + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return prev;  // lane 0 only; read with readfirstlane once needed
  };

  uint32_t prev_u[SMAX];  // counter value seen by each arrival (lane 0); checked at the end
#pragma unroll
  for (int u = 0; u < SMAX; ++u) prev_u[u] = 0;
  f32x4 others[NV];  // late group: the other splits' sum (fast path)
  bool fast = false;

  __syncthreads();  // matches the compute waves' prologue barrier
  for (int u = 0; u < S; ++u) {
    __syncthreads();  // B'(u-1)
    __syncthreads();  // B(u): red holds unit u's tiles
    const int g = group_of(u);
    const bool gv = g < p.groups;
    f32x4 own[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) {
      const float* src = red + 4 * lane + 256 * v;
      f32x4 sum = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
      for (int w = 1; w < WAVES; ++w) sum += *reinterpret_cast<const f32x4*>(src + w * TILE);
      own[v] = sum;
    }
    if (!gv) continue;
    if (!split) {
#pragma unroll
      for (int v = 0; v < NV; ++v) store_c(g, v, own[v]);
      continue;
    }
    if (u < S - 1) {
      // early unit: publish the partial and move on
#pragma unroll
      for (int v = 0; v < NV; ++v) store_packets(pr, packet_off(g, r, v), own[v], kTag);
#pragma unroll
      for (int uu = 0; uu < SMAX; ++uu)
        if (uu == u) prev_u[uu] = arrive(g);
      if (u == S - 2) {
        // Poll the late group's other splits while the compute waves stream
        // the last unit (bounded: CTAs that are not co-resident must not spin
        // forever; on a timeout the counter decides who reduces).
        const int gl = group_of(S - 1);
        if (gl < p.groups) fast = sum_packets(gl, r, p.spin_limit, others);
      }
      continue;
    }
    // late unit
    if (fast) {
#pragma unroll
      for (int v = 0; v < NV; ++v) store_c(g, v, others[v] + own[v]);
      for (int rs = 0; rs < S; ++rs)
        if (rs != r) clear_packets(g, rs);
      // Release the counter without waiting: the S-1 early arrivals and this
      // subtraction net to zero in any order, and no early arrival can see
      // S-1 arrivals before it (so none reduces).
      if (lane == 0)
        __hip_atomic_fetch_add(cnt + g, (uint32_t)(1 - S), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
#pragma unroll
      for (int v = 0; v < NV; ++v) store_packets(pr, packet_off(g, r, v), own[v], kTag);
      prev_u[SMAX - 1] = arrive(g);
    }
  }
  if (!split) return;
  // The last of a group's S arrivals (possible only when its late unit gave
  // up polling) reduces it and resets the counter.
#pragma unroll
  for (int u = 0; u < SMAX; ++u) {
    const bool late = u == SMAX - 1;
    if (late && fast) continue;
    if (!late && u >= S - 1) continue;
    const int g = group_of(late ? S - 1 : u);
    if (g >= p.groups) continue;
    const uint32_t prev = __builtin_amdgcn_readfirstlane(prev_u[u]);
    if ((prev & kArrivals) != (uint32_t)(S - 1)) continue;
    reduce_from_packets(g);
  }
}

// ---- whole-K streaming kernel (M <= 16, K <= 16 * KW) ----------------------
// One CTA per 32-column group and K / KW waves, each owning K range
// w*KW .. w*KW+KW-1 of the group: its weights (32 columns x KW/2 bytes) and
// scales land in its own LDS slot, its activations (16 rows x KW) in VGPRs.
// Every load of the CTA is issued at entry -- no split-K, no ring reuse, no
// cross-CTA protocol -- so the only serial steps after the last byte lands
// are the wave's remaining MFMAs, one barrier and an LDS reduction of the
// waves' partial tiles (in wave order: bit-reproducible).
//
// All VMEM instructions here are asm, counted by hand: the activation loads
// first (4 per 128 K), then the scale DMAs, then the weight DMAs.  A wait
// that publishes loaded registers redefines them (asm "+v"), so no use can
// be scheduled above it.
template <int KW>
struct WholeCfg {
  static_assert(KW == 256 || KW == 512, "K per wave");
  static constexpr int MAXW = 16;             // waves per CTA at most
  static constexpr int STEPS = KW / 128;      // 4-MFMA steps per column block
  static constexpr int CH = KW / 32;          // 16-byte chunks (and scale bytes) per column
  static constexpr int CPD = 2048 / KW;       // columns per weight DMA ([N,K/2])
  static constexpr int NI = 16 / CPD;         // weight DMAs per 16-column block
  static constexpr int SLOT = 32 * KW / 2;    // weight bytes per wave
  static constexpr int W_LOADS = SLOT / 1024;
  static constexpr int SC_W = 32 * CH;        // scale bytes per wave
  static constexpr int SC_LOADS = SC_W / 256;
  static constexpr int A_LOADS = 4 * STEPS;
  static constexpr int VM = A_LOADS + SC_LOADS + W_LOADS;
  static constexpr int LDS = MAXW * (SLOT + SC_W);
  static_assert(VM < 64, "vmcnt range");
  static_assert(SLOT >= 16 * 32 * 4, "a wave's slot holds its 16 x 32 partial tile");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

__device__ __forceinline__ u32x4 asm_load16(const desc_t& d, uint32_t voff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(d) : "memory");
  return v;
}
// s_waitcnt vmcnt(N) that redefines the STEPS x 4 activation registers.
template <int N, int STEPS>
__device__ __forceinline__ void vm_wait_tie(u32x4 (&a)[STEPS][4]) {
  asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory");
#pragma unroll
  for (int t = 0; t < STEPS; ++t)
#pragma unroll
    for (int s = 0; s < 4; ++s) asm volatile("" : "+v"(a[t][s]));
}

template <int LAYOUT, int KW>
__global__ void __launch_bounds__(1024, 1) stream_whole_kernel(StreamArgs p) {
  static_assert(LAYOUT == kLayoutNK || LAYOUT == kLayoutP, "weight layout");
  using Cfg = WholeCfg<KW>;
  constexpr int STEPS = Cfg::STEPS, CH = Cfg::CH, CPD = Cfg::CPD, NI = Cfg::NI, SLOT = Cfg::SLOT;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::LDS];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = (int)blockDim.x >> 6;  // K / KW
  const int g = blockIdx.x;             // column group
  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;
  const int c = lane & 15, q = lane >> 4;
  const int kw0 = wave * KW;
  uint8_t* const ws = smem + wave * SLOT;
  uint8_t* const ss = smem + Cfg::MAXW * SLOT + wave * Cfg::SC_W;

  // Issue order: the first half of the weights, the scales, the activations,
  // the second half.  The weights' HBM requests go out first; the activation
  // loads (L2 hits, 16 rows x KW x 2 bytes per wave -- twice the wave's
  // weight bytes at M = 16) are taken in while those stream, and the first
  // half's compute waits only for them.
  // activations: lane (c, q) holds row c, K kw0 + 128t + 32s + 8q .. +7 in
  // a[t][s] (MFMA (t, s) of the wave's range: the four lanes of a row read 64
  // contiguous bytes per load); the weights are read in the same K order
  u32x4 a[STEPS][4];
  auto issue_a = [&]() __attribute__((always_inline)) {
    const desc_t d = make_desc(p.A);
#pragma unroll
    for (int t = 0; t < STEPS; ++t)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        a[t][s] = asm_load16(d, c < M ? (uint32_t)((c * K + kw0 + 128 * t + 32 * s + 8 * q) * 2) : kOobOffset);
  };
  if constexpr (LAYOUT == kLayoutP) {
    // scales: KW/64 blocks of 64 bytes; weights: KW/64 blocks of 1 KB, both
    // contiguous in the panel
    const desc_t d = make_desc(p.B + ((size_t)g * (K / kPK) + (kw0 >> 6)) * 1024);
#pragma unroll
    for (int i = 0; i < Cfg::W_LOADS / 2; ++i) dma16_nt(d, ws + i * 1024, (uint32_t)(i * 1024 + 16 * lane));
    const desc_t ds = make_desc(p.S + (size_t)g * (K / kPK) * 64 + kw0);
#pragma unroll
    for (int k = 0; k < Cfg::SC_LOADS; ++k) dma4_nt(ds, ss + 256 * k, (uint32_t)(256 * k + 4 * lane));
    issue_a();
#pragma unroll
    for (int i = Cfg::W_LOADS / 2; i < Cfg::W_LOADS; ++i) dma16_nt(d, ws + i * 1024, (uint32_t)(i * 1024 + 16 * lane));
  } else {
    // weights: DMA i of block cb moves CPD whole column segments (KW/2
    // bytes); chunk j of column 16cb + CPD*i + rr lands at 16-byte position
    // (j + rot(i, rr)) % CH of its row (16 distinct bank slots per read)
    const desc_t d = make_desc(p.B + (size_t)g * 32 * Kh);
    const int rr = lane / CH;
    auto issue_w = [&](int cb) __attribute__((always_inline)) {
#pragma unroll
      for (int i = 0; i < NI; ++i) {
        const int col = 16 * cb + CPD * i + rr;
        const int j = ((lane % CH) - chunk_rot<KW>(i, rr)) & (CH - 1);
        const bool ok = g * 32 + col < N;
        dma16_nt(d, ws + (NI * cb + i) * 1024, ok ? (uint32_t)(col * Kh + (kw0 >> 1) + 16 * j) : kOobOffset);
      }
    };
    issue_w(0);
    // scales: [32 columns][CH bytes] of this wave's K range
    {
      const desc_t ds = make_desc(p.S + (size_t)g * 32 * G);
#pragma unroll
      for (int k = 0; k < Cfg::SC_LOADS; ++k) {
        const int byte = 256 * k + 4 * lane;
        const int col = byte / CH, b = byte % CH;
        const bool ok = g * 32 + col < N;
        dma4_nt(ds, ss + 256 * k, ok ? (uint32_t)(col * G + kw0 / 32 + b) : kOobOffset);
      }
    }
    issue_a();
    issue_w(1);
  }

  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  if constexpr (LAYOUT == kLayoutP) {
    // step t needs blocks 2t, 2t + 1 (chunk 4t + q = block 2t + q/2, lane
    // slot 32 (q % 2) + column); its scale sits at the same slot of the
    // block's 64 scale bytes
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      // blocks 0 .. 2t+1 landed: at most min(W/2, W - 2t - 2) loads
      // outstanding (the second half of the weights follows the activations)
      constexpr int W = Cfg::W_LOADS;
      if (t == 0)
        vm_wait_tie<(W / 2 < W - 2 ? W / 2 : W - 2), STEPS>(a);
      else if (t == 1)
        wait_vmcnt<(W / 2 < W - 4 ? W / 2 : (W >= 4 ? W - 4 : 0))>();
      else if (t == 2)
        wait_vmcnt<(W >= 6 ? W - 6 : 0)>();
      else
        wait_vmcnt<0>();
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          // chunk 4t + s = block 2t + s/2, lane slot 32 (s % 2) + column; word q
          const int blk = 2 * t + (s >> 1), slot = 32 * (s & 1) + 16 * cb + c;
          const uint32_t w = *reinterpret_cast<const uint32_t*>(ws + blk * 1024 + slot * 16 + 4 * q);
          const float sc = e8m0_to_f32(ss[blk * 64 + slot]);
          acc[cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a[t][s]), operand_from_word(w, sc), acc[cb]);
        }
      }
    }
  } else {
    const int i_c = c / CPD, rr_c = c % CPD;
    const int rot_c = chunk_rot<KW>(i_c, rr_c);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      if (cb == 0)
        vm_wait_tie<NI, STEPS>(a);  // block 0's weights, scales and activations
      else
        wait_vmcnt<0>();
      // this wave's CH scale bytes of the column: byte j scales chunk j
      uint32_t scw[STEPS];
      if constexpr (STEPS == 2) {
        const u32x2 v2 = *reinterpret_cast<const u32x2*>(ss + (16 * cb + c) * CH);
        scw[0] = v2.x;
        scw[1] = v2.y;
      } else {
        const u32x4 v4 = *reinterpret_cast<const u32x4*>(ss + (16 * cb + c) * CH);
        scw[0] = v4.x;
        scw[1] = v4.y;
        scw[2] = v4.z;
        scw[3] = v4.w;
      }
#pragma unroll
      for (int t = 0; t < STEPS; ++t) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          // word q of chunk 4t + s; its scale is byte s of scw[t]
          const int j = 4 * t + s;
          const uint32_t w = *reinterpret_cast<const uint32_t*>(ws + (NI * cb + i_c) * 1024 + rr_c * (KW / 2) +
                                                                16 * ((j + rot_c) & (CH - 1)) + 4 * q);
          const float sc = e8m0_to_f32(scw[t] >> (8 * s));
          acc[cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a[t][s]), operand_from_word(w, sc), acc[cb]);
        }
      }
    }
  }

  // partial tile of this wave -> its own slot (its weights are consumed), then
  // the sum over waves in wave order
  float* const part = reinterpret_cast<float*>(ws);
#pragma unroll
  for (int cb = 0; cb < 2; ++cb)
#pragma unroll
    for (int i = 0; i < 4; ++i) part[(4 * q + i) * 32 + 16 * cb + c] = acc[cb][i];
  __syncthreads();
  // 128 groups of 4 outputs; a one-wave CTA (K = KW) takes two each
  for (int e4 = threadIdx.x; e4 < 128; e4 += blockDim.x) {
    const int e = 4 * e4;  // row e / 32, columns e % 32 .. +3 of the group
    const int row = e >> 5, col = g * 32 + (e & 31);
    if (row >= M) break;
    f32x4 sum = *reinterpret_cast<const f32x4*>(smem + 4 * e);
    for (int w = 1; w < nw; ++w) sum += *reinterpret_cast<const f32x4*>(smem + w * SLOT + 4 * e);
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = p.ep.any ? epilogue_value(p.ep, sum[i], row, col + i, N) : sum[i];
    if (p.out_bf16) {
      uint16_t* out = static_cast<uint16_t*>(p.C) + (size_t)row * N + col;
      if ((N & 3) == 0 && col + 3 < N) {
        *reinterpret_cast<u32x2*>(out) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < N) out[i] = (uint16_t)bf16_bits_rne(v[i]);
      }
    } else {
      float* out = static_cast<float*>(p.C) + (size_t)row * N + col;
      if ((N & 3) == 0 && col + 3 < N) {
        *reinterpret_cast<f32x4*>(out) = f32x4{v[0], v[1], v[2], v[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < N) out[i] = v[i];
      }
    }
  }
}

template <int KW>
hipError_t launch_whole(int layout, const StreamArgs& a, hipStream_t stream) {
  if (a.M > 16 || a.K % KW != 0 || a.K / KW > WholeCfg<KW>::MAXW) return hipErrorInvalidValue;
  const dim3 block(64 * (a.K / KW));
  if (layout == kLayoutNK)
    hipLaunchKernelGGL((stream_whole_kernel<kLayoutNK, KW>), dim3(a.groups), block, 0, stream, a);
  else if (layout == kLayoutP)
    hipLaunchKernelGGL((stream_whole_kernel<kLayoutP, KW>), dim3(a.groups), block, 0, stream, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

template <int MT, int WAVES, int GCB, int NSLOT, int SMAX, int KW>
hipError_t launch_one(int layout, const StreamArgs& a, hipStream_t stream) {
  using Cfg = StreamCfg<MT, WAVES, GCB, NSLOT, KW>;
  if (a.splits < 1 || a.splits > SMAX) return hipErrorInvalidValue;
  const int grid = a.ctas;
  if (layout == kLayoutNK)
    hipLaunchKernelGGL((stream_kernel<kLayoutNK, MT, WAVES, GCB, NSLOT, SMAX, KW>), dim3(grid), dim3(Cfg::NT), 0,
                       stream, a);
  else if (layout == kLayoutP)
    hipLaunchKernelGGL((stream_kernel<kLayoutP, MT, WAVES, GCB, NSLOT, SMAX, KW>), dim3(grid), dim3(Cfg::NT), 0,
                       stream, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

// (MT, WAVES, GCB, NSLOT, SMAX, KW); index = StreamShape order in the plan table.
#define MXFP4_STREAM_SHAPES(X) \
  X(1, 8, 2, 4, 4, 256)        \
  X(1, 4, 2, 8, 8, 256)        \
  X(2, 4, 2, 8, 8, 256)        \
  X(1, 8, 2, 2, 2, 512)        \
  X(2, 4, 2, 4, 4, 512)

}  // namespace

// The whole-K kernel's shapes: (1, 16, 2, 1, 1, KW) -- one unit per CTA, no ring
// reuse, no split.
bool whole_shape(const StreamShape& s) {
  return s.mt == 1 && s.waves == WholeCfg<512>::MAXW && s.gcb == 2 && s.nslot == 1 && s.smax == 1 &&
         (s.kw == 256 || s.kw == 512);
}

bool stream_shape_available(const StreamShape& s) {
  if (s.resident == 16 || s.resident == 32)
    return s.mt == s.resident / 16 && s.waves == 8 && s.gcb == 8 && s.nslot == 0 && s.smax == 8 && s.kw == 256 &&
           s.direct == 0;
  if (s.resident)
    return s.mt == 1 && s.waves == 16 && s.gcb == 2 && (s.nslot == 0 || (s.nslot == 1 && s.resident == 1)) &&
           s.smax == 1 && s.kw == 512 && s.direct == 0 && (s.resident == 1 || s.resident == 8);
  if (s.direct)
    return s.mt == 1 && s.waves == 8 && s.nslot == 0 && s.smax == 8 &&
           ((s.direct == 16 && s.gcb == 4 && s.kw == 512) || (s.direct == 8 && s.gcb == 2 && s.kw == 1024));
  if (whole_shape(s)) return true;
#define X(MT_, W_, GCB_, NS_, SM_, KW_)                                                              \
  if (s.mt == MT_ && s.waves == W_ && s.gcb == GCB_ && s.nslot == NS_ && s.smax == SM_ && s.kw == KW_) \
    return true;
  MXFP4_STREAM_SHAPES(X)
#undef X
  return false;
}

hipError_t launch_stream(int layout, const StreamShape& s, const StreamArgs& args, hipStream_t stream) {
  if (s.resident)
    return s.nslot == 1 ? launch_resident_dot(layout, args, stream) : launch_resident(s.resident, layout, args, stream);
  if (s.direct) return launch_decode(s.direct, layout, args, stream);
  if (whole_shape(s)) {
    if (args.splits != 1) return hipErrorInvalidValue;
    return s.kw == 512 ? launch_whole<512>(layout, args, stream) : launch_whole<256>(layout, args, stream);
  }
#define X(MT_, W_, GCB_, NS_, SM_, KW_)                                                               \
  if (s.mt == MT_ && s.waves == W_ && s.gcb == GCB_ && s.nslot == NS_ && s.smax == SM_ && s.kw == KW_) \
    return launch_one<MT_, W_, GCB_, NS_, SM_, KW_>(layout, args, stream);
  MXFP4_STREAM_SHAPES(X)
#undef X
  return hipErrorInvalidValue;
}

}  // namespace mxfp4
