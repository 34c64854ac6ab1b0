// Decode kernels with [N, K/2] weights.  The decode kernel (M <= 16):
// activations resident in LDS, weights streamed straight into VGPRs by
// separate waves.  The resident kernel (M <= 8, production for M = 1; its
// notes are at its definition): every weight byte of a CTA loaded into VGPRs
// at entry.
//
// The reference has no kernel for these shapes (every launcher rejects
// M % 64 != 0, csrc/common.h:80-99).  A decode GEMM is a read of the weights
// (M = 16, N = K = 8192: 36.2 MB) plus 2 GFLOP of MFMA work, so its time is
// set by how early and how many bytes the kernel puts in flight and by the
// serial steps after the last byte lands.  Measured on MI355X (cold HBM:
// buffers rotated past the 256 MB MALL; probes, not product code):
//   - a bare 32-36 MB read takes 6.7-8.1 us per launch (about 1.6 us fixed);
//     under that flood the first bytes land ~4 us after issue;
//   - global loads are ~1.1 us faster than buffer loads of the same bytes,
//     and the non-temporal hint helps global loads a little (it slows buffer
//     loads);
//   - activation loads in the MFMA operand layout (16 rows 2K bytes apart per
//     instruction) cost 2.4x the same bytes read 1 KB-contiguous;
//   - activation and weight loads issued by the same wave serialize (11.7 us
//     for 64 MB of L2 activations + 32 MB of weights), while loader waves and
//     weight waves overlap (9.5 us);
//   - a CU's loads enter the memory system in issue order at the rate it
//     accepts them (a wave that issues 16 loads at once is stalled in issue
//     for up to 8 us), and every cross-CTA round trip at the end (publish,
//     poll, store) adds ~1 us.
//
// So a CTA owns CW columns x KR of K with its activation slice (MR rows x KR,
// 128 KB) resident in LDS:
// * 8 loader waves DMA the activation slice (1 KB contiguous per DMA, 16-byte
//   chunk j of row m landing at j ^ (m & 7): conflict-free operand reads;
//   rows past M are skipped), then wait and release barrier B1.  The compute
//   waves issue their loads only after the loaders have issued their DMAs
//   (barrier B0): with the weights first, the activations landed after ~8 us,
//   behind every weight byte of the CU.
// * 8 compute waves each DMA their 1 KB scale block into LDS (an HBM read
//   like the weights: in the loaders' queue it held B1 until the weight flood
//   had drained), then keep 8 weight loads in flight -- CW columns x KR/8 of
//   K in all, 16 bytes per lane (lane (c, q) reads bytes 64t + 16q .. +15 of
//   its column's segment: 16 columns x 64 contiguous bytes per load), global
//   non-temporal loads -- issuing the next as each lands and is consumed
//   (waves that issued all 16 at once sat in issue until ~8 us).
// * The K order inside one MFMA only has to agree between the operands:
//   MFMA (t, s) of a 128-K step t takes K 128t + 32q + 8s .. +7 of the wave's
//   range in lane (c, q): word s of the lane's 16 weight bytes and activation
//   chunk 16t + 4q + s of row c.  Its scale is group 4t + q of the range.
// * Each compute wave writes its partial tile into its own activation range
//   (it alone reads that range), and the CTA sums the 8 tiles in wave order.
// * Two shapes: MR = 8 (32 columns x the whole K up to 8192 per CTA: no
//   split at K <= 8192) and MR = 16 (64 columns x 4096 K: 2 splits at K =
//   8192).  Split CTAs publish their tile as tagged packets to the group's
//   reducer (split S-1), which polls (bounded), adds the splits in split
//   order, writes C, clears the packets and releases the group counter.  If
//   the reducer gives up polling (CTAs not co-resident), it publishes too and
//   the last of the S arrivals on the counter reduces.
// * Out-of-range K ranges are DMAs past the descriptor's range (zeros land in
//   LDS); columns past N load column N-1 and are zeroed.
//
// Result (N = K = 8192, bf16 C, graph-replayed): MR = 8 takes 11.8 us at
// M = 8 against 12.3 us for the whole-K streaming kernel (N = 28672: 39.4
// against 41.0 us), and is the auto plan for 2 <= M <= 8; at M = 1 the
// streaming kernel is faster (10.4 against 11.1 us).  MR = 16 (15.4 us at
// M = 16 against 12.7 us for the split-K streaming kernel) is an explicit
// plan only: its 128 KB activation slice per CU queues ahead of the weights.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

template <int MR, int CW, int KR>
struct DecodeCfg {
  static constexpr int DEPTH = 8;                       // weight loads in flight per compute wave
  static constexpr int CWAVES = 8;                      // compute waves
  static constexpr int LWAVES = 8;                      // loader waves
  static constexpr int NT = 64 * (CWAVES + LWAVES);
  static constexpr int KWV = KR / CWAVES;               // K per compute wave
  static constexpr int T = KWV / 128;                   // 128-K steps per compute wave
  static constexpr int CB = CW / 16;                    // 16-column blocks
  static constexpr int A_ROWB = 2 * KWV;                // activation bytes per row and range
  static constexpr int A_RANGE = MR * A_ROWB;           // LDS bytes per compute wave's range
  static constexpr int A_BYTES = CWAVES * A_RANGE;
  static constexpr int A_DMAS = A_BYTES / 1024 / LWAVES;  // per loader wave
  static constexpr int SW_COL = KWV / 32;               // scale bytes per column and compute wave
  static constexpr int S_BYTES = CWAVES * 1024;         // one 1 KB scale block per compute wave
  static constexpr int TILE = MR * CW;                  // outputs per CTA
  static constexpr int ACTIVE = TILE / 4;               // threads holding 4 outputs
  static constexpr int LDS = A_BYTES + S_BYTES;
  static_assert(A_ROWB % 1024 == 0, "a 1 KB DMA covers part of one row");
  static_assert(A_DMAS * LWAVES * 1024 == A_BYTES && A_DMAS < 48, "whole activation DMAs per loader wave");
  static_assert(CW * SW_COL == 1024 && SW_COL % 16 == 0 && T * CB < 64, "one 1 KB scale DMA per compute wave");
  static_assert(TILE * 4 <= A_RANGE && ACTIVE % 64 == 0 && ACTIVE <= 64 * CWAVES, "partial tiles");
  static_assert(LDS <= 160 * 1024, "LDS budget");
};

template <int MR, int CW, int KR>
__global__ void __launch_bounds__(1024, 1) decode_kernel(StreamArgs p) {
  using Cfg = DecodeCfg<MR, CW, KR>;
  static_assert(Cfg::NT == 1024, "launch bounds");
  constexpr int T = Cfg::T, CB = Cfg::CB, TILE = Cfg::TILE;
  __shared__ __attribute__((aligned(1024))) uint8_t smem[Cfg::LDS];
  __shared__ int s_slow, s_last;
  uint8_t* const alds = smem;
  const uint8_t* const slds = smem + Cfg::A_BYTES;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int S = p.splits;
  const int r = (int)blockIdx.x % S, g = (int)blockIdx.x / S;
  const int M = p.M, N = p.N, K = p.K;
  const int Kh = K >> 1, G = K >> 5;
  const int kr0 = r * KR;
  if (tid == 0) s_slow = 0;

  f32x4 acc[CB];
#pragma unroll
  for (int cb = 0; cb < CB; ++cb) acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (wave >= Cfg::CWAVES) {
    // ============================ loader wave ============================
    const int lw = wave - Cfg::CWAVES;
    const desc_t da = make_desc(p.A);
#pragma unroll
    for (int d = 0; d < Cfg::A_DMAS; ++d) {
      const int D = lw * Cfg::A_DMAS + d;           // 1 KB block of the slice
      const int cw = D / (Cfg::A_RANGE / 1024);     // compute wave's range
      const int o = (D % (Cfg::A_RANGE / 1024)) * 1024;
      const int m = o / Cfg::A_ROWB;
      const int j = ((o % Cfg::A_ROWB) >> 4) + lane;  // LDS chunk position in the row
      const int src = j ^ (m & 7);
      const int k = kr0 + cw * Cfg::KWV;            // first K of the range
      if (m >= M) continue;                         // rows past M are never read
      dma16(da, alds + D * 1024, k < K ? (uint32_t)m * (uint32_t)K * 2u + 2u * (uint32_t)k + 16u * src : kOobOffset);
    }
    __builtin_amdgcn_s_barrier();  // B0: the activation DMAs are queued ahead of every weight load
    wait_vmcnt0();
    __builtin_amdgcn_s_barrier();  // B1: activations in LDS
  } else {
    // ============================ compute wave ===========================
    const int c = lane & 15, q = lane >> 4;
    const int cw = wave;
    const int k0 = kr0 + cw * Cfg::KWV;  // K % KWV == 0: a range is all in or all out
    const bool kok = k0 < K;
    constexpr int NL = T * CB, D = Cfg::DEPTH < NL ? Cfg::DEPTH : NL;
    u32x4 w[NL];
    // weight load i = (t, cb) = (i / CB, i % CB): bytes 64t + 16q .. +15 of
    // the range of column 16cb + c (columns past N read column N-1)
    auto issue = [&](int i) __attribute__((always_inline)) {
      const int t = i / CB, cb = i % CB;
      const int n = CW * g + 16 * cb + c;
      const int nc = n < N ? n : N - 1;
      w[i] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4*>(p.B + (size_t)nc * Kh + (k0 >> 1) + 64 * t + 16 * q));
    };
    __builtin_amdgcn_s_barrier();  // B0
    __builtin_amdgcn_sched_barrier(0);
    if (kok) {
      // this wave's scale block (CW columns x KWV/32 groups = 1 KB) into its
      // LDS slot, ahead of its weights: it lands first, with the first weights
      const int byte = 16 * lane;
      const int cl = byte / Cfg::SW_COL, gi = k0 / 32 + byte % Cfg::SW_COL;
      const int n = CW * g + cl;
      dma16(make_desc(p.S), slds + cw * 1024, n < N ? (uint32_t)n * (uint32_t)G + (uint32_t)gi : kOobOffset);
#pragma unroll
      for (int i = 0; i < D; ++i) issue(i);
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();  // B1 (the weights stay in flight)
    __builtin_amdgcn_sched_barrier(0);
    if (kok) {
      // the scale DMA was issued before the D weight loads: it has landed once
      // at most D are outstanding (an asm wait: the compiler does not see the
      // DMA)
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(D) : "memory");
      __builtin_amdgcn_sched_barrier(0);
      bool nok[CB];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) nok[cb] = CW * g + 16 * cb + c < N;
      const bool rok = c < M;  // activation rows past M are not in LDS: zero operands
      const uint8_t* const arow = alds + cw * Cfg::A_RANGE + (rok ? c : 0) * Cfg::A_ROWB;
      const int swz = c & 7;
#pragma unroll
      for (int t = 0; t < T; ++t) {
        u32x4 a[4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
          a[s] = rok ? *reinterpret_cast<const u32x4*>(arow + 16 * ((16 * t + 4 * q + s) ^ swz))
                     : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          const int i = t * CB + cb;
          // groups 4t .. 4t+3 of the range for column 16cb + c; this lane's is byte q
          const uint32_t sw = *reinterpret_cast<const uint32_t*>(slds + cw * 1024 + (16 * cb + c) * Cfg::SW_COL + 4 * t);
          const float scale = e8m0_to_f32(sw >> (8 * q));
          const u32x4 wv = nok[cb] ? w[i] : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
          for (int s = 0; s < 4; ++s)
            acc[cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a[s]), operand_from_word(wv[s], scale), acc[cb]);
          // keep D loads in flight: the next one is issued as this one is consumed
          if (i + D < NL) {
            __builtin_amdgcn_sched_barrier(0);
            issue(i + D);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
    }
    // the partial tile (rows 4q + i < MR, column 16cb + c) into this wave's
    // own activation range, which no other wave reads
    float* const part = reinterpret_cast<float*>(alds + cw * Cfg::A_RANGE);
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (4 * q + i < MR) part[(4 * q + i) * CW + 16 * cb + c] = acc[cb][i];
  }
  __syncthreads();  // B2: the partial tiles

  // the CTA's sum in wave order: thread tid < ACTIVE owns elements 4 tid .. +3
  const bool active = tid < Cfg::ACTIVE;
  f32x4 own = f32x4{0.f, 0.f, 0.f, 0.f};
  if (active) {
    own = *reinterpret_cast<const f32x4*>(alds + 16 * tid);
#pragma unroll
    for (int v = 1; v < Cfg::CWAVES; ++v) own += *reinterpret_cast<const f32x4*>(alds + v * Cfg::A_RANGE + 16 * tid);
  }
  const int row = tid / (CW / 4), col = CW * g + 4 * (tid % (CW / 4));
  auto store_c = [&](f32x4 x) __attribute__((always_inline)) {
    if (!active || row >= M) return;
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = p.ep.any ? epilogue_value(p.ep, x[i], row, col + i, N) : x[i];
    if (p.out_bf16) {
      uint16_t* out = static_cast<uint16_t*>(p.C) + (size_t)row * N + col;
      if ((N & 3) == 0 && col + 3 < N) {
        *reinterpret_cast<u32x2*>(out) = u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < N) out[i] = (uint16_t)bf16_bits_rne(y[i]);
      }
    } else {
      float* out = static_cast<float*>(p.C) + (size_t)row * N + col;
      if ((N & 3) == 0 && col + 3 < N) {
        *reinterpret_cast<f32x4*>(out) = f32x4{y[0], y[1], y[2], y[3]};
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (col + i < N) out[i] = y[i];
      }
    }
  };
  if (S == 1) {
    store_c(own);
    return;
  }

  // ---- split-K across the group's S CTAs ----
  const __amdgpu_buffer_rsrc_t pr = make_rsrc(p.partials);
  auto packet_off = [&](int rs_) __attribute__((always_inline)) {
    return (uint32_t)((((size_t)g * S + rs_) * TILE + 4 * tid) * 8);
  };
  auto publish = [&]() __attribute__((always_inline)) {
    if (active) store_packets(pr, packet_off(r), own, kTag);
  };
  auto clear = [&](int rs_) __attribute__((always_inline)) {
    if (!active) return;
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, pr, packet_off(rs_), 0, kCPolDevice);
    __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, pr, packet_off(rs_) + 16, 0, kCPolDevice);
  };
  // Split rs_'s packets of this thread, polled until tagged: at most `limit`
  // rounds (limit < 0: 2^20 rounds, only for packets already published,
  // whose stores are in flight).  Whole waves without outputs return at once.
  auto poll = [&](int rs_, int limit, f32x4& val) __attribute__((always_inline)) -> bool {
    if (tid >= Cfg::ACTIVE) {
      val = f32x4{0.f, 0.f, 0.f, 0.f};
      return true;
    }
    for (int it = 0;; ++it) {
      const u32x4 x0 = load_packets(pr, packet_off(rs_)), x1 = load_packets(pr, packet_off(rs_) + 16);
      if (__builtin_amdgcn_ballot_w64(tagged(x0, x1)) == __builtin_amdgcn_ballot_w64(true)) {
        val = packet_values(x0, x1);
        return true;
      }
      if (limit >= 0 ? it >= limit : it >= (1 << 20)) return false;
      __builtin_amdgcn_s_sleep(1);
    }
  };
  // The last of the S arrivals: every split published; sum in split order
  // (NaN instead of a partial sum if a published packet never showed up).
  auto reduce_all = [&]() __attribute__((always_inline)) {
    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
    bool ok = true;
    for (int rs_ = 0; rs_ < S; ++rs_) {
      f32x4 v = own;
      if (rs_ != r) ok = poll(rs_, -1, v) && ok;
      tot = rs_ == 0 ? v : tot + v;
    }
    const float nan = __builtin_nanf("");
    store_c(ok ? tot : f32x4{nan, nan, nan, nan});
    for (int rs_ = 0; rs_ < S; ++rs_) clear(rs_);
    if (tid == 0) __hip_atomic_store(p.counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  auto arrive_and_maybe_reduce = [&]() __attribute__((always_inline)) {
    __syncthreads();  // every wave has issued its packet stores
    if (tid == 0)
      s_last = (int)((__hip_atomic_fetch_add(p.counters + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) &
                      kArrivals) == (uint32_t)(S - 1));
    __syncthreads();
    if (s_last) reduce_all();
  };

  if (r != S - 1) {
    publish();
    arrive_and_maybe_reduce();
    return;
  }
  // reducer: the other splits in split order, then its own
  f32x4 others = f32x4{0.f, 0.f, 0.f, 0.f};
  bool fast = true;
  for (int rs_ = 0; rs_ < S - 1 && fast; ++rs_) {
    f32x4 v;
    fast = poll(rs_, p.spin_limit, v);
    others = rs_ == 0 ? v : others + v;
  }
  if (!fast) s_slow = 1;
  __syncthreads();
  if (s_slow == 0) {
    store_c(others + own);
    for (int rs_ = 0; rs_ < S - 1; ++rs_) clear(rs_);
    // The S - 1 arrivals and this subtraction net to zero in any order, and
    // no arrival can see S - 1 arrivals before it (so none reduces).
    if (tid == 0)
      __hip_atomic_fetch_add(p.counters + g, (uint32_t)(1 - S), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  publish();
  arrive_and_maybe_reduce();
}

using Dec16 = DecodeCfg<16, 64, 4096>;  // M <= 16: 64 columns x 4096 K per CTA
using Dec8 = DecodeCfg<8, 32, 8192>;    // M <= 8: 32 columns x 8192 K per CTA

// ---- resident kernel: every weight byte of the CTA in flight at entry ------
// One CTA of K / 512 waves per 32 columns x the whole K (K <= 8192, no split,
// no workspace).  Wave w owns K range 512w .. 512w+511.  At entry it issues,
// as plain global loads straight into VGPRs: its MR activation rows (1 KB
// each, contiguous), its 2 x 16 scale bytes and its 8 weight loads (16
// columns x 64 contiguous bytes per load, the MFMA operand order: 32
// VGPRs) -- nothing else is in its way, and the loads return in issue order.
// Measured on MI355X (N = K = 8192, graph-replayed, weights rotated past the
// MALL): the weight read alone in this pattern takes 7.9 us (4.3 TB/s); the
// whole kernel 9.6 us at M = 1 against 10.4 us for the whole-K streaming
// kernel (scale loads +0.3 us, activations +0.2 us, the wave reduction
// +0.1 us).  Non-temporal loads were slower here (10.0 us).  With more rows
// the activation bytes per CU grow (M = 8: 128 KB, 11.9 us -- the decode
// kernel above takes 11.7 us), so the auto plan uses it at M = 1.
// * K order: load j = (ct, jj) of lane (c, q) holds bytes 64jj + 16q .. +15
//   of the wave's 256-byte segment of column 16ct + c: K 512w + 128jj + 32q
//   + 0..31.  MFMA (jj, s) takes word s (K .. + 8s .. +7) against activation
//   chunk 16jj + 4q + s of row c; its scale is group 16w + 4jj + q, byte q of
//   word jj of the lane's 16 scale bytes.
// * Activations: the wave writes its rows to its own LDS slice (chunk j of
//   row r at j ^ r: a 16-lane operand read hits 8 distinct 16-byte slots)
//   and reads the MFMA operands back; only lanes with c < M read (the others
//   give zeros).
// * The waves' partial tiles are summed in wave order (bit-reproducible) and
//   stored with the fused epilogue.  Columns past N load column N - 1 and are
//   not stored.
template <int MR>
__global__ void __launch_bounds__(1024, 1) resident_kernel(StreamArgs p) {
  static_assert(MR == 1 || MR == 8, "activation rows");
  __shared__ __attribute__((aligned(16))) uint8_t alds[16 * MR * 1024];
  __shared__ __attribute__((aligned(16))) float red[16][MR * 32];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = (int)(blockDim.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int M = p.M, N = p.N, K = p.K;
  const int col0 = 32 * (int)blockIdx.x;
  const size_t Kh = (size_t)(K >> 1), G = (size_t)(K >> 5);

  // No branch ahead of the loads: rows past M load row M - 1 and are zeroed once
  // landed, and row 0 (M >= 1) is never selected (a branch on M made the
  // first load wait for a second round trip of kernel-argument loads, 10.3
  // against 9.6 us at M = 1, or sank a load below the others and drained
  // them all before the first MFMA).
  u32x4 av[MR];
#pragma unroll
  for (int r = 0; r < MR; ++r)
    av[r] = *reinterpret_cast<const u32x4*>(p.A + (size_t)min(r, M - 1) * K + 512 * w + 8 * lane);
  int cc[2];
  u32x4 sv[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    cc[ct] = min(col0 + 16 * ct + c, N - 1);
    sv[ct] = *reinterpret_cast<const u32x4*>(p.S + (size_t)cc[ct] * G + 16 * w);
  }
  u32x4 wv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    wv[j] = *reinterpret_cast<const u32x4*>(p.B + (size_t)cc[j >> 2] * Kh + 256 * w + 64 * (j & 3) + 16 * q);

  // slots of waves this CTA does not have (K < 8192) add zeros in the reduction
  for (int i = (int)threadIdx.x; i < (16 - nw) * MR * 32; i += (int)blockDim.x) red[nw + i / (MR * 32)][i % (MR * 32)] = 0.f;

  uint8_t* const my = alds + w * MR * 1024;
#pragma unroll
  for (int r = 0; r < MR; ++r)
    *reinterpret_cast<u32x4*>(my + r * 1024 + 16 * (lane ^ r)) = (r == 0 || r < M) ? av[r] : u32x4{0u, 0u, 0u, 0u};
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave reads only its own slice
  __builtin_amdgcn_wave_barrier();

  const int rc = c < MR ? c : 0;
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int ct = j >> 2, jj = j & 3;
    const float f = e8m0_to_f32((sv[ct][jj] >> (8 * q)) & 0xFFu);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 b = operand_from_word(wv[j][s], f);
      const int ch = 16 * jj + 4 * q + s;
      u32x4 a = u32x4{0u, 0u, 0u, 0u};
      if (c < M && c < MR) a = *reinterpret_cast<const u32x4*>(my + rc * 1024 + 16 * (ch ^ rc));
      acc[ct] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a), b, acc[ct]);
    }
  }
  // D lane (c, q) holds rows 4q .. 4q+3 of column c
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * q + i < MR) red[w][(4 * q + i) * 32 + 16 * ct + c] = acc[ct][i];
  __syncthreads();
  for (int e = threadIdx.x; e < MR * 32; e += blockDim.x) {
    const int row = e >> 5, col = col0 + (e & 31);
    if (row >= M || col >= N) continue;
    // all 16 slots read at once and added in wave order (slots past nw hold
    // zeros): a loop bounded by nw issued the reads one round trip at a time,
    // and per-slot conditions cost 22 SGPRs (two CTAs per CU no longer fit)
    float x = red[0][e];
#pragma unroll
    for (int ww = 1; ww < 16; ++ww) x += red[ww][e];
    const float y = p.ep.any ? epilogue_value(p.ep, x, row, col, N) : x;
    if (p.out_bf16)
      static_cast<uint16_t*>(p.C)[(size_t)row * N + col] = (uint16_t)bf16_bits_rne(y);
    else
      static_cast<float*>(p.C)[(size_t)row * N + col] = y;
  }
}

// ---- resident split kernel: 17 <= M <= 32 ------------------------------------
// M = 1 form with whole column segments per load (variant 13).  A bare read
// of the decode weights with 4 columns x 256 contiguous bytes per load takes
// 7.1 us against 7.9 us in the MFMA operand order (16 columns x 64 bytes).
// At M = 1 an MFMA uses one row of 16, so this form drops it: lane (r, e) of
// load j holds bytes 16e .. 16e+15 (K 32e .. 32e+31 of the wave's 512) of
// column 4j + r, converts them with their scale and takes v_dot2_f32_bf16
// products with the same 32 activations in K order; the 16 lanes of a
// column are summed by xor shuffles (8, 4, 2, 1) and the waves in wave order.
// A word as the bf16 pair operand of v_dot2_f32_bf16.  Taken by value: a
// __builtin_bit_cast of a vector component (v.y) read component 0 here.
__device__ __forceinline__ bf16x2 bf16_pair(uint32_t v) { return __builtin_bit_cast(bf16x2, v); }

// OCC = 8 waves per SIMD (<= 64 VGPRs: two 16-wave CTAs share a CU) for grids
// past one CTA per CU; OCC = 1 otherwise (66 VGPRs; measured at M = 1, K =
// 8192: 9.4 against 9.9 us at N = 8192, and 28.7 against 25.9 us at N =
// 28672, where it fits one CTA per CU).
template <int OCC>
__global__ void __launch_bounds__(1024, OCC) resident_dot_kernel(StreamArgs p) {
  __shared__ __attribute__((aligned(16))) float red[16][32];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nw = (int)(blockDim.x >> 6);
  const int r = lane >> 4, e = lane & 15;
  const int N = p.N, K = p.K;
  const int col0 = 32 * (int)blockIdx.x;
  const size_t Kh = (size_t)(K >> 1), G = (size_t)(K >> 5);

  u32x4 av[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) av[s] = *reinterpret_cast<const u32x4*>(p.A + 512 * w + 32 * e + 8 * s);
  uint32_t sb[8];
  u32x4 wv[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) sb[j] = p.S[(size_t)min(col0 + 4 * j + r, N - 1) * G + 16 * w + e];
#pragma unroll
  for (int j = 0; j < 8; ++j)
    wv[j] = *reinterpret_cast<const u32x4*>(p.B + (size_t)min(col0 + 4 * j + r, N - 1) * Kh + 256 * w + 16 * e);

  for (int i = (int)threadIdx.x; i < (16 - nw) * 32; i += (int)blockDim.x) red[nw + i / 32][i % 32] = 0.f;

  float part[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float f = e8m0_to_f32(sb[j]);
    float acc = 0.f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      const uint32_t b0 = fp4x2_to_bf16x2<0>(wv[j][d], f), b1 = fp4x2_to_bf16x2<1>(wv[j][d], f);
      const uint32_t b2 = fp4x2_to_bf16x2<2>(wv[j][d], f), b3 = fp4x2_to_bf16x2<3>(wv[j][d], f);
      acc = __builtin_amdgcn_fdot2_f32_bf16(bf16_pair(b0), bf16_pair(av[d].x), acc, false);
      acc = __builtin_amdgcn_fdot2_f32_bf16(bf16_pair(b1), bf16_pair(av[d].y), acc, false);
      acc = __builtin_amdgcn_fdot2_f32_bf16(bf16_pair(b2), bf16_pair(av[d].z), acc, false);
      acc = __builtin_amdgcn_fdot2_f32_bf16(bf16_pair(b3), bf16_pair(av[d].w), acc, false);
    }
    part[j] = acc;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) part[j] += __shfl_xor(part[j], m, 16);
  if (e == 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j) red[w][4 * j + r] = part[j];
  }
  __syncthreads();
  if (threadIdx.x < 32) {
    const int col = col0 + (int)threadIdx.x;
    if (col >= N) return;
    float x = red[0][threadIdx.x];
#pragma unroll
    for (int ww = 1; ww < 16; ++ww) x += red[ww][threadIdx.x];
    const float y = p.ep.any ? epilogue_value(p.ep, x, 0, col, N) : x;
    if (p.out_bf16)
      static_cast<uint16_t*>(p.C)[col] = (uint16_t)bf16_bits_rne(y);
    else
      static_cast<float*>(p.C)[col] = y;
  }
}

// One CTA of 8 waves per 128 columns x 2048 K (S = ceil(K / 2048) CTAs per
// column group); wave w owns K 256w .. 256w+255 of the CTA's range.  At entry
// every wave issues its 32 activation rows (16 loads of 1 KB: 2 rows x 512 B
// each), 8 x 8 scale bytes and 16 weight loads in the MFMA operand order (8
// column blocks x 2 halves of 128 K: 64 VGPRs), all straight into VGPRs.
// The activations go to the wave's own LDS slice (chunk j of row r at
// j ^ (r & 7)); both 16-row halves run against the same weight registers,
// so the weights are converted once for 32 rows.  Measured on MI355X (N = K
// = 8192, M = 32, graph-replayed): 14.6 us for the kernel body against
// 21.2 us for the split-K streaming kernel, whose 8-byte packets for 4
// splits of 32-column units wrote 25 MB per launch.
// * K order: half h, word s of lane (c, q) holds K k0 + 128h + 32q + 8s .. +7
//   of column 16cb + c (k0 = the wave's first K); activation chunk
//   16h + 4q + s of the wave's slice; scale group 4h + q, byte q of word h
//   of the lane's 8 scale bytes.
// * The 8 wave tiles (32 x 128 fp32) are summed in wave order through the
//   LDS (the activation slices are dead by then); thread t owns elements
//   4t .. 4t+3 and 2048 + 4t .. +3.  K splits meet as plain fp32 partials
//   summed in split order by the last arrival on the group counter (no
//   polling, so nothing assumes the CTAs are co-resident; bit-reproducible).
// * Waves whose K range is past K load the last range and zero their
//   weights; columns past N load column N-1 and are not stored; rows past M
//   load row M-1 and their operands are zeroed when read back (a condition
//   on the stored value let the compiler sink a load below the others and
//   drain them all first).
constexpr int kRsCols = 128, kRsKr = 2048, kRsWaves = 8;

// MT 16-row tiles (M <= 16 MT); MT = 1 fits two CTAs per CU (4 waves per
// SIMD: <= 128 VGPRs; the second launch bound is waves per SIMD).
template <int MT>
__global__ void __launch_bounds__(512, MT == 1 ? 4 : 2) resident_split_kernel(StreamArgs p) {
  constexpr int kRsTile = 16 * MT * kRsCols;  // floats per CTA tile
  __shared__ __attribute__((aligned(16))) uint8_t smem[kRsWaves * MT * 8192];
  __shared__ int s_last;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int S = p.splits;
  const int r = (int)blockIdx.x % S, g = (int)blockIdx.x / S;
  const int M = p.M, N = p.N, K = p.K;
  const size_t Kh = (size_t)(K >> 1), G = (size_t)(K >> 5);
  const int k0 = r * kRsKr + 256 * w;
  const bool kok = k0 < K;  // K % 256 == 0: a wave's range is all in or all out
  const int kl = kok ? k0 : K - 256;
  const int col0 = kRsCols * g;

  u32x4 av[8 * MT];
#pragma unroll
  for (int i = 0; i < 8 * MT; ++i) {
    const int row = min(2 * i + (lane >> 5), M - 1);
    av[i] = *reinterpret_cast<const u32x4*>(p.A + (size_t)row * K + kl + 8 * (lane & 31));
  }
  u32x2 sv[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb)
    sv[cb] = *reinterpret_cast<const u32x2*>(p.S + (size_t)min(col0 + 16 * cb + c, N - 1) * G + kl / 32);
  u32x4 wv[8][2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
      wv[cb][h] = *reinterpret_cast<const u32x4*>(p.B + (size_t)min(col0 + 16 * cb + c, N - 1) * Kh + kl / 2 +
                                                  64 * h + 16 * q);

  uint8_t* const my = smem + w * MT * 8192;
#pragma unroll
  for (int i = 0; i < 8 * MT; ++i) {
    const int row = 2 * i + (lane >> 5), ch = lane & 31;
    *reinterpret_cast<u32x4*>(my + row * 512 + 16 * (ch ^ (row & 7))) = av[i];
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the wave reads only its own slice
  __builtin_amdgcn_wave_barrier();

  f32x4 acc[MT][8];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int cb = 0; cb < 8; ++cb) acc[mt][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int ch = 16 * h + 4 * q + s;
      u32x4 a[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        a[mt] = *reinterpret_cast<const u32x4*>(my + (16 * mt + c) * 512 + 16 * (ch ^ (c & 7)));
        if (16 * mt + c >= M) a[mt] = u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int cb = 0; cb < 8; ++cb) {
        // a wave past K multiplies zero codes by 2^0 (its loaded scales may be 0xFF: NaN)
        const float f = e8m0_to_f32(kok ? (sv[cb][h] >> (8 * q)) & 0xFFu : 127u);
        const bf16x8 b = operand_from_word(kok ? wv[cb][h][s] : 0u, f);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt][cb] = mfma_16x16x32(__builtin_bit_cast(bf16x8, a[mt]), b, acc[mt][cb]);
      }
    }
  __syncthreads();  // every wave has read its activations: the LDS now takes the tiles
  float* const part = reinterpret_cast<float*>(smem) + w * kRsTile;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int cb = 0; cb < 8; ++cb)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[(16 * mt + 4 * q + i) * kRsCols + 16 * cb + c] = acc[mt][cb][i];
  __syncthreads();

  // the CTA's sum in wave order: thread t owns elements 4t .. 4t+3 (v = 0)
  // and 2048 + 4t .. +3 (v = 1)
  f32x4 own[MT];
#pragma unroll
  for (int v = 0; v < MT; ++v) {
    const float* src = reinterpret_cast<const float*>(smem) + 2048 * v + 4 * tid;
    own[v] = *reinterpret_cast<const f32x4*>(src);
#pragma unroll
    for (int ww = 1; ww < kRsWaves; ++ww) own[v] += *reinterpret_cast<const f32x4*>(src + ww * kRsTile);
  }
  auto store_c = [&](const f32x4 (&x)[MT]) __attribute__((always_inline)) {
#pragma unroll
    for (int v = 0; v < MT; ++v) {
      const int e = 2048 * v + 4 * tid;
      const int row = e / kRsCols, col = col0 + e % kRsCols;
      if (row >= M) continue;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = p.ep.any ? epilogue_value(p.ep, x[v][i], row, col + i, N) : x[v][i];
      if (p.out_bf16) {
        uint16_t* out = static_cast<uint16_t*>(p.C) + (size_t)row * N + col;
        if ((N & 3) == 0 && col + 3 < N) {
          *reinterpret_cast<u32x2*>(out) = u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (col + i < N) out[i] = (uint16_t)bf16_bits_rne(y[i]);
        }
      } else {
        float* out = static_cast<float*>(p.C) + (size_t)row * N + col;
        if ((N & 3) == 0 && col + 3 < N) {
          *reinterpret_cast<f32x4*>(out) = f32x4{y[0], y[1], y[2], y[3]};
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (col + i < N) out[i] = y[i];
        }
      }
    }
  };
  if (S == 1) {
    store_c(own);
    return;
  }

  // ---- split-K across the group's S CTAs ----
  // Plain fp32 partials (rows < M) with device-coherent stores; the last of
  // the S arrivals on the group counter sums the splits in split order (its
  // own from registers, every other split's loads in flight together) and
  // resets the counter.  Tagged packets (8 bytes per value, cleared after
  // use) cost 23.2 us here at M = 32: 19 MB of packet traffic per launch.
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(p.partials + (size_t)g * S * kRsTile);
  bool live[MT];
#pragma unroll
  for (int v = 0; v < MT; ++v) {
    live[v] = (2048 * v + 4 * tid) / kRsCols < M;
    if (live[v]) store_coherent(rp, (uint32_t)((r * kRsTile + 2048 * v + 4 * tid) * 4), own[v]);
  }
  if (!splitk_arrive_last(p.counters + g, (uint32_t)S, &s_last, tid)) return;
  f32x4 t[8][MT];
#pragma unroll
  for (int sp = 0; sp < 8; ++sp)
#pragma unroll
    for (int v = 0; v < MT; ++v)
      t[sp][v] = sp < S && sp != r && live[v] ? load_coherent4(rp, (uint32_t)((sp * kRsTile + 2048 * v + 4 * tid) * 4))
                                              : own[v];
  f32x4 tot[MT];
#pragma unroll
  for (int v = 0; v < MT; ++v) tot[v] = t[0][v];
#pragma unroll
  for (int sp = 1; sp < 8; ++sp)
#pragma unroll
    for (int v = 0; v < MT; ++v)
      if (sp < S) tot[v] += t[sp][v];
  store_c(tot);
}

}  // namespace

int64_t resident_splits(int rows, int64_t K) { return rows >= 16 ? (K + kRsKr - 1) / kRsKr : 1; }
int64_t resident_groups(int rows, int64_t N) {
  const int64_t cw = rows >= 16 ? kRsCols : 32;
  return (N + cw - 1) / cw;
}
size_t resident_workspace(int rows, int64_t N, int64_t K) {
  const int64_t S = resident_splits(rows, K);
  return S > 1 ? (size_t)(resident_groups(rows, N) * S * rows * kRsCols * 4) : 0;
}

// Resident kernel shape rules: [N,K/2], 1 <= M <= rows.  rows 1 or 8: K a
// multiple of 512 up to 8192 (K / 512 waves of 64 lanes, no split).  rows 32:
// K a multiple of 256, at most 8 splits of 2048, one counter per 128-column
// group and the partials within 1 GiB.
bool resident_shape_ok(int rows, int layout, int64_t M, int64_t N, int64_t K) {
  if (layout != kLayoutNK || M < 1 || M > rows || N < 1) return false;
  if (rows == 1 || rows == 8) return K >= 512 && K <= 8192 && K % 512 == 0;
  return (rows == 16 || rows == 32) && K >= 256 && K % 256 == 0 && resident_splits(rows, K) <= 8 &&
         resident_groups(rows, N) * 4 <= (int64_t)MXFP4_COUNTER_BYTES &&
         resident_workspace(rows, N, K) <= (size_t)kNumRecords;
}

hipError_t launch_resident_dot(int layout, const StreamArgs& a, hipStream_t stream) {
  if (!resident_shape_ok(1, layout, a.M, a.N, a.K) || a.splits != 1) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)((a.N + 31) / 32), block = (unsigned)(a.K / 512 * 64);
  if (grid > 256)
    hipLaunchKernelGGL(resident_dot_kernel<8>, dim3(grid), dim3(block), 0, stream, a);
  else
    hipLaunchKernelGGL(resident_dot_kernel<1>, dim3(grid), dim3(block), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_resident(int rows, int layout, const StreamArgs& a, hipStream_t stream) {
  if (!resident_shape_ok(rows, layout, a.M, a.N, a.K) || a.splits != resident_splits(rows, a.K))
    return hipErrorInvalidValue;
  if (rows >= 16) {
    if (a.splits > 1 && (!a.partials || !a.counters)) return hipErrorInvalidValue;
    const unsigned grid = (unsigned)(resident_groups(rows, a.N) * a.splits);
    if (rows == 32)
      hipLaunchKernelGGL(resident_split_kernel<2>, dim3(grid), dim3(64 * kRsWaves), 0, stream, a);
    else
      hipLaunchKernelGGL(resident_split_kernel<1>, dim3(grid), dim3(64 * kRsWaves), 0, stream, a);
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((a.N + 31) / 32)), block((unsigned)(a.K / 512 * 64));
  if (rows == 1)
    hipLaunchKernelGGL(resident_kernel<1>, grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL(resident_kernel<8>, grid, block, 0, stream, a);
  return hipGetLastError();
}

int64_t decode_splits(int rows, int64_t K) {
  const int64_t kr = rows <= 8 ? 8192 : 4096;
  return (K + kr - 1) / kr;
}
int64_t decode_groups(int rows, int64_t N) {
  const int64_t cw = rows <= 8 ? 32 : 64;
  return (N + cw - 1) / cw;
}
size_t decode_workspace(int rows, int64_t N, int64_t K) {
  const int64_t S = decode_splits(rows, K);
  const int64_t tile = rows <= 8 ? 8 * 32 : 16 * 64;
  return S > 1 ? (size_t)(decode_groups(rows, N) * S * tile * 8) : 0;
}

// Shape rules: M <= rows (8 or 16), K a multiple of one compute wave's range
// (KR / 8: 1024 or 512 K), at most 8 splits, 32-bit offsets for activations,
// scales and packets, one counter per column group.
bool decode_shape_ok(int rows, int layout, int64_t M, int64_t N, int64_t K) {
  if (rows != 8 && rows != 16) return false;
  const int64_t kwv = rows <= 8 ? 1024 : 512;
  return layout == kLayoutNK && M >= 1 && M <= rows && K >= kwv && K % kwv == 0 && decode_splits(rows, K) <= 8 &&
         M * K * 2 < (int64_t)kOobOffset && N * (K / 32) < (int64_t)kOobOffset &&
         decode_workspace(rows, N, K) <= (size_t)kNumRecords && decode_groups(rows, N) * 4 <= (1 << 20);
}

hipError_t launch_decode(int rows, int layout, const StreamArgs& a, hipStream_t stream) {
  if (!decode_shape_ok(rows, layout, a.M, a.N, a.K) || a.splits != decode_splits(rows, a.K))
    return hipErrorInvalidValue;
  if (a.splits > 1 && (!a.partials || !a.counters)) return hipErrorInvalidValue;
  const unsigned grid = (unsigned)(decode_groups(rows, a.N) * a.splits);
  if (rows <= 8)
    hipLaunchKernelGGL((decode_kernel<8, 32, 8192>), dim3(grid), dim3(Dec8::NT), 0, stream, a);
  else
    hipLaunchKernelGGL((decode_kernel<16, 64, 4096>), dim3(grid), dim3(Dec16::NT), 0, stream, a);
  return hipGetLastError();
}

}  // namespace mxfp4
