// extern "C" entry points (include/mxfp4_mi355x.h): argument checks, the
// 256-CU cost model that picks a kernel plan, workspace layout, launch.
//
// Reference counterparts: dispatch/check_inputs (csrc/mxfp4_ext.cpp:11-48),
// launch_strategy_* (csrc/common.h:43-78), gemm_auto (python/mxfp4_cdna3/
// kernels.py:63-74), shape_supported_* (csrc/common.h:80-99), device_info
// (csrc/mxfp4_ext.cpp:156-168), cost_model.predict (python/mxfp4_cdna3/
// cost_model.py:117-146).
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "mxfp4_kernels.h"
#include "../../include/mxfp4_mi355x.h"

namespace mxfp4 {
namespace {

// ---- MI355X roofline constants (dense, no sparsity) ------------------------
constexpr double kNumCus = 256.0;
constexpr double kHbmBytesPerS = 8.0e12;
constexpr double kMfmaFlopsPerS = 2.5e15;
constexpr double kLaunchS = 2.0e-6;  // fixed per-launch cost folded into every plan
// [N,K/2] -> G rewrite of a via-G plan: fraction of HBM bandwidth it moves its
// bytes (read + write of codes and scales) at
constexpr double kConvertEff = 0.6;

// Tiled kernel families: the first version (mxfp4_tiled.hip), the pipelined
// kernel (mxfp4_tiled_pipe.hip) and the hand-scheduled 128 x 256 kernel
// (mxfp4_tiled_sched.hip; [K/2,N] and G weights with K % 64 == 0, [N,K/2]
// with K % 128 == 0).
constexpr int kFamilyPlain = 0, kFamilyPipe = 1, kFamilySched = 2;

struct TiledVariant {
  TiledShape shape;
  double eff_kn, eff_nk;  // sustained fraction of the 2.5 PF/s peak, per weight layout (measured)
  int ctas_per_cu;        // residency (registers / LDS)
  int family;             // kFamily*: which tiled kernel runs the shape
};

// Tile variants of the tiled family; index = mxfp4_plan.variant.  The
// efficiencies are calibrated on MI355X with seeded random data (A ~ N(0,1),
// uniform E2M1 codes), where power limits the MFMA rate well below peak.
// Variants 6, 7 and 15: the median over the MFMA-bound BASELINE configs
// (dit_up, dit_down, 70B FFN M = 512 / 2048 / 8192) of peak time / measured
// time, fitted from a bench.py --sweep CSV by cost_model.fit_efficiency
// (eff_kn is the [K/2,N] fit; G measures 0.580 / 0.497 / 0.437); 3 and 5
// were measured after the split-K reduction change at M = 48 .. 1024 and
// are scaled with variant 15 at each refit, per layout, so their standing
// against the fitted variants is kept.  The model then picks within 12 % of
// the best measured plan on those shapes.
const TiledVariant kTiled[] = {
    // 0, 1, 2, 4, 8 .. 14: explicit plans only (efficiency 0: never
    // auto-selected); their last calibration predates the store-loop and
    // split-K changes
    {{2, 2, 4}, 0.0, 0.0, 1, kFamilyPlain},         // 0: 256 x 256, 4 waves, 128 x 128 per wave
    {{4, 2, 2}, 0.0, 0.0, 1, kFamilyPlain},         // 1: 256 x 256, 8 waves
    {{2, 2, 2}, 0.0, 0.0, 2, kFamilyPlain},         // 2: 128 x 256
    {{1, 2, 2}, 0.173, 0.150, 2, kFamilyPlain},     // 3:  64 x 256 (re-measured at M = 64 .. 256)
    {{2, 1, 2}, 0.0, 0.0, 2, kFamilyPlain},         // 4: 128 x 128
    {{1, 2, 1}, 0.152, 0.131, 4, kFamilyPlain},     // 5:  32 x 256 (re-measured at M = 48 .. 1024)
    {{4, 2, 2, 4, 3}, 0.501, 0.475, 1, kFamilyPipe}, // 6: pipelined 256 x 256, 8 waves of 64 x 128, 3 stages
    {{2, 2, 2, 4, 3}, 0.431, 0.390, 1, kFamilyPipe}, // 7: pipelined 128 x 256, 4 waves of 64 x 128
    {{4, 2, 2, 4, 3}, 0.0, 0.0, 1, kFamilyPipe},   // 8: = 6 (a 4-stage 256 x 256 ring no longer fits 160 KB)
    {{2, 4, 4, 2, 3}, 0.0, 0.0, 1, kFamilyPipe},   // 9: = 10
    {{2, 4, 4, 2, 3}, 0.0, 0.0, 1, kFamilyPipe},   // 10: pipelined 256 x 256, 8 waves of 128 x 64, 3 stages
    {{2, 2, 2, 4, 4}, 0.0, 0.0, 1, kFamilyPipe},   // 11: as 7 with 4 stages
    {{2, 4, 2, 2, 4}, 0.0, 0.0, 1, kFamilyPipe},   // 12: pipelined 128 x 256, 8 waves of 64 x 64
    {{1, 4, 4, 2, 4}, 0.0, 0.0, 1, kFamilyPipe},   // 13: pipelined 128 x 256, 4 waves of 128 x 64
    {{2, 1, 2, 4, 4}, 0.0, 0.0, 2, kFamilyPipe},   // 14: pipelined 128 x 128, 2 waves
    {{2, 2, 2, 4, 3}, 0.561, 0.491, 2, kFamilySched}, // 15: hand-scheduled 128 x 256, 4 waves of 64 x 128, 2 CTAs / CU
};
constexpr int kNumTiled = sizeof(kTiled) / sizeof(kTiled[0]);

// Shapes of the memory-bound family; index = mxfp4_plan.variant.
// (mt, cb, wpc, u) -- same order as MXFP4_GEMV_SHAPES in mxfp4_gemv.hip.
const GemvShape kGemv[] = {
    {1, 8, 8, 4},  {1, 16, 8, 2}, {1, 8, 16, 2}, {1, 4, 16, 4}, {2, 8, 8, 2}, {2, 4, 16, 2},
    {1, 2, 16, 4}, {2, 2, 16, 2}, {1, 4, 8, 4},  {1, 2, 8, 4},  {2, 4, 8, 2}, {1, 8, 4, 4},
    {1, 2, 16, 2}, {1, 4, 16, 2}, {1, 8, 8, 2},
};
constexpr int kNumGemv = sizeof(kGemv) / sizeof(kGemv[0]);

// Shapes of the streaming split-K family ([N,K/2], M <= 32); index =
// mxfp4_plan.variant.  (mt, waves, gcb, nslot, smax) -- same order as
// MXFP4_STREAM_SHAPES in mxfp4_stream.hip.  Splits are fixed by the shape:
// ceil(K / (waves * 256)).
const StreamShape kStream[] = {
    {1, 8, 2, 4, 4, 256},  // 0: M <= 16, split 2048 K (K <= 8192)
    {1, 4, 2, 8, 8, 256},  // 1: M <= 16, split 1024 K (K <= 8192)
    {2, 4, 2, 8, 8, 256},  // 2: M <= 32, split 1024 K (K <= 8192)
    {1, 8, 2, 2, 2, 512},  // 3: M <= 16, split 4096 K (K <= 8192)
    {2, 4, 2, 4, 4, 512},  // 4: M <= 32, split 2048 K (K <= 8192)
    {1, 16, 2, 1, 1, 512}, // 5: whole K, M <= 16, K <= 8192 (K / 512 waves)
    {1, 16, 2, 1, 1, 256}, // 6: whole K, M <= 16, K <= 4096 (K / 256 waves)
    {1, 8, 4, 0, 8, 512, 16},  // 7: decode kernel, M <= 16, [N,K/2], 64 columns x 4096 K per CTA, K % 512 == 0
    {1, 8, 2, 0, 8, 1024, 8},  // 8: decode kernel, M <= 8, [N,K/2], 32 columns x 8192 K per CTA, K % 1024 == 0
    {1, 16, 2, 0, 1, 512, 0, 1},  // 9: resident kernel, M == 1, [N,K/2], 32 columns x K <= 8192 per CTA, K % 512 == 0
    {1, 16, 2, 0, 1, 512, 0, 8},  // 10: resident kernel, M <= 8 (explicit plans only)
    {2, 8, 8, 0, 8, 256, 0, 32},  // 11: resident split kernel, M <= 32, [N,K/2], 128 columns x 2048 K per CTA, K % 256 == 0
    {1, 8, 8, 0, 8, 256, 0, 16},  // 12: resident split kernel, M <= 16, two CTAs per CU
    {1, 16, 2, 1, 1, 512, 0, 1},  // 13: resident kernel, M == 1, whole-segment loads and dot products
};
constexpr int kNumStream = sizeof(kStream) / sizeof(kStream[0]);
constexpr int kStreamSpin = 4096;  // late-unit polls before counter arbitration
constexpr int64_t kRsrcBytes = 1LL << 30;  // range of one buffer descriptor (mxfp4_device.h kNumRecords)

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

double problem_bytes(int64_t M, int64_t N, int64_t K, int c_bytes) {
  return 2.0 * M * K + N * K / 2.0 + N * K / 32.0 + (double)c_bytes * M * N;
}

// Workspace bytes of the G copy of a via-G plan (codes, then scales).
size_t via_g_bytes(int64_t N, int64_t K) {
  return align_up((size_t)(K / 2) * N, 256) + align_up((size_t)(K / 32) * N, 256);
}
bool via_g_ok(int layout, int64_t N, int64_t K) {
  return layout == kLayoutNK && layout_shape_ok(kLayoutG, N, K) && K % 64 == 0;
}

int64_t stream_splits(const StreamShape& s, int64_t K) { return ceil_div(K, s.k_split()); }
int64_t stream_ctas(const StreamShape& s, int64_t N, int64_t K) {
  const int64_t splits = stream_splits(s, K);
  if (s.direct || s.resident) return ceil_div(N, 16 * s.gcb) * splits;
  return ceil_div(ceil_div(N, 32), splits) * splits;
}
bool stream_plan_ok(int layout, int64_t M, int64_t N, int64_t K, const StreamShape& s) {
  if (s.resident) return resident_shape_ok(s.resident, layout, M, N, K) && stream_splits(s, K) == resident_splits(s.resident, K);
  if (s.direct) return decode_shape_ok(s.direct, layout, M, N, K);
  if ((layout != kLayoutNK && layout != kLayoutP) || M > 16 * s.mt || K % s.kw != 0) return false;
  const int64_t splits = stream_splits(s, K);
  if (splits > s.smax) return false;
  if (splits > 1 && stream_ctas(s, N, K) * 4 > (int64_t)MXFP4_COUNTER_BYTES) return false;
  // the split-K packets are addressed through one buffer descriptor over the
  // partials (32-bit offsets, kNumRecords bytes)
  if (splits > 1 && stream_ctas(s, N, K) * splits * s.tile() * 8 > kRsrcBytes) return false;
  return stream_shape_available(s);
}

int gemv_steps(int layout, int64_t K) { return (int)(layout == kLayoutKN ? K / 32 : ceil_div(K, 128)); }

// Partial-tile floats per CTA of the memory-bound family.
int64_t gemv_tile(const GemvShape& g) { return 16LL * g.mt * 16 * g.cb; }

bool gemv_plan_ok(int layout, int64_t M, int64_t N, const GemvShape& g) {
  if (layout != kLayoutKN && layout != kLayoutNK) return false;
  if (M > 16 * g.mt) return false;
  if (layout == kLayoutKN && (N % 16 != 0 || g.cb < 4)) return false;
  return gemv_shape_available(layout, g);
}

void choose_tiled(int layout, int64_t M, int64_t N, int64_t K, mxfp4_plan* out, size_t max_ws);

// Memory-bound family.  [N,K/2]: 32 columns x the whole K per CTA of 16
// waves (no split needed once N >= 8192).  [K/2,N]: 128 columns per CTA and
// K split so the grid has ~256 CTAs; the split partials cost 8*S*M/K of the
// weight bytes, so S stays small.
void choose_gemv(int layout, int64_t M, int64_t N, int64_t K, mxfp4_plan* out) {
  const bool two = M > 16;
  // 16 < M <= 32 with [N,K/2]: the resident split kernel (variant 11: 128
  // columns x 2048 K per CTA, the weights converted once for 32 rows) first,
  // at any N (K = 8192, M = 17 / 32: 15.3 / 16.2 us at N = 8192 against 21.0
  // / 21.3 us streaming; 28.3 / 30.0 us at N = 16384 against 35.1 / 37.2 us
  // for the GEMV family below).
  // 8 < M <= 16 with [N,K/2] and N >= 16384: its 16-row form (variant 12,
  // two CTAs per CU; K = 8192, M = 16: 23.4 / 39.5 us at N = 16384 / 28672
  // against 24.8 / 42.2 us for the split-K streaming kernel, which stays
  // faster at N = 8192: 12.7 against 14.7 us).
  if ((two || (M > 8 && N >= 16384)) && layout == kLayoutNK) {
    const StreamShape& st = kStream[two ? 11 : 12];
    if (stream_plan_ok(layout, M, N, K, st) && stream_ctas(st, N, K) >= 192) {
      *out = {MXFP4_KERNEL_STREAM, two ? 11 : 12, (int32_t)stream_splits(st, K), 0};
      return;
    }
  }
  // [N,K/2] with enough column groups to fill the chip: the streaming split-K
  // kernel, first choice that fits (measured on MI355X at N = 8192 / 28672,
  // K = 8192: 512-K waves with 2 splits beat 256-K waves with 4; both beat
  // this family by 1.3-1.7x).
  // [N,K/2] with M > 16 and N >= 16384: the GEMV's 128-column CTAs reuse each
  // activation byte over twice the streaming kernel's columns (M = 24 / 32,
  // K = 8192: 32.5 / 33.7 us at N = 16384 and 56.4 / 58.5 us at N = 28672,
  // against 40.0 / 40.5 and 72.9 / 74.2 us streaming; at N = 8192 they tie)
  const bool wide_gemv = two && layout == kLayoutNK && N >= 16384;
  if ((layout == kLayoutNK || layout == kLayoutP) && !wide_gemv) {
    // M <= 8: the whole-K kernel first (256-K waves up to K = 4096).  It
    // reads 32 x K activation bytes per CU, which at M = 16 is twice the CU's
    // weight bytes; there the split-K kernel, which reuses each CTA's K range
    // of activations across two column groups, is faster (measured at
    // N = 8192 / 28672, K = 8192: whole-K 10.6 / 32.3 us at M = 1, 12.4 /
    // 40.7 us at M = 8, 15.8 / 52.7 us at M = 16; split-K 12.7 / 41.5 us at
    // M = 1, 13.1 / 42.7 us at M = 16).
    // 2 <= M <= 8 with [N,K/2]: the decode kernel with the activations in LDS
    // (variant 8) before those (M = 8: 11.8 / 39.4 us against 12.3 / 41.0 us
    // whole-K; at M = 1 the whole-K kernel is faster, 10.4 against 11.1 us).
    // M == 1 with [N,K/2] and K % 512 == 0, K <= 8192: the resident kernel's
    // dot-product form (variant 13) before those (N = 8192 / 28672, K = 8192:
    // 9.4 / 25.9 us against 10.0 / 27.1 us for its MFMA form, variant 9, and
    // 10.4 / 33.6 us whole-K).
    static const int kPrefer1[] = {13, 6, 5, 3, 0, 1}, kPrefer8[] = {8, 6, 5, 3, 0, 1}, kPrefer16[] = {3, 0, 1},
                     kPrefer32[] = {4, 2};
    const int* pref = two ? kPrefer32 : M == 1 ? kPrefer1 : M <= 8 ? kPrefer8 : kPrefer16;
    const int npref = two ? 2 : M == 1 ? 6 : M <= 8 ? 6 : 3;
    for (int i = 0; i < npref; ++i) {
      const StreamShape& st = kStream[pref[i]];
      if (stream_plan_ok(layout, M, N, K, st) && stream_ctas(st, N, K) >= 192) {
        *out = {MXFP4_KERNEL_STREAM, pref[i], (int32_t)stream_splits(st, K), 0};
        return;
      }
    }
  }
  if (layout != kLayoutKN && layout != kLayoutNK) {
    // prepacked layouts the streaming kernel does not take: the pipelined
    // tiled kernel with split-K
    choose_tiled(layout, M, N, K, out, 0);
    return;
  }
  int want;
  if (layout == kLayoutKN)
    // (2,8,8,2) / (1,8,8,4); M <= 16 with N >= 24576: 256-column CTAs and
    // split 2 (N = 28672, K = 8192: 28.5 / 29.9 / 32.2 us at M = 1 / 8 / 16
    // against 29.8 / 32.4 / 35.8 us with 128-column CTAs, which at N = 8192
    // are the faster ones)
    want = two ? 4 : N >= 24576 ? 1 : 0;
  else
    want = two ? (wide_gemv ? 4 : 7) : 6;  // (2,8,8,2) or (2,2,16,2) / (1,2,16,4)
  const GemvShape& g = kGemv[want];
  const int64_t groups = ceil_div(N, 16 * g.cb);
  const int64_t steps = gemv_steps(layout, K);
  int64_t splits = std::max<int64_t>(1, (256 + groups / 2) / groups);
  splits = std::min<int64_t>(splits, std::max<int64_t>(1, steps / g.wpc));
  out->kernel = MXFP4_KERNEL_GEMV;
  out->variant = want;
  out->split_k = (int32_t)splits;
  out->flags = 0;
}

// The G loader uses the [K/2,N] lane map and the panel loader the [N,K/2]
// one (mxfp4_tiled_pipe.hip).
double tiled_eff(const TiledVariant& v, int layout) {
  return layout == kLayoutKN || layout == kLayoutG ? v.eff_kn : v.eff_nk;
}

// Tiled variants a layout may use: the first tiled kernel has only the plain
// loaders, the scheduled kernel the plain and G ones ([N,K/2]: aligned scale
// dwords of K-step pairs), the pipelined kernel all four (its [N,K/2] loader
// reads aligned scale dwords).  The scheduled kernel stores 4 adjacent
// columns per lane and row (8 / 16 bytes): [N,K/2] needs N % 4 == 0 there
// ([K/2,N] has N % 16 == 0 and G N % 128 == 0 already), so that every group
// of 4 is inside the row and aligned.  Its [K/2,N] loader addresses the
// whole K range of a column block from one buffer descriptor (the K step is
// the scalar offset), so the codes must fit the descriptor's range; larger
// [K/2,N] weights take the kernels that rebase per K step.
bool tiled_variant_ok(const TiledVariant& v, int layout, int64_t N, int64_t K) {
  if (v.family == kFamilyPlain) return layout == kLayoutKN || layout == kLayoutNK;
  if (v.family == kFamilySched)
    return K % (layout == kLayoutNK ? 128 : 64) == 0 && N % 4 == 0 &&
           (layout != kLayoutKN || tiled_sched_kn_fits(N, K)) && tiled_sched_available(layout, v.shape);
  if (layout == kLayoutNK) return K % 128 == 0;
  if (layout == kLayoutG) return v.shape.bn() % kGCols == 0;
  return true;
}

double tiled_time(const TiledVariant& v, int layout, int64_t M, int64_t N, int64_t K, int splits) {
  const int bm = v.shape.bm(), bn = v.shape.bn();
  const int64_t tiles = ceil_div(M, bm) * ceil_div(N, bn);
  const int64_t ksteps = ceil_div(K, 64);
  const int64_t per_split = ceil_div(ksteps, splits);
  const int64_t ctas = tiles * ceil_div(ksteps, per_split);
  const double slots = kNumCus * v.ctas_per_cu;
  const double rounds = std::ceil((double)ctas / slots);
  // CTAs per CU in a round, and the CU's MFMA rate at that residency
  // relative to the one the efficiency was calibrated at: SIMDs without a
  // wave idle, and a SIMD with one wave runs at ~0.88 of two (1.68 vs 1.91
  // PF/s on random operands)
  const double share = std::min<double>(v.ctas_per_cu, std::ceil((double)ctas / (rounds * kNumCus)));
  auto fill = [&](double ctas_on_cu) {
    const double per_simd = ctas_on_cu * v.shape.wm * v.shape.wn / 4.0;
    return std::min(1.0, per_simd) * (per_simd >= 2.0 ? 1.0 : 0.88);
  };
  const double cu_rate = kMfmaFlopsPerS / kNumCus * tiled_eff(v, layout) * fill(share) / fill(v.ctas_per_cu);
  const double t_cta = (double)bm * bn * per_split * 64 * 2.0 * share / cu_rate;
  double t = rounds * t_cta;
  const double t_hbm = problem_bytes(M, N, K, 2) / kHbmBytesPerS;
  t = std::max(t, t_hbm);
  // split-K: partial traffic plus the last CTA's serial tail (coherent store,
  // counter, then coherent loads of every split's partial tile at roughly one
  // CU's bandwidth, ~100 GB/s; measured on the 70B FFN at M = 128: split 2
  // 81 us, split 4 92 us).
  if (splits > 1)
    t += 2.0 * tiles * splits * (double)bm * bn * 4.0 / kHbmBytesPerS + 1.5e-6 + splits * (double)bm * bn * 4.0 / 1.0e11;
  return t + kLaunchS;
}

size_t plan_workspace(int layout, int64_t M, int64_t N, int64_t K, const mxfp4_plan& p);

// max_ws: the workspace the call has; a via-G plan ([N,K/2] weights rewritten
// to G first, at kConvertEff of HBM bandwidth) is a candidate only if its
// workspace fits.
void choose_tiled(int layout, int64_t M, int64_t N, int64_t K, mxfp4_plan* out, size_t max_ws) {
  double best = 1e30;
  int bv = 0, bs = 1, bf = 0;
  const int64_t ksteps = ceil_div(K, 64);
  const bool try_g = via_g_ok(layout, N, K);
  const double t_convert =
      2.0 * ((double)(K / 2) * N + (double)(K / 32) * N) / (kHbmBytesPerS * kConvertEff) + kLaunchS;
  for (int pass = 0; pass < (try_g ? 2 : 1); ++pass) {
    const int lay = pass == 0 ? layout : kLayoutG;
    for (int v = 0; v < kNumTiled; ++v) {
      const TiledVariant& tv = kTiled[v];
      if (!tiled_variant_ok(tv, lay, N, K) || tiled_eff(tv, lay) <= 0.0) continue;
      const int64_t tiles = ceil_div(M, tv.shape.bm()) * ceil_div(N, tv.shape.bn());
      for (int s = 1; s <= 16 && s <= ksteps; ++s) {
        if (s > 1 && tiles * 4 > (int64_t)MXFP4_COUNTER_BYTES) break;
        if (pass == 1 && plan_workspace(layout, M, N, K, {MXFP4_KERNEL_TILED, v, s, MXFP4_PLAN_TILED_VIA_G}) > max_ws)
          continue;
        const double t = tiled_time(tv, lay, M, N, K, s) + (pass == 1 ? t_convert : 0.0);
        if (t < best * 0.98) {  // prefer fewer splits / earlier variants / no rewrite on near ties
          best = t;
          bv = v;
          bs = s;
          bf = pass == 1 ? MXFP4_PLAN_TILED_VIA_G : 0;
        }
      }
    }
  }
  out->kernel = MXFP4_KERNEL_TILED;
  out->variant = bv;
  out->split_k = bs;
  out->flags = bf;
}

hipError_t validate_plan(int layout, int64_t M, int64_t N, int64_t K, const mxfp4_plan& p) {
  if (p.split_k < 1) return hipErrorInvalidValue;
  if (p.flags & ~(MXFP4_PLAN_STREAM_NO_POLL | MXFP4_PLAN_TILED_VIA_G)) return hipErrorInvalidValue;
  if ((p.flags & MXFP4_PLAN_TILED_VIA_G) && (p.kernel != MXFP4_KERNEL_TILED || !via_g_ok(layout, N, K)))
    return hipErrorInvalidValue;
  switch (p.kernel) {
    case MXFP4_KERNEL_GENERIC:
      return hipSuccess;
    case MXFP4_KERNEL_GEMV: {
      if (p.variant < 0 || p.variant >= kNumGemv) return hipErrorInvalidValue;
      if (!gemv_plan_ok(layout, M, N, kGemv[p.variant])) return hipErrorInvalidValue;
      const int64_t groups = ceil_div(N, 16 * kGemv[p.variant].cb);
      if (p.split_k > 1 && groups * 4 > (int64_t)MXFP4_COUNTER_BYTES) return hipErrorInvalidValue;
      if (p.split_k > gemv_steps(layout, K)) return hipErrorInvalidValue;
      return hipSuccess;
    }
    case MXFP4_KERNEL_STREAM: {
      if (p.variant < 0 || p.variant >= kNumStream) return hipErrorInvalidValue;
      const StreamShape& s = kStream[p.variant];
      if (!stream_plan_ok(layout, M, N, K, s)) return hipErrorInvalidValue;
      // the split count is fixed by the shape; split_k must restate it
      if (p.split_k != stream_splits(s, K)) return hipErrorInvalidValue;
      return hipSuccess;
    }
    case MXFP4_KERNEL_TILED: {
      if (p.variant < 0 || p.variant >= kNumTiled) return hipErrorInvalidValue;
      if (layout == kLayoutKN && N % 16 != 0) return hipErrorInvalidValue;
      const int lay = (p.flags & MXFP4_PLAN_TILED_VIA_G) ? kLayoutG : layout;
      if (!tiled_variant_ok(kTiled[p.variant], lay, N, K)) return hipErrorInvalidValue;
      const TiledShape& s = kTiled[p.variant].shape;
      const int64_t tiles = ceil_div(M, s.bm()) * ceil_div(N, s.bn());
      if (p.split_k > 1 && tiles * 4 > (int64_t)MXFP4_COUNTER_BYTES) return hipErrorInvalidValue;
      if (p.split_k > ceil_div(K, 64)) return hipErrorInvalidValue;
      return hipSuccess;
    }
    default:
      return hipErrorInvalidValue;
  }
}

// max_ws: the workspace bytes the call can use beyond what the direct plans
// need (only via-G plans are held to it)
void auto_plan(int layout, int64_t M, int64_t N, int64_t K, mxfp4_plan* out, size_t max_ws) {
  if (layout == kLayoutKN && N % 16 != 0) {
    *out = {MXFP4_KERNEL_GENERIC, 0, 1, 0};
  } else if (M <= 32) {
    choose_gemv(layout, M, N, K, out);
  } else {
    choose_tiled(layout, M, N, K, out, max_ws);
  }
}

// [split-K counters][partials] (split_k > 1), then a via-G plan's G copy.
// The G copy starts after the counter region even at split 1: a workspace is
// shared by the calls on its stream (the extension keeps one per stream), and
// every split-K call needs the counters zero on entry.
size_t split_workspace(int layout, int64_t M, int64_t N, int64_t K, const mxfp4_plan& p);
size_t via_g_offset(int layout, int64_t M, int64_t N, int64_t K, const mxfp4_plan& p) {
  return std::max<size_t>(split_workspace(layout, M, N, K, p), MXFP4_COUNTER_BYTES);
}
size_t plan_workspace(int layout, int64_t M, int64_t N, int64_t K, const mxfp4_plan& p) {
  if (p.flags & MXFP4_PLAN_TILED_VIA_G) return via_g_offset(layout, M, N, K, p) + via_g_bytes(N, K);
  return split_workspace(layout, M, N, K, p);
}
size_t split_workspace(int layout, int64_t M, int64_t N, int64_t K, const mxfp4_plan& p) {
  if (p.split_k <= 1) return 0;
  size_t partial = 0;
  if (p.kernel == MXFP4_KERNEL_GEMV) {
    const GemvShape& g = kGemv[p.variant];
    partial = (size_t)ceil_div(N, 16 * g.cb) * p.split_k * gemv_tile(g) * sizeof(float);
  } else if (p.kernel == MXFP4_KERNEL_STREAM) {
    const StreamShape& s = kStream[p.variant];
    // 8-byte (value, tag) packets per partial element
    partial = s.resident ? resident_workspace(s.resident, N, K)
              : s.direct ? decode_workspace(s.direct, N, K)
                         : (size_t)stream_ctas(s, N, K) * p.split_k * s.tile() * 8;
  } else if (p.kernel == MXFP4_KERNEL_TILED) {
    const TiledShape& s = kTiled[p.variant].shape;
    const int64_t ksteps = ceil_div(K, 64);
    const int64_t per = ceil_div(ksteps, p.split_k);
    const int64_t splits = ceil_div(ksteps, per);
    partial = (size_t)(ceil_div(M, s.bm()) * ceil_div(N, s.bn())) * splits * s.bm() * s.bn() *
              sizeof(float);
  }
  (void)layout;
  return partial ? MXFP4_COUNTER_BYTES + align_up(partial, 256) : 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

bool layout_ok(int layout, int64_t N, int64_t K) {
  return layout >= kLayoutKN && layout <= kLayoutP && layout_shape_ok(layout, N, K);
}

hipError_t check_args(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                      int64_t M, int64_t N, int64_t K, int layout) {
  if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
  if (K % 32 != 0) return hipErrorInvalidValue;
  if (M > INT32_MAX || N > INT32_MAX || K > (1LL << 21)) return hipErrorInvalidValue;
  if (!layout_ok(layout, N, K)) return hipErrorInvalidValue;
  if (c_dtype != MXFP4_OUT_F32 && c_dtype != MXFP4_OUT_BF16) return hipErrorInvalidValue;
  if (M * N == 0) return hipSuccess;
  if (!C) return hipErrorInvalidValue;
  if (K > 0 && (!A || !B || !S)) return hipErrorInvalidValue;
  return hipSuccess;
}

// The kernels' view of a caller's epilogue (NULL: none).
hipError_t make_epilogue(const mxfp4_epilogue* in, Epilogue* out) {
  *out = Epilogue{};
  if (!in) return hipSuccess;
  if (in->activation < MXFP4_ACT_NONE || in->activation > MXFP4_ACT_GELU_TANH) return hipErrorInvalidValue;
  if (in->bias_dtype != MXFP4_OUT_F32 && in->bias_dtype != MXFP4_OUT_BF16) return hipErrorInvalidValue;
  if (in->residual_dtype != MXFP4_OUT_F32 && in->residual_dtype != MXFP4_OUT_BF16) return hipErrorInvalidValue;
  const uintptr_t ab = in->bias_dtype == MXFP4_OUT_BF16 ? 1 : 3, ar = in->residual_dtype == MXFP4_OUT_BF16 ? 1 : 3;
  if (((uintptr_t)in->bias & ab) || ((uintptr_t)in->residual & ar)) return hipErrorInvalidValue;
  out->bias = in->bias;
  out->residual = in->residual;
  out->bias_bf16 = in->bias_dtype == MXFP4_OUT_BF16;
  out->res_bf16 = in->residual_dtype == MXFP4_OUT_BF16;
  out->act = in->activation;
  out->any = in->bias != nullptr || in->residual != nullptr || in->activation != MXFP4_ACT_NONE;
  out->res_vec = ((uintptr_t)in->residual & (in->residual_dtype == MXFP4_OUT_BF16 ? 7u : 15u)) == 0;
  return hipSuccess;
}

hipError_t run(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype, int64_t M,
               int64_t N, int64_t K, int layout, const mxfp4_plan* plan_in, const mxfp4_epilogue* ep_in,
               void* workspace, size_t workspace_bytes, hipStream_t stream) {
  // an automatic plan may rewrite [N,K/2] weights to G only in a workspace
  // the caller passed
  const size_t max_ws = workspace && aligned16(workspace) ? workspace_bytes : 0;
  hipError_t e = check_args(A, B, S, C, c_dtype, M, N, K, layout);
  if (e != hipSuccess) return e;
  Epilogue ep;
  e = make_epilogue(ep_in, &ep);
  if (e != hipSuccess) return e;
  if (M * N == 0) return hipSuccess;
  const int out_bf16 = c_dtype == MXFP4_OUT_BF16;
  if (K == 0) {
    // C = act(0 + bias) + residual: the generic kernel with an empty K loop
    if (ep.any) return launch_generic(layout, nullptr, B, S, C, out_bf16, (int)M, (int)N, 0, ep, stream);
    return launch_zero_fill(C, (size_t)M * N * (out_bf16 ? 2 : 4), stream);
  }

  mxfp4_plan plan;
  if (plan_in && plan_in->kernel != MXFP4_KERNEL_AUTO) {
    plan = *plan_in;
  } else {
    auto_plan(layout, M, N, K, &plan, max_ws);
  }
  // The fast families read 16-byte vectors.
  if (plan.kernel != MXFP4_KERNEL_GENERIC &&
      !(aligned16(A) && aligned16(B) && aligned16(S) && aligned16(C))) {
    if (plan_in && plan_in->kernel != MXFP4_KERNEL_AUTO) return hipErrorInvalidValue;
    plan = {MXFP4_KERNEL_GENERIC, 0, 1, 0};
  }
  e = validate_plan(layout, M, N, K, plan);
  if (e != hipSuccess) return e;

  const size_t need = plan_workspace(layout, M, N, K, plan);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need || !aligned16(workspace)))
    return hipErrorInvalidValue;
  uint32_t* counters = static_cast<uint32_t*>(workspace);
  const size_t split_need = split_workspace(layout, M, N, K, plan);
  float* partials =
      split_need ? reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + MXFP4_COUNTER_BYTES) : nullptr;
  if (plan.flags & MXFP4_PLAN_TILED_VIA_G) {
    // the G copy after the split-K region; the tiled kernel then reads it
    uint8_t* g_codes = static_cast<uint8_t*>(workspace) + via_g_offset(layout, M, N, K, plan);
    uint8_t* g_scales = g_codes + align_up((size_t)(K / 2) * N, 256);
    e = launch_convert_nk_to_g(B, S, g_codes, g_scales, (size_t)K, (size_t)N, stream);
    if (e != hipSuccess) return e;
    B = g_codes;
    S = g_scales;
    layout = kLayoutG;
  }

  const uint16_t* A16 = static_cast<const uint16_t*>(A);
  switch (plan.kernel) {
    case MXFP4_KERNEL_GENERIC:
      return launch_generic(layout, A16, B, S, C, out_bf16, (int)M, (int)N, (int)K, ep, stream);
    case MXFP4_KERNEL_GEMV: {
      const GemvShape& g = kGemv[plan.variant];
      GemvArgs a{};
      a.A = A16; a.B = B; a.S = S; a.C = C;
      a.M = (int)M; a.N = (int)N; a.K = (int)K;
      a.out_bf16 = out_bf16;
      a.col_groups = (int)ceil_div(N, 16 * g.cb);
      a.steps = gemv_steps(layout, K);
      a.steps_per_split = (int)ceil_div(a.steps, plan.split_k);
      a.splits = (int)ceil_div(a.steps, a.steps_per_split);
      a.partials = a.splits > 1 ? partials : nullptr;
      a.counters = a.splits > 1 ? counters : nullptr;
      a.ep = ep;
      return launch_gemv(layout, g, a, stream);
    }
    case MXFP4_KERNEL_STREAM: {
      const StreamShape& s = kStream[plan.variant];
      StreamArgs a{};
      a.A = A16; a.B = B; a.S = S; a.C = C;
      a.M = (int)M; a.N = (int)N; a.K = (int)K;
      a.out_bf16 = out_bf16;
      a.splits = (int)stream_splits(s, K);
      a.groups = (int)ceil_div(N, 32);
      a.ctas = (int)stream_ctas(s, N, K);
      a.partials = a.splits > 1 ? partials : nullptr;
      a.counters = a.splits > 1 ? counters : nullptr;
      a.spin_limit = (plan.flags & MXFP4_PLAN_STREAM_NO_POLL) ? 0 : kStreamSpin;
      a.ep = ep;
      return launch_stream(layout, s, a, stream);
    }
    case MXFP4_KERNEL_TILED: {
      const TiledShape& s = kTiled[plan.variant].shape;
      TiledArgs a{};
      a.A = A16; a.B = B; a.S = S; a.C = C;
      a.M = (int)M; a.N = (int)N; a.K = (int)K;
      a.out_bf16 = out_bf16;
      a.tiles_m = (int)ceil_div(M, s.bm());
      a.tiles_n = (int)ceil_div(N, s.bn());
      a.group_m = 4;
      a.ksteps = (int)ceil_div(K, 64);
      a.steps_per_split = (int)ceil_div(a.ksteps, plan.split_k);
      a.splits = (int)ceil_div(a.ksteps, a.steps_per_split);
      a.partials = a.splits > 1 ? partials : nullptr;
      a.counters = a.splits > 1 ? counters : nullptr;
      a.ep = ep;
      switch (kTiled[plan.variant].family) {
        case kFamilySched: return launch_tiled_sched(layout, s, a, stream);
        case kFamilyPipe: return launch_tiled_pipe(layout, s, a, stream);
        default: return launch_tiled(layout, s, a, stream);
      }
    }
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace
}  // namespace mxfp4

// ---- the allocation-free entry point's workspace ------------------------------
// One file-scope device array, loaded with this code object on every GPU the
// library runs on (each GPU holds its own copy at its own address, until the
// process ends): [split-K counters][partials], as the workspace of
// mxfp4_gemm.  In host code `scratch` names a host-side stand-in, never the
// device memory: the entry point uses the address hipGetSymbolAddress gives
// for the current device.
static __device__ __align__(256) uint8_t scratch[MXFP4_NOALLOC_SCRATCH_BYTES];

namespace mxfp4 {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch[kMaxDevices];  // device address of `scratch`, per device

// The current device's scratch, set up on the first call on that device:
// its address, and one zero fill of the whole array (the counters and
// split-K packets must start at zero; every call leaves them at zero), queued
// on `stream` ahead of the call's kernels.  That fill has to run, not be
// recorded: a first call on a device under stream capture is refused.
hipError_t noalloc_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch[dev] == nullptr) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(stream, &cap);
    if (e != hipSuccess) return e;
    if (cap != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (ptr == nullptr) return hipErrorInvalidSymbol;
    e = launch_zero_fill(ptr, MXFP4_NOALLOC_SCRATCH_BYTES, stream);
    if (e != hipSuccess) return e;
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return hipSuccess;
}

}  // namespace
}  // namespace mxfp4

using namespace mxfp4;

extern "C" {

hipError_t mxfp4_select_plan(int64_t M, int64_t N, int64_t K, int b_layout, mxfp4_plan* out) {
  if (!out || M < 0 || N < 0 || K < 0 || K % 32 != 0) return hipErrorInvalidValue;
  if (!layout_ok(b_layout, N, K)) return hipErrorInvalidValue;
  auto_plan(b_layout, M, N, K, out, SIZE_MAX);
  return hipSuccess;
}

hipError_t mxfp4_plan_describe(const mxfp4_plan* plan, char* buf, size_t buf_len) {
  if (!plan || !buf || buf_len == 0) return hipErrorInvalidValue;
  switch (plan->kernel) {
    case MXFP4_KERNEL_GENERIC:
      snprintf(buf, buf_len, "generic");
      return hipSuccess;
    case MXFP4_KERNEL_GEMV:
      if (plan->variant < 0 || plan->variant >= kNumGemv) return hipErrorInvalidValue;
      snprintf(buf, buf_len, "gemv mt%d cb%d wpc%d u%d split%d", kGemv[plan->variant].mt,
               kGemv[plan->variant].cb, kGemv[plan->variant].wpc, kGemv[plan->variant].u,
               plan->split_k);
      return hipSuccess;
    case MXFP4_KERNEL_STREAM: {
      if (plan->variant < 0 || plan->variant >= kNumStream) return hipErrorInvalidValue;
      const StreamShape& s = kStream[plan->variant];
      if (s.resident >= 16)
        snprintf(buf, buf_len, "resident rows%d cols%d kr%d split%d", s.resident, 16 * s.gcb, s.k_split(),
                 plan->split_k);
      else if (s.resident)
        snprintf(buf, buf_len, "resident rows%d cols%d split%d%s", s.resident, 16 * s.gcb, plan->split_k,
                 s.nslot == 1 ? " dot" : "");
      else if (s.direct)
        snprintf(buf, buf_len, "decode rows%d cols%d kr%d split%d", s.direct, 16 * s.gcb, s.k_split(),
                 plan->split_k);
      else if (s.nslot == 1 && s.smax == 1)
        snprintf(buf, buf_len, "stream-whole mt%d kw%d split%d", s.mt, s.kw, plan->split_k);
      else
        snprintf(buf, buf_len, "stream mt%d w%d kw%d kr%d split%d", s.mt, s.waves, s.kw, s.k_split(),
                 plan->split_k);
      return hipSuccess;
    }
    case MXFP4_KERNEL_TILED: {
      if (plan->variant < 0 || plan->variant >= kNumTiled) return hipErrorInvalidValue;
      const TiledShape& s = kTiled[plan->variant].shape;
      const char* via = (plan->flags & MXFP4_PLAN_TILED_VIA_G) ? " via-g" : "";
      if (kTiled[plan->variant].family == kFamilySched)
        snprintf(buf, buf_len, "tiled-sched %dx%d w%dx%d ns%d split%d%s", s.bm(), s.bn(), s.wm, s.wn,
                 s.stages, plan->split_k, via);
      else if (kTiled[plan->variant].family == kFamilyPipe)
        snprintf(buf, buf_len, "tiled-pipe %dx%d w%dx%d ns%d split%d%s", s.bm(), s.bn(), s.wm, s.wn,
                 s.stages, plan->split_k, via);
      else
        snprintf(buf, buf_len, "tiled %dx%d w%dx%d split%d%s", s.bm(), s.bn(), s.wm, s.wn, plan->split_k, via);
      return hipSuccess;
    }
    default:
      return hipErrorInvalidValue;
  }
}

size_t mxfp4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int b_layout,
                                  const mxfp4_plan* plan) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 32 != 0) return 0;
  if (!layout_ok(b_layout, N, K)) return 0;
  mxfp4_plan p;
  if (plan && plan->kernel != MXFP4_KERNEL_AUTO) {
    p = *plan;
    if (validate_plan(b_layout, M, N, K, p) != hipSuccess) return 0;
  } else {
    auto_plan(b_layout, M, N, K, &p, SIZE_MAX);
  }
  return plan_workspace(b_layout, M, N, K, p);
}

hipError_t mxfp4_gemm(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                      int64_t M, int64_t N, int64_t K, int b_layout, void* workspace,
                      size_t workspace_bytes, hipStream_t stream) {
  return run(A, B, S, C, c_dtype, M, N, K, b_layout, nullptr, nullptr, workspace, workspace_bytes, stream);
}

hipError_t mxfp4_gemm_with_plan(const void* A, const uint8_t* B, const uint8_t* S, void* C,
                                int c_dtype, int64_t M, int64_t N, int64_t K, int b_layout,
                                const mxfp4_plan* plan, void* workspace, size_t workspace_bytes,
                                hipStream_t stream) {
  return run(A, B, S, C, c_dtype, M, N, K, b_layout, plan, nullptr, workspace, workspace_bytes, stream);
}

hipError_t mxfp4_gemm_ex(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                         int64_t M, int64_t N, int64_t K, int b_layout, const mxfp4_plan* plan,
                         const mxfp4_epilogue* ep, void* workspace, size_t workspace_bytes,
                         hipStream_t stream) {
  return run(A, B, S, C, c_dtype, M, N, K, b_layout, plan, ep, workspace, workspace_bytes, stream);
}

hipError_t mxfp4_dequant(const uint8_t* B, const uint8_t* S, void* out, int out_dtype, int64_t K,
                         int64_t N, int b_layout, hipStream_t stream) {
  if (K < 0 || N < 0 || K % 32 != 0 || K > INT32_MAX || N > INT32_MAX) return hipErrorInvalidValue;
  if (out_dtype != MXFP4_OUT_F32 && out_dtype != MXFP4_OUT_BF16) return hipErrorInvalidValue;
  if (!layout_ok(b_layout, N, K)) return hipErrorInvalidValue;
  if (K * N == 0) return hipSuccess;
  if (!B || !S || !out) return hipErrorInvalidValue;
  return launch_dequant(b_layout, B, S, out, out_dtype == MXFP4_OUT_BF16, (int)K, (int)N, stream);
}

hipError_t mxfp4_convert_layout(const uint8_t* B, const uint8_t* S, int src_layout, uint8_t* B_out,
                                uint8_t* S_out, int dst_layout, int64_t K, int64_t N,
                                hipStream_t stream) {
  if (K < 0 || N < 0 || K % 32 != 0) return hipErrorInvalidValue;
  if (!layout_ok(src_layout, N, K) || !layout_ok(dst_layout, N, K)) return hipErrorInvalidValue;
  if (K * N == 0) return hipSuccess;
  if (!B || !S || !B_out || !S_out || !aligned16(B_out)) return hipErrorInvalidValue;
  const uint64_t code_bytes = (uint64_t)K / 2 * N, scale_bytes = (uint64_t)K / 32 * N;
  const uint64_t b0 = (uintptr_t)B, b1 = b0 + code_bytes, o0 = (uintptr_t)B_out, o1 = o0 + code_bytes;
  const uint64_t s0 = (uintptr_t)S, s1 = s0 + scale_bytes, t0 = (uintptr_t)S_out, t1 = t0 + scale_bytes;
  if ((b0 < o1 && o0 < b1) || (s0 < t1 && t0 < s1)) return hipErrorInvalidValue;  // overlap
  return launch_convert(src_layout, dst_layout, B, S, B_out, S_out, (size_t)K, (size_t)N, stream);
}

hipError_t mxfp4_quantize(const void* X, int x_dtype, int x_layout, int64_t K, int64_t N, uint8_t* B,
                          uint8_t* S, int b_layout, hipStream_t stream) {
  if (K < 0 || N < 0 || K % 32 != 0) return hipErrorInvalidValue;
  if (x_dtype != MXFP4_IN_F32 && x_dtype != MXFP4_IN_BF16) return hipErrorInvalidValue;
  if (x_layout != kLayoutKN && x_layout != kLayoutNK) return hipErrorInvalidValue;
  if (!layout_ok(b_layout, N, K)) return hipErrorInvalidValue;
  if (K * N == 0) return hipSuccess;
  if (!X || !B || !S || !aligned16(X) || !aligned16(B)) return hipErrorInvalidValue;
  if ((uint64_t)(K / 32) * (uint64_t)N / 256 >= (1ull << 31)) return hipErrorInvalidValue;  // grid size
  return launch_quantize(X, x_dtype == MXFP4_IN_BF16, x_layout, B, S, b_layout, (size_t)K, (size_t)N, stream);
}

int mxfp4_shape_supported(char strategy, int64_t M, int64_t N, int64_t K) {
  int bm, bn, bk = 64;
  switch (strategy) {
    case 'a': case 'b': case 'c': bm = 64; bn = 128; break;
    case 'd': case 'g': case 'h': case 'i': case 'j': case 'k': case 'm': bm = 128; bn = 128; break;
    case 'e': bm = 128; bn = 64; break;
    case 'f': bm = 256; bn = 128; break;
    default: return -1;
  }
  return (M % bm == 0) && (N % bn == 0) && (K % bk == 0) && (K % 32 == 0);
}

hipError_t mxfp4_device_info(int dev, mxfp4_device_info_t* out) {
  if (!out) return hipErrorInvalidValue;
  hipDeviceProp_t prop{};
  hipError_t e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) return e;
  memset(out, 0, sizeof(*out));
  strncpy(out->name, prop.name, sizeof(out->name) - 1);
  strncpy(out->gcn_arch_name, prop.gcnArchName, sizeof(out->gcn_arch_name) - 1);
  out->multi_processor_count = prop.multiProcessorCount;
  out->warp_size = prop.warpSize;
  out->total_global_mem = (int64_t)prop.totalGlobalMem;
  out->shared_mem_per_block = (int64_t)prop.sharedMemPerBlock;
  return hipSuccess;
}

hipError_t mxfp4_gemm_noalloc(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                              int64_t M, int64_t N, int64_t K, int b_layout, hipStream_t stream) {
  hipError_t e = check_args(A, B, S, C, c_dtype, M, N, K, b_layout);
  if (e != hipSuccess) return e;
  void* ws = nullptr;
  e = noalloc_scratch(stream, &ws);
  if (e != hipSuccess) return e;
  // the automatic plan as run() picks it with this workspace: a via-G
  // rewrite only if its G copy fits the scratch
  size_t need = 0;
  if (M > 0 && N > 0 && K > 0) {
    mxfp4_plan p;
    auto_plan(b_layout, M, N, K, &p, MXFP4_NOALLOC_SCRATCH_BYTES);
    need = plan_workspace(b_layout, M, N, K, p);
  }
  if (need > MXFP4_NOALLOC_SCRATCH_BYTES) return hipErrorOutOfMemory;
  return run(A, B, S, C, c_dtype, M, N, K, b_layout, nullptr, nullptr, ws, MXFP4_NOALLOC_SCRATCH_BYTES, stream);
}

const char* mxfp4_version(void) { return "mxfp4_mi355x 0.1.0 (gfx950)"; }

}  // extern "C"
