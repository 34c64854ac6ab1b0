// Device primitives shared by every MXFP4 kernel (gfx950 / CDNA4 only).
//
// Replaces the reference's dequant headers and loaders:
//   csrc/strategy_c_dequant.h:21-74   (FP8-FNUZ LUT dequant)      -> fp4x2_to_bf16x2 (scaled cvt)
//   csrc/strategy_h_dequant.h:24-67   (unscaled perm dequant)      -> fp4x2_to_bf16x2 (scaled cvt)
//   csrc/direct_lds.h:14-17           (VGPR-staged "direct" load)  -> buffer_load_lds16
//   csrc/bf16_gemm.h:18-20            (mfma 16x16x16 bf16)         -> mfma_32x32x16 / mfma_16x16x32
//   csrc/bf16_gemm.h:156-175          (6-XCD remap, props/launch)  -> xcd_chunked_id, tile_of (mxfp4_schedule.h)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "mxfp4_schedule.h"

namespace mxfp4 {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr int kGroup = 32;  // K elements per E8M0 scale
constexpr int kWave = 64;   // CDNA wavefront width

// Offset given to a masked lane of a buffer load: past num_records, so the
// hardware returns zeros (and writes zeros to LDS for the LDS-DMA form).
constexpr uint32_t kOobOffset = 0x80000000u;
constexpr uint32_t kNumRecords = 0x40000000u;

// E8M0 byte -> the scale operand of v_cvt_scalef32_pk_*: the byte goes in
// the fp32 exponent field (as csrc/strategy_h_dequant.h:65-67 does).  The
// convert reads only that field as an OCP MX E8M0 scale, so byte 0 scales by
// 2^-127 (bf16 subnormals are kept: identical to ref.py:69) and byte 255 is
// NaN (ref.py gives +-inf); measured on gfx950 by the exhaustive dequant test.
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return __builtin_bit_cast(float, (e & 0xFFu) << 23);
}

// Byte SEL of w holds two E2M1 codes (low nibble = even K).  Returns the two
// bf16 values code * 2^(e-127), element 0 (low half) from the low nibble.  One
// v_cvt_scalef32_pk_bf16_fp4; exact for every scale byte 0..254 (an E2M1
// value times a power of two fits bf16, subnormals included).
template <int SEL>
__device__ __forceinline__ uint32_t fp4x2_to_bf16x2(uint32_t w, float scale) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, SEL));
}

// Eight K-consecutive codes of one column, given as byte SEL of four words
// r0..r3 (r_i holds K pair i), -> one MFMA bf16x8 operand.
template <int SEL>
__device__ __forceinline__ bf16x8 operand_from_bytes(uint32_t r0, uint32_t r1, uint32_t r2,
                                                     uint32_t r3, float scale) {
  u32x4 v;
  v.x = fp4x2_to_bf16x2<SEL>(r0, scale);
  v.y = fp4x2_to_bf16x2<SEL>(r1, scale);
  v.z = fp4x2_to_bf16x2<SEL>(r2, scale);
  v.w = fp4x2_to_bf16x2<SEL>(r3, scale);
  return __builtin_bit_cast(bf16x8, v);
}

// Eight K-consecutive codes packed in one word (K-contiguous layouts).
__device__ __forceinline__ bf16x8 operand_from_word(uint32_t w, float scale) {
  u32x4 v;
  v.x = fp4x2_to_bf16x2<0>(w, scale);
  v.y = fp4x2_to_bf16x2<1>(w, scale);
  v.z = fp4x2_to_bf16x2<2>(w, scale);
  v.w = fp4x2_to_bf16x2<3>(w, scale);
  return __builtin_bit_cast(bf16x8, v);
}

__device__ __forceinline__ f32x16 mfma_32x32x16(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mfma_16x16x32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Raw buffer resource over [base, base + kNumRecords).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)kNumRecords,
                                           0x00020000);
}

// 16 bytes per lane from global (rsrc + voffset) straight into LDS at
// lds_base + 16 * lane.  lds_base must be wave-uniform.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, void* lds_base,
                                                  uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)lds_base, 16, voffset, 0, 0, 0);
}

__device__ __forceinline__ void wait_vmcnt0() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// s_waitcnt vmcnt(N) with expcnt/lgkmcnt left at their maxima (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// vmcnt(n) for a wave-uniform n known only at run time (0 <= n < 64; larger n
// waits for vmcnt(63)).  A branch chain over immediates.
template <int I = 0>
__device__ __forceinline__ void wait_vmcnt_rt(int n) {
  if constexpr (I < 63) {
    if (n == I) {
      wait_vmcnt<I>();
      return;
    }
    wait_vmcnt_rt<I + 1>(n);
  } else {
    wait_vmcnt<63>();
  }
}

// ---- LDS DMA issued as inline asm ---------------------------------------------
// The compiler treats every LDS read that follows a buffer_load ... lds it
// can see as possibly aliasing it and waits for vmcnt(0) first (it has no
// alias information for one LDS array), which drains a multi-stage ring on
// every step.  The ring kernels therefore issue their global->LDS loads as
// asm the compiler does not track, count them themselves (wait_vmcnt<N>
// before the barrier that publishes a stage) and keep no compiler-visible
// VMEM loads inside the pipelined loop: a compiler-computed vmcnt would not
// count these loads and would drain the ring again.
typedef uint32_t desc_t __attribute__((ext_vector_type(4)));

// Raw buffer descriptor over [base, base + num_records) (stride 0, 32-bit
// data format, as __builtin_amdgcn_make_buffer_rsrc builds it).  base and
// num_records must be wave-uniform.
__device__ __forceinline__ desc_t make_desc(const void* base, uint32_t num_records = kNumRecords) {
  const uint64_t b = reinterpret_cast<uint64_t>(base);
  return desc_t{(uint32_t)b, (uint32_t)(b >> 32) & 0xFFFFu, num_records, 0x00020000u};
}

// 16 bytes per lane: global (desc + voffset) -> LDS lds + 16 * lane.
// M0 (the LDS base of the DMA) is an input operand, so the compiler writes it
// and knows the asm reads it.
__device__ __forceinline__ void dma16(desc_t d, const void* lds, uint32_t voffset) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds"
               :: "v"(voffset), "s"(d), "{m0}"((uint32_t)(uintptr_t)lds) : "memory");
}
// 4 bytes per lane: global (desc + voffset) -> LDS lds + 4 * lane.
__device__ __forceinline__ void dma4(desc_t d, const void* lds, uint32_t voffset) {
  asm volatile("buffer_load_dword %0, %1, 0 offen lds"
               :: "v"(voffset), "s"(d), "{m0}"((uint32_t)(uintptr_t)lds) : "memory");
}
// The same with the non-temporal hint, for bytes read once per launch (the
// decode kernels' weights and scales).  Measured on MI355X in a 36 MB decode
// read: 1.2-1.4 us faster per launch than the same loads without it.
__device__ __forceinline__ void dma16_nt(desc_t d, const void* lds, uint32_t voffset) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen nt lds"
               :: "v"(voffset), "s"(d), "{m0}"((uint32_t)(uintptr_t)lds) : "memory");
}
__device__ __forceinline__ void dma4_nt(desc_t d, const void* lds, uint32_t voffset) {
  asm volatile("buffer_load_dword %0, %1, 0 offen nt lds"
               :: "v"(voffset), "s"(d), "{m0}"((uint32_t)(uintptr_t)lds) : "memory");
}

// Split-K partials cross XCDs, whose L2s are not coherent with each other.
// Instead of __threadfence() (buffer_wbl2 + buffer_inv of the whole L2 on
// gfx950, which flushes every CTA's cached tiles), the partials themselves
// are written and read with SC1 (device-scope coherent) buffer accesses, the
// same cache policy LLVM gives agent-scope atomic loads/stores.  A writer
// waits for its SC1 stores (vmcnt) before the counter increment.
constexpr int kCPolDevice = 16;  // SC1

__device__ __forceinline__ void store_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCPolDevice);
}
__device__ __forceinline__ void store_coherent(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, off, 0, kCPolDevice);
}
__device__ __forceinline__ f32x4 load_coherent4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCPolDevice));
}
__device__ __forceinline__ float load_coherent1(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kCPolDevice));
}

// The lane index computed afresh (v_mbcnt) where the optimizer cannot reuse
// an earlier copy.  A kernel whose main loop takes every VGPR uses it for the
// lane-derived offsets of its epilogue: kept live across the loop they are
// spilled, and each reload's vmcnt(0) wait also waits for every store issued
// before it.
__device__ __forceinline__ int fresh_lane() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// Split-K arrival: every thread's SC1 partial stores have completed when
// thread 0 bumps the tile counter; returns true in the CTA that arrived last
// (it then owns the reduction and resets the counter for the next call).
// tid: the caller's work-item id.
__device__ __forceinline__ bool splitk_arrive_last(uint32_t* counter, uint32_t splits, int* s_flag, int tid) {
  wait_vmcnt0();
  __syncthreads();
  if (tid == 0) {
    const uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = prev == splits - 1;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *s_flag = last;
  }
  __syncthreads();
  // the same word for every thread: wave-uniform to the compiler, so code
  // after a return on it keeps its values in SGPRs
  return __builtin_amdgcn_readfirstlane(*s_flag) != 0;
}
__device__ __forceinline__ bool splitk_arrive_last(uint32_t* counter, uint32_t splits, int* s_flag) {
  return splitk_arrive_last(counter, splits, s_flag, (int)threadIdx.x);
}

// The last CTA's sum of a tile's split partials: Q f32x4 per thread, element
// i of split sp at byte sp * slot + (i * nt + tid) * 16 (tid: the work-item
// id; splitk_sum passes threadIdx.x).  Each
// element's splits are added in split order (bit-reproducible).  The loads go
// GRP elements at a time, one split's GRP loads in flight together: S * Q /
// GRP memory round trips (an element-by-element loop waited for every load,
// S * Q round trips -- 160 us of tail at S = 16).  put(i, sum) stores the
// result.
template <int Q, int GRP = 8, typename Put>
__device__ __forceinline__ void splitk_sum_tid(__amdgpu_buffer_rsrc_t rp, uint32_t slot, int splits, uint32_t nt,
                                               int tid, Put&& put) {
  static_assert(Q % GRP == 0, "whole groups");
#pragma unroll
  for (int g0 = 0; g0 < Q; g0 += GRP) {
    f32x4 sum[GRP];
    for (int sp = 0; sp < splits; ++sp) {
      f32x4 t[GRP];
#pragma unroll
      for (int b = 0; b < GRP; ++b)
        t[b] = load_coherent4(rp, sp * slot + (uint32_t)((g0 + b) * nt + tid) * 16);
#pragma unroll
      for (int b = 0; b < GRP; ++b) sum[b] = sp == 0 ? t[b] : sum[b] + t[b];
    }
#pragma unroll
    for (int b = 0; b < GRP; ++b) put(g0 + b, sum[b]);
  }
}
template <int Q, int GRP = 8, typename Put>
__device__ __forceinline__ void splitk_sum(__amdgpu_buffer_rsrc_t rp, uint32_t slot, int splits, uint32_t nt,
                                           Put&& put) {
  splitk_sum_tid<Q, GRP>(rp, slot, splits, nt, (int)threadIdx.x, put);
}

// ---- split-K partials as tagged packets (streaming and decode kernels) ------
// A published partial element is an 8-byte packet (value, tag), written with
// device-coherent (SC1) stores and polled with SC1 loads, which see a packet
// atomically; the reader needs no store-completion wait from the writer.
// The tag is a quiet-NaN bit pattern with a rare payload, which no finite
// partial that another split-K kernel leaves in the shared workspace can
// equal (workspace words are zero or such partials).
constexpr uint32_t kTag = 0x7FC5A3E1u;
constexpr uint32_t kArrivals = 0xFFFFu;  // counter arrivals field (low half)

// Whole vectors are bit-cast, never single components: hipcc's front end
// lowers __builtin_bit_cast of a vector component (v.y) to a load from the
// vector's first element.
__device__ __forceinline__ void store_packets(__amdgpu_buffer_rsrc_t r, uint32_t off, f32x4 v, uint32_t tag) {
  const u32x4 w = __builtin_bit_cast(u32x4, v);
  const u32x4 lo = {w.x, tag, w.y, tag};
  const u32x4 hi = {w.z, tag, w.w, tag};
  __builtin_amdgcn_raw_buffer_store_b128(lo, r, off, 0, kCPolDevice);
  __builtin_amdgcn_raw_buffer_store_b128(hi, r, off + 16, 0, kCPolDevice);
}
__device__ __forceinline__ u32x4 load_packets(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kCPolDevice);
}
__device__ __forceinline__ bool tagged(u32x4 a, u32x4 b) {
  return a.y == kTag && a.w == kTag && b.y == kTag && b.w == kTag;
}
__device__ __forceinline__ f32x4 packet_values(u32x4 a, u32x4 b) {
  const f32x4 fa = __builtin_bit_cast(f32x4, a), fb = __builtin_bit_cast(f32x4, b);
  return f32x4{fa.x, fa.z, fb.x, fb.z};
}

__device__ __forceinline__ uint32_t bf16_bits_rne(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f);
}

// Two values, one v_cvt_pk_bf16_f32 (the same RNE conversion as
// bf16_bits_rne, which converts one value per instruction).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t{lo, hi}), bf16x2_t));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// ---- fused epilogue -----------------------------------------------------------
// v = act(acc + bias[col]) + residual[row][col], in fp32 (the definitions of
// torch.nn.functional.silu / gelu / gelu(approximate="tanh")).
template <int ACT>
__device__ __forceinline__ float activate_c(float v) {
  if constexpr (ACT == 1)  // SiLU
    return v / (1.0f + expf(-v));
  else if constexpr (ACT == 2)  // GELU (erf)
    return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
  else if constexpr (ACT == 3)  // GELU (tanh)
    return 0.5f * v * (1.0f + tanhf(0.79788456080286536f * (v + 0.044715f * v * v * v)));
  else
    return v;
}
__device__ __forceinline__ float activate(int act, float v) {
  switch (act) {
    case 1: return activate_c<1>(v);
    case 2: return activate_c<2>(v);
    case 3: return activate_c<3>(v);
    default: return v;
  }
}

// Store loops.  A GEMM kernel's store loop is unrolled over every accumulator
// element (128-256 per thread); with the epilogue's math (expf / erff / tanhf)
// inlined per element, one loop is ~25k instructions, and walking it thrashes
// the instruction cache: a 128 x 256 tile's plain bf16 store took 32 us when
// the plain and fused stores shared one loop with a per-element branch.  So
// each kernel writes its loop once, as a lambda over these tags, and calls it
// in separate branches chosen once per thread: the plain stores (OutKind 0 =
// fp32, 1 = bf16) are compact loops that never touch the epilogue code; the
// fused store (StoreKind<true>) is one loop that picks the output type per
// store (OutKind 2).
template <bool F>
struct StoreKind {
  static constexpr bool value = F;
};
template <int V>
struct OutKind {
  static constexpr int value = V;
};

template <typename Ep>
__device__ __forceinline__ float epilogue_value(const Ep& ep, float v, size_t row, size_t col, size_t N) {
  if (ep.bias)
    v += ep.bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(ep.bias)[col])
                      : static_cast<const float*>(ep.bias)[col];
  v = activate(ep.act, v);
  if (ep.residual) {
    const size_t o = row * N + col;
    v += ep.res_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(ep.residual)[o])
                     : static_cast<const float*>(ep.residual)[o];
  }
  return v;
}

}  // namespace mxfp4
