// MXFP4 quantizer: fp32 / bf16 weights -> E2M1 codes + E8M0 scales, in any
// weight layout.  Device counterpart of quantize_mxfp4
// (python/mxfp4_cdna3/ref.py:14-47), bit-exact with it for finite inputs:
//
//   amax  = max |x| over the 32-K group                 (ref.py:24)
//   e     = clip(ceil(log2(max(amax, 1e-38f) / 6)), -127, 127)
//           with the quotient and the log2 rounded to float32 (ref.py:25-28)
//   s     = 2^e (float32; 2^-127 is the subnormal 0x00400000)
//   code  = sign(x/s) << 3 | argmin_i | |x/s| - E2M1[i] |  (first minimum:
//           ties go to the smaller magnitude, ref.py:6-11)
//
// Why not the hardware FP4 converts (v_cvt_scalef32_pk_fp4_*): they round to
// nearest even, which resolves the ties at 0.75, 1.75 and 3.5 upward where
// the reference's argmin keeps the smaller magnitude.  The work is a few
// VALU operations per element against 2-4 bytes of HBM traffic, so the
// explicit argmin costs nothing measurable.
//
// The float32 log2 of the reference (numpy) is not correctly rounded
// everywhere, but ceil() of it equals ceil() of the correctly rounded
// float32 log2 on every quotient within 200 ulps of a power of two (checked
// exhaustively against numpy, the only place the two could differ); the
// kernel computes log2 in double precision and rounds it to float32.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

constexpr uint32_t kSafeMinBits = 0x006CE3EEu;  // float32(1e-38), a subnormal (ref.py:25)

// E2M1 code of a scaled value: the reference's argmin over the 8 magnitudes.
__device__ __forceinline__ uint32_t e2m1_code(float xs) {
  const float mag = __builtin_fabsf(xs);
  const float table[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float best = __builtin_fabsf(mag - table[0]);
  uint32_t idx = 0;
#pragma unroll
  for (int i = 1; i < 8; ++i) {
    const float d = __builtin_fabsf(mag - table[i]);
    if (d < best) {
      best = d;
      idx = (uint32_t)i;
    }
  }
  return ((xs < 0.0f) ? 8u : 0u) | idx;
}

// Scale exponent of a group from the bits of its max |x| (a non-negative float).
__device__ __forceinline__ int group_exponent(uint32_t amax_bits) {
  const uint32_t safe_bits = amax_bits > kSafeMinBits ? amax_bits : kSafeMinBits;
  const float q = __fdiv_rn(__builtin_bit_cast(float, safe_bits), 6.0f);
  const float l = (float)log2((double)q);  // double log2, rounded once to float32
  int e = (int)__builtin_ceilf(l);
  return e < -127 ? -127 : (e > 127 ? 127 : e);
}

// 2^v as float32 for v in [-127, 127].
__device__ __forceinline__ float exp2_int(int v) {
  return v >= -126 ? __builtin_bit_cast(float, (uint32_t)(v + 127) << 23) : __builtin_bit_cast(float, 0x00400000u);
}

// One thread per (column n, 32-K group g).  XL: X is [K, N] (kLayoutKN;
// consecutive threads take consecutive columns, so every row read is
// coalesced) or [N, K] (kLayoutNK; a thread reads its 32 contiguous values).
template <int XL, int DST, bool BF16>
__global__ void __launch_bounds__(256) quantize_kernel(const void* __restrict__ X, uint8_t* __restrict__ B,
                                                       uint8_t* __restrict__ S, size_t K, size_t N) {
  const size_t G = K / 32;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= G * N) return;
  size_t g, n;
  if constexpr (XL == kLayoutKN) {
    g = idx / N;
    n = idx - g * N;
  } else {
    n = idx / G;
    g = idx - n * G;
  }
  float x[32];
  if constexpr (XL == kLayoutKN) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const size_t o = (32 * g + i) * N + n;
      x[i] = BF16 ? __builtin_bit_cast(float, (uint32_t)static_cast<const uint16_t*>(X)[o] << 16)
                  : static_cast<const float*>(X)[o];
    }
  } else if constexpr (BF16) {
    const u32x4* src = reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(X) + n * K + 32 * g);
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const u32x4 w = src[v];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * v + 2 * j] = __builtin_bit_cast(float, w[j] << 16);
        x[8 * v + 2 * j + 1] = __builtin_bit_cast(float, w[j] & 0xFFFF0000u);
      }
    }
  } else {
    const f32x4* src = reinterpret_cast<const f32x4*>(static_cast<const float*>(X) + n * K + 32 * g);
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const f32x4 w = src[v];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[4 * v + j] = w[j];
    }
  }
  uint32_t amax_bits = 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t a = __builtin_bit_cast(uint32_t, x[i]) & 0x7FFFFFFFu;
    amax_bits = a > amax_bits ? a : amax_bits;
  }
  const int e = group_exponent(amax_bits);
  // x / 2^e: dividing by a power of two equals multiplying by its (exact)
  // reciprocal, both rounded once.
  const float inv = exp2_int(-e);
  uint32_t w[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 8; ++b) word |= e2m1_code(x[8 * j + b] * inv) << (4 * b);
    w[j] = word;
  }
  // byte kp = 16g + i holds K 2kp (low nibble) and 2kp + 1
  if constexpr (DST == kLayoutNK || DST == kLayoutP) {
    *reinterpret_cast<u32x4*>(B + code_offset<DST>(16 * g, n, K, N)) = u32x4{w[0], w[1], w[2], w[3]};
  } else if constexpr (DST == kLayoutG) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(B + code_offset<DST>(16 * g + 4 * j, n, K, N)) = w[j];
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) B[(16 * g + i) * N + n] = (uint8_t)(w[i / 4] >> (8 * (i % 4)));
  }
  S[scale_offset<DST>(g, n, K, N)] = (uint8_t)(e + 127);
}

template <int XL, bool BF16>
struct QuantTo {
  template <int DST>
  struct Launch {
    static hipError_t run(const void* X, uint8_t* B, uint8_t* S, size_t K, size_t N, hipStream_t stream) {
      const size_t threads = K / 32 * N;
      hipLaunchKernelGGL((quantize_kernel<XL, DST, BF16>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                         stream, X, B, S, K, N);
      return hipGetLastError();
    }
  };
};

template <int XL, bool BF16>
hipError_t quantize_to(int dst, const void* X, uint8_t* B, uint8_t* S, size_t K, size_t N, hipStream_t stream) {
  switch (dst) {
    case kLayoutKN: return QuantTo<XL, BF16>::template Launch<kLayoutKN>::run(X, B, S, K, N, stream);
    case kLayoutNK: return QuantTo<XL, BF16>::template Launch<kLayoutNK>::run(X, B, S, K, N, stream);
    case kLayoutG: return QuantTo<XL, BF16>::template Launch<kLayoutG>::run(X, B, S, K, N, stream);
    case kLayoutP: return QuantTo<XL, BF16>::template Launch<kLayoutP>::run(X, B, S, K, N, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

hipError_t launch_quantize(const void* X, int x_bf16, int x_layout, uint8_t* B, uint8_t* S, int b_layout,
                           size_t K, size_t N, hipStream_t stream) {
  if (K * N == 0) return hipSuccess;
  if (x_layout == kLayoutKN)
    return x_bf16 ? quantize_to<kLayoutKN, true>(b_layout, X, B, S, K, N, stream)
                  : quantize_to<kLayoutKN, false>(b_layout, X, B, S, K, N, stream);
  if (x_layout == kLayoutNK)
    return x_bf16 ? quantize_to<kLayoutNK, true>(b_layout, X, B, S, K, N, stream)
                  : quantize_to<kLayoutNK, false>(b_layout, X, B, S, K, N, stream);
  return hipErrorInvalidValue;
}

}  // namespace mxfp4
