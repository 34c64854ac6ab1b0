// Dequant tile, generic fallback GEMM and zero fill.
//
// dequant_kernel replaces the reference's dequant-only pass
// (csrc/strategy_a_two_pass.cu:8-37, which writes a bf16 [K, N] scratch) and
// is the device counterpart of ref.py:50-72 (dequantize_mxfp4, axis=0).  It
// uses the same v_cvt_scalef32_pk_bf16_fp4 convert as the GEMM kernels, so
// the bit-exact tile test pins the GEMM's in-register dequant as well.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

// One thread per packed byte (two K-adjacent codes of one column).
template <int LAYOUT>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ B,
                                                      const uint8_t* __restrict__ S, void* out,
                                                      int out_bf16, int K, int N) {
  const size_t total = (size_t)(K / 2) * N;
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  size_t r, n;
  uint32_t byte, sbyte;
  if constexpr (LAYOUT == kLayoutKN) {
    r = idx / N;
    n = idx - r * N;
    byte = B[idx];
    sbyte = S[(r / 16) * N + n];
  } else {
    // Thread order follows [K/2, N] so the writes below stay coalesced.
    r = idx / N;
    n = idx - r * N;
    byte = B[n * (size_t)(K / 2) + r];
    sbyte = S[n * (size_t)(K / 32) + r / 16];
  }
  const uint32_t v = fp4x2_to_bf16x2<0>(byte, e8m0_to_f32(sbyte));
  const size_t o0 = (2 * r) * (size_t)N + n, o1 = o0 + N;
  if (out_bf16) {
    static_cast<uint16_t*>(out)[o0] = (uint16_t)(v & 0xFFFFu);
    static_cast<uint16_t*>(out)[o1] = (uint16_t)(v >> 16);
  } else {
    static_cast<float*>(out)[o0] = __builtin_bit_cast(float, v << 16);
    static_cast<float*>(out)[o1] = __builtin_bit_cast(float, v & 0xFFFF0000u);
  }
}

// One thread per output element; fp32 accumulation in K order.
template <int LAYOUT>
__global__ void __launch_bounds__(256) generic_kernel(const uint16_t* __restrict__ A,
                                                      const uint8_t* __restrict__ B,
                                                      const uint8_t* __restrict__ S, void* C,
                                                      int out_bf16, int M, int N, int K) {
  const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx - (size_t)m * N);
  float acc = 0.f;
  for (int kp = 0; kp < K / 2; ++kp) {
    uint32_t byte, sbyte;
    if constexpr (LAYOUT == kLayoutKN) {
      byte = B[(size_t)kp * N + n];
      sbyte = S[(size_t)(kp / 16) * N + n];
    } else {
      byte = B[(size_t)n * (K / 2) + kp];
      sbyte = S[(size_t)n * (K / 32) + kp / 16];
    }
    const uint32_t w = fp4x2_to_bf16x2<0>(byte, e8m0_to_f32(sbyte));
    const float a0 = __builtin_bit_cast(float, (uint32_t)A[(size_t)m * K + 2 * kp] << 16);
    const float a1 = __builtin_bit_cast(float, (uint32_t)A[(size_t)m * K + 2 * kp + 1] << 16);
    acc = __builtin_fmaf(a0, __builtin_bit_cast(float, w << 16), acc);
    acc = __builtin_fmaf(a1, __builtin_bit_cast(float, w & 0xFFFF0000u), acc);
  }
  if (out_bf16)
    static_cast<uint16_t*>(C)[idx] = (uint16_t)bf16_bits_rne(acc);
  else
    static_cast<float*>(C)[idx] = acc;
}

__global__ void __launch_bounds__(256) zero_fill_kernel(uint8_t* p, size_t bytes) {
  const size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16;
  if (i + 16 <= bytes) {
    *reinterpret_cast<u32x4*>(p + i) = u32x4{0u, 0u, 0u, 0u};
  } else {
    for (size_t j = i; j < bytes; ++j) p[j] = 0;
  }
}

}  // namespace

hipError_t launch_dequant(int layout, const uint8_t* B, const uint8_t* S, void* out, int out_bf16,
                          int K, int N, hipStream_t stream) {
  const size_t total = (size_t)(K / 2) * N;
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (layout == kLayoutKN)
    hipLaunchKernelGGL(dequant_kernel<kLayoutKN>, grid, dim3(256), 0, stream, B, S, out, out_bf16, K, N);
  else if (layout == kLayoutNK)
    hipLaunchKernelGGL(dequant_kernel<kLayoutNK>, grid, dim3(256), 0, stream, B, S, out, out_bf16, K, N);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_generic(int layout, const uint16_t* A, const uint8_t* B, const uint8_t* S,
                          void* C, int out_bf16, int M, int N, int K, hipStream_t stream) {
  const size_t total = (size_t)M * N;
  if (total == 0) return hipSuccess;
  const dim3 grid((unsigned)((total + 255) / 256));
  if (layout == kLayoutKN)
    hipLaunchKernelGGL(generic_kernel<kLayoutKN>, grid, dim3(256), 0, stream, A, B, S, C, out_bf16, M, N, K);
  else if (layout == kLayoutNK)
    hipLaunchKernelGGL(generic_kernel<kLayoutNK>, grid, dim3(256), 0, stream, A, B, S, C, out_bf16, M, N, K);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_zero_fill(void* C, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  const size_t chunks = (bytes + 15) / 16;
  hipLaunchKernelGGL(zero_fill_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, stream,
                     static_cast<uint8_t*>(C), bytes);
  return hipGetLastError();
}

}  // namespace mxfp4
