// Dequant tile, generic fallback GEMM, weight layout conversion and zero fill.
//
// dequant_kernel replaces the reference's dequant-only pass
// (csrc/strategy_a_two_pass.cu:8-37, which writes a bf16 [K, N] scratch) and
// is the device counterpart of ref.py:50-72 (dequantize_mxfp4, axis=0).  It
// uses the same v_cvt_scalef32_pk_bf16_fp4 convert as the GEMM kernels, so
// the bit-exact tile test pins the GEMM's in-register dequant as well.
//
// convert_*_kernel is the device counterpart of prepack_b_mxfp4
// (python/mxfp4_cdna3/ref.py:85-101), generalised to any pair of layouts.
#include "mxfp4_device.h"
#include "mxfp4_kernels.h"

namespace mxfp4 {
namespace {

// Scale byte 0xFF has no finite value: ref.py:69 computes 2**128 in float64
// and casts it to float32 (+inf), so codes 0 and 8 (+-0) give NaN and every
// other code +-inf.  The scaled convert gives NaN for all of them (OCP MX
// treats 0xFF as NaN), so the dequant tile substitutes the reference's bf16
// patterns per nibble; exact in fp32 too (bf16 << 16).
__device__ inline uint32_t e8m0_nan_pair(uint32_t byte) {
  auto one = [](uint32_t c) -> uint32_t { return (c & 7u) == 0 ? 0x7FC0u : (c & 8u) ? 0xFF80u : 0x7F80u; };
  return one(byte & 15u) | (one(byte >> 4) << 16);
}

// Grid-stride loops over `total` items: launches cap the grid at kMaxBlocks
// blocks of 256 threads, so any size fits the grid limits.
constexpr unsigned kMaxBlocks = 1u << 20;
inline unsigned grid_for(size_t items) {
  const size_t blocks = (items + 255) / 256;
  return (unsigned)(blocks < kMaxBlocks ? blocks : kMaxBlocks);
}

// One thread per packed byte (two K-adjacent codes of one column), in
// [K/2, N] order so the writes stay coalesced; the source positions follow
// the weight layout (mxfp4_layout.h).
template <int LAYOUT>
__global__ void __launch_bounds__(256) dequant_kernel(const uint8_t* __restrict__ B,
                                                      const uint8_t* __restrict__ S, void* out,
                                                      int out_bf16, int K, int N) {
  const size_t total = (size_t)(K / 2) * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
      const size_t r = idx / N, n = idx - r * N;
      const uint32_t byte = B[code_offset<LAYOUT>(r, n, K, N)];
      const uint32_t sbyte = S[scale_offset<LAYOUT>(r / 16, n, K, N)];
      uint32_t v = fp4x2_to_bf16x2<0>(byte, e8m0_to_f32(sbyte));
      if (sbyte == 0xFFu) v = e8m0_nan_pair(byte);
      const size_t o0 = (2 * r) * (size_t)N + n, o1 = o0 + N;
      if (out_bf16) {
        static_cast<uint16_t*>(out)[o0] = (uint16_t)(v & 0xFFFFu);
        static_cast<uint16_t*>(out)[o1] = (uint16_t)(v >> 16);
      } else {
        static_cast<float*>(out)[o0] = __builtin_bit_cast(float, v << 16);
        static_cast<float*>(out)[o1] = __builtin_bit_cast(float, v & 0xFFFF0000u);
      }
    }
  }

  // One thread per output element; fp32 accumulation in K order.
template <int LAYOUT>
__global__ void __launch_bounds__(256) generic_kernel(const uint16_t* __restrict__ A,
                                                      const uint8_t* __restrict__ B,
                                                      const uint8_t* __restrict__ S, void* C,
                                                      int out_bf16, int M, int N, int K, Epilogue ep) {
  const size_t total = (size_t)M * N;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int m = (int)(idx / N), n = (int)(idx - (size_t)m * N);
    float acc = 0.f;
    for (int kp = 0; kp < K / 2; ++kp) {
      const uint32_t byte = B[code_offset<LAYOUT>(kp, n, K, N)];
      const uint32_t sbyte = S[scale_offset<LAYOUT>(kp / 16, n, K, N)];
      const uint32_t w = fp4x2_to_bf16x2<0>(byte, e8m0_to_f32(sbyte));
      const float a0 = __builtin_bit_cast(float, (uint32_t)A[(size_t)m * K + 2 * kp] << 16);
      const float a1 = __builtin_bit_cast(float, (uint32_t)A[(size_t)m * K + 2 * kp + 1] << 16);
      acc = __builtin_fmaf(a0, __builtin_bit_cast(float, w << 16), acc);
      acc = __builtin_fmaf(a1, __builtin_bit_cast(float, w & 0xFFFF0000u), acc);
    }
    if (ep.any) acc = epilogue_value(ep, acc, m, n, N);
    if (out_bf16)
      static_cast<uint16_t*>(C)[idx] = (uint16_t)bf16_bits_rne(acc);
    else
      static_cast<float*>(C)[idx] = acc;
  }
}

// Layout conversion of the codes: one thread per 16 destination bytes (one
// 16-byte store).  The 16 bytes' positions (kp, n) follow from the first one
// in every destination layout except [K/2, N] with N % 16 != 0, where the
// row may end inside the vector.  Sources whose 16 bytes are one aligned
// vector as well ([N,K/2] <-> panels) are read as one 16-byte load.
template <int SRC, int DST>
__global__ void __launch_bounds__(256) convert_codes_kernel(const uint8_t* __restrict__ B,
                                                            uint8_t* __restrict__ out, size_t K,
                                                            size_t N) {
  const size_t total = K / 2 * N;
  for (size_t o = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; o < total;
       o += (size_t)gridDim.x * blockDim.x * 16) {
    size_t kp0, n0;
    code_position<DST>(o, K, N, kp0, n0);
    constexpr bool kRun = DST == kLayoutNK || DST == kLayoutP;  // 16 consecutive kp of one column
    if constexpr (kRun && (SRC == kLayoutNK || SRC == kLayoutP)) {
      *reinterpret_cast<u32x4*>(out + o) =
          *reinterpret_cast<const u32x4*>(B + code_offset<SRC>(kp0, n0, K, N));
      continue;
    }
    uint8_t v[16];
    const bool kn_row = DST == kLayoutKN && N % 16 == 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      size_t kp = kp0, n = n0;
      if constexpr (kRun) {
        kp = kp0 + i;
      } else if constexpr (DST == kLayoutG) {
        kp = kp0 + i % 4;
        n = n0 + i / 4;
      } else {
        if (kn_row)
          n = n0 + i;
        else
          code_position<DST>(o + i, K, N, kp, n);
      }
      v[i] = B[code_offset<SRC>(kp, n, K, N)];
    }
    u32x4 w;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      w[j] = (uint32_t)v[4 * j] | ((uint32_t)v[4 * j + 1] << 8) | ((uint32_t)v[4 * j + 2] << 16) |
             ((uint32_t)v[4 * j + 3] << 24);
    *reinterpret_cast<u32x4*>(out + o) = w;
  }
}

// Layout conversion of the scales: one thread per destination byte.
template <int SRC, int DST>
__global__ void __launch_bounds__(256) convert_scales_kernel(const uint8_t* __restrict__ S,
                                                             uint8_t* __restrict__ out, size_t K,
                                                             size_t N) {
  for (size_t o = (size_t)blockIdx.x * blockDim.x + threadIdx.x; o < K / 32 * N;
       o += (size_t)gridDim.x * blockDim.x) {
    size_t g, n;
    scale_position<DST>(o, K, N, g, n);
    out[o] = S[scale_offset<SRC>(g, n, K, N)];
  }
}

// [N,K/2] -> G without byte gathers (the rewrite a via-G GEMM plan runs
// before the tiled kernel, and convert_layout's path for this pair): one
// workgroup per 32 columns (a quarter of a G block) and 64 code dwords (512
// K) with their 16 scale groups, transposed through LDS so that the reads
// (256 contiguous bytes of a column) and the writes (the 32 columns of a G
// chunk row: 128 contiguous bytes) are whole lines, all 16 bytes per lane
// (scale reads too when a column's 16 groups are 16-byte aligned); small
// tiles keep ~9 workgroups per CU in flight on dit_up-sized weights.
// B and B_out 16-byte aligned, N % 128 == 0.
constexpr int kCvW = 64;  // code dwords (8 K each) per workgroup
constexpr int kCvC = 32;  // columns per workgroup
__global__ void __launch_bounds__(256) convert_nk_to_g_kernel(const uint8_t* __restrict__ B,
                                                               const uint8_t* __restrict__ S,
                                                               uint8_t* __restrict__ B_out,
                                                               uint8_t* __restrict__ S_out, int K) {
  // [column][dword] padded to 65 words: a 32-lane pass of the transposed
  // reads (8 column quads x 4 chunk rows) falls on 32 distinct banks;
  // scales [column][group] in 20-byte rows
  __shared__ uint32_t t[kCvC][kCvW + 1];
  __shared__ __attribute__((aligned(16))) uint8_t ts[kCvC][kCvW / 4 + 4];
  const size_t n0 = (size_t)blockIdx.x * kCvC;  // first column
  const size_t nb = n0 / kGCols;
  const int c0 = (int)(n0 % kGCols);              // its place in the G block
  const int kw = K / 8, gk = K / 32;
  const int w0 = (int)blockIdx.y * kCvW;
  const int nw = min(kCvW, kw - w0);  // a multiple of 4 (K % 32 == 0)
  const int g0 = w0 / 4, ng = nw / 4;
  const bool svec = ng == kCvW / 4 && gk % 16 == 0 && ((uintptr_t)S & 15u) == 0;
  for (int i = threadIdx.x; i < kCvC * 16; i += 256) {
    const int col = i >> 4, j = (i & 15) * 4;
    if (j < nw) {
      const u32x4 v = *reinterpret_cast<const u32x4*>(B + (n0 + col) * (size_t)(K / 2) + (size_t)(w0 + j) * 4);
      t[col][j] = v.x;
      t[col][j + 1] = v.y;
      t[col][j + 2] = v.z;
      t[col][j + 3] = v.w;
    }
  }
  if (svec) {
    if (threadIdx.x < kCvC) {
      const int col = threadIdx.x;
      const u32x4 v = *reinterpret_cast<const u32x4*>(S + (n0 + col) * (size_t)gk + g0);
      uint32_t* r = reinterpret_cast<uint32_t*>(&ts[col][0]);  // 20-byte rows: 4-byte aligned
      r[0] = v.x;
      r[1] = v.y;
      r[2] = v.z;
      r[3] = v.w;
    }
  } else {
    for (int i = threadIdx.x; i < kCvC * 16; i += 256) {
      const int col = i >> 4, g = i & 15;
      if (g < ng) ts[col][g] = S[(n0 + col) * (size_t)gk + g0 + g];
    }
  }
  __syncthreads();
  // chunk row w, columns 4q .. 4q+3 of the workgroup's 32: one 16-byte store
  for (int i = threadIdx.x; i < kCvW * (kCvC / 4); i += 256) {
    const int w = i >> 3, q = i & 7;
    if (w < nw) {
      const u32x4 v = {t[4 * q][w], t[4 * q + 1][w], t[4 * q + 2][w], t[4 * q + 3][w]};
      *reinterpret_cast<u32x4*>(B_out + ((nb * kw + w0 + w) * kGCols + c0 + 4 * q) * 4) = v;
    }
  }
  if (threadIdx.x < (kCvW / 4) * (kCvC / 4)) {
    const int g = threadIdx.x >> 3, q = threadIdx.x & 7;
    if (g < ng) {
      const uint32_t v = (uint32_t)ts[4 * q][g] | (uint32_t)ts[4 * q + 1][g] << 8 |
                         (uint32_t)ts[4 * q + 2][g] << 16 | (uint32_t)ts[4 * q + 3][g] << 24;
      *reinterpret_cast<uint32_t*>(S_out + (nb * gk + g0 + g) * kGCols + c0 + 4 * q) = v;
    }
  }
}

// 16 bytes per thread; vector stores when p is 16-byte aligned (C may be a
// view at any element offset), byte stores otherwise and for the tail.
__global__ void __launch_bounds__(256) zero_fill_kernel(uint8_t* p, size_t bytes) {
  for (size_t i = ((size_t)blockIdx.x * blockDim.x + threadIdx.x) * 16; i < bytes;
       i += (size_t)gridDim.x * blockDim.x * 16) {
    if (i + 16 <= bytes && ((uintptr_t)p & 15u) == 0) {
      *reinterpret_cast<u32x4*>(p + i) = u32x4{0u, 0u, 0u, 0u};
    } else {
      const size_t end = i + 16 < bytes ? i + 16 : bytes;
      for (size_t j = i; j < end; ++j) p[j] = 0;
    }
  }
}

}  // namespace

namespace {

template <template <int> class F, typename... Args>
hipError_t by_layout(int layout, Args... args) {
  switch (layout) {
    case kLayoutKN: return F<kLayoutKN>::run(args...);
    case kLayoutNK: return F<kLayoutNK>::run(args...);
    case kLayoutG: return F<kLayoutG>::run(args...);
    case kLayoutP: return F<kLayoutP>::run(args...);
    default: return hipErrorInvalidValue;
  }
}

template <int L>
struct DequantLaunch {
  static hipError_t run(const uint8_t* B, const uint8_t* S, void* out, int out_bf16, int K, int N,
                        hipStream_t stream) {
    const size_t total = (size_t)(K / 2) * N;
    hipLaunchKernelGGL(dequant_kernel<L>, dim3(grid_for(total)), dim3(256), 0, stream,
                       B, S, out, out_bf16, K, N);
    return hipGetLastError();
  }
};

template <int L>
struct GenericLaunch {
  static hipError_t run(const uint16_t* A, const uint8_t* B, const uint8_t* S, void* C, int out_bf16,
                        int M, int N, int K, Epilogue ep, hipStream_t stream) {
    const size_t total = (size_t)M * N;
    hipLaunchKernelGGL(generic_kernel<L>, dim3(grid_for(total)), dim3(256), 0, stream,
                       A, B, S, C, out_bf16, M, N, K, ep);
    return hipGetLastError();
  }
};

template <int SRC>
struct ConvertFrom {
  template <int DST>
  struct To {
    static hipError_t run(const uint8_t* B, const uint8_t* S, uint8_t* B_out, uint8_t* S_out,
                          size_t K, size_t N, hipStream_t stream) {
      if constexpr (SRC == kLayoutNK && DST == kLayoutG) {
        if (((uintptr_t)B & 15u) == 0 && ((uintptr_t)B_out & 15u) == 0 && ((uintptr_t)S_out & 3u) == 0 &&
            K <= (size_t)INT32_MAX)
          return launch_convert_nk_to_g(B, S, B_out, S_out, K, N, stream);
      }
      const size_t vecs = K / 2 * N / 16, sbytes = K / 32 * N;
      hipLaunchKernelGGL((convert_codes_kernel<SRC, DST>), dim3(grid_for(vecs)),
                         dim3(256), 0, stream, B, B_out, K, N);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
      hipLaunchKernelGGL((convert_scales_kernel<SRC, DST>), dim3(grid_for(sbytes)),
                         dim3(256), 0, stream, S, S_out, K, N);
      return hipGetLastError();
    }
  };
};

template <int SRC>
struct ConvertLaunch {
  static hipError_t run(int dst, const uint8_t* B, const uint8_t* S, uint8_t* B_out, uint8_t* S_out,
                        size_t K, size_t N, hipStream_t stream) {
    return by_layout<ConvertFrom<SRC>::template To>(dst, B, S, B_out, S_out, K, N, stream);
  }
};

}  // namespace

hipError_t launch_dequant(int layout, const uint8_t* B, const uint8_t* S, void* out, int out_bf16,
                          int K, int N, hipStream_t stream) {
  if ((size_t)(K / 2) * N == 0) return hipSuccess;
  return by_layout<DequantLaunch>(layout, B, S, out, out_bf16, K, N, stream);
}

hipError_t launch_generic(int layout, const uint16_t* A, const uint8_t* B, const uint8_t* S,
                          void* C, int out_bf16, int M, int N, int K, const Epilogue& ep,
                          hipStream_t stream) {
  if ((size_t)M * N == 0) return hipSuccess;
  return by_layout<GenericLaunch>(layout, A, B, S, C, out_bf16, M, N, K, ep, stream);
}

hipError_t launch_convert(int src_layout, int dst_layout, const uint8_t* B, const uint8_t* S,
                          uint8_t* B_out, uint8_t* S_out, size_t K, size_t N, hipStream_t stream) {
  if (K * N == 0) return hipSuccess;
  return by_layout<ConvertLaunch>(src_layout, dst_layout, B, S, B_out, S_out, K, N, stream);
}

hipError_t launch_convert_nk_to_g(const uint8_t* B, const uint8_t* S, uint8_t* B_out, uint8_t* S_out, size_t K,
                                  size_t N, hipStream_t stream) {
  if (K * N == 0) return hipSuccess;
  if (N % kGCols != 0 || K % 32 != 0 || K > (size_t)INT32_MAX || N / kCvC > (size_t)INT32_MAX ||
      ((uintptr_t)B & 15u) != 0 || ((uintptr_t)B_out & 15u) != 0 || ((uintptr_t)S_out & 3u) != 0)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)(N / kCvC), (unsigned)((K / 8 + kCvW - 1) / kCvW));
  hipLaunchKernelGGL(convert_nk_to_g_kernel, grid, dim3(256), 0, stream, B, S, B_out, S_out, (int)K);
  return hipGetLastError();
}

hipError_t launch_zero_fill(void* C, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return hipSuccess;
  const size_t chunks = (bytes + 15) / 16;
  hipLaunchKernelGGL(zero_fill_kernel, dim3(grid_for(chunks)), dim3(256), 0, stream,
                     static_cast<uint8_t*>(C), bytes);
  return hipGetLastError();
}

}  // namespace mxfp4
