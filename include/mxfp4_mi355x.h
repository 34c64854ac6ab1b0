/*
 * mxfp4_mi355x.h -- C ABI of the MI355X (gfx950) MXFP4-weight x BF16-activation GEMM.
 *
 * This is the drop-in boundary for konradha/cdna3-bench's dequant-GEMM path.
 * The reference binds its kernels through C++-mangled launchers in
 * namespace mxfp4_cdna3 (csrc/common.h:43-78) wrapped by a pybind11/torch
 * extension (csrc/mxfp4_ext.cpp:11-225).  Here every entry point is extern "C"
 * with plain pointers and sizes; the torch extension (_C) and any other FFI
 * (ctypes, cgo, JNI) bind these symbols.
 *
 * Conventions shared by every entry point:
 *   - Device pointers, all on the current HIP device, 16-byte aligned.
 *   - A: bf16 [M, K] row-major.  C: [M, N] row-major, fp32 or bf16.
 *   - Weights: E2M1 codes two per byte (low nibble = even K index) with one
 *     E8M0 scale byte per 32 K elements:
 *       MXFP4_LAYOUT_KN: B [K/2, N], S [K/32, N]   (reference API layout,
 *                        csrc/mxfp4_ext.cpp:21-24)
 *       MXFP4_LAYOUT_NK: B [N, K/2], S [N, K/32]   (K-contiguous weights)
 *       MXFP4_LAYOUT_G:  B [N/128][K/8][128][4], S [N/128][K/32][128]
 *                        (strategy G prepack, python/mxfp4_cdna3/ref.py:85-101;
 *                        needs N % 128 == 0)
 *       MXFP4_LAYOUT_P:  B [N/32][K/64][2][32][16], S [N/32][K/64][2][32]
 *                        (panels: each 32-column x 64-K block of codes is 1 KB
 *                        in wave-lane order -- 16 bytes = 32 K of one column
 *                        per lane -- with its 64 scale bytes in the same lane
 *                        order; needs N % 32 == 0 and K % 64 == 0)
 *     In every layout packed byte kp of column n holds K = 2kp and 2kp + 1 of
 *     that column, and scale byte g scales K = 32g .. 32g + 31.
 *   - K % 32 == 0 (csrc/mxfp4_ext.cpp:28).  Any M >= 0, N >= 0 within the
 *     layout's rule above.
 *   - Launches are asynchronous on `stream`; nothing synchronizes.
 *   - Return value is a hipError_t: hipSuccess, hipErrorInvalidValue for bad
 *     arguments (same convention as the reference launchers, e.g.
 *     csrc/strategy_j_synthesis.cu:178), else the launch error.
 *   - Every element of C is written; C needs no initialisation.
 *   - Results are deterministic: split-K partials are summed in a fixed order.
 */
#ifndef MXFP4_MI355X_H
#define MXFP4_MI355X_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MXFP4_LAYOUT_KN = 0, MXFP4_LAYOUT_NK = 1, MXFP4_LAYOUT_G = 2, MXFP4_LAYOUT_P = 3 };
enum { MXFP4_OUT_F32 = 0, MXFP4_OUT_BF16 = 1 };
enum { MXFP4_IN_F32 = 0, MXFP4_IN_BF16 = 1 };
enum { MXFP4_ACT_NONE = 0, MXFP4_ACT_SILU = 1, MXFP4_ACT_GELU_ERF = 2, MXFP4_ACT_GELU_TANH = 3 };
enum {
  MXFP4_KERNEL_AUTO = 0,    /* cost-model choice */
  MXFP4_KERNEL_GEMV = 1,    /* memory-bound family, M <= 32 */
  MXFP4_KERNEL_TILED = 2,   /* MFMA-bound tiled family */
  MXFP4_KERNEL_GENERIC = 3, /* one thread per output, any N */
  MXFP4_KERNEL_STREAM = 4   /* weight streaming, M <= 32, NK or P layout, K % 256 == 0: split-K
                               (variants 0-4) and whole-K (5, 6: M <= 16) kernels; NK only:
                               decode (7: M <= 16, 8: M <= 8) and resident (9 and 13:
                               M == 1, 10: M <= 8; K % 512 == 0, K <= 8192; 11: M <= 32,
                               12: M <= 16; K % 256 == 0, ceil(K / 2048) <= 8 splits)
                               kernels */
};

/* A launch plan: which kernel family, which tile variant, how many K splits. */
typedef struct mxfp4_plan {
  int32_t kernel;  /* MXFP4_KERNEL_* */
  int32_t variant; /* family-specific tile id (see mxfp4_plan_describe) */
  int32_t split_k; /* >= 1 */
  int32_t flags;   /* 0, or MXFP4_PLAN_* bits below */
} mxfp4_plan;

/*
 * Plan flag for tests of the streaming split-K protocol (MXFP4_KERNEL_STREAM
 * with split_k > 1; ignored otherwise): the late unit of each column group
 * does not poll its partners' partials, so every group is reduced by the
 * last of its arrivals -- the path the kernel takes when a group's CTAs are
 * not resident together.  Results are bit-identical to the default path.
 */
#define MXFP4_PLAN_STREAM_NO_POLL 1

/*
 * Plan flag for MXFP4_KERNEL_TILED with [N,K/2] weights, N % 128 == 0 and
 * K % 64 == 0: the call first rewrites the weights to the G layout in the
 * workspace (after the split-K counters and partials -- the counter region
 * is kept even at split 1, as the workspace may serve other calls: K/2 * N
 * code bytes and K/32 * N scale bytes, each rounded up to 256), then runs the
 * tiled variant on G.  The
 * [N,K/2] operand reads of the tiled kernels are 2-way LDS bank-conflicted;
 * for MFMA-bound shapes the rewrite costs less than it saves.  The automatic
 * plan sets it when the cost model says so and the workspace holds it
 * (mxfp4_gemm_workspace_bytes with a NULL plan counts it; a call with a
 * smaller or no workspace gets the direct plan).  Results are bit-identical
 * to the direct plan's.
 */
#define MXFP4_PLAN_TILED_VIA_G 2

/*
 * Fused epilogue: C = act(A x W + bias) + residual, in fp32, then rounded to
 * C's dtype.  act: SiLU x / (1 + e^-x); GELU 0.5 x (1 + erf(x / sqrt 2));
 * GELU-tanh 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) -- the
 * definitions of torch.nn.functional.silu / gelu.  bias: [N]; residual:
 * [M, N] row-major, may be C itself (each element is read before it is
 * written by the same thread).  NULL pointers skip the term.
 */
typedef struct mxfp4_epilogue {
  const void* bias;       /* [N] or NULL */
  const void* residual;   /* [M, N] or NULL */
  int32_t bias_dtype;     /* MXFP4_OUT_F32 or MXFP4_OUT_BF16 */
  int32_t residual_dtype; /* MXFP4_OUT_F32 or MXFP4_OUT_BF16 */
  int32_t activation;     /* MXFP4_ACT_* */
  int32_t reserved;       /* 0 */
} mxfp4_epilogue;

/* Device properties; replaces device_info (csrc/mxfp4_ext.cpp:156-168). */
typedef struct mxfp4_device_info_t {
  char name[256];
  char gcn_arch_name[256];
  int32_t multi_processor_count;
  int32_t warp_size;
  int64_t total_global_mem;
  int64_t shared_mem_per_block;
} mxfp4_device_info_t;

/*
 * The plan mxfp4_gemm would use for this problem (cost model for 256 CUs,
 * 8 TB/s HBM, 2.5 PF/s dense bf16 MFMA).  Replaces gemm_auto's divisibility
 * cascade (python/mxfp4_cdna3/kernels.py:63-74).
 */
hipError_t mxfp4_select_plan(int64_t M, int64_t N, int64_t K, int b_layout, mxfp4_plan* out);

/* Human-readable description of a plan, e.g. "tiled 256x256 w2x2 split1". */
hipError_t mxfp4_plan_describe(const mxfp4_plan* plan, char* buf, size_t buf_len);

/*
 * Workspace bytes mxfp4_gemm needs for this problem under `plan` (NULL = the
 * auto plan).  The first MXFP4_COUNTER_BYTES bytes hold split-K counters:
 * they must be zero before the first call and every call leaves them zero.
 * Calls that share one workspace must be stream-ordered.
 */
#define MXFP4_COUNTER_BYTES ((size_t)1 << 20)
size_t mxfp4_gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int b_layout,
                                  const mxfp4_plan* plan);

/*
 * C[M,N] = A[M,K] x dequant(B, S)[K,N], fp32 accumulation, C in fp32
 * (c_dtype MXFP4_OUT_F32) or bf16 rounded to nearest even (MXFP4_OUT_BF16).
 * Replaces launch_strategy_{a..m} (csrc/common.h:43-78) and the reference's
 * dispatch (csrc/mxfp4_ext.cpp:36-48); unlike those it accepts every M, N.
 */
hipError_t mxfp4_gemm(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                      int64_t M, int64_t N, int64_t K, int b_layout, void* workspace,
                      size_t workspace_bytes, hipStream_t stream);

/* As mxfp4_gemm with an explicit plan (tuning, tests).  plan->kernel AUTO = mxfp4_gemm. */
hipError_t mxfp4_gemm_with_plan(const void* A, const uint8_t* B, const uint8_t* S, void* C,
                                int c_dtype, int64_t M, int64_t N, int64_t K, int b_layout,
                                const mxfp4_plan* plan, void* workspace, size_t workspace_bytes,
                                hipStream_t stream);

/*
 * mxfp4_gemm_with_plan with a fused epilogue (ep NULL = none; plan NULL =
 * the auto plan).  No counterpart in the reference, whose kernels end in a
 * plain fp32 store (csrc/bf16_gemm.h:136-153); it replaces the separate
 * bias / activation / residual passes a caller would run over C.
 */
hipError_t mxfp4_gemm_ex(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                         int64_t M, int64_t N, int64_t K, int b_layout, const mxfp4_plan* plan,
                         const mxfp4_epilogue* ep, void* workspace, size_t workspace_bytes,
                         hipStream_t stream);

/*
 * mxfp4_gemm without a workspace argument and without any allocation: the
 * split-K workspace is a fixed device array of MXFP4_NOALLOC_SCRATCH_BYTES
 * inside the library, one per GPU, held until the process ends (the first
 * call on a GPU looks up its address and queues one zero fill of it on
 * `stream`).  No counterpart in the reference: it is for callers that cannot
 * allocate -- code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc.  Same plan, results and errors as mxfp4_gemm, plus
 * hipErrorOutOfMemory when the plan's workspace (mxfp4_gemm_workspace_bytes)
 * exceeds MXFP4_NOALLOC_SCRATCH_BYTES (nothing is launched then), and
 * hipErrorStreamCaptureUnsupported when the first call on a GPU comes while
 * `stream` is capturing a graph (that call's zero fill must run, not be
 * recorded; later calls may be captured).  Every call
 * on one GPU shares that GPU's array: calls that overlap in time on one GPU
 * (other streams, other threads) race and must be ordered by the caller.
 */
#define MXFP4_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
hipError_t mxfp4_gemm_noalloc(const void* A, const uint8_t* B, const uint8_t* S, void* C, int c_dtype,
                              int64_t M, int64_t N, int64_t K, int b_layout, hipStream_t stream);

/*
 * out[K, N] = dequant(B, S) as bf16 (out_dtype MXFP4_OUT_BF16) or fp32.
 * Bit-exact device counterpart of dequantize_mxfp4(..., axis=0)
 * (python/mxfp4_cdna3/ref.py:50-72) for every scale byte: 0 scales by
 * 2^-127 (subnormals kept), 255 gives +-inf and NaN for codes 0 and 8, as
 * ref.py's float32 arithmetic does.  Replaces dequant_b_kernel
 * (csrc/strategy_a_two_pass.cu:8-37).
 */
hipError_t mxfp4_dequant(const uint8_t* B, const uint8_t* S, void* out, int out_dtype, int64_t K,
                         int64_t N, int b_layout, hipStream_t stream);

/*
 * Rewrites weights (codes B, scales S) of a K x N matrix from one layout to
 * another on the device: B_out/S_out receive the same bytes at the positions
 * of dst_layout.  Device counterpart of prepack_b_mxfp4
 * (python/mxfp4_cdna3/ref.py:85-101, which the reference runs on the host
 * before upload); any pair of MXFP4_LAYOUT_* works, including the inverse
 * direction.  Both layouts' shape rules apply.  Sources and destinations
 * must not overlap; B_out 16-byte aligned.
 */
hipError_t mxfp4_convert_layout(const uint8_t* B, const uint8_t* S, int src_layout, uint8_t* B_out,
                                uint8_t* S_out, int dst_layout, int64_t K, int64_t N,
                                hipStream_t stream);

/*
 * Quantizes a K x N weight matrix X to MXFP4: codes B and E8M0 scales S in
 * b_layout (any MXFP4_LAYOUT_*, its shape rules apply), one scale per 32 K.
 * X is fp32 or bf16 (x_dtype MXFP4_IN_*), row-major [K, N] (x_layout
 * MXFP4_LAYOUT_KN: quantize_mxfp4(X, axis=0)) or [N, K] (MXFP4_LAYOUT_NK:
 * quantize_mxfp4(X, axis=-1)).  Device counterpart of quantize_mxfp4
 * (python/mxfp4_cdna3/ref.py:14-47), bit-exact with it for finite inputs
 * (argmin ties to the smaller magnitude; float32 ceil(log2(amax / 6))
 * clipped to [-127, 127]); NaN / inf inputs give unspecified codes.  X and
 * B 16-byte aligned.
 */
hipError_t mxfp4_quantize(const void* X, int x_dtype, int x_layout, int64_t K, int64_t N, uint8_t* B,
                          uint8_t* S, int b_layout, hipStream_t stream);

/*
 * The reference's shape predicates (csrc/common.h:80-99), strategy 'c'..'g'
 * (and 'a','b' = 'c'); 1 if supported, 0 if not, -1 for an unknown letter.
 */
int mxfp4_shape_supported(char strategy, int64_t M, int64_t N, int64_t K);

/* Device properties of `dev` (csrc/mxfp4_ext.cpp:156-168). */
hipError_t mxfp4_device_info(int dev, mxfp4_device_info_t* out);

/* Library version string. */
const char* mxfp4_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MXFP4_MI355X_H */
