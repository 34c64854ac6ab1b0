// PyTorch-ROCm extension `mxfp4_cdna3._C`: the reference's operator surface
// (csrc/mxfp4_ext.cpp:1-225) over the C ABI in include/mxfp4_mi355x.h.
//
// Same Python-visible names, arguments, defaults, validation order and error
// strings as the reference:
//   gemm_{a,b,c,d,e,f,h,i,j,k,m}(A, B_packed, B_scales, C=None)   (:50-125)
//   gemm_g(A, B_prep, Bs_prep, C=None)                             (:127-154)
//   device_info(dev_id=0), shape_supported_{c,d,e,f,g}(M, N, K)    (:156-224)
// Every letter keeps the reference's accepted shapes (strategy A/B reject
// shapes outside shape_supported_c with "launch_strategy_x: invalid argument",
// the others raise "Strategy X requires ..."), and all of them run the one
// gfx950 path chosen by the library's cost model; gemm_g reads the G
// prepack directly.  Additions: gemm_auto (every shape with K % 32 == 0),
// gemm (any weight layout, explicit plan), dequant, quantize (device
// quantize_mxfp4), convert_layout (device prepack between layouts),
// select_plan.  C may be fp32 (the reference's
// only dtype) or bf16.
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <map>
#include <mutex>
#include <string>
#include <utility>

#include "mxfp4_mi355x.h"

namespace {

// Split-K workspace per (device, stream): zero-filled on allocation (split-K
// counters and packets must start at zero; every call leaves them at zero)
// and grown on demand.  Calls on one stream run in order, so a stream's
// workspace is never used by two kernels at once.  A grown-out buffer goes
// back to torch's caching allocator, which hands it out again only in the
// order of the stream it was allocated on (this one).  Allocation is refused
// while the stream captures a graph: the zero fill would only be recorded.
std::mutex g_ws_mutex;
std::map<std::pair<int, hipStream_t>, torch::Tensor> g_ws;

torch::Tensor workspace_for(const torch::Tensor& like, hipStream_t stream, size_t bytes) {
  if (bytes == 0) return torch::Tensor();
  std::lock_guard<std::mutex> lock(g_ws_mutex);
  const auto key = std::make_pair((int)like.get_device(), stream);
  auto it = g_ws.find(key);
  if (it == g_ws.end() || (size_t)it->second.numel() < bytes) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    TORCH_CHECK(hipStreamIsCapturing(stream, &status) == hipSuccess, "hipStreamIsCapturing failed");
    TORCH_CHECK(status == hipStreamCaptureStatusNone,
                "mxfp4_cdna3: this call needs a ", bytes, "-byte split-K workspace on the capturing stream; "
                "run it once on that stream before the graph capture (the workspace is kept per stream)");
    size_t want = bytes;
    if (it != g_ws.end()) want = std::max(bytes, (size_t)it->second.numel() * 2);
    g_ws[key] = torch::zeros({(int64_t)want}, like.options().dtype(at::kByte));
    it = g_ws.find(key);
  }
  return it->second;
}

// Layout names of the Python API.
int layout_code(const std::string& layout) {
  if (layout == "kn") return MXFP4_LAYOUT_KN;
  if (layout == "nk") return MXFP4_LAYOUT_NK;
  if (layout == "g") return MXFP4_LAYOUT_G;
  if (layout == "p") return MXFP4_LAYOUT_P;
  TORCH_CHECK(false, "layout must be 'kn', 'nk', 'g' or 'p'");
  return -1;
}

bool prepacked(int layout) { return layout == MXFP4_LAYOUT_G || layout == MXFP4_LAYOUT_P; }

int out_code(const torch::Tensor& C) {
  return C.scalar_type() == at::kBFloat16 ? MXFP4_OUT_BF16 : MXFP4_OUT_F32;
}

// Reference check_inputs (csrc/mxfp4_ext.cpp:11-31), with bf16 C accepted.
hipStream_t check_inputs(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& S,
                         const torch::Tensor& C, int64_t M, int64_t N, int64_t K, int layout) {
  TORCH_CHECK(A.is_cuda() && B.is_cuda() && S.is_cuda() && C.is_cuda(),
              "all tensors must be on GPU");
  TORCH_CHECK(A.scalar_type() == at::kBFloat16, "A must be bfloat16");
  TORCH_CHECK(B.scalar_type() == at::kByte, "B_packed must be uint8");
  TORCH_CHECK(S.scalar_type() == at::kByte, "B_scales must be uint8");
  TORCH_CHECK(C.scalar_type() == at::kFloat || C.scalar_type() == at::kBFloat16,
              "C must be float32 or bfloat16");
  TORCH_CHECK(A.dim() == 2 && A.size(0) == M && A.size(1) == K, "A shape");
  if (layout == MXFP4_LAYOUT_KN) {
    TORCH_CHECK(B.dim() == 2 && B.size(0) == K / 2 && B.size(1) == N, "B_packed shape");
    TORCH_CHECK(S.dim() == 2 && S.size(0) == K / 32 && S.size(1) == N, "B_scales shape");
  } else if (prepacked(layout)) {
    // any shape with the layout's element count (the reference passes flat arrays)
    TORCH_CHECK(B.numel() == K / 2 * N, "B_packed size");
    TORCH_CHECK(S.numel() == K / 32 * N, "B_scales size");
  } else {
    TORCH_CHECK(B.dim() == 2 && B.size(0) == N && B.size(1) == K / 2, "B_packed shape");
    TORCH_CHECK(S.dim() == 2 && S.size(0) == N && S.size(1) == K / 32, "B_scales shape");
  }
  TORCH_CHECK(C.dim() == 2 && C.size(0) == M && C.size(1) == N, "C shape");
  TORCH_CHECK(A.is_contiguous() && B.is_contiguous() && S.is_contiguous() && C.is_contiguous(),
              "tensors must be contiguous");
  TORCH_CHECK(K % 32 == 0, "K must be a multiple of 32");
  TORCH_CHECK(A.get_device() == B.get_device() && A.get_device() == S.get_device() &&
                  A.get_device() == C.get_device(),
              "all tensors must be on the same GPU");
  return c10::hip::getCurrentHIPStream(A.get_device()).stream();
}

void launch(const char* name, const torch::Tensor& A, const torch::Tensor& B,
            const torch::Tensor& S, torch::Tensor& C, int64_t M, int64_t N, int64_t K, int layout,
            const mxfp4_plan* plan, hipStream_t stream, const mxfp4_epilogue* ep = nullptr) {
  const size_t ws_bytes = mxfp4_gemm_workspace_bytes(M, N, K, layout, plan);
  torch::Tensor ws = workspace_for(A, stream, ws_bytes);
  hipError_t err = mxfp4_gemm_ex(A.data_ptr(), static_cast<const uint8_t*>(B.data_ptr()),
                                 static_cast<const uint8_t*>(S.data_ptr()), C.data_ptr(), out_code(C), M, N,
                                 K, layout, plan, ep, ws_bytes ? ws.data_ptr() : nullptr, ws_bytes, stream);
  TORCH_CHECK(err == hipSuccess, name, ": ", hipGetErrorString(err));
}

int activation_code(const c10::optional<std::string>& act) {
  if (!act.has_value() || *act == "none") return MXFP4_ACT_NONE;
  if (*act == "silu") return MXFP4_ACT_SILU;
  if (*act == "gelu") return MXFP4_ACT_GELU_ERF;
  if (*act == "gelu_tanh") return MXFP4_ACT_GELU_TANH;
  TORCH_CHECK(false, "activation must be None, 'silu', 'gelu' or 'gelu_tanh'");
  return MXFP4_ACT_NONE;
}

// Fused epilogue arguments: bias [N], residual [M, N] (fp32 or bf16, on C's device).
mxfp4_epilogue make_epilogue(const torch::Tensor& C, int64_t M, int64_t N, const c10::optional<torch::Tensor>& bias,
                             const c10::optional<std::string>& activation,
                             const c10::optional<torch::Tensor>& residual) {
  mxfp4_epilogue ep{};
  ep.activation = activation_code(activation);
  auto dtype_code = [](const torch::Tensor& t, const char* what) {
    TORCH_CHECK(t.scalar_type() == at::kFloat || t.scalar_type() == at::kBFloat16, what,
                " must be float32 or bfloat16");
    return t.scalar_type() == at::kBFloat16 ? MXFP4_OUT_BF16 : MXFP4_OUT_F32;
  };
  if (bias.has_value()) {
    const auto& b = *bias;
    TORCH_CHECK(b.is_cuda() && b.get_device() == C.get_device(), "bias must be on C's GPU");
    TORCH_CHECK(b.dim() == 1 && b.size(0) == N && b.is_contiguous(), "bias must be a contiguous [N] vector");
    ep.bias = b.data_ptr();
    ep.bias_dtype = dtype_code(b, "bias");
  }
  if (residual.has_value()) {
    const auto& r = *residual;
    TORCH_CHECK(r.is_cuda() && r.get_device() == C.get_device(), "residual must be on C's GPU");
    TORCH_CHECK(r.dim() == 2 && r.size(0) == M && r.size(1) == N && r.is_contiguous(),
                "residual must be a contiguous [M, N] matrix");
    ep.residual = r.data_ptr();
    ep.residual_dtype = dtype_code(r, "residual");
  }
  return ep;
}

// (kernel, variant, split_k[, flags]) of the Python API.
mxfp4_plan plan_from(const std::vector<int64_t>& v) {
  TORCH_CHECK(v.size() == 3 || v.size() == 4, "plan must be (kernel, variant, split_k[, flags])");
  return mxfp4_plan{(int32_t)v[0], (int32_t)v[1], (int32_t)v[2], v.size() == 4 ? (int32_t)v[3] : 0};
}

// Reference dispatch (csrc/mxfp4_ext.cpp:36-48): C=None -> fp32 [M, N].
torch::Tensor dispatch(const char* name, const torch::Tensor& A, const torch::Tensor& B,
                       const torch::Tensor& S, c10::optional<torch::Tensor> C_opt) {
  const int64_t M = A.size(0), K = A.size(1), N = B.size(1);
  torch::Tensor C = C_opt.has_value() ? *C_opt : torch::empty({M, N}, A.options().dtype(at::kFloat));
  auto stream = check_inputs(A, B, S, C, M, N, K, MXFP4_LAYOUT_KN);
  launch(name, A, B, S, C, M, N, K, MXFP4_LAYOUT_KN, nullptr, stream);
  return C;
}

// Strategy A/B: the reference launchers return hipErrorInvalidValue outside
// shape_supported_c (csrc/strategy_a_two_pass.cu:96, strategy_b_lds_dequant.cu:65).
torch::Tensor dispatch_ab(const char* name, const torch::Tensor& A, const torch::Tensor& B,
                          const torch::Tensor& S, c10::optional<torch::Tensor> C_opt) {
  const int64_t M = A.size(0), K = A.size(1), N = B.size(1);
  torch::Tensor C = C_opt.has_value() ? *C_opt : torch::empty({M, N}, A.options().dtype(at::kFloat));
  auto stream = check_inputs(A, B, S, C, M, N, K, MXFP4_LAYOUT_KN);
  TORCH_CHECK(mxfp4_shape_supported('c', M, N, K) == 1, name, ": ",
              hipGetErrorString(hipErrorInvalidValue));
  launch(name, A, B, S, C, M, N, K, MXFP4_LAYOUT_KN, nullptr, stream);
  return C;
}

#define MXFP4_LETTER(fn, letter, pred, msg)                                                   \
  torch::Tensor fn(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& S,   \
                   c10::optional<torch::Tensor> C) {                                          \
    TORCH_CHECK(mxfp4_shape_supported(pred, A.size(0), B.size(1), A.size(1)) == 1, msg);      \
    return dispatch("launch_strategy_" letter, A, B, S, C);                                   \
  }

torch::Tensor gemm_a(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& S,
                     c10::optional<torch::Tensor> C) {
  return dispatch_ab("launch_strategy_a", A, B, S, C);
}
torch::Tensor gemm_b(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& S,
                     c10::optional<torch::Tensor> C) {
  return dispatch_ab("launch_strategy_b", A, B, S, C);
}
MXFP4_LETTER(gemm_c, "c", 'c', "Strategy C requires M%64==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_d, "d", 'd', "Strategy D requires M%128==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_e, "e", 'e', "Strategy E requires M%128==0, N%64==0, K%64==0")
MXFP4_LETTER(gemm_f, "f", 'f', "Strategy F requires M%256==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_h, "h", 'd', "Strategy H requires M%128==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_i, "i", 'd', "Strategy I requires M%128==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_k, "k", 'd', "Strategy K requires M%128==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_j, "j", 'd', "Strategy J requires M%128==0, N%128==0, K%64==0")
MXFP4_LETTER(gemm_m, "m", 'd', "Strategy M requires M%128==0, N%128==0, K%64==0")
#undef MXFP4_LETTER

// Every shape with K % 32 == 0 (the reference's gemm_auto falls back to B,
// which rejects M % 64 != 0: python/mxfp4_cdna3/kernels.py:63-74).
torch::Tensor gemm_auto(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& S,
                        c10::optional<torch::Tensor> C) {
  return dispatch("gemm_auto", A, B, S, C);
}

// Any weight layout ("kn": [K/2,N]/[K/32,N], "nk": [N,K/2]/[N,K/32], "g":
// the strategy-G prepack, "p": panels; g and p in any shape of the right
// size, N = numel / (K/2)), output dtype, and an optional explicit plan
// (kernel, variant, split_k), and a fused epilogue C = act(A W + bias) + residual.
torch::Tensor gemm(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& S,
                   c10::optional<torch::Tensor> C_opt, const std::string& layout,
                   c10::optional<at::ScalarType> out_dtype, c10::optional<std::vector<int64_t>> plan,
                   c10::optional<torch::Tensor> bias, c10::optional<std::string> activation,
                   c10::optional<torch::Tensor> residual) {
  const int lay = layout_code(layout);
  TORCH_CHECK(A.dim() == 2 && (prepacked(lay) || B.dim() == 2), "A shape");
  const int64_t M = A.size(0), K = A.size(1);
  TORCH_CHECK(K % 32 == 0, "K must be a multiple of 32");
  int64_t N;
  if (lay == MXFP4_LAYOUT_KN)
    N = B.size(1);
  else if (lay == MXFP4_LAYOUT_NK)
    N = B.size(0);
  else
    N = K == 0 ? 0 : B.numel() / (K / 2);
  at::ScalarType dt = out_dtype.has_value() ? *out_dtype : at::kFloat;
  torch::Tensor C = C_opt.has_value() ? *C_opt : torch::empty({M, N}, A.options().dtype(dt));
  auto stream = check_inputs(A, B, S, C, M, N, K, lay);
  mxfp4_plan p{MXFP4_KERNEL_AUTO, 0, 1, 0};
  if (plan.has_value()) p = plan_from(*plan);
  const mxfp4_epilogue ep = make_epilogue(C, M, N, bias, activation, residual);
  launch("mxfp4_gemm", A, B, S, C, M, N, K, lay, &p, stream, &ep);
  return C;
}

// G layout (python/mxfp4_cdna3/ref.py:85-101, csrc/mxfp4_ext.cpp:127-154).
torch::Tensor gemm_g(const torch::Tensor& A, const torch::Tensor& B_prep,
                     const torch::Tensor& Bs_prep, c10::optional<torch::Tensor> C_opt) {
  const int64_t M = A.size(0), K = A.size(1);
  TORCH_CHECK(A.is_cuda() && B_prep.is_cuda() && Bs_prep.is_cuda(), "all tensors on GPU");
  TORCH_CHECK(A.scalar_type() == at::kBFloat16, "A bf16");
  TORCH_CHECK(B_prep.scalar_type() == at::kByte, "B_prep uint8");
  TORCH_CHECK(Bs_prep.scalar_type() == at::kByte, "Bs_prep uint8");
  TORCH_CHECK(K % 2 == 0 && B_prep.numel() % (K / 2) == 0,
              "B_prep size not consistent with K/2 byte stride");
  const int64_t N = B_prep.numel() / (K / 2);
  TORCH_CHECK(Bs_prep.numel() == K * N / 32, "Bs_prep size != K*N/32");
  TORCH_CHECK(mxfp4_shape_supported('g', M, N, K) == 1,
              "Strategy G requires M%128==0, N%128==0, K%64==0");
  TORCH_CHECK(A.is_contiguous() && B_prep.is_contiguous() && Bs_prep.is_contiguous(),
              "tensors contiguous");
  torch::Tensor C = C_opt.has_value() ? *C_opt : torch::empty({M, N}, A.options().dtype(at::kFloat));
  TORCH_CHECK((C.scalar_type() == at::kFloat || C.scalar_type() == at::kBFloat16) && C.dim() == 2 &&
                  C.size(0) == M && C.size(1) == N && C.is_contiguous(),
              "C shape/contig");
  TORCH_CHECK(A.get_device() == B_prep.get_device() && A.get_device() == Bs_prep.get_device() &&
                  A.get_device() == C.get_device(),
              "all tensors must be on the same GPU");
  auto stream = c10::hip::getCurrentHIPStream(A.get_device()).stream();
  launch("launch_strategy_g", A, B_prep, Bs_prep, C, M, N, K, MXFP4_LAYOUT_G, nullptr, stream);
  return C;
}

// Shape a layout's code / scale tensors take when this API allocates them.
std::vector<int64_t> code_shape(int layout, int64_t K, int64_t N) {
  switch (layout) {
    case MXFP4_LAYOUT_KN: return {K / 2, N};
    case MXFP4_LAYOUT_NK: return {N, K / 2};
    case MXFP4_LAYOUT_G: return {N / 128, K / 8, 128, 4};
    default: return {N / 32, K / 64, 2, 32, 16};
  }
}
std::vector<int64_t> scale_shape(int layout, int64_t K, int64_t N) {
  switch (layout) {
    case MXFP4_LAYOUT_KN: return {K / 32, N};
    case MXFP4_LAYOUT_NK: return {N, K / 32};
    case MXFP4_LAYOUT_G: return {N / 128, K / 32, 128};
    default: return {N / 32, K / 64, 2, 32};
  }
}

// (K, N) of weights in `layout`: from the 2-D shapes of kn/nk, from K (given,
// or the leading dims of the shapes convert_layout returns) for g/p.
std::pair<int64_t, int64_t> weight_dims(const torch::Tensor& B, int layout, c10::optional<int64_t> K_opt) {
  if (layout == MXFP4_LAYOUT_KN || layout == MXFP4_LAYOUT_NK) {
    TORCH_CHECK(B.dim() == 2, "B must be 2-D for layout kn / nk");
    const bool kn = layout == MXFP4_LAYOUT_KN;
    return {(kn ? B.size(0) : B.size(1)) * 2, kn ? B.size(1) : B.size(0)};
  }
  int64_t K;
  if (K_opt.has_value()) {
    K = *K_opt;
  } else {
    TORCH_CHECK(B.dim() >= 2, "pass K for flat prepacked weights");
    K = B.size(1) * (layout == MXFP4_LAYOUT_G ? 8 : 64);
  }
  TORCH_CHECK(K > 0 && K % 32 == 0 && B.numel() % (K / 2) == 0, "B size not consistent with K");
  return {K, B.numel() / (K / 2)};
}

// Weights rewritten into another layout on the device (prepack / unprepack);
// returns (codes, scales) shaped for dst (code_shape / scale_shape).
py::tuple convert_layout(const torch::Tensor& B, const torch::Tensor& S, const std::string& src,
                         const std::string& dst, c10::optional<int64_t> K_opt) {
  const int ls = layout_code(src), ld = layout_code(dst);
  TORCH_CHECK(B.is_cuda() && S.is_cuda(), "all tensors must be on GPU");
  TORCH_CHECK(B.scalar_type() == at::kByte && S.scalar_type() == at::kByte, "B and S must be uint8");
  TORCH_CHECK(B.is_contiguous() && S.is_contiguous(), "B/S must be contiguous");
  TORCH_CHECK(B.get_device() == S.get_device(), "all tensors must be on the same GPU");
  const auto kn = weight_dims(B, ls, K_opt);
  const int64_t K = kn.first, N = kn.second;
  TORCH_CHECK(K % 32 == 0, "K must be a multiple of 32");
  TORCH_CHECK(S.numel() == K / 32 * N, "B_scales size");
  TORCH_CHECK((ld != MXFP4_LAYOUT_G && ls != MXFP4_LAYOUT_G) || N % 128 == 0, "layout g needs N % 128 == 0");
  TORCH_CHECK((ld != MXFP4_LAYOUT_P && ls != MXFP4_LAYOUT_P) || (N % 32 == 0 && K % 64 == 0),
              "layout p needs N % 32 == 0 and K % 64 == 0");
  torch::Tensor Bo = torch::empty(code_shape(ld, K, N), B.options());
  torch::Tensor So = torch::empty(scale_shape(ld, K, N), S.options());
  auto stream = c10::hip::getCurrentHIPStream(B.get_device()).stream();
  hipError_t err = mxfp4_convert_layout(static_cast<const uint8_t*>(B.data_ptr()),
                                        static_cast<const uint8_t*>(S.data_ptr()), ls,
                                        static_cast<uint8_t*>(Bo.data_ptr()),
                                        static_cast<uint8_t*>(So.data_ptr()), ld, K, N, stream);
  TORCH_CHECK(err == hipSuccess, "mxfp4_convert_layout: ", hipGetErrorString(err));
  return py::make_tuple(Bo, So);
}

// Device quantize_mxfp4 (python/mxfp4_cdna3/ref.py:14-47) of a 2-D fp32 / bf16
// weight: axis 0 -> X is [K, N]; axis -1 (or 1) -> X is [N, K].  Output
// layout default: "kn" for axis 0 and "nk" for axis -1, the shapes the
// reference returns; any layout may be asked for.
py::tuple quantize(const torch::Tensor& X, int64_t axis, c10::optional<std::string> layout) {
  TORCH_CHECK(X.is_cuda(), "X must be on GPU");
  TORCH_CHECK(X.dim() == 2, "X must be 2-D");
  TORCH_CHECK(X.scalar_type() == at::kFloat || X.scalar_type() == at::kBFloat16, "X must be float32 or bfloat16");
  TORCH_CHECK(X.is_contiguous(), "X must be contiguous");
  TORCH_CHECK(axis == 0 || axis == 1 || axis == -1, "axis must be 0 or -1");
  const bool kn_in = axis == 0;
  const int64_t K = kn_in ? X.size(0) : X.size(1), N = kn_in ? X.size(1) : X.size(0);
  TORCH_CHECK(K % 32 == 0, "axis ", axis, " length ", K, " not divisible by 32");
  const int ld = layout.has_value() ? layout_code(*layout) : (kn_in ? MXFP4_LAYOUT_KN : MXFP4_LAYOUT_NK);
  TORCH_CHECK(ld != MXFP4_LAYOUT_G || N % 128 == 0, "layout g needs N % 128 == 0");
  TORCH_CHECK(ld != MXFP4_LAYOUT_P || (N % 32 == 0 && K % 64 == 0), "layout p needs N % 32 == 0 and K % 64 == 0");
  auto opts = X.options().dtype(at::kByte);
  torch::Tensor B = torch::empty(code_shape(ld, K, N), opts);
  torch::Tensor S = torch::empty(scale_shape(ld, K, N), opts);
  auto stream = c10::hip::getCurrentHIPStream(X.get_device()).stream();
  hipError_t err = mxfp4_quantize(X.data_ptr(), X.scalar_type() == at::kBFloat16 ? MXFP4_IN_BF16 : MXFP4_IN_F32,
                                  kn_in ? MXFP4_LAYOUT_KN : MXFP4_LAYOUT_NK, K, N,
                                  static_cast<uint8_t*>(B.data_ptr()), static_cast<uint8_t*>(S.data_ptr()), ld,
                                  stream);
  TORCH_CHECK(err == hipSuccess, "mxfp4_quantize: ", hipGetErrorString(err));
  return py::make_tuple(B, S);
}

torch::Tensor dequant(const torch::Tensor& B, const torch::Tensor& S, const std::string& layout,
                      at::ScalarType out_dtype, c10::optional<int64_t> K_opt) {
  const int lay = layout_code(layout);
  TORCH_CHECK(B.is_cuda() && S.is_cuda(), "all tensors must be on GPU");
  TORCH_CHECK(B.scalar_type() == at::kByte && S.scalar_type() == at::kByte, "B and S must be uint8");
  TORCH_CHECK(out_dtype == at::kFloat || out_dtype == at::kBFloat16, "out_dtype must be float32 or bfloat16");
  TORCH_CHECK(B.is_contiguous() && S.is_contiguous(), "B/S must be contiguous");
  const auto kn_dims = weight_dims(B, lay, K_opt);
  const int64_t K = kn_dims.first, N = kn_dims.second;
  TORCH_CHECK(K % 32 == 0, "K must be a multiple of 32");
  if (lay == MXFP4_LAYOUT_KN || lay == MXFP4_LAYOUT_NK) {
    const bool kn = lay == MXFP4_LAYOUT_KN;
    TORCH_CHECK(S.dim() == 2 && (kn ? (S.size(0) == K / 32 && S.size(1) == N) : (S.size(0) == N && S.size(1) == K / 32)),
                "B_scales shape");
  } else {
    TORCH_CHECK(S.numel() == K / 32 * N, "B_scales size");
  }
  torch::Tensor out = torch::empty({K, N}, B.options().dtype(out_dtype));
  auto stream = c10::hip::getCurrentHIPStream(B.get_device()).stream();
  hipError_t err = mxfp4_dequant(static_cast<const uint8_t*>(B.data_ptr()),
                                 static_cast<const uint8_t*>(S.data_ptr()), out.data_ptr(),
                                 out_dtype == at::kBFloat16 ? MXFP4_OUT_BF16 : MXFP4_OUT_F32, K, N,
                                 lay, stream);
  TORCH_CHECK(err == hipSuccess, "mxfp4_dequant: ", hipGetErrorString(err));
  return out;
}

std::string describe_plan(const std::vector<int64_t>& plan) {
  const mxfp4_plan p = plan_from(plan);
  char buf[128];
  hipError_t err = mxfp4_plan_describe(&p, buf, sizeof(buf));
  TORCH_CHECK(err == hipSuccess, "mxfp4_plan_describe: ", hipGetErrorString(err));
  return std::string(buf);
}

py::tuple select_plan(int64_t M, int64_t N, int64_t K, const std::string& layout) {
  mxfp4_plan p{};
  hipError_t err = mxfp4_select_plan(M, N, K, layout_code(layout), &p);
  TORCH_CHECK(err == hipSuccess, "mxfp4_select_plan: ", hipGetErrorString(err));
  char buf[128];
  mxfp4_plan_describe(&p, buf, sizeof(buf));
  return py::make_tuple(p.kernel, p.variant, p.split_k, std::string(buf));
}

py::dict device_info(int64_t dev_id) {
  mxfp4_device_info_t info{};
  hipError_t err = mxfp4_device_info((int)dev_id, &info);
  TORCH_CHECK(err == hipSuccess, "hipGetDeviceProperties: ", hipGetErrorString(err));
  py::dict d;
  d["name"] = std::string(info.name);
  d["gcn_arch_name"] = std::string(info.gcn_arch_name);
  d["multi_processor_count"] = info.multi_processor_count;
  d["total_global_mem"] = info.total_global_mem;
  d["shared_mem_per_block"] = info.shared_mem_per_block;
  d["warp_size"] = info.warp_size;
  return d;
}

bool shape_supported(char s, int64_t M, int64_t N, int64_t K) {
  return mxfp4_shape_supported(s, M, N, K) == 1;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.doc() = "MXFP4 (E2M1 + E8M0) x BF16 GEMM for MI355X (gfx950)";
  auto abc = [&](const char* name, torch::Tensor (*fn)(const torch::Tensor&, const torch::Tensor&,
                                                       const torch::Tensor&, c10::optional<torch::Tensor>)) {
    m.def(name, fn, py::arg("A"), py::arg("B_packed"), py::arg("B_scales"), py::arg("C") = py::none());
  };
  abc("gemm_a", &gemm_a);
  abc("gemm_b", &gemm_b);
  abc("gemm_c", &gemm_c);
  abc("gemm_d", &gemm_d);
  abc("gemm_e", &gemm_e);
  abc("gemm_f", &gemm_f);
  abc("gemm_h", &gemm_h);
  abc("gemm_i", &gemm_i);
  abc("gemm_k", &gemm_k);
  abc("gemm_j", &gemm_j);
  abc("gemm_m", &gemm_m);
  abc("gemm_auto", &gemm_auto);
  m.def("gemm_g", &gemm_g, py::arg("A"), py::arg("B_prep"), py::arg("Bs_prep"), py::arg("C") = py::none());
  m.def("gemm", &gemm, py::arg("A"), py::arg("B"), py::arg("S"), py::arg("C") = py::none(),
        py::arg("layout") = "kn", py::arg("out_dtype") = py::none(), py::arg("plan") = py::none(),
        py::arg("bias") = py::none(), py::arg("activation") = py::none(), py::arg("residual") = py::none());
  m.def("dequant", &dequant, py::arg("B"), py::arg("S"), py::arg("layout") = "kn",
        py::arg("out_dtype") = at::kBFloat16, py::arg("K") = py::none());
  m.def("quantize", &quantize, py::arg("X"), py::arg("axis") = -1, py::arg("layout") = py::none());
  m.def("convert_layout", &convert_layout, py::arg("B"), py::arg("S"), py::arg("src"), py::arg("dst"),
        py::arg("K") = py::none());
  m.def("describe_plan", &describe_plan, py::arg("plan"));
  m.def("select_plan", &select_plan, py::arg("M"), py::arg("N"), py::arg("K"), py::arg("layout") = "kn");
  m.def("device_info", &device_info, py::arg("dev_id") = 0);
  m.def("shape_supported_c", [](int64_t M, int64_t N, int64_t K) { return shape_supported('c', M, N, K); },
        py::arg("M"), py::arg("N"), py::arg("K"));
  m.def("shape_supported_d", [](int64_t M, int64_t N, int64_t K) { return shape_supported('d', M, N, K); },
        py::arg("M"), py::arg("N"), py::arg("K"));
  m.def("shape_supported_e", [](int64_t M, int64_t N, int64_t K) { return shape_supported('e', M, N, K); },
        py::arg("M"), py::arg("N"), py::arg("K"));
  m.def("shape_supported_f", [](int64_t M, int64_t N, int64_t K) { return shape_supported('f', M, N, K); },
        py::arg("M"), py::arg("N"), py::arg("K"));
  m.def("shape_supported_g", [](int64_t M, int64_t N, int64_t K) { return shape_supported('g', M, N, K); },
        py::arg("M"), py::arg("N"), py::arg("K"));
  m.def("version", []() { return std::string(mxfp4_version()); });
}
