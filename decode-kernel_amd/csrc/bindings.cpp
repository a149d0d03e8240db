// PyTorch-ROCm extension `decode_kernel._cuda` over the C ABI in
// include/decode_kernel/dk_gemv.h.
//
// Same Python surface, argument names, defaults and validation messages as
// the reference binding (csrc/bindings.cpp:10-129). Differences:
//   * every C-ABI status is checked and raised as RuntimeError (the reference
//     printed launch errors and returned garbage, csrc/gemv_w4a16.cu:9-16);
//   * work is issued on the current HIP stream of the tensors' device under a
//     device guard (the reference assumed the current device);
//   * v4 needs no workspace (the reference zeroed a [B, M] fp32 buffer per
//     call, csrc/bindings.cpp:65-68); the reuse path's split-K tiles take
//     one from torch's caching allocator, with no clearing.
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/extension.h>

#include <algorithm>
#include <cstdint>
#include <vector>

#include "decode_kernel/dk_gemv.h"
#include "decode_kernel/dk_mlp.h"

namespace {

constexpr int64_t kGroupSize = DK_GROUP_SIZE;
constexpr int64_t kNibblesPerWord = DK_NIBBLES_PER_WORD;

hipStream_t current_stream(const torch::Tensor& t) {
  return c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

void check_status(int rc, const char* what) {
  TORCH_CHECK(rc == DK_OK, what, " failed (status ", rc, "): ", dk_last_error());
}

// Reference: csrc/bindings.cpp:10-33.
void check_gemv_inputs(const torch::Tensor& packed, const torch::Tensor& scales,
                       const torch::Tensor& x) {
  TORCH_CHECK(packed.is_cuda() && scales.is_cuda() && x.is_cuda(),
              "packed, scales, and x must be CUDA tensors");
  TORCH_CHECK(packed.device() == x.device() && scales.device() == x.device(),
              "packed, scales, and x must be on the same device");
  TORCH_CHECK(packed.scalar_type() == torch::kInt32, "packed must be int32 (uint32 bit pattern)");
  TORCH_CHECK(scales.scalar_type() == torch::kFloat16, "scales must be fp16");
  TORCH_CHECK(x.scalar_type() == torch::kFloat16, "x must be fp16");
  TORCH_CHECK(packed.dim() == 2 && scales.dim() == 2 && x.dim() == 2,
              "packed [M,K/8], scales [M,K/128], x [B,K]");
  TORCH_CHECK(packed.is_contiguous() && scales.is_contiguous() && x.is_contiguous(),
              "packed, scales, and x must be contiguous");
  const int64_t M = packed.size(0);
  const int64_t K = packed.size(1) * kNibblesPerWord;
  TORCH_CHECK(K % kGroupSize == 0, "K must be divisible by group size 128");
  TORCH_CHECK(scales.size(0) == M && scales.size(1) == K / kGroupSize,
              "scales shape must be [M, K/128]");
  TORCH_CHECK(x.size(1) == K, "x.shape[1] must equal K");
  TORCH_CHECK(M <= INT32_MAX && K <= INT32_MAX && x.size(0) <= INT32_MAX,
              "M, K and B must fit in int32");
}

}  // namespace

torch::Tensor gemv_common(torch::Tensor packed, torch::Tensor scales, torch::Tensor x, int version,
                          int split_k, bool reuse_weights, int warps_per_row);

// Reference: csrc/bindings.cpp:37-78.
torch::Tensor w4a16_gemv(torch::Tensor packed, torch::Tensor scales, torch::Tensor x, int version,
                         int split_k, bool reuse_weights, int warps_per_row) {
  return gemv_common(packed, scales, x, version, split_k, reuse_weights, warps_per_row);
}

torch::Tensor gemv_common(torch::Tensor packed, torch::Tensor scales, torch::Tensor x, int version,
                          int split_k, bool reuse_weights, int warps_per_row) {
  check_gemv_inputs(packed, scales, x);
  TORCH_CHECK(version >= 0 && version <= 5, "version must be 0..5");
  TORCH_CHECK(split_k >= 1 && split_k <= 32, "split_k must be in [1, 32]");
  TORCH_CHECK(warps_per_row >= 1 && warps_per_row <= 8, "warps_per_row must be in [1, 8]");
  if (warps_per_row > 1) {
    TORCH_CHECK(version == 1 && !reuse_weights,
                "warps_per_row > 1 is implemented for streaming v1 only");
  }

  const int M = static_cast<int>(packed.size(0));
  const int K = static_cast<int>(packed.size(1) * kNibblesPerWord);
  const int B = static_cast<int>(x.size(0));

  c10::DeviceGuard guard(x.device());
  auto y = torch::empty({B, M}, x.options());
  if (K == 0) return y.zero_();  // empty sums (the reference returned uninitialised y)

  dk_gemv_config cfg;
  cfg.version = version;
  cfg.split_k = split_k;
  cfg.reuse_weights = reuse_weights ? 1 : 0;
  cfg.warps_per_row = warps_per_row;

  // The reuse path's split-K tiles take a workspace from the caching
  // allocator: tickets that carry the call's generation, then fp32 partials,
  // so it needs no clearing (8-byte words keep it 8-byte aligned). No other
  // path, v4 included, takes one.
  const size_t ws_bytes = dk_gemv_workspace_bytes(M, K, B, &cfg);
  torch::Tensor workspace;
  void* ws_ptr = nullptr;
  if (ws_bytes > 0) {
    workspace = torch::empty({static_cast<int64_t>((ws_bytes + 7) / 8)},
                             x.options().dtype(torch::kInt64));
    ws_ptr = workspace.data_ptr();
  }

  const int rc = dk_w4a16_gemv(reinterpret_cast<const uint32_t*>(packed.data_ptr<int32_t>()),
                               reinterpret_cast<const uint16_t*>(scales.data_ptr<at::Half>()),
                               reinterpret_cast<const uint16_t*>(x.data_ptr<at::Half>()),
                               reinterpret_cast<uint16_t*>(y.data_ptr<at::Half>()), M, K, B, &cfg,
                               ws_ptr, ws_bytes, current_stream(x));
  check_status(rc, "w4a16_gemv");
  return y;
}

// Reference: csrc/bindings.cpp:80-86.
void d2d_copy(torch::Tensor src, torch::Tensor dst) {
  TORCH_CHECK(src.is_cuda() && dst.is_cuda(), "src and dst must be CUDA");
  TORCH_CHECK(src.nbytes() == dst.nbytes(), "src/dst size mismatch");
  TORCH_CHECK(src.nbytes() % 16 == 0, "copy size must be a multiple of 16");
  TORCH_CHECK(src.is_contiguous() && dst.is_contiguous(), "src and dst must be contiguous");
  c10::DeviceGuard guard(src.device());
  check_status(dk_d2d_copy(src.data_ptr(), dst.data_ptr(), src.nbytes(), current_stream(src)),
               "d2d_copy");
}

// Reference: csrc/bindings.cpp:88-98.
void stream_read(torch::Tensor src, torch::Tensor partials) {
  TORCH_CHECK(src.is_cuda() && partials.is_cuda(), "src and partials must be CUDA");
  TORCH_CHECK(src.nbytes() % 16 == 0, "buffer size must be a multiple of 16");
  TORCH_CHECK(src.is_contiguous(), "src must be contiguous");
  TORCH_CHECK(partials.scalar_type() == torch::kFloat32, "partials must be fp32");
  TORCH_CHECK(partials.is_contiguous(), "partials must be contiguous");
  const int64_t blocks = partials.numel();
  TORCH_CHECK(blocks >= 1 && blocks <= INT32_MAX, "partials must have one float per block");
  c10::DeviceGuard guard(src.device());
  check_status(dk_stream_read(src.data_ptr(), partials.data_ptr<float>(), src.nbytes(),
                              static_cast<int>(blocks), current_stream(src)),
               "stream_read");
}

// Reference: csrc/bindings.cpp:100-106.
void stream_write(torch::Tensor dst) {
  TORCH_CHECK(dst.is_cuda(), "dst must be CUDA");
  TORCH_CHECK(dst.nbytes() % 16 == 0, "buffer size must be a multiple of 16");
  TORCH_CHECK(dst.is_contiguous(), "dst must be contiguous");
  c10::DeviceGuard guard(dst.device());
  const int blocks = dk_stream_recommended_blocks();
  TORCH_CHECK(blocks > 0, "stream_recommended_blocks failed: ", dk_last_error());
  check_status(dk_stream_write(dst.data_ptr(), dst.nbytes(), blocks, current_stream(dst)),
               "stream_write");
}

// Device quantizer: fp32 W [M, K] on the GPU -> (packed int32 [M, K/8],
// scales fp16 [M, K/128]). Reference: python/decode_kernel/quantize.py:26-51.
std::vector<torch::Tensor> quantize_and_pack(torch::Tensor w) {
  TORCH_CHECK(w.is_cuda(), "w must be a CUDA tensor");
  TORCH_CHECK(w.scalar_type() == torch::kFloat32, "w must be fp32");
  TORCH_CHECK(w.dim() == 2, "weight must be [M, K]");
  TORCH_CHECK(w.size(1) % kGroupSize == 0, "K=", w.size(1), " is not divisible by group_size=128");
  TORCH_CHECK(w.size(0) <= INT32_MAX && w.size(1) <= INT32_MAX, "M and K must fit in int32");
  c10::DeviceGuard guard(w.device());
  auto wc = w.contiguous();
  const int M = static_cast<int>(wc.size(0));
  const int K = static_cast<int>(wc.size(1));
  auto packed = torch::empty({M, K / kNibblesPerWord}, wc.options().dtype(torch::kInt32));
  auto scales = torch::empty({M, K / kGroupSize}, wc.options().dtype(torch::kFloat16));
  check_status(dk_quantize_pack_f32(wc.data_ptr<float>(), M, K,
                                    reinterpret_cast<uint32_t*>(packed.data_ptr<int32_t>()),
                                    reinterpret_cast<uint16_t*>(scales.data_ptr<at::Half>()),
                                    current_stream(wc)),
               "quantize_and_pack");
  return {packed, scales};
}

int stream_recommended_blocks() {
  const int blocks = dk_stream_recommended_blocks();
  TORCH_CHECK(blocks > 0, "stream_recommended_blocks failed: ", dk_last_error());
  return blocks;
}

namespace {

const uint32_t* words(const torch::Tensor& t) {
  return reinterpret_cast<const uint32_t*>(t.data_ptr<int32_t>());
}
const uint16_t* halves(const torch::Tensor& t) {
  return reinterpret_cast<const uint16_t*>(t.data_ptr<at::Half>());
}

// Gate and up are [I, H] in the GEMV format; x is [B, H].
void check_gate_up(const torch::Tensor& gate, const torch::Tensor& gate_scales,
                   const torch::Tensor& up, const torch::Tensor& up_scales,
                   const torch::Tensor& x) {
  check_gemv_inputs(gate, gate_scales, x);
  check_gemv_inputs(up, up_scales, x);
  TORCH_CHECK(gate.sizes() == up.sizes() && gate_scales.sizes() == up_scales.sizes(),
              "gate and up must have the same shape [I, H/8] and scales [I, H/128]");
}

}  // namespace

// h = fp16(silu(gate x) * (up x)): the fused gate/up projection of an MLP
// decode step. No counterpart in the reference (it composes its gemv).
torch::Tensor gate_up_silu(torch::Tensor gate, torch::Tensor gate_scales, torch::Tensor up,
                           torch::Tensor up_scales, torch::Tensor x) {
  check_gate_up(gate, gate_scales, up, up_scales, x);
  const int I = static_cast<int>(gate.size(0));
  const int H = static_cast<int>(gate.size(1) * kNibblesPerWord);
  const int B = static_cast<int>(x.size(0));
  c10::DeviceGuard guard(x.device());
  auto h = torch::empty({B, I}, x.options());
  if (H == 0) return h.zero_();  // g = u = 0 and silu(0) * 0 = 0
  check_status(dk_gate_up_silu(words(gate), halves(gate_scales), words(up), halves(up_scales),
                               halves(x), reinterpret_cast<uint16_t*>(h.data_ptr<at::Half>()), I, H,
                               B, current_stream(x)),
               "gate_up_silu");
  return h;
}

// y = down fp16(silu(gate x) * (up x)): one MLP decode step, two launches.
torch::Tensor mlp_decode(torch::Tensor gate, torch::Tensor gate_scales, torch::Tensor up,
                         torch::Tensor up_scales, torch::Tensor down, torch::Tensor down_scales,
                         torch::Tensor x) {
  check_gate_up(gate, gate_scales, up, up_scales, x);
  const int I = static_cast<int>(gate.size(0));
  const int H = static_cast<int>(gate.size(1) * kNibblesPerWord);
  const int B = static_cast<int>(x.size(0));
  TORCH_CHECK(down.is_cuda() && down_scales.is_cuda() && down.device() == x.device() &&
                  down_scales.device() == x.device(),
              "down and its scales must be CUDA tensors on x's device");
  TORCH_CHECK(down.scalar_type() == torch::kInt32 && down_scales.scalar_type() == torch::kFloat16,
              "down must be int32 and its scales fp16");
  TORCH_CHECK(down.dim() == 2 && down_scales.dim() == 2 && down.is_contiguous() &&
                  down_scales.is_contiguous(),
              "down [H, I/8] and scales [H, I/128] must be contiguous 2-D tensors");
  TORCH_CHECK(I % kGroupSize == 0, "I must be divisible by group size 128");
  TORCH_CHECK(down.size(0) == H && down.size(1) * kNibblesPerWord == I,
              "down must be [H, I/8] for gate/up [I, H/8]");
  TORCH_CHECK(down_scales.size(0) == H && down_scales.size(1) == I / kGroupSize,
              "down scales must be [H, I/128]");
  c10::DeviceGuard guard(x.device());
  auto y = torch::empty({B, H}, x.options());
  if (I == 0) return y.zero_();
  const size_t ws_bytes = dk_mlp_workspace_bytes(I, H, B);
  auto ws = torch::empty({static_cast<int64_t>(ws_bytes / 2) + 8}, x.options());
  check_status(dk_mlp_decode(words(gate), halves(gate_scales), words(up), halves(up_scales),
                             words(down), halves(down_scales), halves(x),
                             reinterpret_cast<uint16_t*>(y.data_ptr<at::Half>()), I, H, B,
                             ws.data_ptr(), ws.nbytes(), current_stream(x)),
               "mlp_decode");
  return y;
}

namespace {

void check_words(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.scalar_type() == torch::kInt32, name, " must be int32 (uint32 bit pattern)");
  TORCH_CHECK(t.dim() == 2 && t.is_contiguous(), name, " must be a contiguous [M, K/8] tensor");
  TORCH_CHECK((t.size(1) * kNibblesPerWord) % kGroupSize == 0,
              "K must be divisible by group size 128");
  TORCH_CHECK(t.size(0) <= INT32_MAX && t.size(1) * kNibblesPerWord <= INT32_MAX,
              "M and K must fit in int32");
}

}  // namespace

// Offline repack into the kernel-native paired layout, and its inverse.
// No counterpart in the reference (its format is the API format here too).
torch::Tensor repack_paired(torch::Tensor packed) {
  check_words(packed, "packed");
  c10::DeviceGuard guard(packed.device());
  auto out = torch::empty_like(packed);
  check_status(dk_repack_paired(words(packed), reinterpret_cast<uint32_t*>(out.data_ptr<int32_t>()),
                                static_cast<int>(packed.size(0)),
                                static_cast<int>(packed.size(1) * kNibblesPerWord),
                                current_stream(packed)),
               "repack_paired");
  return out;
}

torch::Tensor unpack_paired(torch::Tensor paired) {
  check_words(paired, "paired");
  c10::DeviceGuard guard(paired.device());
  auto out = torch::empty_like(paired);
  check_status(dk_unpack_paired(words(paired), reinterpret_cast<uint32_t*>(out.data_ptr<int32_t>()),
                                static_cast<int>(paired.size(0)),
                                static_cast<int>(paired.size(1) * kNibblesPerWord),
                                current_stream(paired)),
               "unpack_paired");
  return out;
}

// The v5 GEMV on paired weights (stamp 25); checks as w4a16_gemv.
torch::Tensor w4a16_gemv_paired(torch::Tensor paired, torch::Tensor scales, torch::Tensor x) {
  check_gemv_inputs(paired, scales, x);
  const int M = static_cast<int>(paired.size(0));
  const int K = static_cast<int>(paired.size(1) * kNibblesPerWord);
  const int B = static_cast<int>(x.size(0));
  c10::DeviceGuard guard(x.device());
  auto y = torch::empty({B, M}, x.options());
  if (K == 0) return y.zero_();
  check_status(dk_w4a16_gemv_paired(words(paired), halves(scales), halves(x),
                                    reinterpret_cast<uint16_t*>(y.data_ptr<at::Half>()), M, K, B,
                                    current_stream(x)),
               "w4a16_gemv_paired");
  return y;
}

int last_kernel_stamp() { return dk_last_kernel_stamp(); }

void empty_kernel() {
  check_status(dk_empty_kernel(c10::hip::getCurrentHIPStream().stream()), "empty_kernel");
}

int64_t workspace_bytes(int64_t M, int64_t K, int64_t B, int version, int split_k,
                        bool reuse_weights, int warps_per_row) {
  dk_gemv_config cfg{version, split_k, reuse_weights ? 1 : 0, warps_per_row};
  return static_cast<int64_t>(
      dk_gemv_workspace_bytes(static_cast<int>(M), static_cast<int>(K), static_cast<int>(B), &cfg));
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("w4a16_gemv", &w4a16_gemv, "W4A16 GEMV", py::arg("packed"), py::arg("scales"),
        py::arg("x"), py::arg("version") = 5, py::arg("split_k") = 4,
        py::arg("reuse_weights") = false, py::arg("warps_per_row") = 1);
  m.def("quantize_and_pack", &quantize_and_pack,
        "fp32 W [M, K] -> (packed int32 [M, K/8], scales fp16 [M, K/128]) on the GPU",
        py::arg("w"));
  m.def("gate_up_silu", &gate_up_silu,
        "Fused MLP gate/up projection: fp16(silu(gate x) * (up x)) -> [B, I]", py::arg("gate"),
        py::arg("gate_scales"), py::arg("up"), py::arg("up_scales"), py::arg("x"));
  m.def("mlp_decode", &mlp_decode,
        "MLP decode step: down fp16(silu(gate x) * (up x)) -> [B, H]", py::arg("gate"),
        py::arg("gate_scales"), py::arg("up"), py::arg("up_scales"), py::arg("down"),
        py::arg("down_scales"), py::arg("x"));
  m.def("repack_paired", &repack_paired,
        "Repack int32 [M, K/8] weights into the kernel-native paired layout", py::arg("packed"));
  m.def("unpack_paired", &unpack_paired, "Inverse of repack_paired (bit for bit)",
        py::arg("paired"));
  m.def("w4a16_gemv_paired", &w4a16_gemv_paired, "v5 W4A16 GEMV on paired-layout weights",
        py::arg("paired"), py::arg("scales"), py::arg("x"));
  m.def("d2d_copy", &d2d_copy, "Aligned device-to-device copy", py::arg("src"), py::arg("dst"));
  m.def("stream_read", &stream_read, "Read-only STREAM sum-reduction (one float partial per block)",
        py::arg("src"), py::arg("partials"));
  m.def("stream_write", &stream_write, "Write-only STREAM fill", py::arg("dst"));
  m.def("stream_recommended_blocks", &stream_recommended_blocks,
        "Block count used by STREAM probes");
  m.def("last_kernel_stamp", &last_kernel_stamp,
        "Dispatch stamp of the GEMV last launched on this device (read and cleared)");
  m.def("empty_kernel", &empty_kernel, "Empty kernel on the current stream (launch floor)");
  m.def("workspace_bytes", &workspace_bytes, "Device workspace bytes a GEMV call needs",
        py::arg("M"), py::arg("K"), py::arg("B"), py::arg("version") = 5, py::arg("split_k") = 4,
        py::arg("reuse_weights") = false, py::arg("warps_per_row") = 1);
  m.attr("ABI_VERSION") = dk_abi_version();
}
