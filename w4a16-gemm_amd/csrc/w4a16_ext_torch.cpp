// PyTorch-ROCm binding: module `w4a16_ext`, function `w4a16_gemv(W, A, sW, zW)`.
//
// Drop-in for the reference's baseline extension (src/baseline/extension.cpp:6-8) and the
// tensor-level half of w4a16_gemv_cuda (src/baseline/kernel.cu:36-72): the same checks in the
// same order with the same messages, the device guard on W's device, a new fp16 [N] output on
// the current stream.  The kernel launch goes through the C ABI of libw4a16_hip.so (w4a16_gemv
// in include/w4a16.h).
//
// Compiled by the host compiler (no hipify, no device code).
#include <torch/extension.h>

#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>

#include "w4a16.h"

torch::Tensor w4a16_gemv_t(torch::Tensor W, torch::Tensor A, torch::Tensor sW, torch::Tensor zW) {
    // kernel.cu:39-52
    TORCH_CHECK(W.is_cuda() && A.is_cuda() && sW.is_cuda() && zW.is_cuda(), "all tensors must be CUDA");
    TORCH_CHECK(W.is_contiguous() && A.is_contiguous() && sW.is_contiguous() && zW.is_contiguous(),
                "all tensors must be contiguous");
    TORCH_CHECK(W.dtype() == torch::kInt32, "W must be int32 (packed)");
    TORCH_CHECK(A.dtype() == torch::kHalf && sW.dtype() == torch::kHalf && zW.dtype() == torch::kHalf,
                "A, sW, zW must be float16");
    TORCH_CHECK(W.dim() == 2 && A.dim() >= 1, "W must be [N, K/8]");
    const int64_t N = W.size(0);
    const int64_t K = A.size(0);
    TORCH_CHECK(K % 8 == 0, "K must be a multiple of 8");
    TORCH_CHECK(W.size(1) == K / 8, "W must be [N, K/8]");
    TORCH_CHECK(sW.numel() == N && zW.numel() == N, "sW, zW must be [N]");
    TORCH_CHECK(A.numel() == K, "A must be [K]");
    TORCH_CHECK(A.device() == W.device() && sW.device() == W.device() && zW.device() == W.device(),
                "W, A, sW and zW must be on the same device");

    const c10::DeviceGuard guard(W.device());
    hipStream_t stream = c10::hip::getCurrentHIPStream(W.device().index()).stream();
    torch::Tensor C = torch::empty({N}, A.options());
    const int rc = w4a16_gemv(W.data_ptr<int32_t>(), reinterpret_cast<const uint16_t*>(A.data_ptr()),
                              reinterpret_cast<const uint16_t*>(sW.data_ptr()),
                              reinterpret_cast<const uint16_t*>(zW.data_ptr()),
                              reinterpret_cast<uint16_t*>(C.data_ptr()), N, K, stream);
    TORCH_CHECK(rc == W4A16_OK, "w4a16_gemv: ", w4a16_last_error());
    return C;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("w4a16_gemv", &w4a16_gemv_t, "W4A16 GEMV (MI355X, exact int8-MFMA accumulation)");
}
