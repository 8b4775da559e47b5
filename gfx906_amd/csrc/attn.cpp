// PyTorch binding for the gfx950 attention forward: attn(q, k, v, scale).
//
// Same Python signature, accept/reject set and ownership as the reference
// binding (attn.cpp:6-21): fp16 CUDA q/k/v of shape [B, H, S, D] with equal B,
// H and D, k.shape == v.shape, D <= 64 and a multiple of 8, or 128, or 512.
// Non-contiguous inputs are copied to contiguous ones; the output is a new
// contiguous [B, H, Sq, D] fp16 tensor on q's device. The kernel runs on the
// current HIP stream and the call returns without synchronising.
//
// Checks the reference binding lacks, all raising RuntimeError: k and v must
// be fp16 on q's device, sizes must fit the kernel's 32-bit indexing, and a
// launch error is reported instead of being dropped.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>
#include <c10/core/DeviceGuard.h>

#include "gfx906_amd_attn.h"

torch::Tensor attn(torch::Tensor q, torch::Tensor k, torch::Tensor v, double scale) {
    TORCH_CHECK(q.is_cuda() && q.dtype() == torch::kHalf, "kernel: q must be a CUDA fp16 tensor");
    TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
                "kernel: q, k and v must be on the same device");
    TORCH_CHECK(k.dtype() == torch::kHalf && v.dtype() == torch::kHalf,
                "kernel: k and v must be fp16");
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "kernel: q/k/v must be 4-D [B,H,S,D]");
    const c10::DeviceGuard guard(q.device());
    TORCH_CHECK(k.sizes() == v.sizes() && q.size(0) == k.size(0) && q.size(1) == k.size(1) &&
                    q.size(3) == k.size(3),
                "kernel: q/k/v shape mismatch");
    const int64_t B = q.size(0), H = q.size(1), Sq = q.size(2), Skv = k.size(2), D = q.size(3);
    TORCH_CHECK((D <= 64 && D > 0 && D % 8 == 0) || D == 128 || D == 512,
                "kernel: head_dim<=64 multiple of 8, 128, or 512");
    TORCH_CHECK(B * H * std::max<int64_t>(Sq, Skv) * D < (int64_t(1) << 40) && Sq < (1 << 30) &&
                    Skv < (1 << 30) && B * H < (1 << 30),
                "kernel: tensor too large");
    auto qc = q.contiguous(), kc = k.contiguous(), vc = v.contiguous();
    auto o = torch::empty_like(qc, qc.options().memory_format(at::MemoryFormat::Contiguous));
    if (o.numel() == 0) return o;
    const int rc = attn_fwd(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), o.data_ptr(), (int)B,
                            (int)H, (int)Sq, (int)Skv, (int)D, (float)scale,
                            c10::hip::getCurrentHIPStream().stream());
    TORCH_CHECK(rc == 0, "kernel: ", attn_last_error() ? attn_last_error() : "launch failed");
    return o;
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("attn", &attn, "fp16 attention forward on gfx950 (q, k, v, scale)");
}
