// PyTorch binding for the gfx950 implicit-GEMM conv3d:
// conv3d(x, w, bias, res, out, dims, xs, os, rs).
//
// Same argument list and meaning as the reference binding
// (hip_conv/conv3d.cpp:30-49): dims = {nB, D, H, W, C, K, T, R, S, sd, sh, sw,
// Z, P, Q}; xs / os / rs = element strides (n, d|z, h|p, w|q) of x, out and
// res, whose channel stride is 1; w is a packed channels_last_3d tensor; the
// Python layer (gfx906_amd.kitchen) validates layouts as the reference's
// gfx906_kitchen.py does. The kernel runs on the current HIP stream without
// synchronising. Beyond the reference binding: fp16 and device checks, and
// the kernel's own argument checks surface as RuntimeError.
#include <c10/hip/HIPStream.h>
#include <c10/core/DeviceGuard.h>

#include "bindings.h"
#include "gfx906_amd_conv3d.h"

void conv3d(torch::Tensor x, torch::Tensor w, c10::optional<torch::Tensor> bias,
            c10::optional<torch::Tensor> res, torch::Tensor out, std::vector<int64_t> dims,
            std::vector<int64_t> xs, std::vector<int64_t> os, std::vector<int64_t> rs) {
    TORCH_CHECK(dims.size() == 15 && xs.size() == 4 && os.size() == 4 && rs.size() == 4,
                "conv3d: bad dims/strides");
    TORCH_CHECK(x.is_cuda() && x.dtype() == torch::kHalf && w.dtype() == torch::kHalf &&
                    out.dtype() == torch::kHalf,
                "conv3d: x, w and out must be CUDA fp16 tensors");
    TORCH_CHECK(w.device() == x.device() && out.device() == x.device(),
                "conv3d: x, w and out must be on the same device");
    TORCH_CHECK(w.is_contiguous(at::MemoryFormat::ChannelsLast3d),
                "conv3d: w must be a packed channels_last_3d tensor");
    for (const auto* t : {&bias, &res})
        if (t->has_value())
            TORCH_CHECK((*t)->device() == x.device() && (*t)->dtype() == torch::kHalf,
                        "conv3d: bias and res must be fp16 on x's device");
    if (bias.has_value())
        TORCH_CHECK(bias->is_contiguous() && bias->numel() == dims[5], "conv3d: bias must be [K]");
    const c10::DeviceGuard guard(x.device());
    const long M = (long)dims[0] * dims[12] * dims[13] * dims[14];
    const int rc = conv3d_fwd(
        x.data_ptr(), w.data_ptr(), bias.has_value() ? bias->data_ptr() : nullptr,
        res.has_value() ? res->data_ptr() : nullptr, out.data_ptr(), (int)dims[0], (int)dims[1],
        (int)dims[2], (int)dims[3], (int)dims[4], (int)dims[5], (int)dims[6], (int)dims[7],
        (int)dims[8], (int)dims[9], (int)dims[10], (int)dims[11], (int)dims[12], (int)dims[13],
        (int)dims[14], M, xs[0], xs[1], xs[2], xs[3], os[0], os[1], os[2], os[3], rs[0], rs[1],
        rs[2], rs[3], c10::hip::getCurrentHIPStream().stream());
    TORCH_CHECK(rc == 0, "kernel: ", conv3d_last_error() ? conv3d_last_error() : "launch failed");
}
