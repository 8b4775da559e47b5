// The torch extension module: attn (attention forward) and conv3d (implicit-GEMM
// conv3d), the ops of the reference's two extensions (attn.cpp:21 and
// hip_conv/conv3d.cpp:53) in one module.
#include "bindings.h"

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("attn", &attn, "fp16/bf16 attention forward on gfx950 (q, k, v, scale, out=None)",
          pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"), pybind11::arg("scale"),
          pybind11::arg("out") = pybind11::none());
    m.def("conv3d", &conv3d,
          "fp16 NDHWC implicit-GEMM conv3d on gfx950 "
          "(x, w, bias, res, out, dims, xs, os, rs)");
}
