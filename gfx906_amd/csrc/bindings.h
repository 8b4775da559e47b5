// Functions of the torch extension module (registered in module.cpp).
#pragma once

#include <torch/extension.h>

#include <vector>

torch::Tensor attn(torch::Tensor q, torch::Tensor k, torch::Tensor v, double scale,
                   c10::optional<torch::Tensor> out);

void conv3d(torch::Tensor x, torch::Tensor w, c10::optional<torch::Tensor> bias,
            c10::optional<torch::Tensor> res, torch::Tensor out, std::vector<int64_t> dims,
            std::vector<int64_t> xs, std::vector<int64_t> os, std::vector<int64_t> rs);
