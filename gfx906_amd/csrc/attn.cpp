// PyTorch binding for the gfx950 attention forward: attn(q, k, v, scale, out=None).
//
// Same Python signature, accept/reject set and ownership as the reference
// binding (attn.cpp:6-21) for its fp16 case: CUDA q/k/v of shape [B, H, S, D]
// with equal B, H and D, k.shape == v.shape, D <= 64 and a multiple of 8, or
// 128, or 512. The output is a new contiguous [B, H, Sq, D] tensor of q's
// dtype on q's device. The kernel runs on the current HIP stream and the call
// returns without synchronising.
//
// Beyond the reference binding:
//  * Problems whose workgroups leave CUs idle (one head of a VAE, short
//    sequences) split the key range over more workgroups and merge the
//    partial results (attn_fwd_split), with a workspace from torch's
//    allocator; results then agree with the unsplit kernel to fp32 rounding.
//  * bf16 q/k/v run natively (bf16 MFMA), with a bf16 output; the reference
//    accepts fp16 only and its hook casts bf16 around it
//    (deploy/gfx906_attention.py:71-75).
//  * Strided inputs are read in place when the head dim is contiguous and
//    the other strides are multiples of 8 elements (16-byte aligned data);
//    only other layouts are copied, where the reference always calls
//    .contiguous() (attn.cpp:15). The VAE's token-contiguous views
//    ([b, c, h*w] seen as [b, 1, h*w, c], deploy/gfx906_attention.py:102-104,
//    D = 512) are read in place, q and out with them, up to Skv = 6400; past
//    that they are copied, on purpose: the in-place kernel needs transposing
//    LDS reads for K and runs 16 query rows per wave, a cost that grows with
//    Skv^2 while the copies grow with Skv (measured on MI355X with split key
//    ranges, in place against copy and the 32-row kernel: 0.115 against 0.127
//    ms at h*w = 4608, 0.161 against 0.169 ms at 6400, 0.226 against 0.192 ms
//    at 7056, 0.775 against 0.605 ms at 16384).
//  * `out`, if given, is written instead of allocating: any [B, H, Sq, D]
//    view of q's dtype and device whose elements do not overlap, e.g. the
//    transpose of a [B, Sq, H, D] buffer or the VAE's [b, 1, h*w, c] view of
//    a [b, c, h, w] output (written in place with the token-contiguous
//    kernel, else through a contiguous temporary when its head dim is
//    strided). It must not overlap k or v (every workgroup of a head reads
//    them); it may be q itself (a workgroup reads its own query rows before
//    writing them).
//  * Checks raising RuntimeError: k and v must match q's dtype and device,
//    sizes must fit the kernel's indexing, and a launch error is reported
//    instead of being dropped.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>
#include <c10/core/DeviceGuard.h>

#include "bindings.h"
#include "gfx906_amd_attn.h"

namespace {

// Element strides {batch, head, seq, head dim} of a 4-D tensor (0 for size-1
// batch/head/seq dims, whose stride is never used).
std::array<long long, 4> strides4(const torch::Tensor& t) {
    std::array<long long, 4> s;
    for (int d = 0; d < 3; ++d) s[d] = t.size(d) == 1 ? 0 : t.stride(d);
    s[3] = t.stride(3);
    return s;
}

// Whether the kernel can read t in place: contiguous head dim, non-negative
// strides that are multiples of 8 elements, 16-byte aligned data, and (for
// k and v) a sequence stride the 32-bit tile offsets can hold.
bool readable_in_place(const torch::Tensor& t, bool kv) {
    if (t.stride(3) != 1) return false;
    if (reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) return false;
    const auto s = strides4(t);
    for (int d = 0; d < 3; ++d)
        if (s[d] < 0 || s[d] % 8) return false;
    return !kv || s[2] <= (1 << 24);
}

// Whether k (or v) is in the token-contiguous D = 512 layout the kernel
// reads in place: sequence stride 1, head-dim stride a multiple of 8 other
// than 1, batch/head strides multiples of 8, 16-byte aligned data, Skv % 8 ==
// 0 and a per-head span below 2^30 elements.
bool token_contiguous_kv(const torch::Tensor& t) {
    const int64_t D = t.size(3), S = t.size(2);
    const auto s = strides4(t);
    if (D != 512 || S % 8 || t.stride(2) != 1 || s[3] == 1 || s[3] % 8) return false;
    if (s[0] % 8 || s[1] % 8 || reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) return false;
    return (D - 1) * s[3] + S < (int64_t(1) << 30);
}

// Largest Skv for which reading token-contiguous k/v in place beats copying
// them (see the file comment).
constexpr int64_t kInPlaceMaxSkv = 6400;

torch::Tensor as_input(const torch::Tensor& t, bool kv) {
    return readable_in_place(t, kv) ? t : t.clone(at::MemoryFormat::Contiguous);
}

}  // namespace

torch::Tensor attn(torch::Tensor q, torch::Tensor k, torch::Tensor v, double scale,
                   c10::optional<torch::Tensor> out) {
    TORCH_CHECK(q.is_cuda() && (q.dtype() == torch::kHalf || q.dtype() == torch::kBFloat16),
                "kernel: q must be a CUDA fp16 or bf16 tensor");
    TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
                "kernel: q, k and v must be on the same device");
    TORCH_CHECK(k.dtype() == q.dtype() && v.dtype() == q.dtype(),
                "kernel: k and v must have q's dtype");
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
    torch::Tensor o;
    if (out.has_value()) {
        o = *out;
        TORCH_CHECK(o.device() == q.device() && o.dtype() == q.dtype(),
                    "kernel: out must have q's dtype and device");
        TORCH_CHECK(o.dim() == 4 && o.size(0) == B && o.size(1) == H && o.size(2) == Sq &&
                        o.size(3) == D,
                    "kernel: out must be [B, H, Sq, D]");
    } else {
        o = torch::empty({B, H, Sq, D}, q.options().memory_format(at::MemoryFormat::Contiguous));
    }
    if (o.numel() == 0) return o;
    // Token-contiguous k and v (D = 512, Skv <= kInPlaceMaxSkv): read in
    // place, q and out with any strides. Otherwise the head dim of every
    // tensor the kernel touches is contiguous: inputs are copied and out
    // staged as needed.
    const bool tl = Skv <= kInPlaceMaxSkv && token_contiguous_kv(k) && token_contiguous_kv(v);
    const auto qi = tl ? q : as_input(q, false);
    const auto ki = tl ? k : as_input(k, true), vi = tl ? v : as_input(v, true);
    const bool staged = !tl && o.stride(3) != 1;
    torch::Tensor oo =
        staged ? torch::empty({B, H, Sq, D}, q.options().memory_format(at::MemoryFormat::Contiguous))
               : o;
    const auto sq = strides4(qi), sk = strides4(ki), sv = strides4(vi), so = strides4(oo);
    const int dtype = q.dtype() == torch::kBFloat16 ? ATTN_DTYPE_BF16 : ATTN_DTYPE_F16;
    // Problems too small to fill the GPU split the key range; the partial
    // results go to a workspace from torch's caching allocator.
    const size_t ws_bytes = attn_split_workspace_bytes((int)B, (int)H, (int)Sq, (int)Skv, (int)D);
    torch::Tensor ws;
    if (ws_bytes) ws = torch::empty({(int64_t)ws_bytes}, q.options().dtype(torch::kUInt8));
    const int rc = attn_fwd_split(qi.data_ptr(), ki.data_ptr(), vi.data_ptr(), oo.data_ptr(), (int)B,
                                  (int)H, (int)Sq, (int)Skv, (int)D, (float)scale,
                                  c10::hip::getCurrentHIPStream().stream(), dtype, sq.data(),
                                  sk.data(), sv.data(), so.data(),
                                  ws_bytes ? ws.data_ptr() : nullptr, ws_bytes);
    TORCH_CHECK(rc == 0, "kernel: ", attn_last_error() ? attn_last_error() : "launch failed");
    if (staged) o.copy_(oo);
    return o;
}

