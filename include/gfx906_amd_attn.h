/* C ABI of the MI355X (gfx950) flash-attention forward.
 *
 * All pointers are device pointers. For launch() and attn_fwd() the tensors
 * are contiguous fp16:
 *   q, o : [B, H, Sq,  D]
 *   k, v : [B, H, Skv, D]
 * attn_fwd_ex() also takes bf16 and per-tensor strides.
 * D must be <= 64 and a multiple of 8, or 128, or 512. Sq != Skv is allowed.
 * o[b,h,i,:] = sum_j softmax_j(scale * <q[b,h,i,:], k[b,h,j,:]>) v[b,h,j,:],
 * rounded to the element type; rows with Skv == 0 are written as zeros.
 * Calls are asynchronous on `stream`. The only state kept between calls is
 * the static scratch of the calls that split key ranges without a caller
 * workspace (launch(), attn_fwd(), attn_fwd_split_static()): a device array
 * of attn_split_scratch_capacity() bytes that is part of the library's code
 * object, so it is held on every GPU where the library's kernels are loaded,
 * until the process ends. Those calls are ordered on the GPU across streams
 * (each waits for the previous one on its device) except under stream
 * capture, where a captured call neither waits nor is waited for: a graph
 * that contains one is ordered only by the stream it is launched on.
 */
#ifndef GFX906_AMD_ATTN_H
#define GFX906_AMD_ATTN_H

#include <stddef.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types for attn_fwd_ex(). */
#define ATTN_DTYPE_F16 0
#define ATTN_DTYPE_BF16 1

/* Drop-in for the reference entry point of the same name and signature:
 * declared at attn.cpp:4-5, defined at attn_kernel.hip:710-742. Returns
 * nothing; on a rejected argument or launch failure no kernel runs and the
 * reason is available from attn_last_error(). When B*H*Sq is too small to
 * fill the GPU (a one-head VAE attention) it splits the key range as
 * attn_fwd_split_static() does, in the static scratch. */
void launch(const void* q, const void* k, const void* v, void* o,
            int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream);

/* Same computation as launch(), returning 0 on success, 1 for a rejected
 * argument (nothing launched) and 2 for a HIP launch error. It replaces the
 * launch-then-check sequence of the reference binding (attn.cpp:17-19), which
 * has no error path of its own. */
int attn_fwd(const void* q, const void* k, const void* v, void* o,
             int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream);

/* attn_fwd() for fp16 or bf16 (dtype = ATTN_DTYPE_F16 / ATTN_DTYPE_BF16,
 * the same type for q, k, v and o) and strided tensors, never splitting the
 * key range (one workgroup per batch, head and query tile). Each *_strides
 * points to four element strides {batch, head, sequence, head dim} of that
 * tensor, or is NULL for the contiguous layout. Strides are non-negative;
 * input strides may be 0 (a tensor broadcast over batch or heads) but no two
 * elements of o may share an address. Two layouts are accepted:
 *  - head dim contiguous (stride 1) for q, k, v and o: q, k, v 16-byte
 *    aligned with other strides multiples of 8 elements, o 8-byte aligned
 *    with multiples of 4; k/v sequence strides at most 2^24;
 *  - D == 512 with token-contiguous k and v (sequence stride 1, head-dim
 *    stride not 1), as in a [b, c, h*w] activation viewed as
 *    [b, 1, h*w, c]: k, v 16-byte aligned, batch/head/head-dim strides
 *    multiples of 8, Skv % 8 == 0, (D-1)*stride_d + Skv < 2^30 per head;
 *    q and o then take any strides (2-byte aligned).
 * Return codes as attn_fwd(). No counterpart in the reference, whose hook
 * casts bf16 to fp16 and back (deploy/gfx906_attention.py:71-75, 99-100) and
 * whose binding copies strided inputs (attn.cpp:15), including the VAE's
 * transposed views (deploy/gfx906_attention.py:102-104). */
int attn_fwd_ex(const void* q, const void* k, const void* v, void* o,
                int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream,
                int dtype, const long long* q_strides, const long long* k_strides,
                const long long* v_strides, const long long* o_strides);

/* Bytes of device workspace attn_fwd_split() needs for this problem on the
 * current device: 0 when the problem's workgroups already fill the GPU (the
 * call then runs as attn_fwd_ex()), else room for the partial results of the
 * split key ranges. No counterpart in the reference. */
size_t attn_split_workspace_bytes(int B, int H, int Sq, int Skv, int D);

/* attn_fwd_ex() that, when B*H*Sq is too small to fill the GPU (a VAE
 * attention over one head, short problems), splits the key range over more
 * workgroups: each writes its unnormalised partial output and running
 * max/sum to `workspace` (device memory, 16-byte aligned, at least
 * attn_split_workspace_bytes() bytes; may be NULL when that is 0) and a
 * second kernel merges them into o. Same arguments and return codes as
 * attn_fwd_ex(), plus 1 for a missing or short workspace. Results agree with
 * attn_fwd_ex() to fp32 rounding of the merge (not bit for bit). Calls on one
 * workspace must not overlap. No counterpart in the reference. */
int attn_fwd_split(const void* q, const void* k, const void* v, void* o,
                   int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream,
                   int dtype, const long long* q_strides, const long long* k_strides,
                   const long long* v_strides, const long long* o_strides,
                   void* workspace, size_t workspace_bytes);

/* attn_fwd_split() that allocates nothing: the split partial results go to
 * the library's static scratch (attn_split_scratch_capacity() bytes, 96 MiB,
 * on every GPU where the library's kernels are loaded, held until the
 * process ends). For callers that cannot allocate device memory: code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.
 * The split count is the best one whose partial results fit the scratch:
 * the same as attn_fwd_split()'s whenever attn_split_workspace_bytes() <=
 * capacity (then the results are bit-identical), fewer splits or none
 * otherwise. Problems that do not split use no scratch. Calls that use the
 * scratch are ordered across streams on one device (see the top of this
 * file); under stream capture the first such call on a device must have
 * been made outside capture (it sets the scratch up), else status 1. Same
 * arguments and return codes as attn_fwd_split() otherwise. No counterpart
 * in the reference. */
int attn_fwd_split_static(const void* q, const void* k, const void* v, void* o,
                          int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream,
                          int dtype, const long long* q_strides, const long long* k_strides,
                          const long long* v_strides, const long long* o_strides);

/* Bytes of the static scratch attn_fwd_split_static() uses. No counterpart in
 * the reference. */
size_t attn_split_scratch_capacity(void);

/* Message for the last failed launch()/attn_fwd()/attn_fwd_ex()/
 * attn_fwd_split()/attn_fwd_split_static() on the calling thread, or NULL if
 * the last call succeeded. No counterpart in the reference, whose launch()
 * (attn_kernel.hip:710-742) never reports errors. */
const char* attn_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
