/* C ABI of the MI355X (gfx950) flash-attention forward.
 *
 * All pointers are device pointers to contiguous fp16 tensors:
 *   q, o : [B, H, Sq,  D]
 *   k, v : [B, H, Skv, D]
 * D must be <= 64 and a multiple of 8, or 128, or 512. Sq != Skv is allowed.
 * o[b,h,i,:] = sum_j softmax_j(scale * <q[b,h,i,:], k[b,h,j,:]>) v[b,h,j,:],
 * rounded to fp16; rows with Skv == 0 are written as zeros.
 * Calls are asynchronous on `stream` and keep no state between calls.
 */
#ifndef GFX906_AMD_ATTN_H
#define GFX906_AMD_ATTN_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Drop-in for the reference entry point of the same name and signature:
 * declared at attn.cpp:4-5, defined at attn_kernel.hip:710-742. Returns
 * nothing; on a rejected argument or launch failure no kernel runs and the
 * reason is available from attn_last_error(). */
void launch(const void* q, const void* k, const void* v, void* o,
            int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream);

/* Same computation as launch(), returning 0 on success, 1 for a rejected
 * argument (nothing launched) and 2 for a HIP launch error. It replaces the
 * launch-then-check sequence of the reference binding (attn.cpp:17-19), which
 * has no error path of its own. */
int attn_fwd(const void* q, const void* k, const void* v, void* o,
             int B, int H, int Sq, int Skv, int D, float scale, hipStream_t stream);

/* Message for the last failed launch()/attn_fwd() on the calling thread, or
 * NULL if the last call succeeded. No counterpart in the reference, whose
 * launch() (attn_kernel.hip:710-742) never reports errors. */
const char* attn_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
