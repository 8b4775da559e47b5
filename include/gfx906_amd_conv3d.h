/* C ABI of the MI355X (gfx950) fp16 conv3d: VALID convolution over NDHWC
 * (channels-innermost) tensors as an implicit GEMM on matrix cores, with a
 * fused fp16 bias and residual epilogue (the comfy_kitchen fp16_conv3d
 * contract the reference serves, gfx906_kitchen.py:167-248).
 *
 *   out[n,k,z,p,q] = bias[k] + res[n,k,z,p,q]
 *                  + sum_{c,t,r,s} x[n,c,z*sd+t,p*sh+r,q*sw+s] * w[k,c,t,r,s]
 *
 * x is indexed with element strides (xsn, xsd, xsh, xsw) and a channel stride
 * of 1; out and res likewise with (os*) and (rs*); w is a packed
 * channels_last_3d [K, C, T, R, S] tensor (memory order K, T, R, S, C). bias
 * and res may be NULL; res may be out itself. Accumulation is fp32, the
 * output rounded to fp16 (RNE). Z = (D-T)/sd + 1, P = (H-R)/sh + 1,
 * Q = (W-S)/sw + 1, M = nB*Z*P*Q.
 * Requirements (checked): C and K multiples of 8; x, w, out and res 16-byte
 * aligned and bias 8-byte aligned; all strides non-negative multiples of 8;
 * T*R*S <= 1024; x and w each span less than 2^31 bytes; M < 2^31 - 256.
 */
#ifndef GFX906_AMD_CONV3D_H
#define GFX906_AMD_CONV3D_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Drop-in for the reference entry point of the same name and argument list
 * (hip_conv/conv3d_kernel.hip:218-233, declared for the binding at
 * hip_conv/conv3d.cpp:18-26). Returns nothing; on a rejected argument or a
 * launch failure no kernel runs and conv3d_last_error() has the reason. */
void launch_conv3d(const void* x, const void* w, const void* bias, const void* res, void* out,
                   int nB, int D, int H, int W, int C, int K,
                   int T, int R, int S, int sd, int sh, int sw,
                   int Z, int P, int Q, long M,
                   long xsn, long xsd, long xsh, long xsw,
                   long osn, long osz, long osp, long osq,
                   long rsn, long rsz, long rsp, long rsq,
                   hipStream_t stream);

/* Same as launch_conv3d(), returning 0 on success, 1 for a rejected argument
 * (nothing launched) and 2 for a HIP launch error. No counterpart in the
 * reference, whose launch_conv3d has no error path. */
int conv3d_fwd(const void* x, const void* w, const void* bias, const void* res, void* out,
               int nB, int D, int H, int W, int C, int K,
               int T, int R, int S, int sd, int sh, int sw,
               int Z, int P, int Q, long M,
               long xsn, long xsd, long xsh, long xsw,
               long osn, long osz, long osp, long osq,
               long rsn, long rsz, long rsp, long rsq,
               hipStream_t stream);

/* Message for the last failed launch_conv3d()/conv3d_fwd() on the calling
 * thread, or NULL if it succeeded. No counterpart in the reference. */
const char* conv3d_last_error(void);

#ifdef __cplusplus
}
#endif

#endif
