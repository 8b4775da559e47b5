// Implicit-GEMM conv3d for AMD MI355X (gfx950 / CDNA4): fp16 NDHWC tensors,
// fp32 accumulation on matrix cores, fused fp16 bias + residual epilogue.
//
// Counterpart of the reference's VALU kernel (hip_conv/conv3d_kernel.hip:49-216,
// v_dot2_f32_f16 over a 128x64 tile), redesigned for CDNA4:
//
//  * GEMM view, transposed: O^T[k][m] = sum_i W[k][i] * X[m][i] with
//    m = ((n*Z + z)*P + p)*Q + q an output voxel, k an output channel and
//    i = ((t*R + r)*S + s)*C + c the reduction index, so that a packed
//    channels_last_3d weight row w[k] is contiguous in i and, with C % 8 == 0,
//    every aligned 8-element group of i lies in one (t, r, s) tap. With W as
//    the A operand of v_mfma_f32_32x32x16_f16, a lane's accumulator holds
//    four runs of four consecutive output channels of one voxel: the
//    channels-innermost output, bias and residual move as 8-byte vectors.
//  * Tiles of 128 channels x 128 voxels x 64 reduction elements, 4 waves of
//    64x64 (2x2 MFMA blocks). Both operand tiles go from HBM into LDS with
//    buffer loads to LDS (no VGPR staging); the input gather uses a per-lane
//    offset (voxel base + tap offset from a per-workgroup table), and lanes
//    past M, K or the reduction length get an out-of-range offset, so the
//    load returns zeros. LDS rows are 128 bytes with 16-byte units
//    XOR-swizzled; two stages, loads of k-tile t+1 in flight during t.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gfx906_amd_conv3d.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))

struct ConvArgs {
    const f16* x;
    const f16* w;
    const f16* bias;
    const f16* res;
    f16* out;
    int C, K, T, R, S, sd, sh, sw, Z, P, Q, M, KG;
    long long xsn, xsd, xsh, xsw, osn, osz, osp, osq, rsn, rsz, rsp, rsq;
    unsigned x_bytes, w_bytes;
};

constexpr int kBCh = 128;              // output channels per workgroup (GEMM rows)
constexpr int kBVx = 128;              // output voxels per workgroup (GEMM columns)
constexpr int kBR = 64;                // reduction elements per k-tile
constexpr int kNT = 256;               // 4 waves
constexpr int kRowB = kBR * 2;         // bytes per LDS row: 8 units of 16 bytes
constexpr int kTile = 128 * kRowB;     // 16 KB: one W or X tile
constexpr int kStage = 2 * kTile;      // W tile, then X tile
constexpr int kMaxTaps = 1024;
constexpr unsigned kOOB = 0xFFFFFFF0u;  // buffer offset past any range: loads zeros

// Unit u of LDS row r sits in slot u ^ swz(r). Two 128-byte rows span the 64
// banks, so 16 consecutive rows read at one unit cover 16 different bank
// groups.
__device__ __forceinline__ int swz(int r) { return (r >> 1) & 7; }

#if defined(__HIP_DEVICE_COMPILE__)
__device__ __forceinline__ f16x8 lds_read16(const char* base, int byte_off) {
    return *(const LDS_AS f16x8*)((const LDS_AS char*)base + byte_off);
}

// Output voxel m -> (n, z, p, q).
struct Voxel {
    int n, z, p, q;
};
__device__ __forceinline__ Voxel voxel(int m, int Z, int P, int Q) {
    Voxel v;
    v.q = m % Q;
    m /= Q;
    v.p = m % P;
    m /= P;
    v.z = m % Z;
    v.n = m / Z;
    return v;
}
#endif

// grid: (ceil(M / 128), ceil(K / 128)); block: 256 threads.
__global__ void __launch_bounds__(kNT, 2) conv3d_mfma(const ConvArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
    __shared__ __attribute__((aligned(1024))) char lds[2 * kStage];
    __shared__ int tapoff[kMaxTaps];  // x element offset of tap (t, r, s)

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int m0 = blockIdx.x * kBVx, k0 = blockIdx.y * kBCh;
    const int RS = a.R * a.S, taps = a.T * RS;
    for (int tp = tid; tp < taps; tp += kNT) {
        const int t = tp / RS, r = (tp - t * RS) / a.S, s = tp - t * RS - r * a.S;
        tapoff[tp] = (int)(t * a.xsd + r * a.xsh + s * a.xsw);
    }

    // Load roles. LDS block b (1 KB, b = wave + 4j) holds rows 8b..8b+7 of a
    // tile; lane l writes row 8b + l/8, slot l%8, so it fetches unit
    // u = (l%8) ^ swz(row) = (l%8) ^ ((4(b&1) + l/16) & 7). b&1 = wave&1, so
    // u is the same in all four of the lane's blocks, and so is the tap of
    // its reduction group.
    const int rsub = lane >> 3;
    const int u = (lane & 7) ^ ((4 * (wave & 1) + (lane >> 4)) & 7);
    unsigned wo[4];  // bytes into w (unused, and possibly wrapped, for rows past K)
    int xo[4];
    bool wv[4], xv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 8 * (wave + 4 * j) + rsub;
        const int k = k0 + row;
        wv[j] = k < a.K;
        wo[j] = ((unsigned)k * (unsigned)a.KG + 8u * (unsigned)u) * 2u;
        const int m = m0 + row;
        xv[j] = m < a.M;
        const Voxel v = voxel(m, a.Z, a.P, a.Q);
        xo[j] = (int)(v.n * a.xsn + (long long)v.z * a.sd * a.xsd +
                      (long long)v.p * a.sh * a.xsh + (long long)v.q * a.sw * a.xsw);
    }
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (int)a.w_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.x, 0, (int)a.x_bytes, 0x00020000);
    __syncthreads();  // tap table ready

    // Loads of the k-tile starting at reduction index i0 into an LDS stage.
    auto issue = [&](int i0, char* dst) __attribute__((always_inline)) {
        const int gi = i0 + 8 * u;
        const bool kin = gi < a.KG;
        int toff = 0;
        if (kin) {
            const int tp = gi / a.C;
            toff = tapoff[tp] + (gi - tp * a.C);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int b = wave + 4 * j;
            const unsigned ow = (wv[j] && kin) ? wo[j] + 2u * (unsigned)i0 : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (LDS_AS void*)(dst + b * 1024), 16, (int)ow,
                                                     0, 0, 0);
            const unsigned ox = (xv[j] && kin) ? (unsigned)(2 * (xo[j] + toff)) : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (LDS_AS void*)(dst + kTile + b * 1024), 16,
                                                     (int)ox, 0, 0, 0);
        }
    };

    // MFMA operand addresses: lane l reads row (32-row block base + l%32),
    // unit 2*ks + l/32 (16 reduction elements per k-step).
    const int g = lane >> 5, r32 = lane & 31;
    const int wch = wave & 1, wvx = wave >> 1;  // channel half, voxel half
    int aaddr[2][4], baddr[2][4];
#pragma unroll
    for (int bl = 0; bl < 2; ++bl)
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const int ra = wch * 64 + bl * 32 + r32, rb = wvx * 64 + bl * 32 + r32;
            aaddr[bl][ks] = ra * kRowB + (((2 * ks + g) ^ swz(ra)) * 16);
            baddr[bl][ks] = rb * kRowB + (((2 * ks + g) ^ swz(rb)) * 16);
        }

    f32x16 acc[2][2];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb)
#pragma unroll
        for (int vb = 0; vb < 2; ++vb) acc[cb][vb] = f32x16{};

    // The stage pointers are restrict-qualified: the stage being filled and
    // the stage being read are disjoint, so reads need not wait for the loads.
    const int nkt = (a.KG + kBR - 1) / kBR;
    auto step = [&](int kt, char* __restrict__ nxt, const char* __restrict__ cur)
        __attribute__((always_inline)) {
        if (kt + 1 < nkt) issue((kt + 1) * kBR, nxt);
        const char* sw = cur;
        const char* sx = cur + kTile;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            f16x8 af[2], bf[2];
#pragma unroll
            for (int bl = 0; bl < 2; ++bl) {
                af[bl] = lds_read16(sw, aaddr[bl][ks]);
                bf[bl] = lds_read16(sx, baddr[bl][ks]);
            }
#pragma unroll
            for (int cb = 0; cb < 2; ++cb)
#pragma unroll
                for (int vb = 0; vb < 2; ++vb)
                    acc[cb][vb] =
                        __builtin_amdgcn_mfma_f32_32x32x16_f16(af[cb], bf[vb], acc[cb][vb], 0, 0, 0);
        }
    };
    issue(0, lds);
    for (int kt = 0; kt < nkt; ++kt) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's part of k-tile kt landed
        __syncthreads();                    // every wave's; k-tile kt-1's stage is free
        step(kt, lds + ((kt + 1) & 1) * kStage, lds + (kt & 1) * kStage);
    }

    // Epilogue: accumulator row 8(r/4) + 4g + r%4 (an output channel), column
    // l%32 (an output voxel); four runs of four channels per lane and voxel.
#pragma unroll
    for (int vb = 0; vb < 2; ++vb) {
        const int m = m0 + wvx * 64 + vb * 32 + r32;
        if (m >= a.M) continue;
        const Voxel v = voxel(m, a.Z, a.P, a.Q);
        const long long oo = v.n * a.osn + v.z * a.osz + v.p * a.osp + v.q * a.osq;
        const long long ro = v.n * a.rsn + v.z * a.rsz + v.p * a.rsp + v.q * a.rsq;
#pragma unroll
        for (int cb = 0; cb < 2; ++cb)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int ch = k0 + wch * 64 + cb * 32 + 8 * rr + 4 * g;
                if (ch >= a.K) continue;
                f32x4 val = {acc[cb][vb][4 * rr], acc[cb][vb][4 * rr + 1], acc[cb][vb][4 * rr + 2],
                             acc[cb][vb][4 * rr + 3]};
                if (a.bias) val += __builtin_convertvector(*(const f16x4*)(a.bias + ch), f32x4);
                if (a.res) val += __builtin_convertvector(*(const f16x4*)(a.res + ro + ch), f32x4);
                *(f16x4*)(a.out + oo + ch) = __builtin_convertvector(val, f16x4);
            }
    }
#endif
}

thread_local char g_err[256];

void set_err(const char* msg) {
    int i = 0;
    for (; msg[i] && i < 255; ++i) g_err[i] = msg[i];
    g_err[i] = 0;
}

int fail(const char* msg) {
    set_err(msg);
    return 1;
}

bool mult8(long v) { return v >= 0 && v % 8 == 0; }

}  // namespace

extern "C" const char* conv3d_last_error(void) { return g_err[0] ? g_err : nullptr; }

extern "C" int conv3d_fwd(const void* x, const void* w, const void* bias, const void* res,
                          void* out, int nB, int D, int H, int W, int C, int K, int T, int R, int S,
                          int sd, int sh, int sw, int Z, int P, int Q, long M, long xsn, long xsd,
                          long xsh, long xsw, long osn, long osz, long osp, long osq, long rsn,
                          long rsz, long rsp, long rsq, hipStream_t stream) {
    g_err[0] = 0;
    if (nB <= 0 || D <= 0 || H <= 0 || W <= 0 || C <= 0 || K <= 0 || T <= 0 || R <= 0 || S <= 0)
        return fail("conv3d: sizes must be positive");
    if (sd <= 0 || sh <= 0 || sw <= 0) return fail("conv3d: strides must be positive");
    if (C % 8 || K % 8) return fail("conv3d: C and K must be multiples of 8");
    if (D < T || H < R || W < S || Z != (D - T) / sd + 1 || P != (H - R) / sh + 1 ||
        Q != (W - S) / sw + 1)
        return fail("conv3d: output size does not match a VALID convolution");
    if (M != (long)nB * Z * P * Q || M >= (1L << 31) - 256)
        return fail("conv3d: M must be nB*Z*P*Q < 2^31 - 256");
    if ((long)T * R * S > kMaxTaps) return fail("conv3d: more than 1024 taps");
    if (!x || !w || !out) return fail("conv3d: null pointer");
    if (((uintptr_t)x | (uintptr_t)w | (uintptr_t)out | (uintptr_t)res) % 16 ||
        (uintptr_t)bias % 8)
        return fail("conv3d: x, w, out, res must be 16-byte and bias 8-byte aligned");
    const long strides[12] = {xsn, xsd, xsh, xsw, osn, osz, osp, osq, rsn, rsz, rsp, rsq};
    for (long s : strides)
        if (!mult8(s)) return fail("conv3d: strides must be non-negative multiples of 8");
    const long KG = (long)C * T * R * S;
    const long x_span = ((nB - 1) * xsn + (D - 1) * xsd + (H - 1) * xsh + (W - 1) * xsw + C) * 2;
    const long w_span = (long)K * KG * 2;
    if (x_span >= (1L << 31) || w_span >= (1L << 31))
        return fail("conv3d: x or w spans 2^31 bytes or more");
    ConvArgs a;
    a.x = (const f16*)x;
    a.w = (const f16*)w;
    a.bias = (const f16*)bias;
    a.res = (const f16*)res;
    a.out = (f16*)out;
    a.C = C;
    a.K = K;
    a.T = T;
    a.R = R;
    a.S = S;
    a.sd = sd;
    a.sh = sh;
    a.sw = sw;
    a.Z = Z;
    a.P = P;
    a.Q = Q;
    a.M = (int)M;
    a.KG = (int)KG;
    a.xsn = xsn;
    a.xsd = xsd;
    a.xsh = xsh;
    a.xsw = xsw;
    a.osn = osn;
    a.osz = osz;
    a.osp = osp;
    a.osq = osq;
    a.rsn = rsn;
    a.rsz = rsz;
    a.rsp = rsp;
    a.rsq = rsq;
    a.x_bytes = (unsigned)x_span;
    a.w_bytes = (unsigned)w_span;
    dim3 grid((unsigned)((M + kBVx - 1) / kBVx), (unsigned)((K + kBCh - 1) / kBCh));
    hipLaunchKernelGGL(conv3d_mfma, grid, dim3(kNT), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        return 2;
    }
    return 0;
}

extern "C" void launch_conv3d(const void* x, const void* w, const void* bias, const void* res,
                              void* out, int nB, int D, int H, int W, int C, int K, int T, int R,
                              int S, int sd, int sh, int sw, int Z, int P, int Q, long M, long xsn,
                              long xsd, long xsh, long xsw, long osn, long osz, long osp, long osq,
                              long rsn, long rsz, long rsp, long rsq, hipStream_t stream) {
    (void)conv3d_fwd(x, w, bias, res, out, nB, D, H, W, C, K, T, R, S, sd, sh, sw, Z, P, Q, M, xsn,
                     xsd, xsh, xsw, osn, osz, osp, osq, rsn, rsz, rsp, rsq, stream);
}
