// Flash-attention forward for AMD MI355X (gfx950 / CDNA4), fp16 in/out.
//
// Computes, per (batch, head) and query row i:
//     o_i = sum_j softmax_j(scale * <q_i, k_j>) * v_j
// on contiguous [B, H, S, D] tensors with Sq != Skv allowed, no mask, no dropout.
// This is the computation behind the reference's `launch` entry point
// (attn_kernel.hip:710-742, dispatch) and its per-D kernels
// (attn_pair_gfx906 attn_kernel.hip:313-512 for D=64/128, attn_d512_gfx906
// attn_kernel.hip:525-708 for D=512, attn_tiled_gfx906 attn_kernel.hip:146-308
// for D<64). The reference kernels run on VALU dot2 instructions; this file
// is a different design built around CDNA4 matrix cores:
//
//  * Scores are computed transposed, S^T = K * Q^T, with
//    v_mfma_f32_32x32x16_f16. In the 32x32 accumulator layout a lane holds one
//    column (one query row) and 16 of the 32 keys of a key block, so the
//    online-softmax state (running max m, running sum l) is a per-lane scalar
//    and the row reductions need a single exchange with lane^32.
//  * The same registers, rounded to fp16, are the B operand of
//    O^T = V^T * P^T. The key order inside each 16-key step of that MFMA
//    follows the accumulator layout; V^T is stored in LDS with the matching
//    key permutation (bits 2 and 3 of the key index swapped), so a lane's A
//    operand is one 16-byte LDS read.
//  * Softmax runs in fp32 with exp2 and scale*log2(e) folded into one FMA.
//    The running max is updated lazily: the O accumulator is rescaled only
//    when a tile's max exceeds the running max by more than 2^8, which keeps
//    every p = exp2(s*c - m) <= 256 (exact in fp16 range) and skips the
//    rescale multiply on almost every tile.
//  * The row sum l is accumulated from the fp16-rounded P (v_dot2_f32_f16
//    against 1.0), so numerator and denominator see the same rounded weights.
//  * Output rows are normalised by 1/l and rounded to fp16 (RNE), as the
//    reference does (attn_kernel.hip:497-511). Rows of a head with Skv == 0
//    are written as zeros (the reference leaves them unwritten).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>

#include "../../include/gfx906_amd_attn.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kLog2e = 1.4426950408889634f;
// Lazy-rescale threshold in log2 units: p never exceeds 2^kTau.
constexpr float kTau = 8.0f;

__device__ __forceinline__ f16x8 ld16(const f16* p) {
    return *reinterpret_cast<const f16x8*>(p);
}
__device__ __forceinline__ void st16(f16* p, f16x8 v) {
    *reinterpret_cast<f16x8*>(p) = v;
}

__device__ __forceinline__ float xor32_max(float x) {
    return fmaxf(x, __shfl_xor(x, 32));
}
__device__ __forceinline__ float xor32_sum(float x) {
    return x + __shfl_xor(x, 32);
}

// Position of key kk (0..15) inside a 16-key step of the V^T tile: bits 2 and
// 3 swapped, so the 8 keys one lane feeds into the PV MFMA are contiguous.
__device__ __forceinline__ constexpr int vt_pos(int kk) {
    return (kk & ~12) | ((kk & 4) << 1) | ((kk & 8) >> 1);
}

// Kernel configuration per head-dim class.
//   DP  : head dim the tiles are built for (64, 128 or 512)
//   NW  : waves per workgroup; each wave owns 32 query rows
//   BN  : keys per K/V tile
template <int DP_, int NW_, int BN_>
struct Cfg {
    static constexpr int DP = DP_;
    static constexpr int NW = NW_;
    static constexpr int BN = BN_;
    static constexpr int BM = NW * 32;           // query rows per workgroup
    static constexpr int NT = NW * 64;           // threads per workgroup
    static constexpr int KS = DP + 8;            // sK row stride (halfs)
    static constexpr int VS = BN + 8;            // sVt row stride (halfs)
    static constexpr int K_CHUNKS = BN * DP / 8; // 16-byte chunks per K tile
    static constexpr int V_TASKS = (DP / 8) * (BN / 4); // 4 keys x 8 dims each
    static constexpr int K_PER_T = (K_CHUNKS + NT - 1) / NT;
    static constexpr int V_PER_T = (V_TASKS + NT - 1) / NT;
    static constexpr int LDS_BYTES = (BN * KS + DP * VS) * 2;
};

// One K/V tile staged in registers between its global load and its LDS store.
template <class C>
struct Stage {
    f16x8 k[C::K_PER_T];
    f16x8 v[C::V_PER_T][4];
};

// Global -> registers for key tile starting at n0. Keys >= Skv and dims >= D
// are loaded as zeros (zero K columns meet zero Q columns; zero V rows meet
// p = 0), so nothing outside the tensors is read.
template <class C, bool PAD>
__device__ __forceinline__ void load_tile(Stage<C>& st, const f16* __restrict__ Kh,
                                          const f16* __restrict__ Vh, int n0, int Skv,
                                          int D, int tid) {
    constexpr int CPR = C::DP / 8;  // chunks per row
#pragma unroll
    for (int i = 0; i < C::K_PER_T; ++i) {
        const int c = tid + i * C::NT;
        const int key = c / CPR, dc = c % CPR;
        f16x8 val = {};
        if ((C::K_CHUNKS % C::NT == 0 || c < C::K_CHUNKS) && n0 + key < Skv &&
            (!PAD || dc * 8 < D))
            val = ld16(Kh + (long)(n0 + key) * D + dc * 8);
        st.k[i] = val;
    }
#pragma unroll
    for (int i = 0; i < C::V_PER_T; ++i) {
        const int t = tid + i * C::NT;
        const int dc = t % CPR, kq = t / CPR;  // 8-dim block, 4-key quad
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = kq * 4 + r;
            f16x8 val = {};
            if ((C::V_TASKS % C::NT == 0 || t < C::V_TASKS) && n0 + key < Skv &&
                (!PAD || dc * 8 < D))
                val = ld16(Vh + (long)(n0 + key) * D + dc * 8);
            st.v[i][r] = val;
        }
    }
}

// Registers -> LDS. K keeps its [key][dim] layout; V is transposed to
// [dim][key] with the vt_pos key permutation inside each 16-key step.
template <class C>
__device__ __forceinline__ void store_tile(const Stage<C>& st, f16* sK, f16* sVt, int tid) {
    constexpr int CPR = C::DP / 8;
#pragma unroll
    for (int i = 0; i < C::K_PER_T; ++i) {
        const int c = tid + i * C::NT;
        if (C::K_CHUNKS % C::NT == 0 || c < C::K_CHUNKS) {
            const int key = c / CPR, dc = c % CPR;
            st16(sK + key * C::KS + dc * 8, st.k[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < C::V_PER_T; ++i) {
        const int t = tid + i * C::NT;
        if (C::V_TASKS % C::NT == 0 || t < C::V_TASKS) {
            const int dc = t % CPR, kq = t / CPR;
            const int key0 = kq * 4;  // 4-aligned, so vt_pos keeps the quad contiguous
            const int pos = (key0 & ~15) + vt_pos(key0 & 15);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f16x4 col = {st.v[i][0][e], st.v[i][1][e], st.v[i][2][e], st.v[i][3][e]};
                *reinterpret_cast<f16x4*>(sVt + (dc * 8 + e) * C::VS + pos) = col;
            }
        }
    }
}

// grid: ceil(Sq / BM) * B*H workgroups, query tiles of one head adjacent;
// block: NW*64 threads.
template <class C, bool PAD>
__global__ void __launch_bounds__(C::NT)
attn_fwd_mfma(const f16* __restrict__ Q, const f16* __restrict__ K,
              const f16* __restrict__ V, f16* __restrict__ O,
              int Sq, int Skv, int D, float c, float qsign) {
    constexpr int DP = C::DP, BN = C::BN;
    constexpr int NQF = DP / 16;  // Q fragments (16 dims each)
    constexpr int NOB = DP / 32;  // 32-dim output blocks
    constexpr int NKB = BN / 32;  // 32-key score blocks per tile
    __shared__ __attribute__((aligned(16))) f16 sK[BN * C::KS];
    __shared__ __attribute__((aligned(16))) f16 sVt[DP * C::VS];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int g = lane >> 5, r32 = lane & 31;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    const long bh = blockIdx.x / nqt;
    const int qt = blockIdx.x % nqt;
    const f16* Qh = Q + bh * (long)Sq * D;
    const f16* Kh = K + bh * (long)Skv * D;
    const f16* Vh = V + bh * (long)Skv * D;
    f16* Oh = O + bh * (long)Sq * D;
    const int qrow = qt * C::BM + wave * 32 + r32;
    const bool live = qrow < Sq;

    // Q^T fragments: B operand (column = this lane's query, k = dims).
    f16x8 qf[NQF];
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
        const int d0 = 16 * s + 8 * g;
        f16x8 val = {};
        if (live && (!PAD || d0 < D)) val = ld16(Qh + (long)qrow * D + d0);
        if (qsign < 0.f) val = -val;  // exact: negative scale -> negated q, |scale|
        qf[s] = val;
    }

    f32x16 oacc[NOB];
#pragma unroll
    for (int b = 0; b < NOB; ++b) oacc[b] = f32x16{};
    float m_run = -INFINITY;  // running max, in units of s*c (log2 domain)
    float l_run = 0.f;        // partial row sum over this lane's keys

    const int ntiles = (Skv + BN - 1) / BN;
    Stage<C> st;
    if (ntiles > 0) load_tile<C, PAD>(st, Kh, Vh, 0, Skv, D, tid);

    for (int t = 0; t < ntiles; ++t) {
        const int n0 = t * BN;
        __syncthreads();
        store_tile<C>(st, sK, sVt, tid);
        __syncthreads();
        if (t + 1 < ntiles) load_tile<C, PAD>(st, Kh, Vh, n0 + BN, Skv, D, tid);

        // S^T = K Q^T over this tile.
        f32x16 sacc[NKB];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            sacc[kb] = f32x16{};
            const f16* kp = sK + (kb * 32 + r32) * C::KS + 8 * g;
#pragma unroll
            for (int s = 0; s < NQF; ++s)
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld16(kp + 16 * s), qf[s],
                                                                  sacc[kb], 0, 0, 0);
        }

        // Tail tile: keys >= Skv take no part in the max and get p = 0.
        const bool tail = n0 + BN > Skv;
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = n0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                if (!tail || key < Skv) mx = fmaxf(mx, sacc[kb][r]);
            }
        mx = xor32_max(mx) * c;

        // Lazy rescale, decided per wave so the branch is uniform.
        if (__any(mx > m_run + kTau)) {
            const float m_new = fmaxf(m_run, mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
            for (int b = 0; b < NOB; ++b) oacc[b] *= alpha;
            l_run *= alpha;
            m_run = m_new;
        }

        // P = exp2(S*c - m), rounded to fp16; l += sum of the rounded values.
#pragma unroll
        for (int ks = 0; ks < BN / 16; ++ks) {
            const int kb = ks >> 1, r0 = 8 * (ks & 1);
            f16x8 pb;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int r = r0 + e;
                float p = __builtin_amdgcn_exp2f(fmaf(sacc[kb][r], c, -m_run));
                if (tail) {
                    const int key = n0 + kb * 32 + 8 * (r >> 2) + 4 * g + (r & 3);
                    if (key >= Skv) p = 0.f;
                }
                pb[e] = (f16)p;
            }
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                f16x2 pp = {pb[e], pb[e + 1]};
                l_run = __builtin_amdgcn_fdot2(pp, f16x2{(f16)1.0f, (f16)1.0f}, l_run, false);
            }
            // O^T += V^T P^T for this 16-key step.
            const f16* vp = sVt + r32 * C::VS + 16 * ks + 8 * g;
#pragma unroll
            for (int b = 0; b < NOB; ++b)
                oacc[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ld16(vp + b * 32 * C::VS), pb,
                                                                 oacc[b], 0, 0, 0);
        }
    }

    const float l = xor32_sum(l_run);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (live) {
        f16* op = Oh + (long)qrow * D;
#pragma unroll
        for (int b = 0; b < NOB; ++b)
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
                const int d0 = 32 * b + 8 * rr + 4 * g;
                if (!PAD || d0 < D) {
                    f16x4 h = {(f16)(oacc[b][4 * rr + 0] * inv), (f16)(oacc[b][4 * rr + 1] * inv),
                               (f16)(oacc[b][4 * rr + 2] * inv), (f16)(oacc[b][4 * rr + 3] * inv)};
                    *reinterpret_cast<f16x4*>(op + d0) = h;
                }
            }
    }
}

using Cfg64 = Cfg<64, 4, 64>;
using Cfg128 = Cfg<128, 4, 64>;
using Cfg512 = Cfg<512, 4, 32>;

thread_local char g_err[256];

void set_err(const char* msg) {
    int i = 0;
    for (; msg[i] && i < 255; ++i) g_err[i] = msg[i];
    g_err[i] = 0;
}

template <class C, bool PAD>
hipError_t launch_cfg(const void* q, const void* k, const void* v, void* o, int B, int H,
                      int Sq, int Skv, int D, float scale, hipStream_t s) {
    dim3 grid((unsigned)((Sq + C::BM - 1) / C::BM) * (unsigned)(B * H));
    const float c = fabsf(scale) * kLog2e;
    const float qsign = scale < 0.f ? -1.f : 1.f;
    hipLaunchKernelGGL((attn_fwd_mfma<C, PAD>), grid, dim3(C::NT), 0, s,
                       (const f16*)q, (const f16*)k, (const f16*)v, (f16*)o, Sq, Skv, D, c,
                       qsign);
    return hipGetLastError();
}

}  // namespace

extern "C" const char* attn_last_error(void) { return g_err[0] ? g_err : nullptr; }

extern "C" int attn_fwd(const void* q, const void* k, const void* v, void* o, int B, int H,
                        int Sq, int Skv, int D, float scale, hipStream_t s) {
    g_err[0] = 0;
    if (B < 0 || H < 0 || Sq < 0 || Skv < 0) {
        set_err("attn: negative size");
        return 1;
    }
    if (!((D <= 64 && D > 0 && D % 8 == 0) || D == 128 || D == 512)) {
        set_err("attn: head_dim must be <=64 and a multiple of 8, or 128, or 512");
        return 1;
    }
    if ((long)B * H * ((Sq + 31) / 32) > 0x7fffffffL) {
        set_err("attn: grid too large");
        return 1;
    }
    if (B == 0 || H == 0 || Sq == 0) return 0;
    if (!q || !o || (Skv > 0 && (!k || !v))) {
        set_err("attn: null pointer");
        return 1;
    }
    hipError_t e;
    if (D == 128)
        e = launch_cfg<Cfg128, false>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    else if (D == 64)
        e = launch_cfg<Cfg64, false>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    else if (D == 512)
        e = launch_cfg<Cfg512, false>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    else
        e = launch_cfg<Cfg64, true>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        return 2;
    }
    return 0;
}

extern "C" void launch(const void* q, const void* k, const void* v, void* o, int B, int H,
                       int Sq, int Skv, int D, float scale, hipStream_t s) {
    (void)attn_fwd(q, k, v, o, B, H, Sq, Skv, D, scale, s);
}
