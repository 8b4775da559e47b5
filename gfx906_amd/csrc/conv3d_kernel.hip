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
//    the A operand of v_mfma_f32_16x16x32_f16, a lane's accumulator holds a
//    run of four consecutive output channels of one voxel: the
//    channels-innermost output, bias and residual move as 8-byte vectors.
//    (The card is power-limited under sustained matrix load; the 16x16x32
//    form costs less energy per FLOP than 32x32x16 and holds a higher clock:
//    +6 % on a VAE decoder layer.)
//  * Tiles of 64*CW channels x 64*NB voxels x KB reduction elements (CW = 2
//    or 4, NB = 2, 3 or 4, KB = 32 or 64; seven configurations, chosen per
//    problem for how the tile count fills the CUs and how long the
//    reduction is), 2*CW waves of 64 x 32*NB (4 x 2NB MFMA blocks): with
//    CW = 2 two workgroups per CU whose barriers are independent, with
//    CW = 4 one workgroup of 8 waves that loads fewer bytes per MFMA.
//    Both operand tiles go from HBM into LDS with buffer loads to LDS (no
//    VGPR staging); the input gather uses a per-lane offset (voxel base +
//    the offset of the lane's tap, advanced incrementally from k-tile to
//    k-tile), and lanes past M, K or the reduction length get an
//    out-of-range offset, so the load returns zeros. LDS rows are 2*KB bytes
//    (with KB = 64 each row is one whole 128-byte line of a weight row or of
//    a voxel's channels) with 16-byte units XOR-swizzled; a ring of two to
//    four stages keeps the loads of the next k-tiles in flight, k-tiles past
//    the end load zeros (so every wait count is static), and the barrier
//    waits for this wave's LDS reads only, not for loads in flight.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "gfx906_amd_conv3d.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
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

constexpr int kMaxTaps = 1024;
constexpr unsigned kOOB = 0xFFFFFFF0u;  // buffer offset past any range: loads zeros

// Per-configuration sizes: NB 32-voxel MFMA blocks per wave, CW waves along
// output channels x 2 along voxels (64*CW channels x 64*NB voxels per
// workgroup), NST stages in the LDS ring, KB reduction elements per k-tile
// (LDS rows of 2*KB bytes: 32 -> 64-byte rows, 64 -> 128-byte rows, so that
// each row of a tile is one whole 128-byte line of the weights or of a voxel).
template <int NB, int NST, int KB, int CW>
struct ConvCfg {
    static constexpr int NW = 2 * CW;               // waves
    static constexpr int NT = 64 * NW;              // threads
    static constexpr int BCH = 64 * CW;             // output channels per workgroup
    static constexpr int ROWB = 2 * KB;             // bytes per LDS row
    static constexpr int UNITS = ROWB / 16;         // 16-byte units per row
    static constexpr int RPB = 1024 / ROWB;         // rows per 1 KB load block
    static constexpr int BVX = 64 * NB;             // output voxels per workgroup
    static constexpr int WTILE = BCH * ROWB;        // bytes of one W tile
    static constexpr int XTILE = BVX * ROWB;        // bytes of one X tile
    static constexpr int WJ = WTILE / 1024 / NW;    // W load blocks per wave per k-tile
    static constexpr int XBLK = XTILE / 1024;       // X load blocks per k-tile
    // X load blocks per wave per k-tile. When the waves do not divide the X
    // blocks, the waves past the last block issue a load of zeros into a
    // 1 KB pad after the X tile instead, so that every wave issues the same
    // number of loads and every wait count stays static.
    static constexpr int XJ = (XBLK + NW - 1) / NW;
    static constexpr int PAD = XJ * NW > XBLK ? 1024 : 0;
    static constexpr int STAGE = WTILE + XTILE + PAD;  // W tile, X tile, pad
    static constexpr int LOADS = WJ + XJ;
    static constexpr int OCC = CW == 2 ? 2 : 1;     // workgroups per CU
    static_assert(KB == 32 || KB == 64, "k-tile");
    static_assert(CW == 2 || CW == 4, "channel waves");
    static_assert(WJ * NW * 1024 == WTILE && XBLK * 1024 == XTILE, "whole load blocks");
    static_assert(NST * STAGE * OCC <= 160 * 1024, "LDS");
    static_assert(NST >= 2 && NST <= 4, "ring depth");
    static_assert((NST - 2) * LOADS < 16, "vmcnt immediate");
};

// Unit u of LDS row r sits in slot u ^ swz(r). 64-byte rows: four rows span
// the 64 banks and rows r, r+4 differ in swz; 128-byte rows: two rows span
// the banks and rows r, r+2, ..., r+14 differ in swz. Either way 16
// consecutive rows read at one unit cover 16 different bank groups.
template <int KB>
__host__ __device__ constexpr int swz(int r) { return KB == 32 ? (r >> 2) & 3 : (r >> 1) & 7; }

#if defined(__HIP_DEVICE_COMPILE__)
// Workgroup barrier for reusing an LDS stage: this wave's LDS reads are
// complete (lgkmcnt(0)), then s_barrier. Unlike __syncthreads() there is no
// release fence: that fence also waits for every outstanding load to LDS
// (vmcnt(0)), including the k-tiles meant to stay in flight. Each wave waits
// for its own part of the k-tile to be read (vmcnt(n)) before this. The
// memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

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

// Tile (voxel tile * channel tiles + channel tile) of workgroup L of n.
// Workgroups go to the 8 XCDs round robin (L % 8), each XCD with its own L2;
// this map gives XCD x the x-th contiguous eighth of the tiles, in order, so
// that the channel tiles of one voxel tile, and neighbouring voxel tiles
// (whose input windows overlap), share one L2.
__device__ __forceinline__ int tile_of(int L, int n) {
    const int xcd = L & 7, pos = L >> 3, base = n >> 3, extra = n & 7;
    return (xcd < extra ? xcd * (base + 1) : extra * (base + 1) + (xcd - extra) * base) + pos;
}

// grid: ceil(M / (64*NB)) * ceil(K / (64*CW)) workgroups (1-D, see tile_of);
// block: 128*CW threads. SMALLC: C < KB, so that one k-tile can cross
// several taps.
// The second launch bound is HIP's minimum waves per SIMD (amdgpu_waves_per_eu):
// OCC workgroups of 2*CW waves over the CU's four SIMDs.
template <int NB, int NST, int KB, int CW, bool SMALLC>
__global__ void __launch_bounds__((ConvCfg<NB, NST, KB, CW>::NT),
                                  (ConvCfg<NB, NST, KB, CW>::OCC * ConvCfg<NB, NST, KB, CW>::NW / 4))
    conv3d_mfma(const ConvArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
    using Cf = ConvCfg<NB, NST, KB, CW>;
    constexpr int STAGE = Cf::STAGE, LOADS = Cf::LOADS, ROWB = Cf::ROWB, UNITS = Cf::UNITS;
    constexpr int RPB = Cf::RPB, WJ = Cf::WJ, XJ = Cf::XJ, NW = Cf::NW;
    // The ring's stages are separate arrays, so that the compiler can tell
    // their accesses apart: a read of one stage never waits for the loads
    // into another.
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[NST > 2 ? STAGE : 16];
    __shared__ __attribute__((aligned(1024))) char st3[NST > 3 ? STAGE : 16];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int m0, k0;
    {
        const int nct = (a.K + Cf::BCH - 1) / Cf::BCH;
        const int t = tile_of(blockIdx.x, gridDim.x), vt = t / nct;
        m0 = vt * Cf::BVX;
        k0 = (t - vt * nct) * Cf::BCH;
    }

    // Load roles. LDS block b (1 KB) holds rows RPB*b..RPB*b+RPB-1 of a tile;
    // lane l writes row RPB*b + l/UNITS, slot l%UNITS, so it fetches unit
    // u = (l%UNITS) ^ swz(row). For the lane's blocks (W blocks wave + NW*j,
    // j < WJ; X blocks wave + NW*j, j < XJ) swz(row) does not depend on j, so
    // u and the tap of the lane's reduction group are the same in all of them.
    const int rsub = lane / UNITS;
    const int u = (lane % UNITS) ^ swz<KB>(RPB * wave + rsub);
    unsigned wo[WJ];  // bytes into w (unused, and possibly wrapped, for rows past K)
    bool wv[WJ];
#pragma unroll
    for (int j = 0; j < WJ; ++j) {
        const int k = k0 + RPB * (wave + NW * j) + rsub;
        wv[j] = k < a.K;
        wo[j] = ((unsigned)k * (unsigned)a.KG + 8u * (unsigned)u) * 2u;
    }
    int xo[XJ];
    bool xv[XJ];
#pragma unroll
    for (int j = 0; j < XJ; ++j) {
        const int m = m0 + RPB * (wave + NW * j) + rsub;
        xv[j] = m < a.M && wave + NW * j < Cf::XBLK;
        const Voxel v = voxel(m, a.Z, a.P, a.Q);
        xo[j] = (int)(v.n * a.xsn + (long long)v.z * a.sd * a.xsd +
                      (long long)v.p * a.sh * a.xsh + (long long)v.q * a.sw * a.xsw);
    }
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.w, 0, (int)a.w_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.x, 0, (int)a.x_bytes, 0x00020000);

    // The lane's reduction group of the next k-tile to issue: reduction index
    // gi = i0 + 8u lies in tap (t, r, s) at channel cc, and the tap starts
    // toff elements into a window (toff = t*xsd + r*xsh + s*xsw). The tap is
    // advanced incrementally, so the loop reads no tap table.
    int gi = 8 * u;
    int cc, ts, tr, toff;
    {
        const int tp = gi / a.C;
        cc = gi - tp * a.C;
        ts = tp % a.S;
        tr = (tp / a.S) % a.R;
        const int tt = tp / (a.S * a.R);
        toff = (int)(tt * a.xsd + tr * a.xsh + ts * a.xsw);
    }
    // Per k-tile the group moves KB = tstep*C + cstep elements on: whole taps
    // (C < KB only), then cstep channels with at most one more tap.
    const int tstep = SMALLC ? KB / a.C : 0;
    const int cstep = KB - tstep * a.C;
    const int dr = (int)(a.xsh - a.S * a.xsw), dt = (int)(a.xsd - a.R * a.xsh);
    // Next tap where `go` holds: s, then r, then t.
    auto next_tap = [&](bool go) __attribute__((always_inline)) {
        ts += go ? 1 : 0;
        toff += go ? (int)a.xsw : 0;
        const bool ws = ts == a.S;
        ts = ws ? 0 : ts;
        tr += ws ? 1 : 0;
        toff += ws ? dr : 0;
        const bool wr = tr == a.R;
        tr = wr ? 0 : tr;
        toff += wr ? dt : 0;
    };

    // Loads of the next k-tile (reduction indices i0 .. i0+KB-1) into an LDS
    // stage, then the lane's group moves on by KB.
    int i0 = 0;
    auto issue = [&](char* dst) __attribute__((always_inline)) {
        const bool kin = gi < a.KG;
#pragma unroll
        for (int j = 0; j < WJ; ++j) {
            const unsigned ow = (wv[j] && kin) ? wo[j] + 2u * (unsigned)i0 : kOOB;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rw, (LDS_AS void*)(dst + (wave + NW * j) * 1024), 16, (int)ow, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < XJ; ++j) {
            const unsigned ox = (xv[j] && kin) ? (unsigned)(2 * (xo[j] + toff + cc)) : kOOB;
            const int blk = wave + NW * j;  // past the X tile: zeros into the pad
            char* xdst = dst + Cf::WTILE + (blk < Cf::XBLK ? blk * 1024 : Cf::XTILE);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (LDS_AS void*)xdst, 16, (int)ox, 0, 0, 0);
        }
        i0 += KB;
        gi += KB;
        if (SMALLC) {  // tstep <= KB / 8 for C >= 8
#pragma unroll
            for (int i = 0; i < KB / 8; ++i) next_tap(i < tstep);
        }
        cc += cstep;
        const bool wrap = cc >= a.C;
        cc -= wrap ? a.C : 0;
        next_tap(wrap);
    };

    // MFMA operand addresses (v_mfma_f32_16x16x32_f16): lane l reads row
    // (16-row block base + l%16), unit 4*ks + l/16 (32 reduction elements per
    // k-step).
    constexpr int KS32 = KB / 32;
    const int g = lane >> 4, r16 = lane & 15;
    const int wch = wave % CW, wvx = wave / CW;  // channel quarter/half, voxel half
    int aaddr[4][KS32], baddr[2 * NB][KS32];
#pragma unroll
    for (int ks = 0; ks < KS32; ++ks) {
#pragma unroll
        for (int bl = 0; bl < 4; ++bl) {
            const int ra = wch * 64 + bl * 16 + r16;
            aaddr[bl][ks] = ra * ROWB + (((4 * ks + g) ^ swz<KB>(ra)) * 16);
        }
#pragma unroll
        for (int bl = 0; bl < 2 * NB; ++bl) {
            const int rb = wvx * 32 * NB + bl * 16 + r16;
            baddr[bl][ks] = Cf::WTILE + rb * ROWB + (((4 * ks + g) ^ swz<KB>(rb)) * 16);
        }
    }

    f32x4 acc[4][2 * NB];
#pragma unroll
    for (int cb = 0; cb < 4; ++cb)
#pragma unroll
        for (int vb = 0; vb < 2 * NB; ++vb) acc[cb][vb] = f32x4{};

    // One k-tile from stage cur, after issuing the loads of the k-tile NST-1
    // ahead into fill (the stage of the k-tile before this one).
    auto step = [&](char* __restrict__ fill, const char* __restrict__ cur)
        __attribute__((always_inline)) {
        // vmcnt(NST-2 k-tiles of loads): this wave's part of the k-tile in cur
        // landed.
        __builtin_amdgcn_s_waitcnt(0x0F70 | ((NST - 2) * LOADS));
        lds_barrier();    // every wave's; the k-tile in fill was consumed
        issue(fill);
        f16x8 af[KS32][4], bf[KS32][2 * NB];
#pragma unroll
        for (int ks = 0; ks < KS32; ++ks) {
#pragma unroll
            for (int bl = 0; bl < 4; ++bl) af[ks][bl] = lds_read16(cur, aaddr[bl][ks]);
#pragma unroll
            for (int bl = 0; bl < 2 * NB; ++bl) bf[ks][bl] = lds_read16(cur, baddr[bl][ks]);
        }
#pragma unroll
        for (int ks = 0; ks < KS32; ++ks)
#pragma unroll
            for (int cb = 0; cb < 4; ++cb)
#pragma unroll
                for (int vb = 0; vb < 2 * NB; ++vb)
                    acc[cb][vb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[ks][cb], bf[ks][vb],
                                                                         acc[cb][vb], 0, 0, 0);
        // With the small-C tap walk, a k-tile's reads hoisted above the
        // previous k-tile's MFMAs push the wave past 256 VGPRs (spills).
        if constexpr (SMALLC) __builtin_amdgcn_sched_barrier(0);
    };
    // k-tile t sits in stage t % NST. The loop runs whole groups of NST
    // k-tiles: k-tiles past the end load zeros and add nothing.
    const int nkt = (a.KG + KB - 1) / KB;
    issue(st0);
    if constexpr (NST == 2) {
        for (int kt = 0; kt < nkt; kt += 2) {
            step(st1, st0);
            step(st0, st1);
        }
    } else if constexpr (NST == 4) {
        issue(st1);
        issue(st2);
        for (int kt = 0; kt < nkt; kt += 4) {
            step(st3, st0);
            step(st0, st1);
            step(st1, st2);
            step(st2, st3);
        }
    } else {
        issue(st1);
        for (int kt = 0; kt < nkt; kt += 3) {
            step(st2, st0);
            step(st0, st1);
            step(st1, st2);
        }
    }
    // The zero loads past the last k-tile must land before the workgroup's
    // LDS is released.
    __builtin_amdgcn_s_waitcnt(0x0F70);

    // Epilogue: accumulator row 4g + r (an output channel), column l%16 (an
    // output voxel); one run of four channels per lane, voxel and block.
#pragma unroll
    for (int vb = 0; vb < 2 * NB; ++vb) {
        const int m = m0 + wvx * 32 * NB + vb * 16 + r16;
        if (m >= a.M) continue;
        const Voxel v = voxel(m, a.Z, a.P, a.Q);
        const long long oo = v.n * a.osn + v.z * a.osz + v.p * a.osp + v.q * a.osq;
        const long long ro = v.n * a.rsn + v.z * a.rsz + v.p * a.rsp + v.q * a.rsq;
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const int ch = k0 + wch * 64 + cb * 16 + 4 * g;
            if (ch >= a.K) continue;
            f32x4 val = acc[cb][vb];
            if (a.bias) val += __builtin_convertvector(*(const f16x4*)(a.bias + ch), f32x4);
            if (a.res) val += __builtin_convertvector(*(const f16x4*)(a.res + ro + ch), f32x4);
            *(f16x4*)(a.out + oo + ch) = __builtin_convertvector(val, f16x4);
        }
    }
#endif
}

// Launches configuration (NB, NST, KB, CW) over the whole problem.
template <int NB, int NST, int KB, int CW>
void launch_cfg(const ConvArgs& a, hipStream_t stream) {
    using Cf = ConvCfg<NB, NST, KB, CW>;
    const unsigned tiles = (unsigned)((a.M + Cf::BVX - 1) / Cf::BVX) *
                           (unsigned)((a.K + Cf::BCH - 1) / Cf::BCH);
    if (a.C < KB)
        hipLaunchKernelGGL((conv3d_mfma<NB, NST, KB, CW, true>), dim3(tiles), dim3(Cf::NT), 0,
                           stream, a);
    else
        hipLaunchKernelGGL((conv3d_mfma<NB, NST, KB, CW, false>), dim3(tiles), dim3(Cf::NT), 0,
                           stream, a);
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

// The kernel configurations: NB, KB, channels per workgroup (64*CW),
// workgroups per CU, relative cost per output element and reduction element
// (fitted on MI355X, see pick_kernel), launcher.
struct ConvKernel {
    int nb, kb, bch, occ;
    double rel;
    void (*launch)(const ConvArgs&, hipStream_t);
};
const ConvKernel kKernels[] = {
    {4, 32, 128, 2, 6.21, launch_cfg<4, 3, 32, 2>}, {3, 64, 128, 2, 6.18, launch_cfg<3, 2, 64, 2>},
    {2, 64, 128, 2, 6.68, launch_cfg<2, 2, 64, 2>}, {4, 32, 256, 1, 4.78, launch_cfg<4, 4, 32, 4>},
    {3, 64, 256, 1, 5.91, launch_cfg<3, 2, 64, 4>}, {2, 64, 256, 1, 5.47, launch_cfg<2, 3, 64, 4>},
    {3, 32, 256, 1, 6.19, launch_cfg<3, 4, 32, 4>},
};
constexpr int kNumKernels = sizeof(kKernels) / sizeof(kKernels[0]);

int find_kernel(int nb, int kb, int bch) {
    for (int i = 0; i < kNumKernels; ++i)
        if (kKernels[i].nb == nb && kKernels[i].kb == kb && kKernels[i].bch == bch) return i;
    return -1;
}

// Kernel configuration for an M x K problem with reduction length KG. Wider
// tiles load fewer bytes per MFMA (the loads into LDS, not the matrix cores,
// bound these kernels); narrower ones fill the CUs better when the tile count
// is small or just past a multiple of the workgroup slots. 64-wide k-tiles
// fetch whole 128-byte lines, 32-wide ones half lines but leave room for a
// deeper ring. Estimated time: R x tile size x (rel x KG / 13824 + 0.355),
// R the workgroups on the busiest CU in units of one workgroup's time (for
// two per CU: half rounds, a workgroup left alone on its CU at the end
// counting 1.3 halves), rel and the per-tile term (start-up and epilogue)
// fitted to six layers on MI355X (VAE decoder 3x3x3 with 128..512 channels,
// a 1x1x1; 3x32x256's rel from its time ratio to 3x64x256 with the 16x16x32
// MFMA kernels, 1.00-1.06 over five layers, so that it is not picked where
// 3x64x256 fits the same tiles).
// GFX906_AMD_CONV_CFG = "<NB>x<KB>" (128 channels) or "<NB>x<KB>x<channels>"
// (a row of kKernels) overrides the choice (testing); it is read on every
// call.
int pick_kernel(long M, int K, long KG) {
    if (const char* e = getenv("GFX906_AMD_CONV_CFG")) {
        int nb = 0, kb = 0, bch = 128;
        if (sscanf(e, "%dx%dx%d", &nb, &kb, &bch) >= 2) {
            const int i = find_kernel(nb, kb, bch);
            if (i >= 0) return i;
        }
    }
    static const int ncu = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        return n;
    }();
    const double kgu = (double)KG / 13824.0;
    int best = 0;
    double best_cost = 1e300;
    for (int i = 0; i < kNumKernels; ++i) {
        const ConvKernel& c = kKernels[i];
        const long tiles = (M + 64 * c.nb - 1) / (64 * c.nb) * ((K + c.bch - 1) / c.bch);
        double r;
        if (c.occ == 2) {
            const long n = (tiles + ncu - 1) / ncu;  // half rounds on the busiest CU
            r = (double)n + (n & 1 ? 0.3 : 0.0);
        } else {
            r = (double)((tiles + ncu - 1) / ncu);
        }
        const double cost = r * 64.0 * c.nb * c.bch * (c.rel * kgu + 0.355);
        if (cost < best_cost) {
            best_cost = cost;
            best = i;
        }
    }
    return best;
}

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
    kKernels[pick_kernel(M, K, KG)].launch(a, stream);
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
