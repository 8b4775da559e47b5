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
//    O^T = V^T * P^T. V stays row-major ([key][dim]) in LDS and the A operand
//    is read with ds_read_b64_tr_b16, whose 16-lane transpose hands each lane
//    four keys of one dim; the key order is chosen to match the accumulator
//    layout of S^T.
//  * K and V tiles go from HBM straight into LDS with buffer loads to LDS
//    (no VGPR staging), through a ring of four stages, two tiles ahead of
//    the compute. Rows are XOR-swizzled in 16-byte units so that the QK^T
//    reads (32 keys x one 16-byte unit) and the transposed V reads (8 keys x
//    64 bytes) are free of LDS bank conflicts.
//  * Each wave is software-pipelined over 32-key blocks: the iteration for
//    block j issues the PV MFMAs of block j-1 and the QK^T MFMAs of block
//    j+1 while the VALU turns the scores of block j into P.
//  * Softmax runs in fp32 with exp2 and scale*log2(e) folded into one FMA.
//    The running max is updated lazily: O is rescaled only when a block's
//    row sum of p = exp2(s*c - m) exceeds 2^15 (the block's max rose well
//    above the running max, or this is the first block), which keeps every p
//    finite in fp16 and skips the rescale on almost every block.
//  * The row sum l is accumulated from the fp16-rounded P (v_dot2_f32_f16
//    against 1.0), so numerator and denominator see the same rounded weights.
//  * Output rows are normalised by 1/l and rounded to fp16 (RNE), as the
//    reference does (attn_kernel.hip:497-511). Rows of a head with Skv == 0
//    are written as zeros (the reference leaves them unwritten).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <type_traits>

#include "gfx906_amd_attn.h"

namespace {

typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

#define LDS_AS __attribute__((address_space(3)))
#define GLOBAL_AS __attribute__((address_space(1)))

constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale: a block whose lane row sum exceeds this takes the exact max.
constexpr float kLsumLimit = 32768.0f;
// Lazy-rescale threshold of the D = 512 kernel in log2 units: p <= 2^kTau.
constexpr float kTau = 8.0f;
constexpr float kPmaxLimit = 256.0f;  // 2^kTau
// sched_group_barrier instruction classes
constexpr int kSgMfma = 0x008, kSgDsRead = 0x100;

__device__ __forceinline__ f16x8 ld_global16(const f16* p) {
    return *reinterpret_cast<const f16x8*>(p);
}

// Three-way max; with NaN-free arithmetic assumed (-fno-honor-nans) the
// backend selects v_max3_f32 for it.
__device__ __forceinline__ float max3(float a, float b, float c) {
    return fmaxf(fmaxf(a, b), c);
}

// 16-byte LDS read at a byte address.
__device__ __forceinline__ f16x8 lds_read16(const char* base, int byte_off) {
    return *(const LDS_AS f16x8*)((const LDS_AS char*)base + byte_off);
}
// Transposed 8-byte LDS read (see the 16-lane mapping in the header comment).
__device__ __forceinline__ f16x4 lds_read_tr(const char* base, int byte_off) {
    fp16x4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (LDS_AS fp16x4_t*)((LDS_AS char*)base + byte_off));
    return __builtin_bit_cast(f16x4, r);
}

// XOR swizzles of the 16-byte unit index within a row.
//  K: the QK^T read takes one unit from 32 consecutive rows, so 16
//     consecutive rows must land on 16 different bank groups.
//  V: the transposed read takes 4 units from 8 consecutive rows; each half
//     wave (4 rows x 4 units) must cover all 16 bank groups.
template <int NU>
__device__ __forceinline__ int kswz(int r) { return NU >= 16 ? (r & 15) : ((r >> 1) & 7); }
template <int NU>
__device__ __forceinline__ int vswz(int r) { return NU >= 16 ? 4 * (r & 3) : 4 * ((r >> 1) & 1); }

// Per-lane byte offsets of the direct HBM->LDS tile loads. Each wave fills
// whole 1 KB LDS blocks (lane i writes 16-byte unit i of its block) for
// BLKS/NW blocks of each K tile and as many of each V tile. The offsets are
// relative to the tile's first row and do not change from tile to tile.
// Units past D (padded head dims) are pointed at unit 0 of the row: finite
// data that meets zero Q columns (K) or feeds unused output columns (V).
template <class C, bool PAD>
__device__ __forceinline__ void tile_offsets(int (&koff)[C::BLKS / C::NW],
                                             int (&voff)[C::BLKS / C::NW], int D, int wave,
                                             int lane) {
#pragma unroll
    for (int i = 0; i < C::BLKS / C::NW; ++i) {
        const int unit = (wave + i * C::NW) * 64 + lane;
        const int row = unit / C::NU, slot = unit % C::NU;
        int ck = slot ^ kswz<C::NU>(row);
        if (PAD && ck * 8 >= D) ck = 0;
        koff[i] = (row * D + ck * 8) * 2;
        int cv = slot ^ vswz<C::NU>(row);
        if (PAD && cv * 8 >= D) cv = 0;
        voff[i] = (row * D + cv * 8) * 2;
    }
}

#if defined(__HIP_DEVICE_COMPILE__)
// Issue the loads of one K (or V) tile starting at key n0 into an LDS stage.
// The buffer descriptor covers exactly the tile's valid rows, so rows past
// Skv read as zeros and nothing outside the tensor is touched; a tile that
// starts at or past Skv has an empty range and fills the stage with zeros.
template <class C>
__device__ __forceinline__ void issue_tile(const f16* __restrict__ X, int n0, int Skv, int D,
                                           char* stage, int wave,
                                           const int (&off)[C::BLKS / C::NW]) {
    // Uniform; readfirstlane keeps the descriptor in SGPRs (a clamp selected
    // as a VALU op would otherwise force a waterfall loop around each load).
    const int bytes = __builtin_amdgcn_readfirstlane(max(0, min(Skv - n0, C::BN)) * D * 2);
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)(X + (long)n0 * D), 0, bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < C::BLKS / C::NW; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LDS_AS void*)(stage + (wave + i * C::NW) * 1024),
                                                 16, off[i], 0, 0, 0);
}

// Max of x over lanes l and l^32 (both halves get the result).
__device__ __forceinline__ float half_swap_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float half_swap_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// P for one 32-key block of S^T (a lane's 16 scores, two 16-key PV steps):
// p = exp2(s*c + nm) rounded to fp16, nm = -(running max). Adds the block's
// row-sum contribution, taken from the fp16-rounded values, to lsum.
__device__ __forceinline__ void block_exp_f16(const f32x16& Sb, f16x8& P0, f16x8& P1, float nm,
                                              float c, float& lsum) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        f16x8& P = h ? P1 : P0;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[8 * h + e], c, nm));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[8 * h + e + 1], c, nm));
            const f16x2 hp = __builtin_convertvector(f32x2{p0, p1}, f16x2);
            P[e] = hp[0];
            P[e + 1] = hp[1];
            lsum = __builtin_amdgcn_fdot2(hp, f16x2{(f16)1.0f, (f16)1.0f}, lsum, false);
        }
    }
}

// Whether a block's P needs the exact-max rescale: some lane's row sum over
// the block exceeds 2^15 or is not finite. Every p <= lsum, so passing the
// test keeps all p finite in fp16; the first block (running max -1e30,
// p = inf) always fails it.
__device__ __forceinline__ bool needs_rescale(float lsum) {
    return __any(!(lsum <= kLsumLimit));
}
#endif

// ---------------------------------------------------------------------------
// D <= 128: software-pipelined waves, 32 * QB query rows each.
//
// The iteration for 32-key block j issues the PV MFMAs of block j-1 and the
// QK^T MFMAs of block j+1 while the VALU turns the scores of block j into P,
// so every stretch of a wave's instruction stream carries matrix and vector
// work (two blocks of S and of P are live). With QB = 2 each K or V fragment
// read from LDS feeds two MFMAs, at twice the accumulator registers.
//
// K/V tiles are 64 keys (two blocks) in a ring of four LDS stages, separate
// arrays so that the compiler can tell their accesses apart (a read of one
// stage then never waits for loads into another). The barrier that opens
// tile w+1 follows the iteration that finished every read of tile w-1, whose
// stage then takes tile w+3: loads run two tiles ahead. Tiles past the end
// are loaded anyway, as zeros (empty buffer range), which keeps every wait
// count static.
//
//   DP  : head dim the tiles are built for (64 or 128; D < 64 is padded)
//   NW  : waves per workgroup
//   QB  : 32-row query blocks per wave
//   OCC : workgroups per CU the register budget is sized for
template <int DP_, int NW_, int QB_, int OCC_>
struct Cfg {
    static constexpr int DP = DP_, NW = NW_, QB = QB_, OCC = OCC_, BN = 64;
    static constexpr int BM = NW * 32 * QB;     // query rows per workgroup
    static constexpr int NT = NW * 64;          // threads per workgroup
    static constexpr int NU = DP / 8;           // 16-byte units per row
    static constexpr int RB = DP * 2;           // bytes per row
    static constexpr int TILE = BN * RB;        // bytes of one K (or V) tile
    static constexpr int STAGE = 2 * TILE;      // K tile, then V tile
    static constexpr int BLKS = TILE / 1024;    // 1 KB direct-load blocks per tile
    static_assert(BLKS % NW == 0, "tile must split evenly over waves");
    static_assert(DP % 32 == 0 && DP <= 128, "head-dim class");
};

// grid: ceil(Sq / BM) * B*H workgroups, query tiles of one head adjacent;
// block: NW*64 threads.

template <class C, bool PAD>
__global__ void __launch_bounds__(C::NT, C::OCC)
attn_fwd_pipe(const f16* __restrict__ Q, const f16* __restrict__ K,
             const f16* __restrict__ V, f16* __restrict__ O,
             int Sq, int Skv, int D, float c, float qsign) {
#if defined(__HIP_DEVICE_COMPILE__)
    constexpr int DP = C::DP, NU = C::NU, RB = C::RB, TILE = C::TILE, QB = C::QB;
    constexpr int NQF = DP / 16;  // Q fragments (16 dims each) per query block
    constexpr int NOB = DP / 32;  // 32-dim output blocks
    constexpr int LPT = C::BLKS / C::NW;  // loads per wave per K (or V) tile
    static_assert(2 * LPT < 16, "vmcnt immediate");
    constexpr int kWaitNext = 0x0F70 | (2 * LPT);  // vmcnt(one tile of loads)
    __shared__ __attribute__((aligned(1024))) char st0[C::STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[C::STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[C::STAGE];
    __shared__ __attribute__((aligned(1024))) char st3[C::STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = lane >> 5, r32 = lane & 31;
    const int j16 = lane & 15, G = lane >> 4;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    const long bh = blockIdx.x / nqt;
    const int qt = blockIdx.x % nqt;
    const f16* Qh = Q + bh * (long)Sq * D;
    const f16* Kh = K + bh * (long)Skv * D;
    const f16* Vh = V + bh * (long)Skv * D;
    f16* Oh = O + bh * (long)Sq * D;
    const int qrow0 = qt * C::BM + wave * 32 * QB + r32;  // this lane's rows: qrow0 + 32 qb
    const int ntiles = (Skv + C::BN - 1) / C::BN;

    // Q^T fragments (B operands), loaded before any tile so that the tile
    // waits below also cover them. Negative scale: sign bits flipped.
    f16x8 qf[QB][NQF];
    const unsigned qneg = qsign < 0.f ? 0x80008000u : 0u;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int s = 0; s < NQF; ++s) {
            const int d0 = 16 * s + 8 * g, row = qrow0 + 32 * qb;
            f16x8 val = {};
            if (row < Sq && (!PAD || d0 < D)) val = ld_global16(Qh + (long)row * D + d0);
            qf[qb][s] = __builtin_bit_cast(f16x8, __builtin_bit_cast(u32x4, val) ^ qneg);
        }

    f32x16 oacc[QB][NOB];
    float m_run[QB], l_run[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
#pragma unroll
        for (int b = 0; b < NOB; ++b) oacc[qb][b] = f32x16{};
        // Running max in units of s*c (log2 domain). It starts finite so that
        // a masked key (score -inf) gives p = 0 rather than NaN.
        m_run[qb] = -1e30f;
        l_run[qb] = 0.f;
    }

    if (ntiles > 0) {
        int koff[LPT], voff[LPT];
        tile_offsets<C, PAD>(koff, voff, D, wave, lane);
        auto issue = [&](int t, char* dst) __attribute__((always_inline)) {
            issue_tile<C>(Kh, t * C::BN, Skv, D, dst, wave, koff);
            issue_tile<C>(Vh, t * C::BN, Skv, D, dst + TILE, wave, voff);
        };
        int kaddr[8];
        {
            const int kl = g ^ kswz<NU>(r32);
#pragma unroll
            for (int s = 0; s < 8; ++s) kaddr[s] = r32 * RB + (((2 * s) & 15) ^ kl) * 16;
        }
        int vaddr[4];
        {
            const int vrow = 4 * g + (j16 >> 2);
            const int vv = NU >= 16 ? (j16 >> 2) : (j16 >> 3);
            const int w = 2 * (G & 1) + ((j16 & 3) >> 1);
#pragma unroll
            for (int b = 0; b < 4; ++b)
                vaddr[b] = vrow * RB + (4 * (b ^ vv) + w) * 16 + 8 * (j16 & 1);
        }

        // S^T of 32-key block kb of the tile in stage st, both query blocks.
        auto qk = [&](const char* st, int kb, f32x16 (&S)[QB]) __attribute__((always_inline)) {
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) S[qb] = f32x16{};
#pragma unroll
            for (int s = 0; s < NQF; ++s) {
                const f16x8 a = lds_read16(st, kaddr[s & 7] + kb * 32 * RB + ((2 * s) & ~15) * 16);
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
                    S[qb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[qb][s], S[qb], 0, 0, 0);
            }
        };
        // O^T += V^T P^T for 32-key block kb of the tile in stage st.
        auto pv = [&](const char* st, int kb, const f16x8 (&P)[QB][2]) __attribute__((always_inline)) {
            const char* sv = st + TILE;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
#pragma unroll
                for (int b = 0; b < NOB; ++b) {
                    const int off = (2 * kb + ks) * 16 * RB + (b & ~3) * 64;
                    const f16x4 lo = lds_read_tr(sv, vaddr[b & 3] + off);
                    const f16x4 hi = lds_read_tr(sv, vaddr[b & 3] + off + 8 * RB);
                    const f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
                    for (int qb = 0; qb < QB; ++qb)
                        oacc[qb][b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, P[qb][ks], oacc[qb][b], 0, 0, 0);
                }
        };
        // Scores of keys >= Skv (block keys key0..key0+31) to -inf. Taken
        // for the last one or two blocks only; a branch at the start of an
        // iteration, so the iteration's MFMAs and VALU work stay in one
        // scheduling region.
        auto mask = [&](f32x16 (&S)[QB], int key0) __attribute__((always_inline)) {
            if (key0 + 32 > Skv) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int key = key0 + 8 * (r >> 2) + 4 * g + (r & 3);
                        if (key >= Skv) S[qb][r] = -INFINITY;
                    }
            }
        };
        // P of one 32-key block for every query block, with the lazy rescale:
        // when a row sum fails the test, the exact max of the block's scores
        // is taken, O and l are rescaled and P is recomputed (a per-wave
        // branch, so it stays uniform). Any rescale of O comes after the PV
        // MFMAs issued before this call.
        auto softmax = [&](f32x16 (&S)[QB], f16x8 (&P)[QB][2]) __attribute__((always_inline)) {
            float lp[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) {
                lp[qb] = 0.f;
                block_exp_f16(S[qb], P[qb][0], P[qb][1], -m_run[qb], c, lp[qb]);
            }
            float lmax = lp[0];
#pragma unroll
            for (int qb = 1; qb < QB; ++qb) lmax = fmaxf(lmax, lp[qb]);
            if (__builtin_expect(needs_rescale(lmax), 0)) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    float mx = -INFINITY;
#pragma unroll
                    for (int r = 0; r < 16; r += 2) mx = max3(mx, S[qb][r], S[qb][r + 1]);
                    mx = half_swap_max(mx) * c;
                    const float m_new = fmaxf(m_run[qb], mx);
                    const float alpha = __builtin_amdgcn_exp2f(m_run[qb] - m_new);
#pragma unroll
                    for (int b = 0; b < NOB; ++b) oacc[qb][b] *= alpha;
                    l_run[qb] *= alpha;
                    m_run[qb] = m_new;
                    lp[qb] = 0.f;
                    block_exp_f16(S[qb], P[qb][0], P[qb][1], -m_new, c, lp[qb]);
                }
            }
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) l_run[qb] += lp[qb];
        };

        f32x16 Sa[QB], Sb[QB];
        f16x8 Pa[QB][2], Pb[QB][2];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) Pb[qb][ks] = f16x8{};  // block -1: no keys

        // Tile w (blocks 2w, 2w+1) in stage cur; prev holds tile w-1, nxt
        // tile w+1; fill (the stage of tile w-1) takes tile w+3.
        auto tile = [&](int w, const char* prev, const char* cur, const char* nxt, char* fill)
                __attribute__((always_inline)) {
            mask(Sa, w * C::BN);
            pv(prev, 1, Pb);   // block 2w-1
            qk(cur, 1, Sb);    // block 2w+1
            softmax(Sa, Pa);   // block 2w
            __builtin_amdgcn_s_waitcnt(kWaitNext);  // own loads of tile w+1 done
            __syncthreads();                        // every wave's; tile w-1 consumed
            issue(w + 3, fill);
            mask(Sb, w * C::BN + 32);
            pv(cur, 0, Pa);    // block 2w
            qk(nxt, 0, Sa);    // block 2w+2
            softmax(Sb, Pb);   // block 2w+1
        };

        // Prologue: tiles 0 and 1 in flight, stage 3's V zeroed for the PV
        // of block -1 (P = 0, and 0 * garbage could be NaN), tile 2 issued
        // once tile 0 is in, then S of block 0.
        issue(0, st0);
        issue(1, st1);
        for (int i = tid; i < TILE / 16; i += C::NT)
            *reinterpret_cast<u32x4*>(st3 + TILE + 16 * i) = u32x4{};
        __builtin_amdgcn_s_waitcnt(kWaitNext);
        __syncthreads();
        issue(2, st2);
        qk(st0, 0, Sa);

        // Tile w sits in stage w % 4. The loop runs whole groups of four
        // tiles: tiles past the end hold zeros and are masked to p = 0 (at
        // most three per workgroup). A single exit keeps the register
        // allocation of the loop body intact; exits after each tile do not.
        for (int w0 = 0;; w0 += 4) {
            tile(w0 + 0, st3, st0, st1, st3);
            tile(w0 + 1, st0, st1, st2, st0);
            tile(w0 + 2, st1, st2, st3, st1);
            tile(w0 + 3, st2, st3, st0, st2);
            if (w0 + 4 >= ntiles) break;
        }
        pv(st3, 1, Pb);  // block 2w+1 of the last tile
        // The zero-range loads past the end must land before the workgroup's
        // LDS is released.
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }

#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
        const int row = qrow0 + 32 * qb;
        const float l = half_swap_sum(l_run[qb]);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        if (row < Sq) {
            f16* op = Oh + (long)row * D;
#pragma unroll
            for (int b = 0; b < NOB; ++b)
#pragma unroll
                for (int rr = 0; rr < 4; ++rr) {
                    const int d0 = 32 * b + 8 * rr + 4 * g;
                    if (!PAD || d0 < D) {
                        const f16x2 h0 = __builtin_convertvector(
                            f32x2{oacc[qb][b][4 * rr + 0] * inv, oacc[qb][b][4 * rr + 1] * inv}, f16x2);
                        const f16x2 h1 = __builtin_convertvector(
                            f32x2{oacc[qb][b][4 * rr + 2] * inv, oacc[qb][b][4 * rr + 3] * inv}, f16x2);
                        const f16x4 h = {h0[0], h0[1], h1[0], h1[1]};
                        *reinterpret_cast<f16x4*>(op + d0) = h;
                    }
                }
        }
    }
#endif
}

// ---------------------------------------------------------------------------
// D = 512: 16x16x32 MFMA tiles, 16 query rows per wave.
//
// With 32 query rows a wave would need a 256-register O accumulator; with 16
// rows O^T is 32 blocks of 16x16 (128 registers) and two waves fit per SIMD.
// Lane l = 16*g + i holds query i of the wave: the S^T = K Q^T accumulator of
// a 16-key block gives it keys 4g..4g+3, so row reductions combine the four
// lanes i, i+16, i+32, i+48. A 32-key tile is two score blocks feeding one
// 16x16x32 PV step, whose B operand takes keys 4g..4g+3 of block 0 and of
// block 1; V^T is read with ds_read_b64_tr_b16 in that key order.
struct Cfg512 {
    static constexpr int DP = 512, NW = 8, BN = 32, BM = NW * 16, NT = NW * 64;
    static constexpr int RB = DP * 2;  // bytes of one K or V row in HBM
    // LDS rows are padded instead of swizzled (one direct-load instruction
    // fills exactly one row, so the padding costs nothing): with a 1040-byte
    // K stride the QK^T read (16 rows, one 16-byte unit each) and with a
    // 1056-byte V stride the transposed read (8 rows x 32 bytes per half
    // wave) touch every bank group once.
    static constexpr int KS = RB + 16, VS = RB + 32;
    static constexpr int KTILE = BN * KS, VTILE = BN * VS, STAGE = KTILE + VTILE;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int NLD = BN / NW;  // rows loaded per wave per tile, per tensor
};

#if defined(__HIP_DEVICE_COMPILE__)
// Sum / max over lanes i, i+16, i+32, i+48.
__device__ __forceinline__ float quad_group_sum(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}
__device__ __forceinline__ float quad_group_max(float x) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}
#endif

#if defined(__HIP_DEVICE_COMPILE__)
// Rare path of the D = 512 kernel: the tile's scores exceed the running max by
// more than kTau. Returns the new max, the rescale factor for O and l, and P
// and the tile's row sum recomputed with the new max. Kept out of line (and
// away from O, which stays in registers) so the hot loop does not reserve
// registers for it.
struct Rescale512 {
    f16x8 P;
    float m, alpha, l_tile;
};
__device__ __attribute__((noinline)) Rescale512 d512_rescale(f32x4 S0, f32x4 S1, float m_run,
                                                             float c) {
    float mx = fmaxf(max3(S0[0], S0[1], S0[2]), max3(S0[3], S1[0], S1[1]));
    mx = quad_group_max(max3(mx, S1[2], S1[3])) * c;
    Rescale512 r;
    r.m = fmaxf(m_run, mx);
    r.alpha = __builtin_amdgcn_exp2f(m_run - r.m);
    const float nm = -r.m;
    float lsum = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const f32x4& Sb = u < 2 ? S0 : S1;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1)], c, nm));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1) + 1], c, nm));
        const f16x2 hp = __builtin_convertvector(f32x2{p0, p1}, f16x2);
        r.P[2 * u] = hp[0];
        r.P[2 * u + 1] = hp[1];
        lsum = __builtin_amdgcn_fdot2(hp, f16x2{(f16)1.0f, (f16)1.0f}, lsum, false);
    }
    r.l_tile = lsum;
    return r;
}
#endif

// grid: ceil(Sq / 128) * B*H workgroups; block: 512 threads.
__global__ void __launch_bounds__(Cfg512::NT, 1)
attn_fwd_d512(const f16* __restrict__ Q, const f16* __restrict__ K,
              const f16* __restrict__ V, f16* __restrict__ O,
              int Sq, int Skv, float c, float qsign) {
#if defined(__HIP_DEVICE_COMPILE__)
    using C = Cfg512;
    constexpr int D = C::DP, BN = C::BN, RB = C::RB, NLD = C::NLD;
    static_assert(NLD * C::NW == BN && D * 2 == 64 * 16, "one row per load instruction");
    constexpr int NQF = D / 32;  // Q fragments (32 dims each)
    constexpr int NOB = D / 16;  // 16-dim output blocks
    __shared__ __attribute__((aligned(1024))) char lds[C::LDS];  // 2 stages x (K, V)

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    const long bh = blockIdx.x / nqt;
    const int qt = blockIdx.x % nqt;
    const f16* Qh = Q + bh * (long)Sq * D;
    const f16* Kh = K + bh * (long)Skv * D;
    const f16* Vh = V + bh * (long)Skv * D;
    f16* Oh = O + bh * (long)Sq * D;
    const int qrow = qt * C::BM + wave * 16 + i;
    const bool live = qrow < Sq;

    auto stage = [&](int t) { return lds + (t & 1) * C::STAGE; };
    // Direct loads: one instruction per K or V row; lane l fetches dims
    // 8l..8l+7. Rows past Skv read as zeros (the descriptor covers the valid
    // rows only).
    auto issue = [&](int t, char* dst) __attribute__((always_inline)) {
        const int bytes = min(Skv - t * BN, BN) * RB;
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void*)(Kh + (long)t * BN * D), 0, bytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void*)(Vh + (long)t * BN * D), 0, bytes, 0x00020000);
#pragma unroll
        for (int n = 0; n < NLD; ++n) {
            const int row = wave + n * C::NW;  // wave-uniform
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LDS_AS void*)(dst + row * C::KS), 16,
                                                     lane * 16, row * RB, 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (LDS_AS void*)(dst + C::KTILE + row * C::VS),
                                                     16, lane * 16, row * RB, 0, 0);
        }
    };
    const int ntiles = (Skv + BN - 1) / BN;
    if (ntiles > 0) issue(0, stage(0));

    // Q^T fragments (B operand: column = this lane's query, k = dims 32s+8g..).
    f16x8 qf[NQF];
    const unsigned qneg = qsign < 0.f ? 0x80008000u : 0u;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
        f16x8 val = {};
        if (live) val = ld_global16(Qh + (long)qrow * D + 32 * s + 8 * g);
        qf[s] = __builtin_bit_cast(f16x8, __builtin_bit_cast(u32x4, val) ^ qneg);
    }

    // K read: row kb*16 + i, dims 32s + 8g.. ; V^T read (transposed, per
    // 16-lane group g): row 4g + i/4 (+16 for the second key half), dims
    // 16*db + 4*(i%4)..
    const int kbase = i * C::KS + g * 16;
    const int vbase = (4 * g + (i >> 2)) * C::VS + 8 * (i & 3);

    f32x4 oacc[NOB];
#pragma unroll
    for (int b = 0; b < NOB; ++b) oacc[b] = f32x4{};
    float m_run = -1e30f;  // running max (log2 units); finite, see attn_fwd_mfma
    float l_run = 0.f;

    // P (B operand of the PV step) from the two score blocks, with running max -nm.
    auto make_p = [&](const f32x4 (&S)[2], f16x8& P, float nm, float& lsum, f16x2& pm)
        __attribute__((always_inline)) {
        f16x2 hp[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f32x4& Sb = S[u >> 1];
            const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1)], c, nm));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1) + 1], c, nm));
            hp[u] = __builtin_convertvector(f32x2{p0, p1}, f16x2);
            P[2 * u] = hp[u][0];
            P[2 * u + 1] = hp[u][1];
            lsum = __builtin_amdgcn_fdot2(hp[u], f16x2{(f16)1.0f, (f16)1.0f}, lsum, false);
        }
        pm = __builtin_elementwise_maximum(pm, __builtin_elementwise_maximum(
                                                   __builtin_elementwise_maximum(hp[0], hp[1]),
                                                   __builtin_elementwise_maximum(hp[2], hp[3])));
    };

    auto tile = [&](int t, char* __restrict__ nxt, const char* __restrict__ cur)
        __attribute__((always_inline)) {
        if (t + 1 < ntiles) issue(t + 1, nxt);
        const char* sk = cur;
        const char* sv = cur + C::KTILE;
        f32x4 S[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 Sp[2] = {f32x4{}, f32x4{}};
#pragma unroll
            for (int s = 0; s < NQF; ++s) {
                const f16x8 a = lds_read16(sk, kbase + kb * 16 * C::KS + s * 64);
                Sp[s & 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, qf[s], Sp[s & 1], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(kSgDsRead, 4, 0);
#pragma unroll
            for (int n = 0; n < NQF - 4; ++n) {
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
                __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
            }
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 4, 0);
            S[kb] = Sp[0] + Sp[1];
        }
        if (t * BN + BN > Skv) {  // last, partial tile
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (t * BN + kb * 16 + 4 * g + r >= Skv) S[kb][r] = -INFINITY;
        }
        if (t == 0) {  // first tile: start from its exact max (O is still zero)
            float mx = fmaxf(max3(S[0][0], S[0][1], S[0][2]), max3(S[0][3], S[1][0], S[1][1]));
            m_run = quad_group_max(max3(mx, S[1][2], S[1][3])) * c;
        }
        f16x8 P;
        float l_tile = 0.f;
        f16x2 pm = {(f16)0.0f, (f16)0.0f};
        make_p(S, P, -m_run, l_tile, pm);
        const float pmax = fmaxf((float)pm[0], (float)pm[1]);
        // The O rescale runs on every tile (alpha = 1.0 exactly unless the rare
        // path ran): a conditional in-place rescale of the 128-register
        // accumulator costs more registers than two waves per SIMD allow, while
        // 128 multiplies per tile hide under its 64 MFMAs.
        float alpha = 1.f;
        if (__builtin_expect(__any(pmax > kPmaxLimit), 0)) {
            const Rescale512 r = d512_rescale(S[0], S[1], m_run, c);
            alpha = r.alpha;
            l_run *= r.alpha;
            m_run = r.m;
            P = r.P;
            l_tile = r.l_tile;
        }
#pragma unroll
        for (int b = 0; b < NOB; ++b) oacc[b] *= alpha;
        l_run += l_tile;
        // O^T += V^T P^T, one 16x16x32 MFMA per 16-dim block.
#pragma unroll
        for (int b = 0; b < NOB; ++b) {
            const f16x4 lo = lds_read_tr(sv, vbase + 32 * b);
            const f16x4 hi = lds_read_tr(sv, vbase + 32 * b + 16 * C::VS);
            const f16x8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            oacc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, P, oacc[b], 0, 0, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, 4, 0);
#pragma unroll
        for (int n = 0; n < NOB - 2; ++n) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 1, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
    };

    for (int t = 0; t < ntiles; ++t) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): tile t landed (this wave's part)
        __syncthreads();                    // ... every wave's; stage t+1 free
        tile(t, stage(t + 1), stage(t));
    }

    const float l = quad_group_sum(l_run);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (live) {
        f16* op = Oh + (long)qrow * D + 4 * g;
#pragma unroll
        for (int b = 0; b < NOB; ++b) {
            const f16x2 h0 = __builtin_convertvector(f32x2{oacc[b][0] * inv, oacc[b][1] * inv}, f16x2);
            const f16x2 h1 = __builtin_convertvector(f32x2{oacc[b][2] * inv, oacc[b][3] * inv}, f16x2);
            const f16x4 h = {h0[0], h0[1], h1[0], h1[1]};
            *reinterpret_cast<f16x4*>(op + 16 * b) = h;
        }
    }
#endif
}

// Tile configurations per head-dim class (waves per workgroup, keys per
// tile, waves per SIMD); the macros exist for tuning sweeps.
thread_local char g_err[256];

void set_err(const char* msg) {
    int i = 0;
    for (; msg[i] && i < 255; ++i) g_err[i] = msg[i];
    g_err[i] = 0;
}

using Cfg128 = Cfg<128, 8, 1, 1>;  // 128 KB of LDS: one workgroup, two waves per SIMD
using Cfg64 = Cfg<64, 8, 1, 2>;    // 64 KB: two workgroups, four waves per SIMD

template <class C, bool PAD>
hipError_t launch_pipe(const void* q, const void* k, const void* v, void* o, int B, int H,
                      int Sq, int Skv, int D, float scale, hipStream_t s) {
    dim3 grid((unsigned)((Sq + C::BM - 1) / C::BM) * (unsigned)(B * H));
    const float c = fmaxf(fabsf(scale) * kLog2e, 1e-30f);  // see launch_cfg
    const float qsign = scale < 0.f ? -1.f : 1.f;
    hipLaunchKernelGGL((attn_fwd_pipe<C, PAD>), grid, dim3(C::NT), 0, s, (const f16*)q,
                       (const f16*)k, (const f16*)v, (f16*)o, Sq, Skv, D, c, qsign);
    return hipGetLastError();
}

hipError_t launch_d512(const void* q, const void* k, const void* v, void* o, int B, int H, int Sq,
                       int Skv, float scale, hipStream_t s) {
    dim3 grid((unsigned)((Sq + Cfg512::BM - 1) / Cfg512::BM) * (unsigned)(B * H));
    const float c = fmaxf(fabsf(scale) * kLog2e, 1e-30f);  // see launch_cfg
    const float qsign = scale < 0.f ? -1.f : 1.f;
    hipLaunchKernelGGL(attn_fwd_d512, grid, dim3(Cfg512::NT), 0, s, (const f16*)q,
                       (const f16*)k, (const f16*)v, (f16*)o, Sq, Skv, c, qsign);
    return hipGetLastError();
}

// Validates the arguments; returns 0 and the workspace size, or 1 with the
// error message set.
// Validates the arguments; returns 0, or 1 with the error message set.
int check_args(const void* q, const void* k, const void* v, void* o, int B, int H, int Sq,
               int Skv, int D) {
    if (B < 0 || H < 0 || Sq < 0 || Skv < 0) {
        set_err("attn: negative size");
        return 1;
    }
    if (!((D <= 64 && D > 0 && D % 8 == 0) || D == 128 || D == 512)) {
        set_err("attn: head_dim must be <=64 and a multiple of 8, or 128, or 512");
        return 1;
    }
    if ((long)B * H * ((Sq + 31) / 32) > 0x7fffffffL || (long)B * H > 65535) {
        set_err("attn: grid too large");
        return 1;
    }
    if (B == 0 || H == 0 || Sq == 0) return 0;
    if (!q || !o || (Skv > 0 && (!k || !v))) {
        set_err("attn: null pointer");
        return 1;
    }
    return 0;
}

int run(const void* q, const void* k, const void* v, void* o, int B, int H, int Sq, int Skv,
        int D, float scale, hipStream_t s) {
    hipError_t e;
    if (D == 128)
        e = launch_pipe<Cfg128, false>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    else if (D == 64)
        e = launch_pipe<Cfg64, false>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    else if (D == 512)
        e = launch_d512(q, k, v, o, B, H, Sq, Skv, scale, s);
    else
        e = launch_pipe<Cfg64, true>(q, k, v, o, B, H, Sq, Skv, D, scale, s);
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        return 2;
    }
    return 0;
}

}  // namespace

extern "C" const char* attn_last_error(void) { return g_err[0] ? g_err : nullptr; }

extern "C" int attn_fwd(const void* q, const void* k, const void* v, void* o, int B, int H,
                        int Sq, int Skv, int D, float scale, hipStream_t s) {
    g_err[0] = 0;
    if (check_args(q, k, v, o, B, H, Sq, Skv, D)) return 1;
    if (B == 0 || H == 0 || Sq == 0) return 0;
    return run(q, k, v, o, B, H, Sq, Skv, D, scale, s);
}

extern "C" void launch(const void* q, const void* k, const void* v, void* o, int B, int H,
                       int Sq, int Skv, int D, float scale, hipStream_t s) {
    (void)attn_fwd(q, k, v, o, B, H, Sq, Skv, D, scale, s);
}
