// Flash-attention forward for AMD MI355X (gfx950 / CDNA4), fp16 or bf16 in/out.
//
// Computes, per (batch, head) and query row i:
//     o_i = sum_j softmax_j(scale * <q_i, k_j>) * v_j
// on [B, H, S, D] tensors (any batch / head / sequence strides, unit stride
// along D; for D = 512 also token-contiguous K and V, unit stride along S)
// with Sq != Skv allowed, no mask, no dropout; grids too small for the GPU
// split the key range and merge the partial results. This is the
// computation behind the reference's `launch` entry point
// (attn_kernel.hip:710-742, dispatch) and its per-D kernels
// (attn_pair_gfx906 attn_kernel.hip:313-512 for D=64/128, attn_d512_gfx906
// attn_kernel.hip:525-708 for D=512, attn_tiled_gfx906 attn_kernel.hip:146-308
// for D<64). The reference kernels run on VALU dot2 instructions over
// contiguous fp16; this file is a different design built around CDNA4 matrix
// cores:
//
//  * Scores are computed transposed, S^T = K * Q^T, with
//    v_mfma_f32_16x16x32_{f16,bf16} (the card is power-limited under
//    sustained matrix load, and this form costs less energy per FLOP than
//    the 32x32x16 one). In the 16x16 accumulator layout a lane holds one
//    column (one query row) and 4 keys of each 16-key block, so the
//    online-softmax state is per lane, kept equal over the four lanes that
//    share a query, and row reductions combine four lanes.
//  * The same registers, rounded to the input type, are the B operand of
//    O^T = V^T * P^T. V stays row-major ([key][dim]) in LDS and the A operand
//    is read with ds_read_b64_tr_b16, whose 16-lane transpose hands each lane
//    four keys of one dim; the key order is chosen to match the accumulator
//    layout of S^T.
//  * K and V tiles go from HBM straight into LDS with buffer loads to LDS
//    (no VGPR staging), through a ring of four stages, two tiles ahead of
//    the compute. Rows are XOR-swizzled in 16-byte units so that the QK^T
//    reads (16 keys x one 16-byte unit per 16 lanes) and the transposed V
//    reads (4 keys x 32 bytes per 16 lanes) are free of LDS bank conflicts.
//  * Each wave is software-pipelined over 32-key blocks: the iteration for
//    block j issues the PV MFMAs of block j-1 and the QK^T MFMAs of block
//    j+1 while the VALU turns the scores of block j into P.
//  * Softmax runs in fp32 with exp2 and scale*log2(e) folded into one FMA.
//    P = exp2(s*c - m) is computed with the running max m and tested: when
//    some rounded p exceeds a limit, the block's exact max is taken and O,
//    l and P follow (a wave-uniform branch). D = 128 updates m lazily
//    (limit 2^15: every p stays finite in fp16, and the rescale is skipped
//    on almost every block); D <= 64 keeps the exact running max (limit 1:
//    a row's dominant weight is exactly 1.0); D = 512 uses limit 2^8.
//  * The row sum l is accumulated from the rounded P, so numerator and
//    denominator see the same rounded weights: for D <= 128 on the matrix
//    pipe (one more 16x16x32 MFMA per column block, A = a 0/1 row selector),
//    for D = 512 with v_dot2_f32_{f16,bf16} against 1.0.
//  * D = 512 runs 32 query rows per wave at one wave per SIMD, its O^T
//    accumulator in AGPRs (attn_fwd_d512w), so that each K or V fragment read
//    from LDS feeds two MFMAs.
//  * Output rows are normalised by 1/l and rounded to the input type (RNE),
//    as the reference does for fp16 (attn_kernel.hip:497-511). Rows of a head
//    with Skv == 0 are written as zeros (the reference leaves them unwritten).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <math.h>
#include <type_traits>
#include <algorithm>
#include <mutex>
#include <stdlib.h>

#include "gfx906_amd_attn.h"

namespace {

typedef _Float16 f16;
typedef __bf16 bf16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __fp16 fp16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

#define LDS_AS __attribute__((address_space(3)))

constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale of the D = 128 kernel: a block with some p above this takes
// the exact max.
constexpr float kPLazyLimit = 32768.0f;
// Lazy-rescale threshold of the D = 512 kernel: a tile whose largest p
// exceeds 2^8 takes the exact max.
constexpr float kPmaxLimit = 256.0f;
// sched_group_barrier instruction classes
constexpr int kSgMfma = 0x008, kSgDsRead = 0x100;

// Strides of one tensor in elements: batch, head, sequence, head dim. The
// head dim is contiguous (d == 1) except in the token-contiguous D = 512
// layout (attn_fwd_d512<T, true>).
struct Strides {
    long long b, h, s, d;
};

// Kernel arguments. c = |scale| * log2(e) (at least 1e-30); qsign < 0 for a
// negative scale, applied as negated q.
struct KArgs {
    const void* q;
    const void* k;
    const void* v;
    void* o;
    Strides sq, sk, sv, so;
    int H, Sq, Skv, D;
    float c, qsign;
    // Split key range (kernels instantiated with SPLIT): workgroup split s of
    // nsplit takes keys [s*split_len, (s+1)*split_len) and writes its
    // unnormalised O (fp32) to ws_o[s][bh][row][0..D) and its (m, l) to
    // ws_ml[s][bh][row][0..1]; attn_combine merges them.
    int BH, nsplit, split_len;
    float* ws_o;
    float* ws_ml;
    // Every output row starts 16-byte aligned (o and its batch, head and
    // sequence strides): the D <= 128 kernels then write O through LDS as
    // whole 16-byte pieces of consecutive rows.
    int o16;
    // Load Q through LDS, as K (whole rows), in the D = 64 and 128 kernels:
    // set for q sequence strides up to 2^24 elements and more than 1024 keys
    // for D <= 64, 256 for D = 128 (measured: +1 % north star and c2; at 512
    // keys, with the Q tile prefetched into L2, D = 128 +1.1 % and D = 64 +-0,
    // where before the prefetch the two extra barriers cost more than the
    // gathered global loads).
    int q_lds;
    // Compute units of the device: with the kernel's workgroups per CU, how
    // many workgroups are resident at once (the D = 128 ring kernel and the
    // D <= 64 one with the tile max prefetch the Q tile of the workgroup that
    // starts after them into L2).
    int ncu;
};

#if defined(__HIP_DEVICE_COMPILE__)
// Per-element-type operations: vectors, MFMAs, packed RNE conversion from
// fp32 and a dot2 against (1, 1) accumulating in fp32.
template <class T>
struct Elem;
template <>
struct Elem<f16> {
    using x8 = f16x8;
    using x4 = f16x4;
    using x2 = f16x2;
    static __device__ __forceinline__ f32x4 mma16(x8 a, x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ x2 cvt2(float a, float b) {
        return __builtin_convertvector(f32x2{a, b}, x2);
    }
    static __device__ __forceinline__ float sum2(x2 h, float acc) {
        return __builtin_amdgcn_fdot2(h, x2{(f16)1.0f, (f16)1.0f}, acc, false);
    }
};
template <>
struct Elem<bf16> {
    using x8 = bf16x8;
    using x4 = bf16x4;
    using x2 = bf16x2;
    static __device__ __forceinline__ f32x4 mma16(x8 a, x8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ __forceinline__ x2 cvt2(float a, float b) {
        return __builtin_convertvector(f32x2{a, b}, x2);
    }
    static __device__ __forceinline__ float sum2(x2 h, float acc) {
        return __builtin_amdgcn_fdot2_f32_bf16(h, x2{(bf16)1.0f, (bf16)1.0f}, acc, false);
    }
};

// O^T accumulation of attn_fwd_d512w with the accumulator pinned to AGPRs:
// its 256 accumulator registers fill the AGPR file, and the 128 registers of
// Q and the score accumulators must stay in VGPRs, a split the compiler's
// own register assignment does not find. The instruction is therefore
// written out, and with it the wait states the compiler's hazard recognizer
// inserts around MFMAs it knows of (it does not look into asm):
//  * a VALU write of an operand (P, O at initialisation or after a rescale)
//    needs 2 wait states before the MFMA reads it: agpr_fence2 and
//    vgpr_fence2 below follow those writes, tied to them by data dependence;
//  * a VALU read or write of an MFMA's accumulator registers (the rescale,
//    the epilogue, copies the register allocator places at block
//    boundaries) needs the MFMA to have completed (12 wait states on gfx950
//    for an 8-pass MFMA, 20 for 16 passes): the last MFMA of every tile
//    carries 24 wait states (DRAIN), ahead of the rescale, the epilogue and
//    any copy the register allocator places at the loop's edges (draining
//    only after the last tile instead makes the allocator split O's live
//    ranges around the two forms, with copies right after MFMAs). The asm
//    statements are volatile, so nothing moves between an MFMA and that
//    delay.
// The MFMA's srcA (V from LDS) is ordered by the compiler's lgkmcnt waits,
// which cover inline-asm operands. tests/test_d512w_hazards.py checks the
// compiled kernel for both rules. The fences also tie O (and P) to AGPRs
// (VGPRs) where the kernel's own VALU work touches them, which keeps the
// register allocator from giving O VGPR homes there (it spills otherwise).
template <class T, bool DRAIN = false>
__device__ __forceinline__ void mma16_agpr(f32x4& acc, typename Elem<T>::x8 a,
                                           typename Elem<T>::x8 b) {
    if constexpr (std::is_same<T, f16>::value) {
        if constexpr (DRAIN)
            asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+a"(acc) : "v"(a), "v"(b));
        else
            asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    } else {
        if constexpr (DRAIN)
            asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
                         : "+a"(acc) : "v"(a), "v"(b));
        else
            asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
    }
}
// 2 wait states after a VALU write, before an MFMA reads the registers.
__device__ __forceinline__ void agpr_fence2(f32x4& x) { asm("s_nop 1" : "+a"(x)); }
template <class X8>
__device__ __forceinline__ void vgpr_fence2(X8& x, X8& y) { asm("s_nop 1" : "+v"(x), "+v"(y)); }
// 24 wait states after an MFMA wrote the registers, before a VALU reads them.
__device__ __forceinline__ void agpr_fence24(f32x4& a, f32x4& b, f32x4& c, f32x4& d) {
    asm("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+a"(a), "+a"(b), "+a"(c), "+a"(d));
}

// 16-byte global load of 8 elements.
template <class T>
__device__ __forceinline__ typename Elem<T>::x8 ld_global16(const T* p) {
    return *reinterpret_cast<const typename Elem<T>::x8*>(p);
}

// Workgroup barrier for the LDS ring: this wave's LDS reads and writes are
// complete (lgkmcnt(0)), then s_barrier. __syncthreads() would add a release
// fence that also waits for every load to LDS still in flight (vmcnt(0)),
// which drains the tiles meant to stay in flight across the barrier. Each
// wave first waits for its own part of the tile it needs (vmcnt(n)); the
// barrier then orders every wave's part before the reads that follow. The
// memory clobber keeps the compiler from moving LDS accesses across it
// (the s_waitcnt and s_barrier builtins alone are not memory operations to
// the optimiser).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Three-way max. fmaxf in the default IEEE mode quiets its operands first
// (a v_max_f32 x, x, x per operand not known to come from arithmetic, e.g.
// MFMA results); the IEEE 754-2019 maximum propagates NaN instead and maps
// to gfx950's v_maximum3_f32 with no such step.
__device__ __forceinline__ float max3(float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float max2(float a, float b) {
    return __builtin_elementwise_maximum(a, b);
}

// 16-byte LDS read at a byte address.
template <class T>
__device__ __forceinline__ typename Elem<T>::x8 lds_read16(const char* base, int byte_off) {
    return *(const LDS_AS typename Elem<T>::x8*)((const LDS_AS char*)base + byte_off);
}
// Two transposed 8-byte LDS reads (ds_read_b64_tr_b16: within each 16-lane
// group, lane i gets element i%4 of the 8 bytes read by lanes 4e+i/4) joined
// into one MFMA operand. The read moves 16-bit elements whatever their type.
template <class T>
__device__ __forceinline__ typename Elem<T>::x8 lds_read_tr2(const char* base, int lo_off,
                                                              int hi_off) {
    const fp16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (LDS_AS fp16x4_t*)((LDS_AS char*)base + lo_off));
    const fp16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4f16(
        (LDS_AS fp16x4_t*)((LDS_AS char*)base + hi_off));
    const u32x2 l = __builtin_bit_cast(u32x2, lo), h = __builtin_bit_cast(u32x2, hi);
    return __builtin_bit_cast(typename Elem<T>::x8, u32x4{l[0], l[1], h[0], h[1]});
}

// The lane's index in its wave, computed where it is used: a volatile asm,
// which the compiler can neither hoist out of a loop nor share between uses,
// so nothing holds the value in a register in between (the D <= 64 kernels
// run at their 128-VGPR limit and spilled such values around the main loop).
__device__ __forceinline__ int lane_id_here() {
    int x;
    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(x));
    return x;
}

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
    x = max2(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false,
                                                    false);
    return max2(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Q^T fragment: 8 elements of a query row with the sign flipped for a
// negative scale (exact for fp16 and bf16 alike: bit 15 of each element).
template <class T>
__device__ __forceinline__ typename Elem<T>::x8 q_fragment(const T* p, bool load, unsigned qneg) {
    typename Elem<T>::x8 val = {};
    if (load) val = ld_global16(p);
    return __builtin_bit_cast(typename Elem<T>::x8, __builtin_bit_cast(u32x4, val) ^ qneg);
}

// Q rows of one workgroup through a range-checked buffer descriptor: the
// loads are unconditional (no per-row branch, so the compiler does not merge
// them with a zero value through copies that wait for the data), and rows
// past `valid_rows` or offsets past the range (kQOutOfRange) read as zeros.
// The caller applies the sign of a negative scale later, once the prologue
// waits for its loads anyway: an XOR right after the loads would hold back
// every later load of the prologue behind them.
constexpr unsigned kQOutOfRange = 0x80000000u;
template <class T>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t q_rsrc(const T* row0, int valid_rows,
                                                        long long ss, int D) {
    const int bytes = valid_rows > 0 ? (int)(((valid_rows - 1) * ss + D) * 2) : 0;
    return __builtin_amdgcn_make_buffer_rsrc((void*)row0, 0, __builtin_amdgcn_readfirstlane(bytes),
                                             0x00020000);
}
template <class T>
__device__ __forceinline__ typename Elem<T>::x8 q_load(__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(typename Elem<T>::x8,
                              __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}
template <class X8>
__device__ __forceinline__ void q_negate(X8& f, unsigned qneg) {
    f = __builtin_bit_cast(X8, __builtin_bit_cast(u32x4, f) ^ qneg);
}

// Whether some element of a block's rounded P (two 8-element operands, all
// non-negative) exceeds `lim` or is NaN, in any lane of the wave. The first
// block (running max -1e30, p = inf) always does. A tree of
// v_pk_maximum3_f16 over the eight packed registers (4 instructions), then
// one compare per half. bf16 has no packed maximum; its registers go
// through the same tree read as fp16: non-negative values of either type
// order as their 16-bit patterns, so the fp16 maximum of the patterns is the
// pattern of the bf16 maximum, compared with the limit's bf16 pattern read as
// fp16 (7.0 for 2^15). A bf16 inf or NaN reads as an fp16 NaN, which the
// maximum propagates and the compare flags, as it does every pattern above
// the limit's. (Seven packed 16-bit integer maxima before: bit-identical
// decisions, three more instructions per block.)
template <class T>
__device__ __forceinline__ bool p_above(const typename Elem<T>::x8 (&P)[2], float lim) {
    const u32x4 a = __builtin_bit_cast(u32x4, P[0]), b = __builtin_bit_cast(u32x4, P[1]);
    auto h = [](unsigned u) { return __builtin_bit_cast(f16x2, u); };
    auto mx = [](f16x2 x, f16x2 y) { return __builtin_elementwise_maximum(x, y); };
    const f16x2 x = mx(mx(h(a[0]), h(a[1])), h(a[2]));
    const f16x2 y = mx(mx(h(a[3]), h(b[0])), h(b[1]));
    const f16x2 z = mx(mx(h(b[2]), h(b[3])), x);
    const f16x2 r = mx(y, z);
    f16 lh;
    if constexpr (std::is_same<T, f16>::value)
        lh = (f16)lim;
    else
        lh = __builtin_bit_cast(f16, (bf16)lim);
    return __any(!(r[0] <= lh) || !(r[1] <= lh));
}
#endif

// XOR swizzles of the 16-byte unit index within a row.
//  K: the QK^T read takes one unit from 16 consecutive rows per 16-lane
//     group, so 16 consecutive rows must land on 16 different bank groups.
//  V: the transposed read takes 2 units from 4 consecutive rows per 16-lane
//     group; each half wave (8 rows x 2 units) must cover all 16 bank groups.
template <int NU>
__device__ __forceinline__ int kswz(int r) { return NU >= 16 ? (r & 15) : ((r >> 1) & 7); }
template <int NU>
__device__ __forceinline__ int vswz(int r) { return NU >= 16 ? 2 * (r & 7) : 2 * ((r >> 1) & 3); }

// ---------------------------------------------------------------------------
// D <= 128: software-pipelined waves, 32 query rows each.
//
// The iteration for 32-key block j issues the PV MFMAs of block j-1 and the
// QK^T MFMAs of block j+1 while the VALU turns the scores of block j into P,
// so every stretch of a wave's instruction stream carries matrix and vector
// work (two blocks of S and of P are live).
//
// K/V tiles are 64 keys (two blocks) in a ring of four LDS stages, each
// stage's K and V tiles separate arrays, so that the compiler can tell their
// accesses apart (a read of one array then never waits for loads into
// another), with the four K arrays first: for D = 128 every K read then
// reaches its array through the 16-bit immediate offset of one address
// register, and every V read through one register that holds its address
// plus 64 KiB (no address arithmetic in the loop: NS +1.7 %, c2 +1.7 %,
// together with a scalar clamp of the tile rows). The barrier that opens
// tile w+1 follows the iteration that finished every read of tile w-1, whose
// stage then takes tile w+3: loads run two tiles ahead. Tiles past the end
// are loaded anyway, as zeros (empty buffer range), which keeps every wait
// count static.
//
//   DP  : head dim the tiles are built for (64 or 128; D < 64 is padded)
//   NW  : waves per workgroup
//   OCC : workgroups per CU the register budget is sized for
template <int DP_, int NW_, int OCC_>
struct Cfg {
    static constexpr int DP = DP_, NW = NW_, OCC = OCC_, BN = 64;
    static constexpr int BM = NW * 32;          // query rows per workgroup
    static constexpr int NT = NW * 64;          // threads per workgroup
    static constexpr int NU = DP / 8;           // 16-byte units per row
    static constexpr int RB = DP * 2;           // bytes per LDS row
    static constexpr int TILE = BN * RB;        // bytes of one K (or V) tile
    static constexpr int BLKS = TILE / 1024;    // 1 KB direct-load blocks per tile
    static_assert(BLKS % NW == 0, "tile must split evenly over waves");
    static_assert(DP % 32 == 0 && DP <= 128, "head-dim class");
};

// Per-lane byte offsets of the direct HBM->LDS tile loads. Each wave fills
// whole 1 KB LDS blocks (lane i writes 16-byte unit i of its block) for
// BLKS/NW blocks of each K tile and as many of each V tile. The offsets are
// relative to the tile's first row (rows kss / vss elements apart in HBM)
// and do not change from tile to tile. Units past D (padded head dims) are
// pointed at unit 0 of the row: finite data that meets zero Q columns (K) or
// feeds unused output columns (V).
template <class C, bool PAD>
__device__ __forceinline__ void tile_offsets(int (&koff)[C::BLKS / C::NW],
                                             int (&voff)[C::BLKS / C::NW], int D, int kss,
                                             int vss, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < C::BLKS / C::NW; ++i) {
        const int unit = (wave + i * C::NW) * 64 + lane;
        const int row = unit / C::NU, slot = unit % C::NU;
        int ck = slot ^ kswz<C::NU>(row);
        if (PAD && ck * 8 >= D) ck = 0;
        koff[i] = (row * kss + ck * 8) * 2;
        int cv = slot ^ vswz<C::NU>(row);
        if (PAD && cv * 8 >= D) cv = 0;
        voff[i] = (row * vss + cv * 8) * 2;
    }
}

#if defined(__HIP_DEVICE_COMPILE__)
// Issue the loads of one K (or V) tile starting at key n0 into an LDS stage
// (rows ss elements apart). The buffer descriptor covers exactly the tile's
// valid rows, so rows past Skv read as zeros and nothing outside the tensor
// is touched; a tile that starts at or past Skv has an empty range and fills
// the stage with zeros.
template <class C, class T>
__device__ __forceinline__ void issue_tile(const T* __restrict__ X, int n0, int Skv, int D,
                                           long long ss, char* stage, int wave,
                                           const int (&off)[C::BLKS / C::NW]) {
    // Uniform; written as a min and a select (scalar instructions) rather than
    // a clamp, which is selected as a vector med3 and then needs a
    // readfirstlane; readfirstlane keeps the descriptor in SGPRs either way (a
    // VGPR descriptor would force a waterfall loop around each load).
    const int rows = min(Skv - n0, C::BN);
    const int bytes =
        __builtin_amdgcn_readfirstlane(rows > 0 ? (int)(((rows - 1) * ss + D) * 2) : 0);
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)(X + n0 * ss), 0, bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < C::BLKS / C::NW; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LDS_AS void*)(stage + (wave + i * C::NW) * 1024),
                                                 16, off[i], 0, 0, 0);
}
#endif

// MFMA tiling. Every 32x32 block of S^T = K Q^T and of O^T += V^T P^T is
// computed as four v_mfma_f32_16x16x32 blocks rather than one
// v_mfma_f32_32x32x16: under sustained matrix load the card is
// power-limited, and the 16x16x32 form does the same work for less energy
// (a quarter of the accumulator registers read and written per instruction,
// for half the FLOPs), so the card holds a higher clock (c2: 2.07 against
// 1.88 GHz).
//
// Per wave: 32 query rows as two 16-column blocks nb. Per 32-key block S^T is
// 2 (16-key halves kb) x 2 (nb) accumulators; a lane holds, for query
// 16nb + l%16, keys 16kb + 4(l/16) + 0..3. Those 8 keys, rounded, are the k
// slots 8(l/16)..+7 of the PV step's B operand, and the transposed V^T read
// supplies the same key order, so P never leaves registers. A query's keys
// are spread over four lanes (l%16 + 16j): its running max is kept equal in
// all four, its row sum is kept per lane and added up at the end.
//
// P of one 32-key block for one column block (a lane's 8 scores, keys
// 4g..4g+3 then 16+4g..): p = exp2(s*c + nm) rounded to the element type,
// nm = -(running max). SUM: adds the row-sum contribution, taken from the
// rounded values, to acc (v_dot2 against 1.0); otherwise the row sum comes
// from an MFMA (below).
#if defined(__HIP_DEVICE_COMPILE__)
template <class T, bool SUM>
__device__ __forceinline__ void block_exp(const f32x4& S0, const f32x4& S1,
                                          typename Elem<T>::x8& P, float nm, float c,
                                          float& acc) {
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const f32x4& Sb = e < 4 ? S0 : S1;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[e & 3], c, nm));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[(e & 3) + 1], c, nm));
        const typename Elem<T>::x2 hp = Elem<T>::cvt2(p0, p1);
        P[e] = hp[0];
        P[e + 1] = hp[1];
        if constexpr (SUM) acc = Elem<T>::sum2(hp, acc);
    }
}
#endif

// grid: ceil(Sq / BM) * B*H (* nsplit with SPLIT) workgroups, query tiles of
// one head adjacent (the splits of one query tile adjacent); block: NW*64
// threads. The second launch bound is HIP's minimum waves per SIMD
// (amdgpu_waves_per_eu): OCC workgroups of NW waves over the CU's four SIMDs.
template <class C, bool PAD, class T, bool SPLIT, bool TILEMAX>
__global__ void __launch_bounds__(C::NT, C::OCC * C::NW / 4)
attn_fwd_pipe(const KArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
    using E = Elem<T>;
    using x8 = typename E::x8;
    constexpr int DP = C::DP, NU = C::NU, RB = C::RB, TILE = C::TILE;
    constexpr int NQF = DP / 32;          // Q fragments (32 dims each) per column block
    constexpr int NOB = DP / 16;          // 16-dim output blocks
    constexpr int LPT = C::BLKS / C::NW;  // loads per wave per K (or V) tile
    static_assert(2 * LPT < 16, "vmcnt immediate");
    constexpr int kWaitNext = 0x0F70 | (2 * LPT);  // vmcnt(one tile of loads)
    // The ring: K and V tiles of stage s in ks and vs, eight separate arrays
    // (the compiler then tells loads into one from reads of another apart).
    __shared__ __attribute__((aligned(1024))) char k0[TILE];
    __shared__ __attribute__((aligned(1024))) char k1[TILE];
    __shared__ __attribute__((aligned(1024))) char k2[TILE];
    __shared__ __attribute__((aligned(1024))) char k3[TILE];
    __shared__ __attribute__((aligned(1024))) char v0[TILE];
    __shared__ __attribute__((aligned(1024))) char v1[TILE];
    __shared__ __attribute__((aligned(1024))) char v2[TILE];
    __shared__ __attribute__((aligned(1024))) char v3[TILE];
    // Destination of the Q prefetch below (never read).
    __shared__ __attribute__((aligned(256))) char qpf[C::NW * 256];

    const int Sq = a.Sq, D = a.D;
    const float c = a.c;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    // Work item w = (head, key split, query tile), query tiles consecutive;
    // consecutive items go to one XCD when the grid divides by 8 (the
    // dispatcher deals workgroup w to XCD w % 8), so an XCD's L2 streams the
    // K/V of as few heads as possible (c2 +2 %).
    int w = blockIdx.x;
    if ((gridDim.x & 7) == 0) w = (w & 7) * (int)(gridDim.x >> 3) + (w >> 3);
    const int qt = w % nqt;
    int bh = w / nqt, split = 0;
    if constexpr (SPLIT) {
        split = bh % a.nsplit;
        bh /= a.nsplit;
    }
    const int b = bh / a.H, h = bh - b * a.H;
    // This workgroup's keys: [kv0, kv0 + Skv) of the head.
    const int kv0 = SPLIT ? split * a.split_len : 0;
    const int Skv = SPLIT ? max(0, min(a.Skv - kv0, a.split_len)) : a.Skv;
    const T* Qh = (const T*)a.q + b * a.sq.b + h * a.sq.h;
    const T* Kh = (const T*)a.k + b * a.sk.b + h * a.sk.h + kv0 * a.sk.s;
    const T* Vh = (const T*)a.v + b * a.sv.b + h * a.sv.h + kv0 * a.sv.s;
    T* Oh = (T*)a.o + b * a.so.b + h * a.so.h;
    const int qrow0 = qt * C::BM + wave * 32 + i;  // this lane's rows: qrow0 + 16 nb
    const int ntiles = (Skv + C::BN - 1) / C::BN;

    // Q^T fragments (B operands: column = query 16nb + l%16, k = dims
    // 32s + 8(l/16)..+7). Through LDS (below) when q_lds is set.
    x8 qf[2][NQF];
    const unsigned qneg = a.qsign < 0.f ? 0x80008000u : 0u;
    const bool q_lds = !PAD && a.q_lds && ntiles > 0;
    // Register path: the sign of a negative scale is applied after the
    // prologue's barrier (q_negate below), so that the Q loads overlap the
    // first K/V tiles' instead of being waited for before those are issued.
    if (!q_lds) {
        const int qrows = min(Sq - qt * C::BM, C::BM);
        if ((long long)(C::BM - 1) * a.sq.s * 2 + DP * 2 < (1LL << 31)) {  // (uniform)
            const __amdgpu_buffer_rsrc_t qr =
                q_rsrc(Qh + (long long)qt * C::BM * a.sq.s, qrows, a.sq.s, D);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int s = 0; s < NQF; ++s) {
                    const int d0 = 32 * s + 8 * g, r = wave * 32 + 16 * nb + i;
                    const unsigned off = r < qrows && (!PAD || d0 < D)
                                             ? (unsigned)((r * a.sq.s + d0) * 2)
                                             : kQOutOfRange;
                    qf[nb][s] = q_load<T>(qr, off);
                }
        } else {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int s = 0; s < NQF; ++s) {
                    const int d0 = 32 * s + 8 * g, row = qrow0 + 16 * nb;
                    qf[nb][s] =
                        q_fragment(Qh + row * a.sq.s + d0, row < Sq && (!PAD || d0 < D), 0u);
                }
        }
    }

    f32x4 oacc[NOB][2];
    // Row sums on the matrix pipe: lacc[nb] += A1 * P with A1 = 1 in row 0
    // and 0 elsewhere, so accumulator row 0 (lane l%16 of lane group 0)
    // holds the running sum of the rounded p of query 16nb + l%16. Two
    // 16x16x32 MFMAs per block replace eight v_dot2, which the matrix pipe
    // cannot overlap (measured: +1.5 % north star; D = 64, where they add 12 %
    // of the block's matrix work, +6 % c5 and +1 % c3 with the exact running
    // max below, whose rescales add VALU work).
    constexpr bool kLazy = DP == 128;
    // D <= 64 with TILEMAX: the running max is raised once per 64-key tile,
    // over both its blocks, before the first block's P (short key ranges,
    // where the max rises on most blocks: c3 +7 %, c1 +3 %); without it, once
    // per 32-key block (long key ranges, where it rarely rises and the tile
    // max's wait for the second block's scores costs more: c5 -2 %).
    constexpr bool kTileMax = !kLazy && TILEMAX;
    // Running max of each query column block. D = 128 keeps a lazy one, in
    // log2 units (s*c), raised only when some p exceeds 2^15 (rare after the
    // first blocks: every p stays finite in fp16); it starts at -1e30
    // (finite, so that a masked key, score -inf, gives p = 0). D <= 64 keeps
    // the exact running max, in score units (s), starting at -inf (the first
    // block's scores always exceed it), so that the dominant weight of a
    // row is exactly 1.0 in fp16: with a stale max it carries a rounding
    // error of up to 2^-11 relative, which on sharp rows with |o| near 4 and
    // above (c3: q, k ~ 2 N(0,1), 512 keys) moves the output past the 2e-3
    // bar.
    float m_run[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) oacc[ob][nb] = f32x4{};
        m_run[nb] = kLazy ? -1e30f : -INFINITY;
    }
    f32x4 lacc[2] = {f32x4{}, f32x4{}};
    x8 aone;
#pragma unroll
    for (int e = 0; e < 8; ++e) aone[e] = (T)(i == 0 ? 1.0f : 0.0f);

    if (ntiles > 0) {
        int koff[LPT], voff[LPT];
        tile_offsets<C, PAD>(koff, voff, D, (int)a.sk.s, (int)a.sv.s, wave, lane);
        auto issue = [&](int t, char* kdst, char* vdst) __attribute__((always_inline)) {
            issue_tile<C>(Kh, t * C::BN, Skv, D, a.sk.s, kdst, wave, koff);
            issue_tile<C>(Vh, t * C::BN, Skv, D, a.sv.s, vdst, wave, voff);
        };
        // K (and Q) read: row 16kb + l%16 of a 32-key block, dims 32s + 8(l/16)..
        int kaddr[NQF];
        {
            const int kl = kswz<NU>(i);
#pragma unroll
            for (int s = 0; s < NQF; ++s) kaddr[s] = i * RB + ((4 * s + g) ^ kl) * 16;
        }
        // V^T read (two ds_read_b64_tr_b16): lane 4e + j of group g reads row
        // 4g + e (+16 for the block's second key half), dims 16ob + 4j..+3, so
        // lane l receives dim 16ob + l%16 of keys 4g..4g+3 (16 + 4g..).
        int vaddr[NOB];
        constexpr int kVBias = 4 * TILE >= 65536 ? 65536 : 0;
        {
            const int vrow = 4 * g + (i >> 2);
            const int vx = vswz<NU>(vrow) >> 1;
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) {
                // Held as vaddr + 64 KiB, opaque to the compiler: the V arrays
                // follow the 64 KiB of K arrays (D = 128), so every V read then
                // takes its array's place as an immediate offset from these
                // registers instead of an address add per read and tile.
                vaddr[ob] = vrow * RB + (ob ^ vx) * 32 + (i & 3) * 8 + kVBias;
                asm volatile("" : "+v"(vaddr[ob]));
            }
        }

        // L2 prefetch of the Q tile of the workgroup that starts after this
        // one on the same XCD: with R = CUs x workgroups per CU resident,
        // workgroup blockIdx + R (R a multiple of 8, so the same XCD, whose L2
        // it then reads). Issued in the last group of four key tiles, so the
        // lines arrive while this workgroup finishes, instead of as a burst of
        // every new workgroup's Q loads at once. One dword per 128-byte line,
        // through a range-checked descriptor into a scratch LDS area that is
        // never read: no fault past the tensor, no registers held. Every wave
        // issues exactly one such load whether or not there is a workgroup to
        // prefetch for (then through an empty range: no memory access), since
        // the waits of the group's next two tiles count it.
        auto prefetch_next_q = [&]() __attribute__((always_inline)) {
            const long long resident = (long long)a.ncu * C::OCC;
            const long long nb = (long long)blockIdx.x + resident;
            const long long span = (long long)(C::BM - 1) * a.sq.s * 2 + DP * 2;
            const T* base = (const T*)a.q;
            int bytes = 0, off = 0;
            if (resident > 0 && (resident & 7) == 0 && nb < (long long)gridDim.x &&
                span < (1LL << 31)) {  // (uniform)
                int w2 = (int)nb;
                if ((gridDim.x & 7) == 0) w2 = (w2 & 7) * (int)(gridDim.x >> 3) + (w2 >> 3);
                const int qt2 = w2 % nqt;
                int bh2 = w2 / nqt;
                if constexpr (SPLIT) bh2 /= a.nsplit;
                const int b2 = bh2 / a.H, h2 = bh2 - b2 * a.H;
                const int rows = min(Sq - qt2 * C::BM, C::BM);
                bytes = (int)((rows - 1) * a.sq.s * 2 + D * 2);
                base += b2 * a.sq.b + h2 * a.sq.h + (long long)qt2 * C::BM * a.sq.s;
                constexpr int LPR = DP * 2 / 128;         // 128-byte lines per row
                constexpr int LPW = C::BM * LPR / C::NW;  // lines per wave (64 or 32)
                const int l = wave * LPW + (lane_id_here() & (LPW - 1));
                off = (int)((l / LPR) * a.sq.s * 2) + (l % LPR) * 128;
            }
            const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                (void*)base, 0, __builtin_amdgcn_readfirstlane(bytes), 0x00020000);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LDS_AS void*)(qpf + wave * 256), 4, off,
                                                     0, 0, 0);
        };

        // PV MFMAs left to the QK^T step that follows (see pv; for D = 64,
        // 2 and 4 measured -0.5 and -1.2 % on c5).
        constexpr int kPvTail = DP == 128 ? 4 : 0;
        // S^T of 32-key block blk of the K tile kt.
        auto qk = [&](const char* kt, int blk, f32x4 (&S)[2][2]) __attribute__((always_inline)) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) S[kb][nb] = f32x4{};
#pragma unroll
            for (int s = 0; s < NQF; ++s)
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const x8 kf = lds_read16<T>(kt, kaddr[s] + (32 * blk + 16 * kb) * RB);
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) S[kb][nb] = E::mma16(kf, qf[nb][s], S[kb][nb]);
                }
            // K reads interleaved with the MFMAs: A fragments ahead, then one
            // more per MFMA pair (measured against the compiler's own order:
            // D = 64 with A = 3, +2 % c5; D = 128 with A = 2, +0.8 % north
            // star and c2, where A = 1 lost 4 % and A = 3, 4 did not gain).
            // The first A reads go out while the last kPvTail MFMAs of the
            // PV step before are still to issue (see pv).
            {
                constexpr int A = DP == 64 ? 3 : 2;
                __builtin_amdgcn_sched_group_barrier(kSgDsRead, A, 0);
                if constexpr (kPvTail > 0) __builtin_amdgcn_sched_group_barrier(kSgMfma, kPvTail, 0);
#pragma unroll
                for (int n = 0; n < 2 * NQF - A; ++n) {
                    __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
                    __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 2 * A, 0);
            }
        };
        // O^T += V^T P^T for 32-key block blk of the V tile sv.
        auto pv = [&](const char* sv, int blk, const x8 (&P)[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) {
                const int off = vaddr[ob] - kVBias + 32 * blk * RB;
                const x8 vf = lds_read_tr2<T>(sv, off, off + 16 * RB);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) oacc[ob][nb] = E::mma16(vf, P[nb], oacc[ob][nb]);
            }

            // kVAhead V fragments ahead of the MFMAs that use them, then one
            // more per MFMA pair (measured: +4 % north star against the
            // compiler's own order; D = 128 four ahead, +0.2-0.35 % north star
            // and c2 over three, two ahead -0.7 %). Every PV step is followed
            // by a QK^T step, whose first K reads are placed ahead of this
            // step's last kPvTail MFMAs (D = 128: +1.2 % north star and c2
            // with 4 or 6, -5 % with 8, which also holds back QK^T MFMAs).
            constexpr int kVAhead = DP == 128 ? 4 : 3;  // V fragments, two reads each
            __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2 * kVAhead, 0);
#pragma unroll
            for (int n = 0; n < NOB - kVAhead; ++n) {
                __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
                __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 0);
            }
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 2 * kVAhead - kPvTail, 0);
        };
        // Scores of keys >= Skv (block keys key0..key0+31) to -inf, for the
        // last one or two blocks only.
        // (D <= 64 recomputes the lane's key offset here, see lane_id_here;
        // D = 128 keeps its register, which its code layout is tuned around.)
        auto mask = [&](f32x4 (&S)[2][2], int key0) __attribute__((always_inline)) {
            if constexpr (DP <= 64) {
                if (key0 + 32 > Skv) {
                    const int gm = lane_id_here() >> 4;
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (key0 + 16 * kb + 4 * gm + r >= Skv) S[kb][nb][r] = -INFINITY;
                }
            } else {
                if (key0 + 32 > Skv) {
#pragma unroll
                    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                            for (int r = 0; r < 4; ++r)
                                if (key0 + 16 * kb + 4 * g + r >= Skv) S[kb][nb][r] = -INFINITY;
                }
            }
        };
        // O, l and m of column block nb move to the running max m_new
        // (m_run's units).
        auto rescale = [&](int nb, float m_new) __attribute__((always_inline)) {
            const float alpha =
                __builtin_amdgcn_exp2f(kLazy ? m_run[nb] - m_new : (m_run[nb] - m_new) * c);
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) oacc[ob][nb] *= alpha;
            if constexpr (kLazy)
                lacc[nb] *= alpha;
            else
                lacc[nb][0] *= alpha;  // rows 1-3 of the row-sum accumulator stay 0
            m_run[nb] = m_new;
        };
        auto lane_max = [&](const f32x4 (&S)[2][2], int nb) __attribute__((always_inline)) {
            const float mx = max3(S[0][nb][0], S[0][nb][1], S[0][nb][2]);
            const float my = max3(S[0][nb][3], S[1][nb][0], S[1][nb][1]);
            return max2(max3(mx, S[1][nb][2], S[1][nb][3]), my);
        };
        // The lane's largest score over a whole 64-key tile (blocks S and S2).
        auto lane_max2 = [&](const f32x4 (&S)[2][2], const f32x4 (&S2)[2][2], int nb)
            __attribute__((always_inline)) {
            const float a0 = max3(S[0][nb][0], S[0][nb][1], S[0][nb][2]);
            const float a1 = max3(S[0][nb][3], S[1][nb][0], S[1][nb][1]);
            const float a2 = max3(S[1][nb][2], S[1][nb][3], S2[0][nb][0]);
            const float a3 = max3(S2[0][nb][1], S2[0][nb][2], S2[0][nb][3]);
            const float a4 = max3(S2[1][nb][0], S2[1][nb][1], S2[1][nb][2]);
            return max2(max3(a0, a1, a2), max3(a3, a4, S2[1][nb][3]));
        };
        // P of one 32-key block. Any rescale of O comes after the PV MFMAs
        // issued before this call.
        //  D = 128 (lazy max): P is computed with the running max first and
        //  tested; when some rounded p exceeds 2^15 (rare after the first
        //  blocks) each query takes its exact block max and O, l and P follow
        //  (a wave-uniform branch).
        //  D <= 64 (exact running max, in score units): the lane's largest
        //  score is compared with the running max before any exponential;
        //  when some query's block max rises above it, the queries take their
        //  exact block max and O and l are rescaled, then P is computed once.
        //  Maxima rise often on short key ranges (most blocks of c3), where
        //  computing P first would compute it twice. A dominant key then
        //  gives p = exp2(fma(s, c, -RN(s*c))), within 2^-20 of 1, which
        //  rounds to exactly 1.0.
        auto softmax = [&](f32x4 (&S)[2][2], x8 (&P)[2]) __attribute__((always_inline)) {
            float lp[2];  // unused: the row sums come from the MFMAs below
            if constexpr (kLazy) {
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    block_exp<T, false>(S[0][nb], S[1][nb], P[nb], -m_run[nb], c, lp[nb]);
                if (__builtin_expect(p_above<T>(P, kPLazyLimit), 0)) {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        rescale(nb, max2(m_run[nb], quad_group_max(lane_max(S, nb)) * c));
                        block_exp<T, false>(S[0][nb], S[1][nb], P[nb], -m_run[nb], c, lp[nb]);
                    }
                }
            } else {
                // Each column block moves only when one of its queries' max
                // rose (+0.8 % c3 against moving both together).
                const float lm[2] = {lane_max(S, 0), lane_max(S, 1)};
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    if (__any(lm[nb] > m_run[nb]))
                        rescale(nb, max2(m_run[nb], quad_group_max(lm[nb])));
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    block_exp<T, false>(S[0][nb], S[1][nb], P[nb], -m_run[nb] * c, c, lp[nb]);
            }
            // Row sums of this block's P: issued here, where the wave's
            // stream is mostly VALU work (+0.6 % north star against issuing
            // them with the PV MFMAs), after any rescale of lacc.
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) lacc[nb] = E::mma16(aone, P[nb], lacc[nb]);
        };
        // D <= 64 with TILEMAX: P of a tile's two blocks. The first call (S2,
        // the tile's second block, non-null) raises the running max to the
        // max over both blocks, then computes S's P; the second (S2 null)
        // computes the second block's P with no test. On the workgroup's first
        // tile (`first`, wave-uniform) O and l are still exactly zero and the
        // running max is -inf: the max is raised with no rescale (the rescale
        // would multiply zeros by exp2(-inf) = 0; c3 rescales on most of its
        // eight tiles, so this drops about one in seven).
        auto softmax_tile = [&](f32x4 (&S)[2][2], x8 (&P)[2], const f32x4 (*S2)[2][2],
                                bool first) __attribute__((always_inline)) {
            float lp[2];  // unused: the row sums come from the MFMAs below
            if (S2) {
                const float lm[2] = {lane_max2(S, *S2, 0), lane_max2(S, *S2, 1)};
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
                    if (__any(lm[nb] > m_run[nb])) {
                        const float m_new = max2(m_run[nb], quad_group_max(lm[nb]));
                        if (first)
                            m_run[nb] = m_new;
                        else
                            rescale(nb, m_new);
                    }
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
                block_exp<T, false>(S[0][nb], S[1][nb], P[nb], -m_run[nb] * c, c, lp[nb]);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) lacc[nb] = E::mma16(aone, P[nb], lacc[nb]);
        };

        f32x4 Sa[2][2], Sb[2][2];
        x8 Pa[2], Pb[2];
        Pb[0] = x8{};  // block -1: no keys
        Pb[1] = x8{};

        // Tile w (blocks 2w, 2w+1) in stage cur (K tile kc, V tile vc); vp
        // holds V of tile w-1, kn K of tile w+1; the stage of tile w-1 (kf,
        // vf) takes tile w+3. PF: issue the Q prefetch after tile w+3's loads;
        // EX: one prefetch load younger than tile w+1's loads is in flight
        // (the wait leaves it).
        auto tile = [&](auto pf, auto ex, int w, const char* vp, const char* kc, const char* vc,
                        const char* kn, char* kf, char* vf) __attribute__((always_inline)) {
            constexpr bool PF = decltype(pf)::value;
            constexpr int EX = decltype(ex)::value;
            mask(Sa, w * C::BN);
            pv(vp, 1, Pb);     // block 2w-1
            qk(kc, 1, Sb);     // block 2w+1
            if constexpr (kTileMax) {
                mask(Sb, w * C::BN + 32);
                softmax_tile(Sa, Pa, &Sb, w == 0);  // block 2w, max over blocks 2w and 2w+1
            } else {
                softmax(Sa, Pa);            // block 2w
            }
            __builtin_amdgcn_s_waitcnt(kWaitNext + EX);  // own loads of tile w+1 done
            lds_barrier();                               // every wave's; tile w-1 consumed
            issue(w + 3, kf, vf);
            if constexpr (PF) prefetch_next_q();
            if constexpr (!kTileMax) mask(Sb, w * C::BN + 32);
            pv(vc, 0, Pa);     // block 2w
            qk(kn, 0, Sa);     // block 2w+2
            if constexpr (kTileMax)
                softmax_tile(Sb, Pb, nullptr, false);  // block 2w+1
            else
                softmax(Sb, Pb);                // block 2w+1
        };

        // Prologue: tiles 0 and 1 in flight, stage 3's V zeroed for the PV of
        // block -1 (P = 0, and 0 * garbage could be NaN), tile 2 issued once
        // tile 0 is in, then S of block 0. Q through LDS: the workgroup's 256
        // query rows as four K-shaped tiles of 64 rows (whole rows per load,
        // the K swizzle) in stages 2 and 3, free until tile 2 is issued; each
        // wave then reads its fragments with the QK^T read pattern (query row
        // for key row).
        if constexpr (!PAD) {
            if (q_lds) {
                static_assert(C::BM == 4 * C::BN, "four Q tiles per workgroup");
                static_assert(4 * LPT < 16, "vmcnt immediate");
                int qoff[LPT], qoff_unused[LPT];
                tile_offsets<C, false>(qoff, qoff_unused, D, (int)a.sq.s, (int)a.sq.s,
                                             wave, lane);
#pragma unroll
                for (int m = 0; m < 4; ++m)
                    issue_tile<C>(Qh, qt * C::BM + m * C::BN, Sq, D, a.sq.s,
                                  m == 0 ? k2 : m == 1 ? v2 : m == 2 ? k3 : v3, wave, qoff);
            }
        }
        issue(0, k0, v0);
        issue(1, k1, v1);
        if constexpr (!PAD) {
            if (q_lds) {
                __builtin_amdgcn_s_waitcnt(0x0F70 | (4 * LPT));  // this wave's Q loads landed
                lds_barrier();                                  // every wave's
                const char* qsrc =
                    ((wave >> 1) == 0 ? k2 : (wave >> 1) == 1 ? v2 : (wave >> 1) == 2 ? k3 : v3) +
                    (wave & 1) * 32 * RB;
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int s = 0; s < NQF; ++s) {
                        const x8 f = lds_read16<T>(qsrc, kaddr[s] + 16 * nb * RB);
                        qf[nb][s] = __builtin_bit_cast(x8, __builtin_bit_cast(u32x4, f) ^ qneg);
                    }
                lds_barrier();  // every wave's Q reads are done: stages 2 and 3 are free
            }
        }
        for (int z = tid; z < TILE / 16; z += C::NT)
            *reinterpret_cast<u32x4*>(v3 + 16 * z) = u32x4{};
        __builtin_amdgcn_s_waitcnt(kWaitNext);
        lds_barrier();
        if (!q_lds && qneg) {  // (uniform)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                for (int s = 0; s < NQF; ++s) q_negate(qf[nb][s], qneg);
        }
        issue(2, k2, v2);
        qk(k0, 0, Sa);

        // Whole groups of four tiles (tiles past the end hold zeros and are
        // masked to p = 0); a single exit keeps the loop's register
        // allocation intact. With kPrefetchQ the last group issues the Q
        // prefetch in its first tile; the waits of its next two tiles leave
        // that load in flight, the last tile's wait (for loads issued after
        // it) takes it. Not for D <= 64 without the tile max (long key
        // ranges, where the prefetch would save a negligible share and its
        // second copy of the group makes the kernel spill at 128 VGPRs).
        constexpr bool kPrefetchQ = kLazy || kTileMax;
        using B0 = std::integral_constant<bool, false>;
        using B1 = std::integral_constant<bool, true>;
        using E0 = std::integral_constant<int, 0>;
        using E1 = std::integral_constant<int, 1>;
        for (int w0 = 0;; w0 += 4) {
            if (kPrefetchQ && w0 + 4 >= ntiles) {
                tile(B1{}, E0{}, w0 + 0, v3, k0, v0, k1, k3, v3);
                tile(B0{}, E1{}, w0 + 1, v0, k1, v1, k2, k0, v0);
                tile(B0{}, E1{}, w0 + 2, v1, k2, v2, k3, k1, v1);
                tile(B0{}, E0{}, w0 + 3, v2, k3, v3, k0, k2, v2);
                break;
            }
            tile(B0{}, E0{}, w0 + 0, v3, k0, v0, k1, k3, v3);
            tile(B0{}, E0{}, w0 + 1, v0, k1, v1, k2, k0, v0);
            tile(B0{}, E0{}, w0 + 2, v1, k2, v2, k3, k1, v1);
            tile(B0{}, E0{}, w0 + 3, v2, k3, v3, k0, k2, v2);
            if (!kPrefetchQ && w0 + 4 >= ntiles) break;
        }
        pv(v3, 1, Pb);   // block 2w+1 of the last tile
        // The zero-range loads past the end must land before the workgroup's
        // LDS is released.
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }

    // Lane indices of the epilogue. D <= 64 runs at 128 VGPRs, and values
    // kept from the prologue would hold registers across the main loop (two
    // were spilled around it): they are recomputed from the lane id.
    int lane_e = lane, ie = i, ge = g, qrow0e = qrow0;
    if constexpr (DP <= 64) {
        lane_e = lane_id_here();
        ie = lane_e & 15;
        ge = lane_e >> 4;
        qrow0e = qt * C::BM + wave * 32 + ie;
    }
    if constexpr (SPLIT) {  // unnormalised O and (m, l) of this key range
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int row = qrow0e + 16 * nb;
            const float l = quad_group_sum(lacc[nb][0]);
            if (row < Sq) {
                const long long r = ((long long)split * a.BH + bh) * Sq + row;
                float* wo = a.ws_o + r * D;
#pragma unroll
                for (int ob = 0; ob < NOB; ++ob) {
                    const int d0 = 16 * ob + 4 * ge;
                    if (!PAD || d0 < D) *reinterpret_cast<f32x4*>(wo + d0) = oacc[ob][nb];
                }
                const float m = kLazy ? m_run[nb] : m_run[nb] * c;  // log2 units
                if (ge == 0) *reinterpret_cast<f32x2*>(a.ws_ml + 2 * r) = f32x2{m, l};
            }
        }
        return;
    }
    if (!PAD && a.o16) {
        // O through LDS: each wave writes its rows, in the element type, to a
        // row-major staging area (rows padded by 16 bytes) in the ring it no
        // longer reads, then stores them as 16-byte pieces of consecutive
        // rows. The barrier makes sure every wave is done with the ring.
        constexpr int RS = DP * 2 + 16;   // staging row stride, bytes
        constexpr int CPR = DP * 2 / 16;  // 16-byte pieces per row
        static_assert(32 * RS <= TILE, "a wave's staging per ring array");
        lds_barrier();
        char* const stg = wave == 0 ? k0 : wave == 1 ? k1 : wave == 2 ? k2 : wave == 3 ? k3 :
                          wave == 4 ? v0 : wave == 5 ? v1 : wave == 6 ? v2 : v3;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const float l = quad_group_sum(lacc[nb][0]);
            const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) {
                const int d0 = 16 * ob + 4 * ge;
                const auto h0 = E::cvt2(oacc[ob][nb][0] * inv, oacc[ob][nb][1] * inv);
                const auto h1 = E::cvt2(oacc[ob][nb][2] * inv, oacc[ob][nb][3] * inv);
                *reinterpret_cast<LDS_AS typename E::x4*>(
                    (LDS_AS char*)stg + (16 * nb + ie) * RS + d0 * 2) =
                    typename E::x4{h0[0], h0[1], h1[0], h1[1]};
            }
        }
        const int row0 = qrow0e - ie;  // this wave's first row
#pragma unroll
        for (int j = 0; j < 32 * CPR / 64; ++j) {
            const int cidx = 64 * j + lane_e, r = cidx / CPR, col = cidx - r * CPR;
            const u32x4 val = *reinterpret_cast<const LDS_AS u32x4*>((const LDS_AS char*)stg +
                                                                     r * RS + col * 16);
            if (row0 + r < Sq) {
                // D <= 64: non-temporal stores (O is not read again; c3, whose
                // three rounds of short workgroups store 50 MB, +1.4 %; D = 128
                // mixed, -0.6 % north star, +1 % c2: not used there).
                u32x4* dst = reinterpret_cast<u32x4*>(Oh + (row0 + r) * a.so.s + col * 8);
                if constexpr (DP <= 64)
                    __builtin_nontemporal_store(val, dst);
                else
                    *dst = val;
            }
        }
        return;
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int row = qrow0e + 16 * nb;
        const float l = quad_group_sum(lacc[nb][0]);
        const float inv = l > 0.f ? 1.f / l : 0.f;
        if (row < Sq) {
            T* op = Oh + row * a.so.s;
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) {
                const int d0 = 16 * ob + 4 * ge;
                if (!PAD || d0 < D) {
                    const auto h0 = E::cvt2(oacc[ob][nb][0] * inv, oacc[ob][nb][1] * inv);
                    const auto h1 = E::cvt2(oacc[ob][nb][2] * inv, oacc[ob][nb][3] * inv);
                    *reinterpret_cast<typename E::x4*>(op + d0) =
                        typename E::x4{h0[0], h0[1], h1[0], h1[1]};
                }
            }
        }
    }
#endif
}

// ---------------------------------------------------------------------------
// D <= 64 with a short key range: K and V resident in LDS, persistent
// workgroups.
//
// When a head's whole K and V fit in LDS (up to 10 tiles of 64 keys, 160 KB,
// i.e. Skv <= 640), one workgroup of 16 waves per CU loads them once and runs
// the query tiles assigned to it back to back (512 rows per tile, 32 per
// wave, the same per-wave block pipeline and softmax as attn_fwd_pipe, so
// the results are bit-identical). The main loop issues no loads into LDS and
// no barriers: the waves drift apart, and one wave's Q loads and O stores
// overlap the other waves' matrix work. A barrier is needed only when the
// workgroup moves on to another head's K/V. Workgroup g of G takes query
// tiles [g*n/G, (g+1)*n/G) of the n = B*H*ceil(Sq/512) tiles, head-major.
struct CfgRes {
    static constexpr int DP = 64, NW = 16, BN = 64, BM = NW * 32, NT = NW * 64;
    static constexpr int NU = DP / 8, RB = DP * 2, TILE = BN * RB, STAGE = 2 * TILE;
    static constexpr int MAX_TILES = 10;  // 10 x 16 KB = 160 KB, all of a CU's LDS
};

template <bool PAD, class T>
__global__ void __launch_bounds__(CfgRes::NT, 1) attn_fwd_kvres(const KArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
    using C = CfgRes;
    using Ring = Cfg<64, 8, 2>;  // tile geometry and load offsets shared with the ring kernel
    using E = Elem<T>;
    using x8 = typename E::x8;
    constexpr int DP = C::DP, NU = C::NU, RB = C::RB, TILE = C::TILE, STAGE = C::STAGE;
    constexpr int NQF = DP / 32, NOB = DP / 16;
    static_assert(Ring::TILE == TILE && Ring::BLKS / Ring::NW == 1, "one 1 KB block per wave");
    __shared__ __attribute__((aligned(1024))) char kv[C::MAX_TILES * STAGE];

    const int Sq = a.Sq, D = a.D, Skv = a.Skv;
    const float c = a.c;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    const int ntiles = (Skv + C::BN - 1) / C::BN;
    const long long items = (long long)a.BH * nqt;
    const int first = (int)(items * blockIdx.x / gridDim.x);
    const int last = (int)(items * (blockIdx.x + 1) / gridDim.x);
    const unsigned qneg = a.qsign < 0.f ? 0x80008000u : 0u;

    // Loads of a head's K/V: waves 0-7 fill 1 KB block (wave % 8) of every K
    // tile, waves 8-15 the same block of every V tile; rows past Skv load
    // zeros.
    int koff[1], voff[1];
    tile_offsets<Ring, PAD>(koff, voff, D, (int)a.sk.s, (int)a.sv.s, wave & 7, lane);
    // K (and Q) read: row 16kb + l%16 of a 32-key block, dims 32s + 8(l/16)..
    int kaddr[NQF];
#pragma unroll
    for (int s = 0; s < NQF; ++s) kaddr[s] = i * RB + ((4 * s + g) ^ kswz<NU>(i)) * 16;
    // V^T read (two ds_read_b64_tr_b16), as in attn_fwd_pipe.
    int vaddr[NOB];
    {
        const int vrow = 4 * g + (i >> 2);
        const int vx = vswz<NU>(vrow) >> 1;
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) vaddr[ob] = vrow * RB + (ob ^ vx) * 32 + (i & 3) * 8;
    }

    f32x4 oacc[NOB][2], lacc[2];  // O^T and the row sums (MFMA, row 0), as attn_fwd_pipe
    float m_run[2];               // exact running max in score units, as attn_fwd_pipe for D <= 64
    x8 qf[2][NQF];
    x8 aone;
#pragma unroll
    for (int e = 0; e < 8; ++e) aone[e] = (T)(i == 0 ? 1.0f : 0.0f);

    auto qk = [&](const char* st, int blk, f32x4 (&S)[2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) S[kb][nb] = f32x4{};
#pragma unroll
        for (int s = 0; s < NQF; ++s)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const x8 kf = lds_read16<T>(st, kaddr[s] + (32 * blk + 16 * kb) * RB);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) S[kb][nb] = E::mma16(kf, qf[nb][s], S[kb][nb]);
            }
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, 3, 0);
#pragma unroll
        for (int n = 0; n < 2 * NQF - 3; ++n) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, 6, 0);
    };
    auto pv = [&](const char* st, int blk, const x8 (&P)[2]) __attribute__((always_inline)) {
        const char* sv = st + TILE;
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
            const int off = vaddr[ob] + 32 * blk * RB;
            const x8 vf = lds_read_tr2<T>(sv, off, off + 16 * RB);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) oacc[ob][nb] = E::mma16(vf, P[nb], oacc[ob][nb]);
        }
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, 6, 0);
#pragma unroll
        for (int n = 0; n < NOB - 3; ++n) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRead, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, 6, 0);
    };
    auto mask = [&](f32x4 (&S)[2][2], int key0) __attribute__((always_inline)) {
        if (key0 + 32 > Skv) {
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int nb = 0; nb < 2; ++nb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (key0 + 16 * kb + 4 * (lane_id_here() >> 4) + r >= Skv)
                            S[kb][nb][r] = -INFINITY;
        }
    };
    // The lane's largest score over a whole 64-key tile (blocks S and S2).
    auto lane_max2 = [&](const f32x4 (&S)[2][2], const f32x4 (&S2)[2][2], int nb)
        __attribute__((always_inline)) {
        const float a0 = max3(S[0][nb][0], S[0][nb][1], S[0][nb][2]);
        const float a1 = max3(S[0][nb][3], S[1][nb][0], S[1][nb][1]);
        const float a2 = max3(S[1][nb][2], S[1][nb][3], S2[0][nb][0]);
        const float a3 = max3(S2[0][nb][1], S2[0][nb][2], S2[0][nb][3]);
        const float a4 = max3(S2[1][nb][0], S2[1][nb][1], S2[1][nb][2]);
        return max2(max3(a0, a1, a2), max3(a3, a4, S2[1][nb][3]));
    };
    // As attn_fwd_pipe's softmax for D <= 64: the maximum is taken over the
    // tile's two blocks (S and S2) before the first block's P (S2 non-null)
    // and not again before the second's (S2 null); on an item's first tile
    // (`first`) it is raised with no rescale of the still-zero O and l.
    auto softmax = [&](f32x4 (&S)[2][2], x8 (&P)[2], const f32x4 (*S2)[2][2], bool first)
        __attribute__((always_inline)) {
        float lm[2] = {0.f, 0.f};
        if (S2) {
            lm[0] = lane_max2(S, *S2, 0);
            lm[1] = lane_max2(S, *S2, 1);
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            if (S2 && __any(lm[nb] > m_run[nb])) {
                const float m_new = max2(m_run[nb], quad_group_max(lm[nb]));
                if (!first) {
                    const float alpha = __builtin_amdgcn_exp2f((m_run[nb] - m_new) * c);
#pragma unroll
                    for (int ob = 0; ob < NOB; ++ob) oacc[ob][nb] *= alpha;
                    lacc[nb][0] *= alpha;  // rows 1-3 of the row-sum accumulator stay 0
                }
                m_run[nb] = m_new;
            }
        }
        float lp[2];  // unused: the row sums come from the MFMAs below
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            block_exp<T, false>(S[0][nb], S[1][nb], P[nb], -m_run[nb] * c, c, lp[nb]);
            lacc[nb] = E::mma16(aone, P[nb], lacc[nb]);
        }
    };

    int cur_bh = -1;
    for (int item = first; item < last; ++item) {
        const int bh = item / nqt, qt = item - bh * nqt;
        const int b = bh / a.H, h = bh - b * a.H;
        if (bh != cur_bh) {  // (re)load this head's K/V; wave-uniform, the same in every wave
            if (cur_bh >= 0) lds_barrier();  // every wave is done with the previous head
            cur_bh = bh;
            const T* Kh = (const T*)a.k + b * a.sk.b + h * a.sk.h;
            const T* Vh = (const T*)a.v + b * a.sv.b + h * a.sv.h;
            for (int t = 0; t < ntiles; ++t) {
                if (wave < 8)
                    issue_tile<Ring>(Kh, t * C::BN, Skv, D, a.sk.s, kv + t * STAGE, wave, koff);
                else
                    issue_tile<Ring>(Vh, t * C::BN, Skv, D, a.sv.s, kv + t * STAGE + TILE,
                                     wave - 8, voff);
            }
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's loads landed
            lds_barrier();                      // ... and every wave's
        }
        const T* Qh = (const T*)a.q + b * a.sq.b + h * a.sq.h;
        T* Oh = (T*)a.o + b * a.so.b + h * a.so.h;
        const int qrow0 = qt * C::BM + wave * 32 + i;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
            for (int s = 0; s < NQF; ++s) {
                const int d0 = 32 * s + 8 * g, row = qrow0 + 16 * nb;
                qf[nb][s] = q_fragment(Qh + row * a.sq.s + d0, row < Sq && (!PAD || d0 < D), qneg);
            }
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) oacc[ob][nb] = f32x4{};
            lacc[nb] = f32x4{};
            m_run[nb] = -INFINITY;
        }

        // Block pipeline over the resident tiles, as attn_fwd_pipe's tile():
        // the iteration for block j issues the PV MFMAs of block j-1 and the
        // QK^T MFMAs of block j+1 around the softmax of block j. The QK^T of
        // the block after the last one reads tile 0 and is discarded.
        f32x4 Sa[2][2], Sb[2][2];
        x8 Pa[2], Pb[2];
        if (ntiles > 0) {  // (no keys: the row sums stay 0 and the rows are written as zeros)
        qk(kv, 0, Sa);
        for (int t = 0; t < ntiles; ++t) {
            const char* cur = kv + t * STAGE;
            const char* nxt = t + 1 < ntiles ? cur + STAGE : kv;
            mask(Sa, t * C::BN);
            if (t > 0) pv(cur - STAGE, 1, Pb);  // block 2t-1
            qk(cur, 1, Sb);                     // block 2t+1
            mask(Sb, t * C::BN + 32);
            softmax(Sa, Pa, &Sb, t == 0);       // block 2t (max over 2t, 2t+1)
            pv(cur, 0, Pa);                     // block 2t
            qk(nxt, 0, Sa);                     // block 2t+2
            softmax(Sb, Pb, nullptr, false);    // block 2t+1
        }
        pv(kv + (ntiles - 1) * STAGE, 1, Pb);  // block 2 ntiles - 1
        }

        // (lane indices recomputed here, see lane_id_here)
        const int le = lane_id_here(), ge = le >> 4;
        const int qrow0e = qt * C::BM + wave * 32 + (le & 15);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int row = qrow0e + 16 * nb;
            const float l = quad_group_sum(lacc[nb][0]);
            const float inv = l > 0.f ? 1.f / l : 0.f;
            if (row < Sq) {
                T* op = Oh + row * a.so.s;
#pragma unroll
                for (int ob = 0; ob < NOB; ++ob) {
                    const int d0 = 16 * ob + 4 * ge;
                    if (!PAD || d0 < D) {
                        const auto h0 = E::cvt2(oacc[ob][nb][0] * inv, oacc[ob][nb][1] * inv);
                        const auto h1 = E::cvt2(oacc[ob][nb][2] * inv, oacc[ob][nb][3] * inv);
                        *reinterpret_cast<typename E::x4*>(op + d0) =
                            typename E::x4{h0[0], h0[1], h1[0], h1[1]};
                    }
                }
            }
        }
    }
    // Loads past the end were never issued; nothing is in flight here.
#endif
}

// ---------------------------------------------------------------------------
// D = 512: 16x16x32 MFMA tiles, 16 query rows per wave.
//
// With 32 query rows a wave would need a 256-register O accumulator; with 16
// rows O^T is 32 blocks of 16x16 (128 registers) and two waves fit per SIMD.
// A lane holds 4 keys of each 16-key score block (16x16 accumulator layout:
// rows 4(l/16)..+3, column l%16), so row reductions combine four lanes.
struct Cfg512 {
    static constexpr int DP = 512, NW = 8, BN = 32, BM = NW * 16, NT = NW * 64;
    static constexpr int RB = DP * 2;  // bytes of one K or V row
    // LDS rows are padded instead of swizzled (one direct-load instruction
    // fills exactly one row, so the padding costs nothing). A 1056-byte
    // stride makes both the QK^T read (16 rows, one 16-byte unit each) and
    // the transposed V read (8 rows x 32 bytes per half wave) free of bank
    // conflicts on gfx950 (rocprofv3 SQ_LDS_BANK_CONFLICT = 0 for both
    // patterns; a 1040-byte stride gives the K read 2-way conflicts).
    static constexpr int KS = RB + 32, VS = RB + 32;
    static constexpr int KTILE = BN * KS, VTILE = BN * VS, STAGE = KTILE + VTILE;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int NLD = BN / NW;  // rows loaded per wave per tile, per tensor
};

// Token-contiguous layout (k and v with sequence stride 1, the head dim
// strided: the VAE's [b, c, h*w] activations seen as [b, 1, h*w, c]). A tile
// arrives as K^T and V^T, 512 dim rows of 32 keys (64 bytes, four 16-byte
// key chunks) each, through the same direct loads, 1 KB blocks of 16 dim
// rows. Chunk c of row r sits in slot c ^ tswz(r) of the row in a K^T tile
// and in slot c ^ vswz512(r) in a V^T tile. The keys of the score blocks are
// permuted (tkey) so that each lane's P holds 8 consecutive keys, making a
// V^T fragment one 16-byte read; the transposed K reads of the two 16-lane
// groups served together fall on complementary 8-byte halves of the slots.
// Both read patterns measure free of bank conflicts on gfx950 (rocprofv3
// SQ_LDS_BANK_CONFLICT = 0; the V^T read with the K^T swizzle, or with
// (r >> 2) & 3, has 2-way conflicts).
struct Cfg512T {
    static constexpr int ROWB = Cfg512::BN * 2;    // 64 bytes: one dim row of a tile
    static constexpr int TILE = Cfg512::DP * ROWB;  // 32 KB: K^T or V^T of one tile
    static constexpr int STAGE = 2 * TILE;
    static constexpr int LDS = 2 * STAGE;
    static constexpr int LPW = TILE / 1024 / Cfg512::NW;  // 1 KB loads per wave, tensor, tile
};

// Slot swizzle of the token-contiguous K^T tiles: bit 2 of the row to bit 1 of
// the slot, bit 3 to bit 0.
__host__ __device__ constexpr int tswz(int r) { return (((r >> 2) & 1) << 1) | ((r >> 3) & 1); }
// Slot swizzle of the token-contiguous V^T tiles.
__host__ __device__ constexpr int vswz512(int r) { return (r >> 1) & 3; }
// Key held in row 4j + t of score block kb (j, t < 4) in the token-contiguous
// kernel: lane group g's rows of blocks 0 and 1 are keys 8g..8g+7.
__host__ __device__ constexpr int tkey(int kb, int j, int t) { return 8 * j + 4 * ((j + kb) & 1) + t; }

#if defined(__HIP_DEVICE_COMPILE__)
// Rare path of the D = 512 kernel: the tile's scores exceed the running max by
// more than 8 (log2 units, p > kPmaxLimit). Returns the new max, the rescale
// factor for O and l, and P
// and the tile's row sum recomputed with the new max. Kept out of line (and
// away from O, which stays in registers) so the hot loop does not reserve
// registers for it.
template <class T>
struct Rescale512 {
    typename Elem<T>::x8 P;
    float m, alpha, l_tile;
};
template <class T>
__device__ __attribute__((noinline)) Rescale512<T> d512_rescale(f32x4 S0, f32x4 S1, float m_run,
                                                                float c) {
    float mx = fmaxf(max3(S0[0], S0[1], S0[2]), max3(S0[3], S1[0], S1[1]));
    mx = quad_group_max(max3(mx, S1[2], S1[3])) * c;
    Rescale512<T> r;
    r.m = fmaxf(m_run, mx);
    r.alpha = __builtin_amdgcn_exp2f(m_run - r.m);
    const float nm = -r.m;
    float lsum = 0.f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const f32x4& Sb = u < 2 ? S0 : S1;
        const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1)], c, nm));
        const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1) + 1], c, nm));
        const auto hp = Elem<T>::cvt2(p0, p1);
        r.P[2 * u] = hp[0];
        r.P[2 * u + 1] = hp[1];
        lsum = Elem<T>::sum2(hp, lsum);
    }
    r.l_tile = lsum;
    return r;
}
#endif

// grid: ceil(Sq / 128) * B*H workgroups; block: 512 threads. TL: k and v in
// the token-contiguous layout (Cfg512T), q and o read and written element by
// element with any strides.
template <class T, bool TL, bool SPLIT>
__global__ void __launch_bounds__(Cfg512::NT, 1)
attn_fwd_d512(const KArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
    using C = Cfg512;
    using E = Elem<T>;
    using x8 = typename E::x8;
    constexpr int D = C::DP, BN = C::BN, NLD = C::NLD;
    static_assert(NLD * C::NW == BN && D * 2 == 64 * 16, "one row per load instruction");
    constexpr int NQF = D / 32;  // Q fragments (32 dims each)
    constexpr int NOB = D / 16;  // 16-dim output blocks
    constexpr int STAGE = TL ? Cfg512T::STAGE : C::STAGE;
    constexpr int VOFF = TL ? Cfg512T::TILE : C::KTILE;  // V (V^T) tile within a stage
    __shared__ __attribute__((aligned(1024))) char lds[TL ? Cfg512T::LDS : C::LDS];  // 2 x (K, V)

    const int Sq = a.Sq;
    const float c = a.c;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    int wg = blockIdx.x, split = 0;
    if constexpr (SPLIT) {
        split = wg % a.nsplit;
        wg /= a.nsplit;
    }
    const int bh = wg / nqt;
    const int qt = wg % nqt;
    const int b = bh / a.H, h = bh - b * a.H;
    // This workgroup's keys: [kv0, kv0 + Skv) of the head.
    const int kv0 = SPLIT ? split * a.split_len : 0;
    const int Skv = SPLIT ? max(0, min(a.Skv - kv0, a.split_len)) : a.Skv;
    const T* Qh = (const T*)a.q + b * a.sq.b + h * a.sq.h;
    const T* Kh = (const T*)a.k + b * a.sk.b + h * a.sk.h + kv0 * a.sk.s;
    const T* Vh = (const T*)a.v + b * a.sv.b + h * a.sv.h + kv0 * a.sv.s;
    T* Oh = (T*)a.o + b * a.so.b + h * a.so.h;
    const long long kss = a.sk.s, vss = a.sv.s;
    const int qrow = qt * C::BM + wave * 16 + i;
    const bool live = qrow < Sq;

    auto stage = [&](int t) { return lds + (t & 1) * STAGE; };
    // Direct loads: one instruction per K or V row; lane l fetches dims
    // 8l..8l+7. Rows past Skv read as zeros (the descriptor covers the valid
    // rows only).
    // Token-contiguous layout: lane l of 1 KB block j writes dim row
    // 16j + l/4, slot l%4, so it fetches key chunk tu = (l%4) ^ tswz(row) of
    // K and tv = (l%4) ^ vswz512(row) of V, the same in every block; chunks
    // at or past Skv load zeros. Byte offsets of the lane's rows at key 0
    // (the host keeps them below 2^31).
    const int tu = (lane & 3) ^ ((((lane >> 4) & 1) << 1) | ((lane >> 5) & 1));
    const int tv = (lane & 3) ^ ((lane >> 3) & 3);
    unsigned ktrow[TL ? Cfg512T::LPW : 1], vtrow[TL ? Cfg512T::LPW : 1];
    __amdgpu_buffer_rsrc_t rkt, rvt;
    if constexpr (TL) {
#pragma unroll
        for (int n = 0; n < Cfg512T::LPW; ++n) {
            const long long row = 16 * (wave + n * C::NW) + (lane >> 2);
            ktrow[n] = (unsigned)((row * a.sk.d + 8 * tu) * 2);
            vtrow[n] = (unsigned)((row * a.sv.d + 8 * tv) * 2);
        }
        const int kb = __builtin_amdgcn_readfirstlane((int)(((D - 1) * a.sk.d + Skv) * 2));
        const int vb = __builtin_amdgcn_readfirstlane((int)(((D - 1) * a.sv.d + Skv) * 2));
        rkt = __builtin_amdgcn_make_buffer_rsrc((void*)Kh, 0, kb, 0x00020000);
        rvt = __builtin_amdgcn_make_buffer_rsrc((void*)Vh, 0, vb, 0x00020000);
    }
    auto issue = [&](int t, char* dst) __attribute__((always_inline)) {
        if constexpr (TL) {
            const int k0 = t * BN;
            const bool kin = k0 + 8 * tu < Skv, vin = k0 + 8 * tv < Skv;
#pragma unroll
            for (int n = 0; n < Cfg512T::LPW; ++n) {
                const int blk = wave + n * C::NW;
                const unsigned ok = kin ? ktrow[n] + 2u * (unsigned)k0 : 0xFFFFFFF0u;
                const unsigned ov = vin ? vtrow[n] + 2u * (unsigned)k0 : 0xFFFFFFF0u;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rkt, (LDS_AS void*)(dst + blk * 1024), 16,
                                                         (int)ok, 0, 0, 0);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    rvt, (LDS_AS void*)(dst + Cfg512T::TILE + blk * 1024), 16, (int)ov, 0, 0, 0);
            }
            return;
        }
        const int rows = min(Skv - t * BN, BN);
        const int kbytes = (int)(((rows - 1) * kss + D) * 2);
        const int vbytes = (int)(((rows - 1) * vss + D) * 2);
        const __amdgpu_buffer_rsrc_t rk =
            __builtin_amdgcn_make_buffer_rsrc((void*)(Kh + t * BN * kss), 0, kbytes, 0x00020000);
        const __amdgpu_buffer_rsrc_t rv =
            __builtin_amdgcn_make_buffer_rsrc((void*)(Vh + t * BN * vss), 0, vbytes, 0x00020000);
#pragma unroll
        for (int n = 0; n < NLD; ++n) {
            const int row = wave + n * C::NW;  // wave-uniform
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (LDS_AS void*)(dst + row * C::KS), 16,
                                                     lane * 16, (int)(row * kss * 2), 0, 0);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (LDS_AS void*)(dst + C::KTILE + row * C::VS),
                                                     16, lane * 16, (int)(row * vss * 2), 0, 0);
        }
    };
    const int ntiles = (Skv + BN - 1) / BN;
    if (ntiles > 0) issue(0, stage(0));

    // Q^T fragments (B operand: column = this lane's query, k = dims 32s+8g..).
    x8 qf[NQF];
    const unsigned qneg = a.qsign < 0.f ? 0x80008000u : 0u;
#pragma unroll
    for (int s = 0; s < NQF; ++s) {
        if constexpr (TL) {  // any strides: eight element loads
            x8 val = {};
            if (live)
#pragma unroll
                for (int e = 0; e < 8; ++e) val[e] = Qh[qrow * a.sq.s + (32 * s + 8 * g + e) * a.sq.d];
            qf[s] = __builtin_bit_cast(x8, __builtin_bit_cast(u32x4, val) ^ qneg);
        } else {
            qf[s] = q_fragment(Qh + qrow * a.sq.s + 32 * s + 8 * g, live, qneg);
        }
    }

    // K read: row kb*16 + i, dims 32s + 8g.. ; V^T read (transposed, per
    // 16-lane group g): row 4g + i/4 (+16 for the second key half), dims
    // 16*db + 4*(i%4)..
    const int kbase = i * C::KS + g * 16;
    const int vbase = (4 * g + (i >> 2)) * C::VS + 8 * (i & 3);
    // Token-contiguous layout. K^T read (ds_read_b64_tr_b16, two per
    // fragment, h = 0, 1): lane 4e + j of group g reads keys tkey(kb, j, 0..3)
    // of dim row 32s + 8g + 4h + e (chunk j, half (j + kb) & 1; the row's
    // swizzle is tswz = 2h + g%2), so lane i receives key tkey(kb, i/4, i%4),
    // dims 32s + 8g + 4h + 0..3. V^T read: dim row 16ob + i, keys 8g..8g+7
    // (chunk g), one 16-byte read from slot g ^ vswz512(i).
    int ktb[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
            ktb[h][kb] = (8 * g + 4 * h + (i >> 2)) * Cfg512T::ROWB +
                         (((i & 3) ^ ((h << 1) | (g & 1))) * 16) + (((i & 3) + kb) & 1) * 8;
    const int vtb = i * Cfg512T::ROWB + ((g ^ vswz512(i)) * 16);

    f32x4 oacc[NOB];
#pragma unroll
    for (int ob = 0; ob < NOB; ++ob) oacc[ob] = f32x4{};
    float m_run = -1e30f;  // running max (log2 units); finite so masked keys give p = 0
    float l_run = 0.f;

    // P (B operand of the PV step) from the two score blocks, with running
    // max -nm; pm tracks the largest p.
    auto make_p = [&](const f32x4 (&S)[2], x8& P, float nm, float& lsum, f32x2& pm)
        __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f32x4& Sb = S[u >> 1];
            const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1)], c, nm));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1) + 1], c, nm));
            const auto hp = E::cvt2(p0, p1);
            P[2 * u] = hp[0];
            P[2 * u + 1] = hp[1];
            lsum = E::sum2(hp, lsum);
            pm[u & 1] = max3(pm[u & 1], p0, p1);
        }
    };

    auto tile = [&](int t, char* __restrict__ nxt, const char* __restrict__ cur)
        __attribute__((always_inline)) {
        if (t + 1 < ntiles) issue(t + 1, nxt);
        const char* sk = cur;
        const char* sv = cur + VOFF;
        f32x4 S[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            f32x4 Sp[2] = {f32x4{}, f32x4{}};
#pragma unroll
            for (int s = 0; s < NQF; ++s) {
                x8 kf;
                if constexpr (TL)
                    kf = lds_read_tr2<T>(sk, ktb[0][kb] + s * 32 * Cfg512T::ROWB,
                                         ktb[1][kb] + s * 32 * Cfg512T::ROWB);
                else
                    kf = lds_read16<T>(sk, kbase + kb * 16 * C::KS + s * 64);
                Sp[s & 1] = E::mma16(kf, qf[s], Sp[s & 1]);
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
                for (int r = 0; r < 4; ++r) {
                    const int key = TL ? tkey(kb, g, r) : kb * 16 + 4 * g + r;
                    if (t * BN + key >= Skv) S[kb][r] = -INFINITY;
                }
        }
        if (t == 0) {  // first tile: start from its exact max (O is still zero)
            float mx = fmaxf(max3(S[0][0], S[0][1], S[0][2]), max3(S[0][3], S[1][0], S[1][1]));
            m_run = quad_group_max(max3(mx, S[1][2], S[1][3])) * c;
        }
        x8 P;
        float l_tile = 0.f;
        f32x2 pm = {0.f, 0.f};
        make_p(S, P, -m_run, l_tile, pm);
        const float pmax = fmaxf(pm[0], pm[1]);
        // The O rescale runs on every tile (alpha = 1.0 exactly unless the rare
        // path ran): a conditional in-place rescale of the 128-register
        // accumulator costs more registers than two waves per SIMD allow, while
        // 128 multiplies per tile hide under its 64 MFMAs.
        float alpha = 1.f;
        if (__builtin_expect(__any(!(pmax <= kPmaxLimit)), 0)) {
            const Rescale512<T> r = d512_rescale<T>(S[0], S[1], m_run, c);
            alpha = r.alpha;
            l_run *= r.alpha;
            m_run = r.m;
            P = r.P;
            l_tile = r.l_tile;
        }
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) oacc[ob] *= alpha;
        l_run += l_tile;
        if constexpr (TL) {  // odd lane groups: block 1 holds keys 8g..8g+3
            const u32x4 pw = __builtin_bit_cast(u32x4, P);
            const bool sw = g & 1;
            P = __builtin_bit_cast(x8, u32x4{sw ? pw[2] : pw[0], sw ? pw[3] : pw[1],
                                             sw ? pw[0] : pw[2], sw ? pw[1] : pw[3]});
        }
        // O^T += V^T P^T, one 16x16x32 MFMA per 16-dim block.
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
            x8 vf;
            if constexpr (TL)
                vf = lds_read16<T>(sv, vtb + ob * 16 * Cfg512T::ROWB);
            else
                vf = lds_read_tr2<T>(sv, vbase + 32 * ob, vbase + 32 * ob + 16 * C::VS);
            oacc[ob] = E::mma16(vf, P, oacc[ob]);
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
    if constexpr (SPLIT) {  // unnormalised O and (m, l) of this key range
        if (live) {
            const long long r = ((long long)split * a.BH + bh) * Sq + qrow;
            float* wo = a.ws_o + r * D;
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) *reinterpret_cast<f32x4*>(wo + 16 * ob + 4 * g) = oacc[ob];
            if (g == 0) *reinterpret_cast<f32x2*>(a.ws_ml + 2 * r) = f32x2{m_run, l};
        }
        return;
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (live) {
        T* op = Oh + qrow * a.so.s;
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
            const auto h0 = E::cvt2(oacc[ob][0] * inv, oacc[ob][1] * inv);
            const auto h1 = E::cvt2(oacc[ob][2] * inv, oacc[ob][3] * inv);
            const int d0 = 16 * ob + 4 * g;
            if constexpr (TL) {  // any strides: four element stores
                op[(d0 + 0) * a.so.d] = h0[0];
                op[(d0 + 1) * a.so.d] = h0[1];
                op[(d0 + 2) * a.so.d] = h1[0];
                op[(d0 + 3) * a.so.d] = h1[1];
            } else {
                *reinterpret_cast<typename E::x4*>(op + d0) = typename E::x4{h0[0], h0[1], h1[0], h1[1]};
            }
        }
    }
#endif
}

// ---------------------------------------------------------------------------
// D = 512, wide waves: 32 query rows per wave, one wave per SIMD.
//
// In attn_fwd_d512 (16 rows per wave) every K or V fragment read from LDS
// feeds one MFMA: 1 KB of LDS per 16x16x32 MFMA, more than the LDS delivers
// at the matrix pipe's rate (16-byte reads about 190 bytes per clock per CU,
// the transposed V reads about 120, against 256 needed). Here each fragment
// feeds two MFMAs (one per 16-row column block), halving LDS bytes per FLOP.
// The O^T accumulator (32 rows x 512 dims, fp32) is 256 registers and Q is
// 128, so the wave runs alone on its SIMD (512 registers, the accumulator in
// AGPRs); the D = 512 work per tile (128 MFMAs against 16 exponentials per
// lane) leaves the VALU little to hide behind a second wave.
//
// K and V tiles of 32 keys have two LDS buffers each. The iteration for tile
// t runs the QK^T MFMAs of tile t+1 (K buffer (t+1)&1) in the same basic
// block as the softmax of tile t (scores from the previous iteration), then
// the PV MFMAs of tile t (V buffer t&1); K(t+2) and V(t+1) load meanwhile
// into the buffers the barrier opening the iteration released. Loads past
// the last tile have an empty buffer range and write zeros, so every
// iteration has the same instruction stream.
//
// The arithmetic is attn_fwd_d512's, operation for operation: the same two
// MFMA chains per score block, P, row sums, rescale test (per 16-row column
// block, the rows of one attn_fwd_d512 wave) and O accumulation, so the two
// kernels' outputs are bit-identical.
struct Cfg512W {
    static constexpr int DP = 512, NW = 4, BN = 32, BM = NW * 32, NT = NW * 64;
    static constexpr int KS = Cfg512::KS, VS = Cfg512::VS;  // padded rows (bank-conflict free)
    static constexpr int TILE = BN * KS;                   // one K or V tile
    static constexpr int NLD = BN / NW;                    // rows per wave per tile, per tensor
};
static_assert(Cfg512W::BM == Cfg512::BM, "same query tiling as attn_fwd_d512 (grid, split plan)");

// grid: ceil(Sq / 128) * B*H workgroups (times nsplit); block: 256 threads.
template <class T, bool SPLIT>
__global__ void __launch_bounds__(Cfg512W::NT, 1)
attn_fwd_d512w(const KArgs a) {
#if defined(__HIP_DEVICE_COMPILE__)
    using C = Cfg512W;
    using E = Elem<T>;
    using x8 = typename E::x8;
    constexpr int D = C::DP, BN = C::BN, NLD = C::NLD;
    constexpr int NQF = D / 32;  // Q fragments (32 dims each) per column block
    constexpr int NOB = D / 16;  // 16-dim output blocks
    static_assert(2 * NLD == 16, "prologue wait counts");
    __shared__ __attribute__((aligned(1024))) char kb0[C::TILE];
    __shared__ __attribute__((aligned(1024))) char kb1[C::TILE];
    __shared__ __attribute__((aligned(1024))) char vb0[C::TILE];
    __shared__ __attribute__((aligned(1024))) char vb1[C::TILE];

    const int Sq = a.Sq;
    const float c = a.c;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int i = lane & 15, g = lane >> 4;
    const int nqt = (Sq + C::BM - 1) / C::BM;
    // Workgroup w runs on XCD w % 8 (the dispatcher deals workgroups to the
    // eight XCDs in turn). When the grid divides by 8, consecutive work items
    // go to one XCD, and work items enumerate the query tiles of one K/V range
    // (head, split) consecutively: an XCD's L2 then streams the K/V of as few
    // heads as possible, each tile once for all its workgroups.
    int w = blockIdx.x;
    if ((gridDim.x & 7) == 0) w = (w & 7) * (int)(gridDim.x >> 3) + (w >> 3);
    const int qt = w % nqt;
    int bh = w / nqt, split = 0;
    if constexpr (SPLIT) {
        split = bh % a.nsplit;
        bh /= a.nsplit;
    }
    const int b = bh / a.H, h = bh - b * a.H;
    const int kv0 = SPLIT ? split * a.split_len : 0;
    const int Skv = SPLIT ? max(0, min(a.Skv - kv0, a.split_len)) : a.Skv;
    const T* Qh = (const T*)a.q + b * a.sq.b + h * a.sq.h;
    const T* Kh = (const T*)a.k + b * a.sk.b + h * a.sk.h + kv0 * a.sk.s;
    const T* Vh = (const T*)a.v + b * a.sv.b + h * a.sv.h + kv0 * a.sv.s;
    T* Oh = (T*)a.o + b * a.so.b + h * a.so.h;
    const long long kss = a.sk.s, vss = a.sv.s;
    const int qrow0 = qt * C::BM + wave * 32 + i;  // this lane's rows: qrow0 + 16 rb
    const int ntiles = (Skv + BN - 1) / BN;
    // Direct loads of tile t of X into dst: one instruction per 1 KB row,
    // lane l fetching dims 8l..8l+7 of rows wave + 4n. The descriptor covers
    // the tile's valid rows only (none past the last tile), so the rest read
    // as zeros.
    auto issue = [&](const T* X, long long ss, int t, char* dst) __attribute__((always_inline)) {
        const int rows = min(Skv - t * BN, BN);
        const int bytes = rows > 0 ? (int)(((rows - 1) * ss + D) * 2) : 0;
        const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(X + (rows > 0 ? t * BN * ss : 0)), 0, bytes, 0x00020000);
#pragma unroll
        for (int n = 0; n < NLD; ++n) {
            const int row = wave + n * C::NW;  // wave-uniform
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LDS_AS void*)(dst + row * C::KS), 16,
                                                     lane * 16, (int)(row * ss * 2), 0, 0);
        }
    };

    // Q^T fragments (B operands: column = query 16rb + l%16, k = dims
    // 32s + 8(l/16)..+7).
    // Issue order Q, K(0), V(0), K(1): the prologue waits for the first two.
    // Q goes through a range-checked descriptor where the workgroup's rows
    // span less than 2 GiB; the sign of a negative scale is applied after the
    // prologue's barrier, so that no wait for Q comes before the tiles are
    // issued. (With the predicated fallback for larger spans, the compiler
    // waits for every load in flight before the descriptor loads, so nothing
    // is issued before Q.)
    x8 qf[2][NQF];
    const unsigned qneg = a.qsign < 0.f ? 0x80008000u : 0u;
    if ((long long)(C::BM - 1) * a.sq.s * 2 + D * 2 < (1LL << 31)) {  // (uniform)
        const int qrows = ntiles > 0 ? min(Sq - qt * C::BM, C::BM) : 0;
        const __amdgpu_buffer_rsrc_t qr =
            q_rsrc(Qh + (long long)qt * C::BM * a.sq.s, qrows, a.sq.s, D);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int s = 0; s < NQF; ++s) {
                const int r = wave * 32 + 16 * rb + i;
                const unsigned off =
                    r < qrows ? (unsigned)((r * a.sq.s + 32 * s + 8 * g) * 2) : kQOutOfRange;
                qf[rb][s] = q_load<T>(qr, off);
            }
    } else {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int s = 0; s < NQF; ++s) {
                const int row = qrow0 + 16 * rb;
                qf[rb][s] = q_fragment(Qh + row * a.sq.s + 32 * s + 8 * g, row < Sq && ntiles > 0, 0u);
            }
    }
    // Issued whatever the key count (with no keys the descriptors are empty
    // and the wait after the loop covers them): loads under a condition here
    // make the compiler assume, after the barrier, that the Q loads may be
    // the last ones issued, and wait for V(0) and K(1) in the first QK^T.
    issue(Kh, kss, 0, kb0);
    issue(Vh, vss, 0, vb0);
    issue(Kh, kss, 1, kb1);

    // K read: row 16kb + i, dims 32s + 8g..; V^T read (transposed, per
    // 16-lane group g): rows 4g + i/4 and 16 + 4g + i/4, dims 16ob + 4(i%4)..
    const int kbase = i * C::KS + g * 16;
    const int vbase = (4 * g + (i >> 2)) * C::VS + 8 * (i & 3);

    // S^T = K Q^T of one tile, per column block rb and 16-key block kb, in
    // two MFMA chains (even and odd Q fragments) added at the end.
    // K fragments in flight in the QK^T step: each read is issued six
    // fragments (12 MFMAs, about 190 cycles) ahead of its use, which covers
    // the LDS latency a single wave per SIMD cannot hide otherwise
    // (measured on MI355X against 2, 4, 8 and 10 in flight). The softmax
    // VALU work of the same basic block is left to the scheduler: pinning it
    // between the MFMAs or ahead of them was measured slower.
    constexpr int NKQ = 6;
    auto qk = [&](const char* __restrict__ kt, f32x4 (&S)[2][2]) __attribute__((always_inline)) {
        constexpr int NF = 2 * NQF;  // fragments: 16 per 16-key block
        auto kread = [&](int f) __attribute__((always_inline)) {
            return lds_read16<T>(kt, kbase + (f / NQF) * 16 * C::KS + (f % NQF) * 64);
        };
        x8 kq[NKQ];
#pragma unroll
        for (int j = 0; j < NKQ; ++j) kq[j] = kread(j);
        f32x4 Sp[2][2];
#pragma unroll
        for (int f = 0; f < NF; ++f) {
            const int kb = f / NQF, s = f % NQF;
            if (s == 0) Sp[0][0] = Sp[0][1] = Sp[1][0] = Sp[1][1] = f32x4{};
            const x8 kf = kq[f % NKQ];
            if (f + NKQ < NF) kq[f % NKQ] = kread(f + NKQ);
            Sp[0][s & 1] = E::mma16(kf, qf[0][s], Sp[0][s & 1]);
            Sp[1][s & 1] = E::mma16(kf, qf[1][s], Sp[1][s & 1]);
            if (s == NQF - 1) {
                S[0][kb] = Sp[0][0] + Sp[0][1];
                S[1][kb] = Sp[1][0] + Sp[1][1];
            }
        }
        __builtin_amdgcn_sched_group_barrier(kSgDsRead, NKQ, 0);
#pragma unroll
        for (int f = 0; f < NF - NKQ; ++f) {
            __builtin_amdgcn_sched_group_barrier(kSgMfma, 2, 0);
            __builtin_amdgcn_sched_group_barrier(kSgDsRead, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(kSgMfma, 2 * NKQ, 0);
    };

    // V^T fragment of 16-dim block ob.
    // V^T fragments in flight in the PV step (two transposed reads each; 8
    // measured best against 4 and 6).
    constexpr int NVQ = 8;
    auto vread = [&](const char* vt, int ob) __attribute__((always_inline)) {
        return lds_read_tr2<T>(vt, vbase + 32 * ob, vbase + 32 * ob + 16 * C::VS);
    };

    // P of one column block from its two score blocks, with running max
    // -nm; pm tracks the largest p and lsum sums the rounded p.
    auto make_p = [&](const f32x4 (&S)[2], x8& P, float nm, float& lsum, f32x2& pm)
        __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const f32x4& Sb = S[u >> 1];
            const float p0 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1)], c, nm));
            const float p1 = __builtin_amdgcn_exp2f(fmaf(Sb[2 * (u & 1) + 1], c, nm));
            const auto hp = E::cvt2(p0, p1);
            P[2 * u] = hp[0];
            P[2 * u + 1] = hp[1];
            lsum = E::sum2(hp, lsum);
            pm[u & 1] = max3(pm[u & 1], p0, p1);
        }
    };

    f32x4 oacc[2][NOB];
#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
            oacc[rb][ob] = f32x4{};
            agpr_fence2(oacc[rb][ob]);
        }
    // Running max (log2 units; finite, so masked keys give p = 0) and row sum.
    float m_run[2] = {-1e30f, -1e30f}, l_run[2] = {0.f, 0.f};

    // The last tile's keys past Skv score -inf.
    auto mask_tail = [&](int t, f32x4 (&S)[2][2]) __attribute__((always_inline)) {
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (t * BN + kb * 16 + 4 * g + r >= Skv) S[rb][kb][r] = -INFINITY;
    };

    f32x4 S[2][2];  // scores of the tile the next iteration turns into P
    // Iteration t: scores S of tile t in registers; K(t+1) in kc, V(t) in vc;
    // K(t+2) loads into kf and V(t+1) into vf. P of tile t and the QK^T
    // MFMAs of tile t+1 share a basic block; the rescale test of tile t (a
    // rare branch) follows, then the PV MFMAs of tile t. Interleaving the
    // softmax VALU work with the PV MFMAs instead (a single wave per SIMD
    // issues both) was measured 3 % slower.
    auto iter = [&](int t, char* __restrict__ kf, const char* __restrict__ kc,
                    const char* __restrict__ vc, char* __restrict__ vf) __attribute__((always_inline)) {
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): this wave's K(t+1) and V(t) rows
        lds_barrier();                      // ... every wave's; K(t) and V(t-1) buffers free
        issue(Kh, kss, t + 2, kf);
        issue(Vh, vss, t + 1, vf);
        x8 P[2];
        float lt[2] = {0.f, 0.f};
        f32x2 pm[2] = {{0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) make_p(S[rb], P[rb], -m_run[rb], lt[rb], pm[rb]);
        const bool up0 = __any(!(fmaxf(pm[0][0], pm[0][1]) <= kPmaxLimit));
        const bool up1 = __any(!(fmaxf(pm[1][0], pm[1][1]) <= kPmaxLimit));
        f32x4 Sn[2][2];
        qk(kc, Sn);
        // The first V^T fragments, read before the rare-path branch so that
        // their LDS latency overlaps it.
        x8 vq[NVQ];
#pragma unroll
        for (int j = 0; j < NVQ; ++j) vq[j] = vread(vc, j);
        if (__builtin_expect(up0 || up1, 0)) {
#pragma unroll
            for (int rb = 0; rb < 2; ++rb) {
                if (rb == 0 ? !up0 : !up1) continue;
                // The exact max of the tile's rows; O, l and P follow.
                float mx = fmaxf(max3(S[rb][0][0], S[rb][0][1], S[rb][0][2]),
                                 max3(S[rb][0][3], S[rb][1][0], S[rb][1][1]));
                mx = quad_group_max(max3(mx, S[rb][1][2], S[rb][1][3])) * c;
                const float m_new = fmaxf(m_run[rb], mx);
                const float alpha = __builtin_amdgcn_exp2f(m_run[rb] - m_new);
#pragma unroll
                for (int ob = 0; ob < NOB; ob += 4)
                    agpr_fence24(oacc[rb][ob], oacc[rb][ob + 1], oacc[rb][ob + 2], oacc[rb][ob + 3]);
#pragma unroll
                for (int ob = 0; ob < NOB; ++ob) {
                    oacc[rb][ob] *= alpha;
                    agpr_fence2(oacc[rb][ob]);
                }
                l_run[rb] *= alpha;
                m_run[rb] = m_new;
                lt[rb] = 0.f;
                f32x2 pm2 = {0.f, 0.f};
                make_p(S[rb], P[rb], -m_new, lt[rb], pm2);
            }
        }
        l_run[0] += lt[0];
        l_run[1] += lt[1];
        // O^T += V^T P^T: one V^T fragment per 16-dim block, two MFMAs, with
        // NVQ fragments in flight (the MFMAs are volatile asm, so the LDS
        // reads keep their place in this order).
        vgpr_fence2(P[0], P[1]);
#pragma unroll
        for (int ob = 0; ob < NOB; ++ob) {
            const x8 vfr = vq[ob % NVQ];
            if (ob + NVQ < NOB) vq[ob % NVQ] = vread(vc, ob + NVQ);
            mma16_agpr<T>(oacc[0][ob], vfr, P[0]);
            if (ob + 1 < NOB)
                mma16_agpr<T>(oacc[1][ob], vfr, P[1]);
            else
                mma16_agpr<T, true>(oacc[1][ob], vfr, P[1]);
        }
        if ((t + 2) * BN > Skv) mask_tail(t + 1, Sn);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) S[rb][kb] = Sn[rb][kb];
    };

    if (ntiles > 0) {
        // Prologue: this wave's K(0) rows and Q have landed once at most the
        // 16 loads of V(0) and K(1) are in flight; then every wave's. Scores
        // of tile 0 and their exact max.
        __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16)
        lds_barrier();
        if (qneg) {  // (uniform)
#pragma unroll
            for (int rb = 0; rb < 2; ++rb)
#pragma unroll
                for (int s = 0; s < NQF; ++s) q_negate(qf[rb][s], qneg);
        }
        qk(kb0, S);
        if (BN > Skv) mask_tail(0, S);
#pragma unroll
        for (int rb = 0; rb < 2; ++rb) {
            const float mx = fmaxf(max3(S[rb][0][0], S[rb][0][1], S[rb][0][2]),
                                   max3(S[rb][0][3], S[rb][1][0], S[rb][1][1]));
            m_run[rb] = quad_group_max(max3(mx, S[rb][1][2], S[rb][1][3])) * c;
        }
        for (int t = 0; t < ntiles; t += 2) {
            iter(t, kb0, kb1, vb0, vb1);
            if (t + 1 < ntiles) iter(t + 1, kb1, kb0, vb1, vb0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the (empty) loads past the end

#pragma unroll
    for (int rb = 0; rb < 2; ++rb)
#pragma unroll
        for (int ob = 0; ob < NOB; ob += 4)
            agpr_fence24(oacc[rb][ob], oacc[rb][ob + 1], oacc[rb][ob + 2], oacc[rb][ob + 3]);
    // The output leaves through LDS: each wave writes its 32 rows, in the
    // element type, to a row-major staging area in the ring array of its
    // index (rows padded by 16 bytes), then stores them as whole rows, 1 KB
    // per instruction. A lane's accumulators hold pieces of 16 rows, which
    // stored directly reach memory as 8-byte pieces of 16 rows per
    // instruction (measured on MI355X: 64 workgroups of 128 rows over 128
    // keys 0.0222 -> 0.0182 ms, 8 rounds of them 0.234 -> 0.211 ms, c4
    // +0.7 %). The split path's fp32 partial rows, 64-byte pieces, gained
    // nothing from staging and are stored directly, as is an output whose
    // rows are not 16-byte aligned.
    // The epilogue's addresses derive from the lane index read here, so the
    // compiler cannot compute them ahead of the main loop and keep them live
    // across it (it spilled them otherwise).
    int lane_e = lane;
    asm volatile("" : "+v"(lane_e));
    const int ie = lane_e & 15, ge = lane_e >> 4;
    const int row0 = qt * C::BM + wave * 32;  // this wave's first row
    const bool staged = !SPLIT && a.o16;
    if (staged) lds_barrier();  // every wave is done with the ring
    char* const stg = wave == 0 ? kb0 : wave == 1 ? kb1 : wave == 2 ? vb0 : vb1;
#pragma unroll
    for (int rb = 0; rb < 2; ++rb) {
        const int qrow = row0 + 16 * rb + ie;
        const float l = quad_group_sum(l_run[rb]);
        if constexpr (SPLIT) {  // unnormalised O and (m, l) of this key range
            if (qrow < Sq) {
                const long long r = ((long long)split * a.BH + bh) * Sq + qrow;
                float* wo = a.ws_o + r * D;
#pragma unroll
                for (int ob = 0; ob < NOB; ++ob)
                    *reinterpret_cast<f32x4*>(wo + 16 * ob + 4 * ge) = oacc[rb][ob];
                if (ge == 0) *reinterpret_cast<f32x2*>(a.ws_ml + 2 * r) = f32x2{m_run[rb], l};
            }
        } else if (staged) {
            constexpr int RS = D * 2 + 16;
            static_assert(32 * RS <= C::TILE, "a wave's 32 rows per ring array");
            const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
            for (int ob = 0; ob < NOB; ++ob) {
                const auto h0 = E::cvt2(oacc[rb][ob][0] * inv, oacc[rb][ob][1] * inv);
                const auto h1 = E::cvt2(oacc[rb][ob][2] * inv, oacc[rb][ob][3] * inv);
                *reinterpret_cast<LDS_AS typename E::x4*>(
                    (LDS_AS char*)stg + (16 * rb + ie) * RS + (16 * ob + 4 * ge) * 2) =
                    typename E::x4{h0[0], h0[1], h1[0], h1[1]};
            }
        } else {
            const float inv = l > 0.f ? 1.f / l : 0.f;
            if (qrow < Sq) {
                T* op = Oh + qrow * a.so.s;
#pragma unroll
                for (int ob = 0; ob < NOB; ++ob) {
                    const auto h0 = E::cvt2(oacc[rb][ob][0] * inv, oacc[rb][ob][1] * inv);
                    const auto h1 = E::cvt2(oacc[rb][ob][2] * inv, oacc[rb][ob][3] * inv);
                    *reinterpret_cast<typename E::x4*>(op + 16 * ob + 4 * ge) =
                        typename E::x4{h0[0], h0[1], h1[0], h1[1]};
                }
            }
        }
    }
    if constexpr (!SPLIT) {
        if (staged) {
            constexpr int RS = D * 2 + 16;
            constexpr int CPR = D * 2 / 16;  // 16-byte pieces per row (one per lane)
            static_assert(CPR == 64, "one row per store instruction");
#pragma unroll
            for (int r = 0; r < 32; ++r) {
                const u32x4 val = *reinterpret_cast<const LDS_AS u32x4*>(
                    (const LDS_AS char*)stg + r * RS + lane_e * 16);
                if (row0 + r < Sq)
                    *reinterpret_cast<u32x4*>(Oh + (row0 + r) * a.so.s + lane_e * 8) = val;
            }
        }
    }
#endif
}

// Merge of the split key ranges: per output row, with m* the largest
// running max of its splits and w_s = exp2(m_s - m*),
//     o = sum_s w_s O_s / sum_s w_s l_s
// rounded to the element type. One thread per row and 4 consecutive dims.
// The loads of up to kCombBatch splits go out together before any of them is
// used: a problem small enough to be split leaves few waves per CU, so a loop
// that waited for each split's data in turn would pay one memory latency per
// split. The sums still run over s in ascending order.
constexpr int kCombBatch = 4;
struct CombArgs {
    const float* ws_o;
    const float* ws_ml;
    void* o;
    Strides so;
    int H, Sq, D, BH, nsplit;
};

template <class T>
__global__ void __launch_bounds__(256) attn_combine(const CombArgs c) {
#if defined(__HIP_DEVICE_COMPILE__)
    using E = Elem<T>;
    const int dq = c.D / 4;
    const long long rows = (long long)c.BH * c.Sq;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * dq) return;
    const long long row = idx / dq;
    const int d0 = (int)(idx - row * dq) * 4;
    const int ns = c.nsplit;
    const f32x2* ml = reinterpret_cast<const f32x2*>(c.ws_ml);
    float mx = -3.0e38f;
    for (int s0 = 0; s0 < ns; s0 += 2 * kCombBatch) {
        float m[2 * kCombBatch];
#pragma unroll
        for (int u = 0; u < 2 * kCombBatch; ++u)
            if (s0 + u < ns) m[u] = ml[(s0 + u) * rows + row][0];
#pragma unroll
        for (int u = 0; u < 2 * kCombBatch; ++u)
            if (s0 + u < ns) mx = fmaxf(mx, m[u]);
    }
    f32x4 acc = {};
    float l = 0.f;
    for (int s0 = 0; s0 < ns; s0 += kCombBatch) {
        f32x2 mlv[kCombBatch];
        f32x4 ov[kCombBatch];
#pragma unroll
        for (int u = 0; u < kCombBatch; ++u)
            if (s0 + u < ns) {
                const long long r = (s0 + u) * rows + row;
                mlv[u] = ml[r];
                ov[u] = *reinterpret_cast<const f32x4*>(c.ws_o + r * c.D + d0);
            }
#pragma unroll
        for (int u = 0; u < kCombBatch; ++u)
            if (s0 + u < ns) {
                const float w = __builtin_amdgcn_exp2f(mlv[u][0] - mx);
                acc += w * ov[u];
                l += w * mlv[u][1];
            }
    }
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const auto h0 = E::cvt2(acc[0] * inv, acc[1] * inv);
    const auto h1 = E::cvt2(acc[2] * inv, acc[3] * inv);
    const int bh = (int)(row / c.Sq), srow = (int)(row - (long long)bh * c.Sq);
    const int b = bh / c.H, h = bh - b * c.H;
    T* op = (T*)c.o + b * c.so.b + h * c.so.h + srow * c.so.s + d0 * c.so.d;
    if (c.so.d == 1 && (reinterpret_cast<uintptr_t>(op) & 7) == 0) {
        *reinterpret_cast<typename E::x4*>(op) = typename E::x4{h0[0], h0[1], h1[0], h1[1]};
    } else {
        op[0] = h0[0];
        op[c.so.d] = h0[1];
        op[2 * c.so.d] = h1[0];
        op[3 * c.so.d] = h1[1];
    }
#endif
}

thread_local char g_err[256];

void set_err(const char* msg) {
    int i = 0;
    for (; msg[i] && i < 255; ++i) g_err[i] = msg[i];
    g_err[i] = 0;
}

using Cfg128 = Cfg<128, 8, 1>;  // 128 KB of LDS: one workgroup, two waves per SIMD
using Cfg64 = Cfg<64, 8, 2>;    // 64 KB: two workgroups, four waves per SIMD

int cu_count();

// Query tiles of the K/V-resident kernel.
long long kvres_items(const KArgs& a) {
    return (long long)a.BH * ((a.Sq + CfgRes::BM - 1) / CfgRes::BM);
}

// Workgroups for attn_fwd_kvres on an unsplit D <= 64 problem, or 0 when the
// ring kernel serves it. The resident kernel needs the head's K/V to fit in
// LDS (1 <= Skv <= 640) and, by default, at least as many 512-row query tiles
// as CUs (fewer leave CUs idle; the ring kernel, split if need be, spreads
// such problems wider); it then runs one workgroup per CU. The environment
// variable GFX906_AMD_ATTN_KVRES overrides the choice for tests: 0 = ring
// kernel, 1 = resident kernel whatever the tile count, n > 1 = resident
// kernel on at most n workgroups (several tiles, and heads, per workgroup).
long long kvres_grid(const KArgs& a) {
    if (a.D > 64 || a.Skv < 1 || a.Skv > CfgRes::MAX_TILES * CfgRes::BN) return 0;
    const long long items = kvres_items(a), cus = cu_count();
    const char* env = getenv("GFX906_AMD_ATTN_KVRES");
    const long long force = env ? atoll(env) : -1;
    if (force == 0) return 0;
    if (force == 1) return std::min(items, cus);
    if (force > 1) return std::min(items, force);
    // The ring kernel runs whole groups of four 64-key tiles: with a multiple
    // of four tiles it is the faster of the two (c3, 8 tiles: 0.076 against
    // 0.082 ms on MI355X); otherwise its padding tiles cost more than the
    // resident kernel saves (2 x 16 x 4096 queries, 77 keys: 0.018 against
    // 0.014 ms; 640 keys: 0.109 against 0.100 ms).
    const int ntiles = (a.Skv + CfgRes::BN - 1) / CfgRes::BN;
    return items >= cus && ntiles % 4 ? cus : 0;
}

// D = 512 with row-contiguous K/V runs attn_fwd_d512w (32 rows per wave);
// GFX906_AMD_ATTN_D512W=0 selects attn_fwd_d512 (16 rows per wave) instead,
// for tests (the two are bit-identical).
bool d512_wide() {
    const char* env = getenv("GFX906_AMD_ATTN_D512W");
    return !(env && env[0] == '0' && env[1] == 0);
}

// D <= 64 ring kernel: keys per workgroup up to which the running max is
// raised once per 64-key tile (attn_fwd_pipe's TILEMAX). Measured on MI355X
// against the per-block max (interleaved): c3 (512 keys) +7 %, c1 +3 %,
// 4096 keys +2.4 %, c5 (131072 keys) -2 %. The K/V-resident kernel (at most
// 640 keys) always does, and so matches the ring kernel bit for bit. The
// environment variable GFX906_AMD_ATTN_TILEMAX=0/1 forces either (tests).
constexpr int kTileMaxKeys = 8192;
bool tile_max(int keys) {
    const char* env = getenv("GFX906_AMD_ATTN_TILEMAX");
    if (env && (env[0] == '0' || env[0] == '1') && env[1] == 0) return env[0] == '1';
    return keys <= kTileMaxKeys;
}

template <class T, bool SPLIT>
void launch_kernel(const KArgs& a, unsigned nwg, bool tl, hipStream_t s) {
    const int D = a.D;
    if (D == 512) {
        dim3 grid((unsigned)((a.Sq + Cfg512::BM - 1) / Cfg512::BM) * nwg);
        if (tl)
            hipLaunchKernelGGL((attn_fwd_d512<T, true, SPLIT>), grid, dim3(Cfg512::NT), 0, s, a);
        else if (d512_wide())
            hipLaunchKernelGGL((attn_fwd_d512w<T, SPLIT>), grid, dim3(Cfg512W::NT), 0, s, a);
        else
            hipLaunchKernelGGL((attn_fwd_d512<T, false, SPLIT>), grid, dim3(Cfg512::NT), 0, s, a);
    } else if (D == 128) {
        dim3 grid((unsigned)((a.Sq + Cfg128::BM - 1) / Cfg128::BM) * nwg);
        hipLaunchKernelGGL((attn_fwd_pipe<Cfg128, false, T, SPLIT, false>), grid, dim3(Cfg128::NT),
                           0, s, a);
    } else {
        if constexpr (!SPLIT) {
            if (const long long wgs = kvres_grid(a)) {
                const dim3 grid((unsigned)wgs);
                if (D == 64)
                    hipLaunchKernelGGL((attn_fwd_kvres<false, T>), grid, dim3(CfgRes::NT), 0, s, a);
                else
                    hipLaunchKernelGGL((attn_fwd_kvres<true, T>), grid, dim3(CfgRes::NT), 0, s, a);
                return;
            }
        }
        dim3 grid((unsigned)((a.Sq + Cfg64::BM - 1) / Cfg64::BM) * nwg);
        const bool tm = tile_max(SPLIT ? a.split_len : a.Skv);
        if (D == 64 && tm)
            hipLaunchKernelGGL((attn_fwd_pipe<Cfg64, false, T, SPLIT, true>), grid, dim3(Cfg64::NT),
                               0, s, a);
        else if (D == 64)
            hipLaunchKernelGGL((attn_fwd_pipe<Cfg64, false, T, SPLIT, false>), grid,
                               dim3(Cfg64::NT), 0, s, a);
        else if (tm)
            hipLaunchKernelGGL((attn_fwd_pipe<Cfg64, true, T, SPLIT, true>), grid, dim3(Cfg64::NT),
                               0, s, a);
        else
            hipLaunchKernelGGL((attn_fwd_pipe<Cfg64, true, T, SPLIT, false>), grid, dim3(Cfg64::NT),
                               0, s, a);
    }
}

// Launches the kernel for the whole problem, or (a.nsplit > 1) its split
// key ranges and the merge.
template <class T>
hipError_t launch_t(const KArgs& a, bool tl, hipStream_t s) {
    if (a.nsplit <= 1) {
        launch_kernel<T, false>(a, (unsigned)a.BH, tl, s);
        return hipGetLastError();
    }
    launch_kernel<T, true>(a, (unsigned)a.BH * (unsigned)a.nsplit, tl, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    CombArgs c;
    c.ws_o = a.ws_o;
    c.ws_ml = a.ws_ml;
    c.o = a.o;
    c.so = a.so;
    c.H = a.H;
    c.Sq = a.Sq;
    c.D = a.D;
    c.BH = a.BH;
    c.nsplit = a.nsplit;
    const long long threads = (long long)a.BH * a.Sq * (a.D / 4);
    hipLaunchKernelGGL((attn_combine<T>), dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s,
                       c);
    return hipGetLastError();
}

// Number of CUs of the current device.
int cu_count() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
        return 256;
    return n;
}

// Split of the key range for problems whose grid leaves CUs idle (fewer
// workgroups than slots: one per CU for D = 128 and 512, two for D <= 64),
// with at least four key tiles per split. The count minimises an estimate of
// the run time in tile times of one workgroup: rounds of workgroups over the
// slots x (tiles per split, rounded up to the kernel's loop step: four tiles
// for D <= 128, two for D = 512, + kSplitFixedTiles for a workgroup's prologue
// and epilogue), x kSplitAloneRate when a D <= 64 round leaves every CU one
// workgroup (its tiles then run faster), plus the HBM traffic of the partial
// results (fp32 O written by the split kernel and read back by attn_combine)
// at kSplitTileBytes per tile time. The constants are fitted to interleaved
// timings on the MI355X. Filling the slots exactly is what matters most: one
// D = 512 head of 9216 queries (72 query tiles) in 4 splits is 288
// workgroups, two rounds for 1.125 rounds of work; 3 splits run in one and
// take 0.187 instead of 0.287 ms.
constexpr double kSplitFixedTiles = 2.0;
constexpr double kSplitAloneRate = 0.7;
constexpr double kSplitTileBytes = 11.0e6;
struct SplitPlan {
    int nsplit, split_len;
};
size_t split_ws_bytes(const SplitPlan& p, int B, int H, int Sq, int D);
// ws_cap bounds the workspace of the chosen plan (the static scratch's size
// for callers that pass none); counts whose partial results do not fit are
// skipped, down to no split at all. GFX906_AMD_ATTN_NSPLIT=n (tests) asks
// for n key ranges instead of the estimate's choice, on any grid: as many
// as there are key tiles at most, fewer where n does not divide them into
// non-empty ranges of whole tiles (the same rule as below), and no split
// when n = 1 or when the partial results would not fit ws_cap.
SplitPlan plan_split(int B, int H, int Sq, int Skv, int D, size_t ws_cap = (size_t)-1) {
    const int bm = D == 512 ? Cfg512::BM : (D == 128 ? Cfg128::BM : Cfg64::BM);
    const int bn = D == 512 ? Cfg512::BN : Cfg128::BN;
    const int per_cu = D == 512 || D == 128 ? 1 : 2;
    const long long units = (long long)B * H * ((Sq + bm - 1) / bm);
    if (Skv == 0 || units == 0) return {1, 0};
    const int tiles = (Skv + bn - 1) / bn;
    if (const char* env = getenv("GFX906_AMD_ATTN_NSPLIT")) {
        const long long n = atoll(env);
        if (n >= 1) {
            const int per = (int)((tiles + std::min<long long>(n, tiles) - 1) /
                                  std::min<long long>(n, tiles));
            const SplitPlan p{(tiles + per - 1) / per, per * bn};
            return p.nsplit > 1 && split_ws_bytes(p, B, H, Sq, D) <= ws_cap ? p : SplitPlan{1, 0};
        }
    }
    const long long slots = (long long)cu_count() * per_cu;
    if (units >= slots) return {1, 0};
    const double partial_bytes = 2.0 * B * H * (double)Sq * D * 4;  // per split
    const long long cus = cu_count();
    const int step = D == 512 ? 2 : 4;
    auto estimate = [&](int ns, int per) {
        const long long wgs = units * ns, rounds = (wgs + slots - 1) / slots;
        const double rate = per_cu == 2 && wgs <= cus ? kSplitAloneRate : 1.0;
        const int run = (per + step - 1) / step * step;
        return rounds * (run + kSplitFixedTiles) * rate +
               (ns > 1 ? ns * partial_bytes / kSplitTileBytes : 0.0);
    };
    SplitPlan best{1, 0};
    double best_t = estimate(1, tiles);
    // The search stops at eight times the count that fills the slots once
    // (eight rounds of workgroups), and at 1024 splits (a few microseconds of
    // host time per call at most).
    const long long fill = (slots + units - 1) / units;
    const int max_ns = (int)std::min<long long>(std::min<long long>(tiles / 4, 8 * fill), 1024);
    for (int ns = 2; ns <= max_ns; ++ns) {
        const int per = (tiles + ns - 1) / ns;  // tiles per split
        if ((tiles + per - 1) / per != ns) continue;  // would leave a split empty
        if (split_ws_bytes({ns, per * bn}, B, H, Sq, D) > ws_cap) break;  // grows with ns
        const double t = estimate(ns, per);
        if (t < best_t) {
            best_t = t;
            best = {ns, per * bn};
        }
    }
    return best;
}

size_t split_ws_bytes(const SplitPlan& p, int B, int H, int Sq, int D) {
    if (p.nsplit <= 1) return 0;
    const size_t rows = (size_t)p.nsplit * B * H * Sq;
    return rows * D * 4 + rows * 2 * 4 + 16;
}

// Whether two elements of an output tensor can share an address: the
// (stride, size) pairs of its four dims, sorted by stride, must each step
// past everything the smaller ones span. Dims of size 1 are ignored.
bool output_overlaps(const Strides& s, int B, int H, int Sq, int D) {
    long long st[4] = {s.b, s.h, s.s, s.d};
    long long n[4] = {B, H, Sq, D};
    for (int i = 0; i < 4; ++i)
        for (int j = i + 1; j < 4; ++j)
            if (st[j] < st[i]) {
                long long t = st[i];
                st[i] = st[j];
                st[j] = t;
                t = n[i];
                n[i] = n[j];
                n[j] = t;
            }
    long long extent = 1;
    for (int i = 0; i < 4; ++i) {
        if (n[i] <= 1) continue;
        if (st[i] < extent) return true;
        extent = st[i] * (n[i] - 1) + extent;
    }
    return false;
}

// Whether k and v use the token-contiguous D = 512 layout: sequence stride 1
// (so a 32-key run of one dim is 64 contiguous bytes) and a strided head dim.
bool token_contiguous(const Strides& sk, const Strides& sv, int D) {
    return D == 512 && sk.s == 1 && sv.s == 1 && sk.d != 1 && sv.d != 1;
}

int fail(const char* msg) {
    set_err(msg);
    return 1;
}

// Validates the arguments; returns 0, or 1 with the error message set.
int check_args(const void* q, const void* k, const void* v, void* o, int B, int H, int Sq,
               int Skv, int D, int dtype, const Strides& sq, const Strides& sk,
               const Strides& sv, const Strides& so) {
    if (B < 0 || H < 0 || Sq < 0 || Skv < 0) return fail("attn: negative size");
    if (!((D <= 64 && D > 0 && D % 8 == 0) || D == 128 || D == 512))
        return fail("attn: head_dim must be <=64 and a multiple of 8, or 128, or 512");
    if (dtype != ATTN_DTYPE_F16 && dtype != ATTN_DTYPE_BF16)
        return fail("attn: dtype must be ATTN_DTYPE_F16 or ATTN_DTYPE_BF16");
    // One workgroup per (batch, head, query tile) in grid.x; HIP bounds
    // grid.x * block size by 2^32 (512 threads per workgroup; query tiles
    // of 128 rows for D = 512, 256 otherwise).
    if ((long long)B * H * ((Sq + (D == 512 ? 127 : 255)) / (D == 512 ? 128 : 256)) * 512 >=
        (1LL << 32))
        return fail("attn: grid too large");
    if (B == 0 || H == 0 || Sq == 0) return 0;
    if (!q || !o || (Skv > 0 && (!k || !v))) return fail("attn: null pointer");
    const Strides* all[4] = {&sq, &sk, &sv, &so};
    for (const Strides* s : all)
        if (s->b < 0 || s->h < 0 || s->s < 0 || s->d < 0)
            return fail("attn: strides must be non-negative");
    if (token_contiguous(sk, sv, D)) {
        // k, v: direct loads of 16-byte key runs; q, o: element access.
        const Strides* kv[2] = {&sk, &sv};
        for (const Strides* s : kv)
            if (s->b % 8 || s->h % 8 || s->d % 8)
                return fail("attn: token-contiguous k/v need batch/head/dim strides that are "
                            "multiples of 8 elements");
        if (((uintptr_t)k | (uintptr_t)v) % 16 || ((uintptr_t)q | (uintptr_t)o) % 2)
            return fail("attn: token-contiguous k/v must be 16-byte aligned");
        if (Skv % 8) return fail("attn: token-contiguous k/v need Skv % 8 == 0");
        if ((long long)(D - 1) * sk.d + Skv >= (1LL << 30) ||
            (long long)(D - 1) * sv.d + Skv >= (1LL << 30))
            return fail("attn: token-contiguous k/v span 2^30 elements or more per head");
        if (output_overlaps(so, B, H, Sq, D)) return fail("attn: o strides make output elements overlap");
        return 0;
    }
    if (sq.d != 1 || sk.d != 1 || sv.d != 1 || so.d != 1)
        return fail("attn: the head dim must be contiguous (stride 1), except for D == 512 with "
                    "token-contiguous k and v");
    // 16-byte vector loads of q, k, v and 8-byte stores of o.
    const Strides* in[3] = {&sq, &sk, &sv};
    for (const Strides* s : in)
        if (s->b % 8 || s->h % 8 || s->s % 8)
            return fail("attn: q/k/v strides must be non-negative multiples of 8 elements");
    if (so.b % 4 || so.h % 4 || so.s % 4)
        return fail("attn: o strides must be non-negative multiples of 4 elements");
    if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)v) % 16 || (uintptr_t)o % 8)
        return fail("attn: q/k/v must be 16-byte and o 8-byte aligned");
    // K/V tile offsets and buffer ranges are 32-bit: 64 rows of the sequence
    // stride must stay below 2^31 bytes.
    if (sk.s > (1 << 24) || sv.s > (1 << 24))
        return fail("attn: k/v sequence stride above 2^24 elements");
    if (output_overlaps(so, B, H, Sq, D)) return fail("attn: o strides make output rows overlap");
    return 0;
}

Strides contiguous(int H, int S, int D) {
    return Strides{(long long)H * S * D, (long long)S * D, D, 1};
}

}  // namespace

extern "C" const char* attn_last_error(void) { return g_err[0] ? g_err : nullptr; }

namespace {

// Workspace of the calls that split without a caller workspace
// (attn_fwd_split_static, and launch() / attn_fwd() for grids too small for
// the GPU): the split-key partial results live in this file-scope device
// array. It is part of the library's code object, so every GPU on which any
// kernel of the library is loaded holds its own copy (kScratchBytes) until
// the process ends, whether or not a call ever uses it. Host code must not
// pass `scratch` itself to a kernel (on the host it names a stand-in, not
// device memory): it uses the device address that hipGetSymbolAddress
// returns, looked up once per device. The kernels write every workspace
// entry the merge reads within the same call, so nothing is cleared between
// calls.
//
// Calls that use the array are ordered on the GPU, whatever streams they are
// issued on: each records `done` on its stream after its kernels, and a call
// on another stream first makes its stream wait for that event (the host
// lock keeps wait, launches and record of one call together, so the calls
// form one chain per device). A call made under stream capture neither
// waits nor records (an event recorded outside the graph cannot order its
// replays): a graph that contains one is ordered only by the stream it is
// launched on, and must not run concurrently with other calls that use the
// array on that device.
constexpr size_t kScratchBytes = size_t(96) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
struct DevScratch {
    void* ptr;           // device address of `scratch`
    hipEvent_t done;     // recorded after the last call outside capture that used it
    hipStream_t last;    // the stream of that call
    bool recorded;
};
std::mutex g_scratch_mu;
DevScratch g_scratch[kMaxDevices];

// Device of `stream` (the current device for the null stream), or -1 with
// the error message set.
int stream_device(hipStream_t stream) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess && stream) e = hipStreamGetDevice(stream, &dev);
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        return -1;
    }
    if (dev < 0 || dev >= kMaxDevices) {
        set_err("attn: device index beyond the scratch table");
        return -1;
    }
    return dev;
}

// Looks up `scratch` on device dev and creates its ordering event, once.
// Caller holds g_scratch_mu. Returns 0, or 2 with the error message set.
int scratch_setup(int dev) {
    DevScratch& d = g_scratch[dev];
    if (d.ptr) return 0;
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e == hipSuccess && dev != cur) e = hipSetDevice(dev);
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        return 2;
    }
    void* p = nullptr;
    hipEvent_t ev = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && !p) e = hipErrorInvalidSymbol;
    // The event only orders kernels of this device on two of its streams
    // (hipStreamWaitEvent); nothing on the host or on another device inspects
    // it, so its record needs no system-scope fence: the kernels' own release
    // at their end makes the scratch visible to the device's later kernels.
    // Without the fence a call that splits costs about 2 us less of GPU time
    // (measured on MI355X: B1 H1 S1024 D64 through launch() 16.3 -> 14.5 us).
    if (e == hipSuccess)
        e = hipEventCreateWithFlags(&ev, hipEventDisableTiming | hipEventDisableSystemFence);
    if (dev != cur) {
        const hipError_t r = hipSetDevice(cur);
        if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) {
        if (ev) (void)hipEventDestroy(ev);
        set_err(hipGetErrorString(e));
        return 2;
    }
    d.ptr = p;
    d.done = ev;
    d.last = nullptr;
    d.recorded = false;
    return 0;
}

// attn_fwd_ex (workspace_bytes == SIZE_MAX: never split), attn_fwd_split
// (caller workspace) and, with use_scratch, attn_fwd_split_static, launch()
// and attn_fwd() (workspace: the static scratch, split plans bounded by its
// size).
int attn_fwd_impl(const void* q, const void* k, const void* v, void* o, int B, int H, int Sq,
                  int Skv, int D, float scale, hipStream_t stream, int dtype,
                  const long long* q_strides, const long long* k_strides,
                  const long long* v_strides, const long long* o_strides, void* workspace,
                  size_t workspace_bytes, bool use_scratch = false) {
    g_err[0] = 0;
    auto pick = [](const long long* p, Strides dflt) {
        return p ? Strides{p[0], p[1], p[2], p[3]} : dflt;
    };
    const Strides sq = pick(q_strides, contiguous(H, Sq, D));
    const Strides sk = pick(k_strides, contiguous(H, Skv, D));
    const Strides sv = pick(v_strides, contiguous(H, Skv, D));
    const Strides so = pick(o_strides, contiguous(H, Sq, D));
    if (check_args(q, k, v, o, B, H, Sq, Skv, D, dtype, sq, sk, sv, so)) return 1;
    if (B == 0 || H == 0 || Sq == 0) return 0;
    KArgs a;
    a.q = q;
    a.k = k;
    a.v = v;
    a.o = o;
    a.sq = sq;
    a.sk = sk;
    a.sv = sv;
    a.so = so;
    a.H = H;
    a.Sq = Sq;
    a.Skv = Skv;
    a.D = D;
    // Masked keys carry score -inf and rely on c > 0 (-inf * 0 is NaN). For
    // scale == 0, c = 1e-30 gives exp2(s*c - m) == 1.0f exactly for every
    // finite score, i.e. the same uniform weights as c == 0.
    a.c = fmaxf(fabsf(scale) * kLog2e, 1e-30f);
    a.qsign = scale < 0.f ? -1.f : 1.f;
    a.BH = B * H;
    a.nsplit = 1;
    a.split_len = 0;
    a.ws_o = nullptr;
    a.ws_ml = nullptr;
    a.o16 = (uintptr_t)o % 16 == 0 && so.b % 8 == 0 && so.h % 8 == 0 && so.s % 8 == 0 && so.d == 1;
    a.q_lds = sq.s <= (1LL << 24) && Skv > (D == 128 ? 256 : 1024);
    a.ncu = cu_count();
    SplitPlan p{1, 0};
    if (workspace_bytes != (size_t)-1)  // split the keys if it pays
        p = plan_split(B, H, Sq, Skv, D, use_scratch ? kScratchBytes : (size_t)-1);
    const size_t need = split_ws_bytes(p, B, H, Sq, D);
    DevScratch* ds = nullptr;
    std::unique_lock<std::mutex> lock(g_scratch_mu, std::defer_lock);
    bool capturing = false;
    if (need && use_scratch) {
        const int dev = stream_device(stream);
        if (dev < 0) return 2;
        hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
        hipError_t e = hipStreamIsCapturing(stream, &st);
        if (e != hipSuccess) {
            set_err(hipGetErrorString(e));
            return 2;
        }
        capturing = st != hipStreamCaptureStatusNone;
        lock.lock();
        ds = &g_scratch[dev];
        if (!ds->ptr) {
            if (capturing)
                return fail("attn: the static scratch of this device is set up by the first call "
                            "that splits outside stream capture; make one such call before "
                            "capturing");
            const int rc = scratch_setup(dev);
            if (rc) return rc;
        }
        if (!capturing && ds->recorded && ds->last != stream &&
            (e = hipStreamWaitEvent(stream, ds->done, 0)) != hipSuccess) {
            set_err(hipGetErrorString(e));
            return 2;
        }
        workspace = ds->ptr;
        workspace_bytes = kScratchBytes;
    }
    if (need) {
        if (!workspace || workspace_bytes < need || (uintptr_t)workspace % 16) {
            set_err("attn: workspace missing, misaligned or smaller than "
                    "attn_split_workspace_bytes()");
            return 1;
        }
        a.nsplit = p.nsplit;
        a.split_len = p.split_len;
        a.ws_o = (float*)workspace;
        a.ws_ml = a.ws_o + (size_t)p.nsplit * B * H * Sq * D;
    }
    const bool tl = token_contiguous(sk, sv, D);
    hipError_t e = dtype == ATTN_DTYPE_BF16 ? launch_t<bf16>(a, tl, stream)
                                            : launch_t<f16>(a, tl, stream);
    if (e == hipSuccess && ds && !capturing) {
        e = hipEventRecord(ds->done, stream);
        if (e == hipSuccess) {
            ds->last = stream;
            ds->recorded = true;
        }
    }
    if (e != hipSuccess) {
        set_err(hipGetErrorString(e));
        return 2;
    }
    return 0;
}

}  // namespace

extern "C" int attn_fwd_ex(const void* q, const void* k, const void* v, void* o, int B, int H,
                           int Sq, int Skv, int D, float scale, hipStream_t stream, int dtype,
                           const long long* q_strides, const long long* k_strides,
                           const long long* v_strides, const long long* o_strides) {
    return attn_fwd_impl(q, k, v, o, B, H, Sq, Skv, D, scale, stream, dtype, q_strides, k_strides,
                         v_strides, o_strides, nullptr, (size_t)-1);
}

extern "C" size_t attn_split_workspace_bytes(int B, int H, int Sq, int Skv, int D) {
    if (B <= 0 || H <= 0 || Sq <= 0 || Skv <= 0 ||
        !((D <= 64 && D > 0 && D % 8 == 0) || D == 128 || D == 512))
        return 0;
    return split_ws_bytes(plan_split(B, H, Sq, Skv, D), B, H, Sq, D);
}

extern "C" int attn_fwd_split(const void* q, const void* k, const void* v, void* o, int B, int H,
                              int Sq, int Skv, int D, float scale, hipStream_t stream, int dtype,
                              const long long* q_strides, const long long* k_strides,
                              const long long* v_strides, const long long* o_strides,
                              void* workspace, size_t workspace_bytes) {
    if (workspace_bytes == (size_t)-1) workspace_bytes -= 1;
    return attn_fwd_impl(q, k, v, o, B, H, Sq, Skv, D, scale, stream, dtype, q_strides, k_strides,
                         v_strides, o_strides, workspace, workspace_bytes);
}

extern "C" size_t attn_split_scratch_capacity(void) { return kScratchBytes; }

extern "C" int attn_fwd_split_static(const void* q, const void* k, const void* v, void* o, int B,
                                     int H, int Sq, int Skv, int D, float scale,
                                     hipStream_t stream, int dtype, const long long* q_strides,
                                     const long long* k_strides, const long long* v_strides,
                                     const long long* o_strides) {
    return attn_fwd_impl(q, k, v, o, B, H, Sq, Skv, D, scale, stream, dtype, q_strides, k_strides,
                         v_strides, o_strides, nullptr, 0, true);
}

extern "C" int attn_fwd(const void* q, const void* k, const void* v, void* o, int B, int H,
                        int Sq, int Skv, int D, float scale, hipStream_t s) {
    return attn_fwd_impl(q, k, v, o, B, H, Sq, Skv, D, scale, s, ATTN_DTYPE_F16, nullptr, nullptr,
                         nullptr, nullptr, nullptr, 0, true);
}

extern "C" void launch(const void* q, const void* k, const void* v, void* o, int B, int H,
                       int Sq, int Skv, int D, float scale, hipStream_t s) {
    (void)attn_fwd(q, k, v, o, B, H, Sq, Skv, D, scale, s);
}
