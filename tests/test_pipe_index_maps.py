"""CPU checks of the index maps of the D <= 128 attention kernel
(attn_fwd_pipe in gfx906_amd/csrc/attn_kernel.hip), restated from the kernel
source for both head-dim classes (DP = 64 and 128); the GPU parity tests
check the kernel itself:

* the direct HBM->LDS tile loads (tile_offsets: lane l of 1 KB block b writes
  LDS bytes 1024 b + 16 l, i.e. row (64 b + l) / NU, slot (64 b + l) % NU,
  fetching the row's 16-byte unit slot ^ swizzle(row)) and the K read
  (row 16 kb + l%16, unit 4 s + l/16) give exactly the A operand of
  v_mfma_f32_16x16x32 (lane l: row l%16, k = 8 (l/16) .. +7) for S^T = K Q^T,
  and the same read on a Q tile gives the B operand;
* the transposed V reads (two ds_read_b64_tr_b16: in each 16-lane group lane
  i receives element i%4 of the 8 bytes read by lanes 4e + i/4, e = 0..3)
  give the A operand of O^T += V^T P^T with the key order of P (k slot
  8g + e holds key 4g + e, slot 8g + 4 + e key 16 + 4g + e: the 16x16
  accumulator rows 4g + e of the two 16-key halves of S^T);
* both reads are free of bank conflicts in a 64-bank model (16 lanes of
  16-byte reads, 32 lanes of 8-byte reads served together), and the swizzle
  of the previous 32x32 design fails that model for the new V read (the
  GPU's SQ_LDS_BANK_CONFLICT counter, 0 in the main loop, is the final word);
* the epilogue's staging writes and 16-byte read-back cover each output row
  and dim of a wave exactly once.
"""

import numpy as np
import pytest

BN = 64  # keys per tile


def kswz(nu, r):
    return (r & 15) if nu >= 16 else ((r >> 1) & 7)


def vswz(nu, r):
    return 2 * (r & 7) if nu >= 16 else 2 * ((r >> 1) & 3)


def fill(T, dp, swz):
    """LDS image (uint16, row-major [64][dp]) written by the direct loads of
    one tile T[key][dim]."""
    nu = dp // 8
    lds = np.zeros(BN * dp, dtype=np.uint16)
    for unit in range(BN * nu):  # = (wave + i*NW)*64 + lane over all loads
        row, slot = divmod(unit, nu)
        u = slot ^ swz(nu, row)
        assert 0 <= u < nu
        lds[unit * 8: unit * 8 + 8] = T[row, 8 * u: 8 * u + 8]
    return lds


def kaddr(dp, s, lane):
    nu, rb = dp // 8, dp * 2
    i, g = lane & 15, lane >> 4
    return i * rb + ((4 * s + g) ^ kswz(nu, i)) * 16


def vaddr(dp, ob, lane):
    nu, rb = dp // 8, dp * 2
    i, g = lane & 15, lane >> 4
    vrow = 4 * g + (i >> 2)
    vx = vswz(nu, vrow) >> 1
    return vrow * rb + (ob ^ vx) * 32 + (i & 3) * 8


def rd(lds, byte, n):
    assert byte % 2 == 0 and 0 <= byte and byte + 2 * n <= lds.size * 2
    return lds[byte // 2: byte // 2 + n]


def tr_read(lds, addrs):
    """ds_read_b64_tr_b16 over 64 lanes: addrs[l] is lane l's byte address."""
    raw = [rd(lds, a, 4) for a in addrs]
    out = []
    for lane in range(64):
        g, i = lane >> 4, lane & 15
        out.append([raw[16 * g + 4 * e + i // 4][i % 4] for e in range(4)])
    return out


@pytest.fixture(scope="module", params=[64, 128])
def case(request):
    dp = request.param
    rng = np.random.default_rng(dp)
    K = rng.integers(0, 65535, size=(BN, dp)).astype(np.uint16)
    V = rng.integers(0, 65535, size=(BN, dp)).astype(np.uint16)
    return dp, K, V, fill(K, dp, kswz), fill(V, dp, vswz)


def test_k_reads_give_the_a_operand(case):
    dp, K, _, lk, _ = case
    rb = dp * 2
    for blk in range(2):
        for kb in range(2):
            for s in range(dp // 32):
                for lane in range(64):
                    i, g = lane & 15, lane >> 4
                    got = rd(lk, kaddr(dp, s, lane) + (32 * blk + 16 * kb) * rb, 8)
                    want = K[32 * blk + 16 * kb + i, 32 * s + 8 * g: 32 * s + 8 * g + 8]
                    assert list(got) == list(want)


def test_q_reads_through_lds_give_the_b_operand(case):
    # Q tiles are loaded as K tiles; wave w reads rows 32 (w%2) + 16 nb + l%16
    # of tile w/2 (stage offsets are whole tiles).
    dp, Q, _, lq, _ = case
    rb = dp * 2
    for w2 in range(2):
        for nb in range(2):
            for s in range(dp // 32):
                for lane in range(64):
                    i, g = lane & 15, lane >> 4
                    got = rd(lq, w2 * 32 * rb + kaddr(dp, s, lane) + 16 * nb * rb, 8)
                    want = Q[32 * w2 + 16 * nb + i, 32 * s + 8 * g: 32 * s + 8 * g + 8]
                    assert list(got) == list(want)


def test_v_reads_give_the_a_operand_in_p_key_order(case):
    dp, _, V, _, lv = case
    rb = dp * 2
    # P's k slots (block_exp): 8g + e <- key 4g + e, 8g + 4 + e <- key 16 + 4g + e
    p_keys = {g: [4 * g + e for e in range(4)] + [16 + 4 * g + e for e in range(4)]
              for g in range(4)}
    assert sorted(k for g in range(4) for k in p_keys[g]) == list(range(32))
    for blk in range(2):
        for ob in range(dp // 16):
            lo = tr_read(lv, [vaddr(dp, ob, l) + 32 * blk * rb for l in range(64)])
            hi = tr_read(lv, [vaddr(dp, ob, l) + 32 * blk * rb + 16 * rb for l in range(64)])
            for lane in range(64):
                i, g = lane & 15, lane >> 4
                got = list(lo[lane]) + list(hi[lane])
                want = [V[32 * blk + k, 16 * ob + i] for k in p_keys[g]]
                assert got == want


def banks(addrs, nbytes):
    return [(a // 4 + k) % 64 for a in addrs for k in range(nbytes // 4)]


@pytest.mark.parametrize("dp", [64, 128])
def test_reads_are_bank_conflict_free(dp):
    for s in range(dp // 32):
        for grp in range(4):  # 16 lanes of 16-byte reads
            b = banks([kaddr(dp, s, 16 * grp + i) for i in range(16)], 16)
            assert len(set(b)) == len(b) == 64
    for ob in range(dp // 16):
        for half in range(2):  # 32 lanes of 8-byte reads
            b = banks([vaddr(dp, ob, 32 * half + j) for j in range(32)], 8)
            assert len(set(b)) == len(b) == 64


def test_planted_swizzle_mistake_conflicts():
    # The V swizzle of the 32x32x16 design, 4 (r & 3), maps rows r and r + 4
    # of a half wave's 8 rows to the same units under the new read.
    dp, rb = 128, 256
    addrs = []
    for j in range(32):
        i, g = j & 15, j >> 4
        vrow = 4 * g + (i >> 2)
        vx = (4 * (vrow & 3)) >> 1
        addrs.append(vrow * rb + (0 ^ vx) * 32 + (i & 3) * 8)
    b = banks(addrs, 8)
    assert len(set(b)) < len(b)


@pytest.mark.parametrize("dp", [64, 128])
def test_staged_output_covers_each_element_once(dp):
    rs, cpr = dp * 2 + 16, dp * 2 // 16
    assert 32 * rs <= 64 * dp * 2  # a wave's staging fits one ring array (a 64-key tile)
    written = {}
    for nb in range(2):
        for ob in range(dp // 16):
            for lane in range(64):
                i, g = lane & 15, lane >> 4
                d0 = 16 * ob + 4 * g
                for e in range(4):
                    a = (16 * nb + i) * rs + (d0 + e) * 2
                    assert a not in written
                    written[a] = (16 * nb + i, d0 + e)
    assert sorted(written.values()) == [(r, d) for r in range(32) for d in range(dp)]
    pieces = set()
    for j in range(32 * cpr // 64):
        for lane in range(64):
            c = 64 * j + lane
            r, col = divmod(c, cpr)
            for e in range(8):
                assert written[r * rs + col * 16 + 2 * e] == (r, 8 * col + e)
            pieces.add((r, col))
    assert len(pieces) == 32 * cpr
