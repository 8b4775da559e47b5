"""CPU checks of two index maps the HIP kernels rely on, restated from the
kernel source (the GPU parity tests check the kernels themselves):

* the token-contiguous D = 512 attention tiles (attn_fwd_d512<T, true>): the
  direct loads' chunk choice, the transposed K reads (ds_read_b64_tr_b16: in
  each 16-lane group, lane i receives element i%4 of the 8 bytes read by lanes
  4e + i/4, e = 0..3) and the V^T reads deliver exactly the MFMA operands, P's
  key order matches V^T's, the transposed K reads keep a 64-bank model free
  of conflicts and the V^T reads cover each block's units once (rocprofv3's
  SQ_LDS_BANK_CONFLICT on the GPU is the final word on banks: the swizzles
  were chosen by that counter);
* conv3d's incremental tap tracking (conv3d_mfma) agrees with the direct
  division-based index for every k-tile and lane group, and its load roles
  for both k-tile widths (32 and 64 reduction elements) fill every LDS slot
  once, with whole rows fetched by neighbouring lanes and conflict-free
  operand reads.
"""

import numpy as np
import pytest

D, BN, ROWB = 512, 32, 64


def tswz(r):
    return (((r >> 2) & 1) << 1) | ((r >> 3) & 1)


def tkey(kb, j, t):
    return 8 * j + 4 * ((j + kb) & 1) + t


def vswz(r):
    return (r >> 1) & 3


def fill_tile_v(T):
    """LDS image (uint16) of one V^T tile written by the direct loads: as
    fill_tile, with the V^T swizzle: lane l fetches chunk (l%4) ^ vswz(row)."""
    lds = np.zeros(D * BN, dtype=np.uint16)
    for blk in range(32):
        for lane in range(64):
            row = 16 * blk + lane // 4
            tv = (lane & 3) ^ ((lane >> 3) & 3)
            assert tv == (lane & 3) ^ vswz(row)
            base = blk * 1024 + lane * 16
            lds[base // 2: base // 2 + 8] = T[row, 8 * tv: 8 * tv + 8]
    return lds


def fill_tile(T):
    """LDS image (uint16) of one K^T tile written by the direct loads:
    lane l of 1 KB block blk (= wave + 8n) writes bytes blk*1024 + 16l, i.e.
    row 16*blk + l/4, slot l%4, fetching key chunk tu = (l%4) ^ tswz(row)."""
    lds = np.zeros(D * BN, dtype=np.uint16)
    for blk in range(32):
        for lane in range(64):
            row = 16 * blk + lane // 4
            tu = (lane & 3) ^ ((((lane >> 4) & 1) << 1) | ((lane >> 5) & 1))
            assert tu == (lane & 3) ^ tswz(row)
            base = blk * 1024 + lane * 16
            assert base == row * ROWB + (lane & 3) * 16
            lds[base // 2: base // 2 + 8] = T[row, 8 * tu: 8 * tu + 8]
    return lds


def ktr_addr(s, kb, g, h, i):
    row = 32 * s + 8 * g + 4 * h + (i >> 2)
    return row * ROWB + (((i & 3) ^ ((h << 1) | (g & 1))) * 16) + (((i & 3) + kb) & 1) * 8


def vt_addr(ob, g, i):
    return (16 * ob + i) * ROWB + ((g ^ vswz(i)) * 16)


@pytest.fixture(scope="module")
def tiles():
    rng = np.random.default_rng(0)
    K = rng.integers(0, 65535, size=(BN, D)).astype(np.uint16)  # [key][dim]
    V = rng.integers(0, 65535, size=(BN, D)).astype(np.uint16)
    return K, V, fill_tile(K.T.copy()), fill_tile_v(V.T.copy())


def test_transposed_k_reads_give_the_qk_operand(tiles):
    K, _, lk, _ = tiles
    for s in range(16):
        for kb in range(2):
            for g in range(4):
                reads = {(h, i): lk[ktr_addr(s, kb, g, h, i) // 2:][:4]
                         for h in range(2) for i in range(16)}
                for i in range(16):
                    got = [reads[(h, 4 * e + i // 4)][i % 4] for h in range(2) for e in range(4)]
                    key = tkey(kb, i >> 2, i & 3)
                    want = [K[key, 32 * s + 8 * g + 4 * h + e] for h in range(2) for e in range(4)]
                    assert got == want


def test_vt_reads_match_p_key_order(tiles):
    _, V, _, lv = tiles
    for g in range(4):  # P after the odd-group swap holds keys 8g..8g+7 in order
        b0 = [tkey(0, g, r) for r in range(4)]
        b1 = [tkey(1, g, r) for r in range(4)]
        assert (b1 + b0 if g & 1 else b0 + b1) == list(range(8 * g, 8 * g + 8))
    for ob in range(32):
        for g in range(4):
            for i in range(16):
                got = list(lv[vt_addr(ob, g, i) // 2:][:8])
                assert got == [V[8 * g + e, 16 * ob + i] for e in range(8)]
    keys = sorted(tkey(kb, j, t) for kb in range(2) for j in range(4) for t in range(4))
    assert keys == list(range(BN))


def conflict_free(addrs, nbytes):
    banks = [(a // 4 + k) % 64 for a in addrs for k in range(nbytes // 4)]
    return len(banks) == len(set(banks))


def test_reads_are_bank_conflict_free():
    for s in (0, 7):
        for kb in range(2):
            for h in range(2):
                for half in range(2):  # 32 lanes served together
                    addrs = [ktr_addr(s, kb, g, h, i) for g in (2 * half, 2 * half + 1)
                             for i in range(16)]
                    assert conflict_free(addrs, 8)
    for ob in (0, 9):
        # the V^T read's 64 lanes cover the block's 64 units once
        assert sorted(vt_addr(ob, g, i) for g in range(4) for i in range(16)) == \
            [ob * 1024 + 16 * u for u in range(64)]


def test_planted_swizzle_mistake_conflicts():
    # The swizzle of the previous design ((row >> 2) & 3) with this key order
    # puts both lane groups on the same halves.
    addrs = []
    for g in (0, 1):
        for i in range(16):
            row = 8 * g + (i >> 2)
            addrs.append(row * ROWB + (((i & 3) ^ ((row >> 2) & 3)) * 16) + ((i & 3) & 1) * 8)
    assert not conflict_free(addrs, 8)


# -- conv3d taps -------------------------------------------------------------------------

def tap_walk(C, T, R, S, xsd, xsh, xsw, kbr=32):
    """Per lane group u: (gi, cc, toff) of every k-tile, as the kernel advances them."""
    KG = C * T * R * S
    nkt = -(-KG // kbr)
    small = C < kbr
    for u in range(kbr // 8):
        gi = 8 * u
        tp = gi // C
        cc, ts, tr = gi - tp * C, tp % S, (tp // S) % R
        toff = (tp // (S * R)) * xsd + tr * xsh + ts * xsw
        tstep = kbr // C if small else 0
        cstep = kbr - tstep * C
        dr, dt = xsh - S * xsw, xsd - R * xsh

        def next_tap(go):
            nonlocal ts, tr, toff
            ts += go
            toff += xsw if go else 0
            ws = ts == S
            ts = 0 if ws else ts
            tr += ws
            toff += dr if ws else 0
            wr = tr == R
            tr = 0 if wr else tr
            toff += dt if wr else 0

        for _ in range(-(-nkt // 4) * 4):
            yield gi, cc, toff, KG
            gi += kbr
            if small:
                for i in range(kbr // 8):
                    next_tap(i < tstep)
            cc += cstep
            wrap = cc >= C
            cc -= C if wrap else 0
            next_tap(wrap)


@pytest.mark.parametrize("kbr", [32, 64])
@pytest.mark.parametrize("C", [8, 16, 24, 32, 40, 56, 64, 96, 512])
@pytest.mark.parametrize("trs", [(1, 1, 1), (3, 3, 3), (1, 3, 3), (2, 3, 2), (5, 2, 3)])
def test_conv3d_tap_tracking_matches_division(C, trs, kbr):
    T, R, S = trs
    xsd, xsh, xsw = 7919 * C, 131 * C, C
    for gi, cc, toff, KG in tap_walk(C, T, R, S, xsd, xsh, xsw, kbr):
        if gi >= KG:
            continue
        tp = gi // C
        t, r, s = tp // (R * S), (tp // S) % R, tp % S
        assert (cc, toff) == (gi % C, t * xsd + r * xsh + s * xsw)


def conv_swz(kb, r):
    return (r >> 2) & 3 if kb == 32 else (r >> 1) & 7


CONV_KERNELS = [(4, 32, 2), (3, 64, 2), (2, 64, 2), (4, 32, 4), (3, 64, 4), (2, 64, 4),
                (3, 32, 4)]  # NB, KB, CW


@pytest.mark.parametrize("nb,kb,cw", CONV_KERNELS)
def test_conv3d_load_roles_and_operand_reads(nb, kb, cw):
    rowb, units, nw = 2 * kb, kb // 8, 2 * cw
    rpb = 1024 // rowb
    wtile, xtile = 64 * cw * rowb, 64 * nb * rowb
    for tile_bytes in (wtile, xtile):
        tblk = tile_bytes // 1024
        nblk = -(-tblk // nw)  # loads per wave; past tblk: zeros into the pad
        assert tile_bytes == wtile and nblk * nw == tblk or tile_bytes == xtile
        seen = {}
        for wave in range(nw):
            for lane in range(64):
                rsub = lane // units
                u = (lane % units) ^ conv_swz(kb, rpb * wave + rsub)
                for j in range(nblk):
                    blk = wave + nw * j
                    if blk >= tblk:
                        continue
                    row, slot = rpb * blk + rsub, lane % units
                    assert blk * 1024 + 16 * lane == row * rowb + 16 * slot
                    assert u == slot ^ conv_swz(kb, row)  # same unit in every block j
                    seen[(row, slot)] = u
        rows = tile_bytes // rowb
        assert len(seen) == rows * units  # every slot written once
        # neighbouring lanes fetch whole rows: all units of a row, each once
        for row in range(rows):
            assert sorted(seen[(row, sl)] for sl in range(units)) == list(range(units))
        # operand reads (v_mfma_f32_16x16x32_f16): row base + l%16, unit
        # 4ks + l/16, 16 lanes served together
        for base in range(0, rows, 16):
            for ks in range(kb // 32):
                for q in range(4):
                    addrs = []
                    for lane in range(16 * q, 16 * q + 16):
                        r, unit = base + lane % 16, 4 * ks + lane // 16
                        slot = unit ^ conv_swz(kb, r)
                        assert seen[(r, slot)] == unit  # the read finds its unit
                        addrs.append(r * rowb + 16 * slot)
                    assert conflict_free(addrs, 16)


def tile_of(L, n):
    xcd, pos, base, extra = L & 7, L >> 3, n >> 3, n & 7
    return (xcd * (base + 1) if xcd < extra else extra * (base + 1) + (xcd - extra) * base) + pos


@pytest.mark.parametrize("n", [1, 5, 8, 13, 242, 484, 1024, 1490])
def test_conv3d_xcd_tile_map_is_a_permutation_in_contiguous_eighths(n):
    tiles = [tile_of(L, n) for L in range(n)]
    assert sorted(tiles) == list(range(n))
    for x in range(8):  # XCD x (workgroups L = x mod 8) gets one contiguous run, in order
        run = tiles[x::8]
        assert run == list(range(run[0], run[0] + len(run))) if run else True
