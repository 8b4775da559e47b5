"""Code-generation checks of attn_fwd_pipe's main loop (D = 128, no split).

The north-star kernel's speed depends on how little non-MFMA work its main
loop carries besides the softmax: each VALU instruction there competes with
the MFMAs for the SIMD's issue slots. Two layout decisions keep address
arithmetic out of the loop, and nothing but the compiler's output shows that
they hold:

* the ring's four K tiles are the kernel's first 64 KiB of LDS, so every K
  read takes its array's place as a 16-bit immediate offset;
* the V read registers hold their addresses plus 64 KiB (opaque to the
  compiler), so every V read into the V arrays above 64 KiB does too;

and the tile loads' row clamp is a scalar min and select. This test compiles
the kernel source to gfx950 assembly with the build's own flags, finds the
main loop of the D = 128 fp16 and bf16 kernels (the loop with four
workgroup barriers), leaves out the key-mask and rescale blocks (taken on
the last tiles and rarely), and counts the VALU instructions per wave and
32-key block: 16 FMA, 16 exponentials, 8 conversions, the packed maxima of
the rescale test and 2 compares, with at most a couple of others.
"""

import collections
import re
import subprocess

import pytest

from gfx906_amd import build


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("asm") / "attn_kernel.s"
    cmd = [build.hipcc(), *build.HIP_FLAGS, "--cuda-device-only", "-S", f"-I{build.INCLUDE}",
           str(build.CSRC / "attn_kernel.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip(f"hipcc unavailable or failed: {res.stderr[-500:]}")
    return out.read_text()


def functions(asm, pattern):
    out = {}
    for m in re.finditer(r"^(_Z\w+):[^\n]*\n(.*?)^\.Lfunc_end", asm, re.S | re.M):
        if re.search(pattern, m.group(1)):
            out[m.group(1)] = m.group(2).split("\n")
    return out


def main_loop(lines):
    """The lines of the loop that holds four s_barrier, without the blocks
    that its forward conditional branches skip (key masks, rare rescales)."""
    headers = [i for i, l in enumerate(lines) if "Loop Header" in l]
    for h in headers:
        label = lines[h].split(":")[0]
        latches = [i for i, l in enumerate(lines)
                   if re.match(r"\ts_c?branch\w* " + re.escape(label) + r"$", l)]
        if not latches:
            continue
        body = lines[h:max(latches) + 1]
        if sum("s_barrier" in l for l in body) != 4:
            continue
        inside = {l.split(":")[0] for l in body if l.startswith(".LBB")}
        kept, skip = [], None
        for l in body[:-1]:
            if skip:
                if l.startswith(skip + ":"):
                    skip = None
                continue
            m = re.match(r"\ts_cbranch_\w+ (\.LBB\w+)$", l)
            # a forward branch to a label inside the loop skips a block; the
            # rare rescale blocks sit after the loop and return into it
            if m and m.group(1) != label and m.group(1) in inside:
                skip = m.group(1)
            kept.append(l)
        return kept
    return None


def counts(body):
    c = collections.Counter()
    for l in body:
        if l.startswith("\t") and not l.startswith(("\t;", "\t.")):
            c[l.split()[0]] += 1
    return c


KERNELS = r"attn_fwd_pipeINS_3CfgILi128ELi8ELi1EEELb0E(DF16_|DF16b)Lb0ELb0EEE"


def test_d128_main_loop_instruction_mix(kernel_asm):
    funcs = functions(kernel_asm, KERNELS)
    assert len(funcs) == 2, list(funcs)  # fp16 and bf16, unsplit
    for name, lines in funcs.items():
        body = main_loop(lines)
        assert body is not None, name
        c = counts(body)
        blocks = 8  # four 64-key tiles of two 32-key blocks each
        mfma = sum(v for k, v in c.items() if k.startswith("v_mfma"))
        assert mfma == 34 * blocks, (name, mfma)  # 16 QK^T, 16 PV, 2 row sums
        assert c["v_exp_f32_e32"] == 16 * blocks, name
        valu = sum(v for k, v in c.items() if k.startswith("v_") and not k.startswith("v_mfma"))
        # 16 FMA + 16 exp + 8 cvt + 4 packed maxima (v_pk_maximum3_f16, bf16
        # patterns read as fp16) + 2 compares = 46 per block
        assert valu <= 47 * blocks, (name, valu / blocks, c.most_common(12))
        # no LDS address arithmetic and no vector clamp of the tile rows
        addr = c["v_add_u32_e32"] + c["v_or_b32_e32"] + c["v_med3_i32"] + c["v_readfirstlane_b32"]
        assert addr <= 2, (name, addr)
        # every LDS read of K and V is one instruction with an immediate offset
        assert c["ds_read_b128"] == 8 * blocks and c["ds_read_b64_tr_b16"] == 16 * blocks, name


RESOURCES = re.compile(r"^(_Z\w+):.*?^\.Lfunc_end\d+:.*?; TotalNumVgprs: (\d+)\n; ScratchSize: (\d+)"
                       r".*?; Occupancy: (\d+)", re.S | re.M)
# Waves per SIMD each kernel is designed for (its register budget).
OCCUPANCY = [("attn_fwd_pipeINS_3CfgILi128", 2), ("attn_fwd_pipeINS_3CfgILi64", 4),
             ("attn_fwd_d512w", 1), ("attn_fwd_d512I", 2), ("attn_fwd_kvres", 4),
             ("attn_combine", 8)]


def test_kernels_do_not_spill(kernel_asm):
    """A scratch reload in a ring kernel's loop comes with a vmcnt(0) wait, which
    drains the tile loads in flight: no attention kernel may use scratch. (The
    D <= 64 kernels run at their 128-VGPR limit; they recompute lane indices
    after the main loop instead of keeping them in registers across it.)"""
    seen = set()
    for m in RESOURCES.finditer(kernel_asm):
        name, vgprs, scratch, occ = m.group(1), int(m.group(2)), int(m.group(3)), int(m.group(4))
        want = [o for pat, o in OCCUPANCY if pat in name]
        if not want:
            continue
        seen.add(next(pat for pat, _ in OCCUPANCY if pat in name))
        assert occ >= want[0] and vgprs <= 512 // want[0], (name, vgprs, occ)
        assert scratch == 0, (name, scratch)
    assert seen == {pat for pat, _ in OCCUPANCY}, seen


@pytest.fixture(scope="module")
def conv_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("asm") / "conv3d_kernel.s"
    cmd = [build.hipcc(), *build.HIP_FLAGS, "--cuda-device-only", "-S", f"-I{build.INCLUDE}",
           str(build.CSRC / "conv3d_kernel.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip(f"hipcc unavailable or failed: {res.stderr[-500:]}")
    return out.read_text()


def test_conv3d_kernels_do_not_spill(conv_asm):
    """Every conv3d tile configuration keeps two waves per SIMD and no scratch
    (the small-C 4x32x256 kernel spilled before its k-tile scheduling barrier)."""
    found = [(m.group(1), int(m.group(2)), int(m.group(3)), int(m.group(4)))
             for m in RESOURCES.finditer(conv_asm) if "conv3d_mfma" in m.group(1)]
    assert len(found) == 14, len(found)  # seven configurations, each for small and large C
    for name, vgprs, scratch, occ in found:
        assert scratch == 0 and occ >= 2 and vgprs <= 256, (name, vgprs, scratch, occ)
