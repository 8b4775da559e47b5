"""Static hazard check of attn_fwd_d512w's hand-written MFMAs.

The D = 512 wide kernel issues its PV MFMAs as inline asm (to keep the O^T
accumulator in AGPRs), and the compiler's hazard recognizer does not look
into asm. The kernel provides the wait states itself; this test compiles the
kernel source to gfx950 assembly with the build's own flags and checks every
path through the compiled code against the two gfx950 rules it relies on:

* after an asm MFMA, no instruction may read or write its accumulator
  registers until the MFMA has completed: 12 wait states before a VALU
  access on gfx950 for an 8-pass MFMA, 20 for a 16-pass one; the check asks
  for REQ_AFTER = 20 whatever the pass count;
* before an asm MFMA, no VALU instruction may have written one of its source
  registers (srcA, srcB, srcC) within REQ_BEFORE = 2 wait states.

Wait states are counted conservatively: one per instruction, N + 1 for
s_nop N. Paths follow fall-through and branch edges, loops included. The
checker itself is pinned on planted mistakes.
"""

import re
import subprocess

import pytest

from gfx906_amd import build

REQ_AFTER = 20
REQ_BEFORE = 2

_REG = re.compile(r"\b([va])(?:\[(\d+):(\d+)\]|(\d+)(?!\w))")


def regs(operands):
    out = set()
    for m in _REG.finditer(operands):
        kind = m.group(1)
        if m.group(4) is not None:
            out.add((kind, int(m.group(4))))
        else:
            out.update((kind, r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
    return out


class Instr:
    def __init__(self, text, in_asm):
        self.text = text
        parts = text.split(None, 1)
        self.op = parts[0]
        self.args = parts[1] if len(parts) > 1 else ""
        self.in_asm = in_asm
        first = self.args.split(",")[0] if self.args else ""
        self.dst = regs(first)
        self.all = regs(self.args)
        self.is_asm_mfma = in_asm and self.op.startswith("v_mfma") and any(
            k == "a" for k, _ in self.dst)

    @property
    def wait_states(self):
        if self.op == "s_nop":
            return int(self.args.strip(), 0) + 1
        return 1


def parse_functions(asm, name_part):
    """{function name: (instructions, label -> index)} for functions whose
    symbol contains name_part."""
    funcs = {}
    for m in re.finditer(r"^(\S*%s\S*):" % re.escape(name_part), asm, re.M):
        end = asm.find(".Lfunc_end", m.end())
        body = asm[m.end():end]
        instrs, labels, in_asm = [], {}, False
        for line in body.split("\n"):
            s = line.strip()
            if s.startswith(";;#ASMSTART"):
                in_asm = True
                continue
            if s.startswith(";;#ASMEND"):
                in_asm = False
                continue
            if not s or s.startswith(";") or s.startswith("."):
                lab = re.match(r"^(\.L\w+):", s)
                if lab:
                    labels[lab.group(1)] = len(instrs)
                continue
            s = s.split(";")[0].strip()
            if s:
                instrs.append(Instr(s, in_asm))
        funcs[m.group(1)] = (instrs, labels)
    return funcs


def successors(instrs, labels, i):
    ins = instrs[i]
    if ins.op == "s_endpgm":
        return []
    if ins.op == "s_branch":
        return [labels[ins.args.strip()]]
    if ins.op.startswith("s_cbranch"):
        return [i + 1, labels[ins.args.strip()]]
    return [i + 1] if i + 1 < len(instrs) else []


def predecessors(instrs, labels):
    pred = {i: [] for i in range(len(instrs))}
    for i in range(len(instrs)):
        for j in successors(instrs, labels, i):
            if j < len(instrs):
                pred[j].append(i)
    return pred


def check_function(instrs, labels):
    """Violations of the two rules around every asm MFMA, as strings."""
    bad = []
    pred = predecessors(instrs, labels)
    for i, mf in enumerate(instrs):
        if not mf.is_asm_mfma:
            continue
        acc = mf.dst
        # Forward: nothing touches the accumulator until REQ_AFTER wait states.
        seen = {}
        stack = [(j, 0) for j in successors(instrs, labels, i)]
        while stack:
            j, used = stack.pop()
            if j >= len(instrs) or used >= REQ_AFTER or seen.get(j, -1) >= REQ_AFTER - used:
                continue
            seen[j] = REQ_AFTER - used
            ins = instrs[j]
            if ins.all & acc:
                bad.append(f"{mf.text}  ->  {ins.text}  after {used} wait states")
                continue
            for k in successors(instrs, labels, j):
                stack.append((k, used + ins.wait_states))
        # Backward: no VALU write of a source within REQ_BEFORE wait states.
        srcs = mf.all
        seen = set()
        stack = [(j, 0) for j in pred[i]]
        while stack:
            j, used = stack.pop()
            if used >= REQ_BEFORE or (j, used) in seen:
                continue
            seen.add((j, used))
            ins = instrs[j]
            if ins.op.startswith("v_") and ins.dst & srcs:
                bad.append(f"{ins.text}  ->  {mf.text}  after {used} wait states")
                continue
            stack.extend((k, used + ins.wait_states) for k in pred[j])
    return bad


def _synthetic(body):
    return "k:\n" + body + "\n.Lfunc_end0:\n"


def test_checker_catches_planted_mistakes():
    mfma = ";;#ASMSTART\n\tv_mfma_f32_16x16x32_f16 a[0:3], v[4:7], v[8:11], a[0:3]\n;;#ASMEND\n"
    # An AGPR read right after the MFMA.
    f = parse_functions(_synthetic(mfma + "\tv_accvgpr_read_b32 v0, a2\n\ts_endpgm"), "k")["k"]
    assert len(check_function(*f)) == 1
    # ... also when reached through a branch, and a write counts too.
    asm = mfma + "\ts_branch .LBB0_1\n\ts_nop 7\n.LBB0_1:\n\tv_accvgpr_mov_b32 a3, a9\n\ts_endpgm"
    assert len(check_function(*parse_functions(_synthetic(asm), "k")["k"])) == 1
    # A VALU write of srcB one instruction before the MFMA.
    asm = "\tv_cvt_pk_f16_f32 v9, v1, v2\n" + mfma + "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_endpgm"
    assert len(check_function(*parse_functions(_synthetic(asm), "k")["k"])) == 1
    # Enough wait states in both directions: clean.
    asm = ("\tv_cvt_pk_f16_f32 v9, v1, v2\n\ts_nop 1\n" + mfma +
           "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\tv_accvgpr_read_b32 v0, a2\n\ts_endpgm")
    assert check_function(*parse_functions(_synthetic(asm), "k")["k"]) == []
    # A loop back-edge: the MFMA at the loop's end reaches the read at its top.
    asm = (".LBB0_1:\n\tv_accvgpr_read_b32 v0, a1\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n" + mfma +
           "\ts_cbranch_scc1 .LBB0_1\n\ts_endpgm")
    assert len(check_function(*parse_functions(_synthetic(asm), "k")["k"])) == 1


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory):
    out = tmp_path_factory.mktemp("asm") / "attn_kernel.s"
    cmd = [build.hipcc(), *build.HIP_FLAGS, "--cuda-device-only", "-S", f"-I{build.INCLUDE}",
           str(build.CSRC / "attn_kernel.hip"), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        pytest.skip(f"hipcc unavailable or failed: {res.stderr[-500:]}")
    return out.read_text()


def test_compiled_d512w_respects_mfma_hazards(kernel_asm):
    funcs = parse_functions(kernel_asm, "attn_fwd_d512w")
    assert len(funcs) == 4  # fp16/bf16 x split/unsplit
    for name, (instrs, labels) in funcs.items():
        n = sum(i.is_asm_mfma for i in instrs)
        assert n >= 64, (name, n)  # the PV MFMAs of at least one tile
        bad = check_function(instrs, labels)
        assert not bad, f"{name}: " + "\n".join(bad[:10])
