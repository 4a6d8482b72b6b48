"""Generated-code checks of the head_dim-256 attention kernel (CPU; needs hipcc).

The kernel accumulates O^T in AGPRs through inline-assembly MFMAs
(mfma16x16x32_agpr2 in csrc/common.h).  The compiler's hazard recognizer does
not see inside inline assembly, so the code carries its own wait states; these
tests compile attn_fwd256.hip with the library's flags and check the emitted
gfx950 assembly:

* every compiler-generated instruction that names an AGPR comes at least 18
  wait states after the last inline-asm MFMA, counted from the start of its
  basic block (a block may be entered right after any MFMA), so the VALU
  reads of the accumulators (rescale, epilogue) and any copy of them wait for
  the matrix core;
* no VALU instruction writes an A, B or C operand register of an inline-asm
  MFMA fewer than two wait states before it on any path into it (the pairs
  carry no s_nop of their own);
* the kernel uses no scratch and no packed-fp32 VALU forms.
"""

import os
import re
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__ as G  # noqa: E402

# the head_dim-256 instances, bf16 and fp16
KERNELS = ["_ZN5ugbsa20attn_fwd_pipe_kernelINS_8ElemBf16ELi256ELi4ELb1ELb1ELb1E",
           "_ZN5ugbsa20attn_fwd_pipe_kernelINS_7ElemF16ELi256ELi4ELb1ELb1ELb1E"]
MIN_WAIT_STATES = 18


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not os.path.exists(G.HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("isa")
    src = os.path.join(G.CSRC, "attn_fwd256.hip")
    cmd = [G.HIPCC, *G.FLAGS, "--cuda-device-only", "-S", src, "-o", str(d / "k.s")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return (d / "k.s").read_text()


def kernel_body(text, kernel):
    lines = text.split("\n")
    start = next(i for i, l in enumerate(lines) if l.startswith(kernel) and l.split(";")[0].rstrip().endswith(":"))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
    return lines[start + 1:end]


def _blocks(body):
    """Basic blocks of a kernel body: (label or None, lines, successor labels,
    falls through)."""
    blocks, cur, label = [], [], None
    def close(succ, falls):
        blocks.append((label, cur, succ, falls))
    for line in body:
        s = line.split(";")[0].strip()
        if s.endswith(":") and not s.startswith(";"):
            if cur or label is not None:
                close([], True)
            cur, label = [], s[:-1]
            continue
        cur.append(line)
        op = s.split()[0] if s else ""
        if op == "s_branch" or op.startswith("s_cbranch"):
            close([s.split()[1]], op != "s_branch")
            cur, label = [], None
    close([], False)
    return blocks


def _scan(lines, since, bad):
    """Walk one block from `since` wait states after the last inline-asm MFMA;
    append early AGPR accesses to bad (if given); return the state at its end
    and the counts of MFMAs and checked instructions."""
    in_asm = False
    mfmas = checked = 0
    agpr = re.compile(r"\ba\[?\d")
    for line in lines:
        raw = line.strip()
        if raw.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if raw.startswith(";;#ASMEND"):
            in_asm = False
            continue
        s = line.split(";")[0].strip()
        if not s or s.startswith("."):
            continue
        op = s.split()[0]
        if in_asm:
            if op.startswith("v_mfma"):
                mfmas += 1
                since = 0
            else:
                since += int(s.split()[1]) + 1 if op == "s_nop" else 1
            continue
        if agpr.search(s):
            checked += 1
            if bad is not None and since < MIN_WAIT_STATES:
                bad.append((s, since))
        since += int(s.split()[1]) + 1 if op == "s_nop" else 1
    return since, mfmas, checked


def agpr_hazards(body):
    """(instruction, wait states) of every compiler instruction that names an
    AGPR fewer than MIN_WAIT_STATES wait states after an inline-asm MFMA on
    some path through the kernel's control flow; plus the counts of
    inline-asm MFMAs and of checked instructions."""
    blocks = _blocks(body)
    index = {b[0]: i for i, b in enumerate(blocks) if b[0] is not None}
    preds = [[] for _ in blocks]
    for i, (_, _, succ, falls) in enumerate(blocks):
        for lab in succ:
            preds[index[lab]].append(i)
        if falls and i + 1 < len(blocks):
            preds[i + 1].append(i)
    big = 1 << 30
    entry = [big] * len(blocks)
    out = [big] * len(blocks)
    changed = True
    while changed:              # wait states only shrink along paths: a fixpoint
        changed = False
        for i, (_, lines, _, _) in enumerate(blocks):
            e = min([out[p] for p in preds[i]], default=big)
            o = _scan(lines, e, None)[0]
            if (e, o) != (entry[i], out[i]):
                entry[i], out[i], changed = e, o, True
    bad, mfmas, checked = [], 0, 0
    for i, (_, lines, _, _) in enumerate(blocks):
        _, m, c = _scan(lines, entry[i], bad)
        mfmas, checked = mfmas + m, checked + c
    return bad, mfmas, checked


@pytest.mark.parametrize("kernel", KERNELS)
def test_agpr_accesses_wait_for_the_matrix_cores(asm, kernel):
    bad, mfmas, checked = agpr_hazards(kernel_body(asm, kernel))
    assert not bad, bad[:5]
    assert mfmas >= 64 and checked >= 256, (mfmas, checked)


def test_hazard_check_flags_an_early_read():
    # the checker itself, on hand-written snippets
    body = [";;#ASMSTART", "s_nop 1", "v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]",
            ";;#ASMEND", "v_mov_b32_e32 v9, v8", "v_accvgpr_read_b32 v10, a2"]
    bad, _, _ = agpr_hazards(body)
    assert bad == [("v_accvgpr_read_b32 v10, a2", 1)]
    drained = body[:4] + [";;#ASMSTART", "s_nop 7", "s_nop 7", "s_nop 7", ";;#ASMEND"] + body[4:]
    assert agpr_hazards(drained)[0] == []
    # a loop whose back edge reaches an AGPR read straight after the MFMA
    loop = [".LBB0_1:", "v_accvgpr_read_b32 v10, a2"] + drained[4:-1] + body[:4] + \
           ["s_cbranch_scc1 .LBB0_1", "s_endpgm"]
    assert agpr_hazards(loop)[0] == [("v_accvgpr_read_b32 v10, a2", 1)]
    assert agpr_hazards(loop[:-2] + drained[4:9] + loop[-2:])[0] == []


VALU_TO_MFMA_WAIT_STATES = 2


def _regs(operand):
    """Register set {(file, index)} of one operand text (v7, a[4:7], ...)."""
    m = re.match(r"([va])\[(\d+):(\d+)\]", operand)
    if m:
        return {(m.group(1), i) for i in range(int(m.group(2)), int(m.group(3)) + 1)}
    m = re.match(r"([va])(\d+)$", operand)
    return {(m.group(1), int(m.group(2)))} if m else set()


def _instrs(lines):
    """(instruction, inside inline asm) of a block's lines, labels and
    directives dropped."""
    out, in_asm = [], False
    for line in lines:
        raw = line.strip()
        if raw.startswith(";;#ASMSTART"):
            in_asm = True
        elif raw.startswith(";;#ASMEND"):
            in_asm = False
        else:
            s = line.split(";")[0].strip()
            if s and not s.startswith("."):
                out.append((s, in_asm))
    return out


def operand_write_hazards(body):
    """(writer, MFMA, wait states between them) for every VALU instruction
    that writes an operand register of an inline-asm MFMA fewer than
    VALU_TO_MFMA_WAIT_STATES wait states before it, on any path through the
    kernel's control flow; plus the number of inline-asm MFMAs."""
    blocks = _blocks(body)
    ins = [_instrs(b[1]) for b in blocks]
    index = {b[0]: i for i, b in enumerate(blocks) if b[0] is not None}
    preds = [[] for _ in blocks]
    for i, (_, _, succ, falls) in enumerate(blocks):
        for lab in succ:
            preds[index[lab]].append(i)
        if falls and i + 1 < len(blocks):
            preds[i + 1].append(i)
    bad, mfmas = [], 0
    for i in range(len(blocks)):
        for k, (s, in_asm) in enumerate(ins[i]):
            if not (in_asm and s.startswith("v_mfma")):
                continue
            mfmas += 1
            ops = [o.strip() for o in s.split(None, 1)[1].split(",")]
            srcs = set().union(*(_regs(o) for o in ops[1:4]))
            stack, seen = [(i, k - 1, 0)], set()
            while stack:
                bi, j, ws = stack.pop()
                while j >= 0 and ws < VALU_TO_MFMA_WAIT_STATES:
                    p = ins[bi][j][0]
                    op = p.split()[0]
                    if op.startswith("v_") and len(p.split()) > 1:
                        if _regs(p.split(None, 1)[1].split(",")[0].strip()) & srcs:
                            bad.append((p, s, ws))
                    ws += int(p.split()[1], 0) + 1 if op == "s_nop" else 1
                    j -= 1
                if j < 0 and ws < VALU_TO_MFMA_WAIT_STATES:
                    for q in preds[bi]:
                        if (q, ws) not in seen:
                            seen.add((q, ws))
                            stack.append((q, len(ins[q]) - 1, ws))
    return bad, mfmas


@pytest.mark.parametrize("kernel", KERNELS)
def test_asm_mfma_operands_not_written_just_before(asm, kernel):
    bad, mfmas = operand_write_hazards(kernel_body(asm, kernel))
    assert not bad, bad[:5]
    assert mfmas >= 64, mfmas


def test_operand_hazard_check_flags_a_late_write():
    # the checker itself, on hand-written snippets
    mfma = [";;#ASMSTART", "v_mfma_f32_16x16x32_bf16 a[0:3], v[0:3], v[4:7], a[0:3]", ";;#ASMEND"]
    body = ["v_cvt_pk_bf16_f32 v5, v8, v9", "v_mov_b32_e32 v20, v21"] + mfma
    assert operand_write_hazards(body) == ([("v_cvt_pk_bf16_f32 v5, v8, v9", mfma[1], 1)], 1)
    assert operand_write_hazards(body[:1] + ["s_nop 1"] + body[1:])[0] == []
    # an accumulator written by v_accvgpr_write at the end of a predecessor block
    # (the branch back to the MFMA is the one wait state between them)
    loop = [".LBB0_1:"] + mfma + ["s_cbranch_scc1 .LBB0_2", "v_accvgpr_write_b32 a2, v3",
                                  "s_branch .LBB0_1", ".LBB0_2:", "s_endpgm"]
    assert operand_write_hazards(loop)[0] == [("v_accvgpr_write_b32 a2, v3", mfma[1], 1)]
    # writes of other registers, or of the operands two wait states earlier, pass
    assert operand_write_hazards(["v_mov_b32_e32 v4, v9", "v_add_f32_e32 v30, v1, v2",
                                  "v_mov_b32_e32 v31, v1"] + mfma)[0] == []


@pytest.mark.parametrize("kernel", KERNELS)
def test_no_scratch_and_no_packed_fp32(asm, kernel):
    body = "\n".join(kernel_body(asm, kernel))
    assert not re.search(r"\bv_pk_(add|mul|fma)_f32\b", body)
    assert "scratch_" not in body
    meta = asm[asm.index(".amdgpu_metadata"):]
    entries = [e for e in re.split(r"\n  - \.", meta) if re.search(r"\.name:\s+" + kernel, e)]
    assert len(entries) == 1
    m = re.search(r"\.private_segment_fixed_size:\s+(\d+)", entries[0])
    assert m and int(m.group(1)) == 0
