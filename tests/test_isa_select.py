"""Generated-code checks of the selection kernel (CPU; needs hipcc).

The launched select_kernel instances run at about 180-234 VGPRs and the
compiler parks some scalar values (kernel arguments, addresses) in VGPR lanes
(`v_writelane_b32` / `v_readlane_b32`, SGPR spills) rather than in scratch.
These tests compile select.hip with the library's flags and check, for the
instances the BASELINE configs launch, that:

* no SGPR spill instruction sits in a basic block the compiler marks as part
  of a loop — the spills are straight-line code run once per (tile, head)
  row (the prologue and the selection phase), not per plane chunk;
* the MFMA scoring loop is found (so the check above is not vacuous);
* no scratch memory and no packed-fp32 VALU forms.
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

# select_kernel<ElemBf16, D, QUEST, KP, STREAM=false, ROWS=false>: c2 / c4
# Quest (128, true, 128), c3 Quest (128, true, 256), c4 K-mean (128, false,
# 128 / 256), c5 K-mean at head_dim 256 (256, false, 256)
PREFIX = "_ZN5ugbsa13select_kernelINS_8ElemBf16E"
INSTANCES = ["Li128ELb1ELi128ELb0ELb0", "Li128ELb1ELi256ELb0ELb0", "Li128ELb0ELi128ELb0ELb0",
             "Li128ELb0ELi256ELb0ELb0", "Li256ELb0ELi256ELb0ELb0"]
LABEL = re.compile(r"^(\.LBB\d+_\d+:|; %bb\.\d+:)")


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if not os.path.exists(G.HIPCC) and shutil.which("hipcc") is None:
        pytest.skip("hipcc not available")
    d = tmp_path_factory.mktemp("isa_select")
    src = os.path.join(G.CSRC, "select.hip")
    cmd = [G.HIPCC, *G.FLAGS, "--cuda-device-only", "-S", src, "-o", str(d / "k.s")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return (d / "k.s").read_text()


def kernel_body(text, kernel):
    lines = text.split("\n")
    start = next(i for i, l in enumerate(lines)
                 if l.startswith(kernel) and l.split(";")[0].rstrip().endswith(":"))
    end = next(i for i in range(start, len(lines)) if lines[i].startswith(".Lfunc_end"))
    return lines[start + 1:end]


def loop_membership(body):
    """(instruction, in_loop) for every instruction of a kernel body, from the
    compiler's block annotations: a block is in a loop when its label line (or
    the comment line right after it) says "Loop Header" or "in Loop:"."""
    out, in_loop = [], False
    for k, line in enumerate(body):
        if LABEL.match(line):
            note = line
            if k + 1 < len(body) and body[k + 1].strip().startswith("; =>"):
                note += body[k + 1]
            in_loop = "Loop Header" in note or "in Loop:" in note
            continue
        s = line.split(";")[0].strip()
        if s and not s.startswith("."):
            out.append((s, in_loop))
    return out


def spills_in_loops(body):
    ins = loop_membership(body)
    spills = [s for s, _ in ins if s.startswith(("v_writelane", "v_readlane"))]
    inside = [s for s, lp in ins if lp and s.startswith(("v_writelane", "v_readlane"))]
    mfma_in_loop = sum(1 for s, lp in ins if lp and s.startswith("v_mfma"))
    return spills, inside, mfma_in_loop


def test_spill_check_flags_a_spill_in_a_loop():
    body = ["v_writelane_b32 v1, s2, 0",
            ".LBB0_1:                                ; =>This Inner Loop Header: Depth=1",
            "v_mfma_f32_16x16x32_bf16 v[0:3], v[4:7], v[8:11], v[0:3]",
            "v_readlane_b32 s3, v1, 0",
            "s_cbranch_scc1 .LBB0_1",
            "; %bb.2:",
            "v_readlane_b32 s4, v1, 0",
            "s_endpgm"]
    spills, inside, mfmas = spills_in_loops(body)
    assert len(spills) == 3 and inside == ["v_readlane_b32 s3, v1, 0"] and mfmas == 1
    # the loop annotation on the line after a label
    body2 = [".LBB0_1:", "                 ; =>  This Inner Loop Header: Depth=2"] + body[2:]
    assert spills_in_loops(body2)[1] == ["v_readlane_b32 s3, v1, 0"]


@pytest.mark.parametrize("inst", INSTANCES)
def test_select_spills_stay_out_of_loops(asm, inst):
    spills, inside, mfmas = spills_in_loops(kernel_body(asm, PREFIX + inst))
    assert mfmas >= 16, "the MFMA scoring loop was not found"
    assert not inside, inside[:5]
    print(f"{inst}: {len(spills)} SGPR spill instructions, all outside loops")


@pytest.mark.parametrize("inst", INSTANCES)
def test_select_no_scratch_and_no_packed_fp32(asm, inst):
    kernel = PREFIX + inst
    body = "\n".join(kernel_body(asm, kernel))
    assert not re.search(r"\bv_pk_(add|mul|fma)_f32\b", body)
    assert "scratch_" not in body
    meta = asm[asm.index(".amdgpu_metadata"):]
    entries = [e for e in re.split(r"\n  - \.", meta) if re.search(r"\.name:\s+" + kernel, e)]
    assert len(entries) == 1
    m = re.search(r"\.private_segment_fixed_size:\s+(\d+)", entries[0])
    assert m and int(m.group(1)) == 0
