"""MFMA result reads in the compiled kernels (CPU: hipcc's gfx950 assembly).

The hardware does not interlock a vector-ALU read of an MFMA's destination, so the
compiler inserts wait states; it has been seen to insert too few when a branch
separates the MFMA from the read (a read two wait states after the last P V MFMA gave
stale outputs of one-tile sequences).  This test compiles pd_kernels.hip to assembly
with the library's flags and follows every control-flow path after each v_mfma for 40
instructions: every vector-ALU read of the MFMA's destination must come at least
MIN_WAIT_STATES wait states after it, the fewest the compiler places on straight-line
paths of these kernels.  The checker itself is pinned on a small planted case.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "paged-decode-lab_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
MIN_WAIT_STATES = 8
HORIZON = 40


def _regs(tok):
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def _operands(text):
    parts = text.split(None, 1)
    op = parts[0]
    if len(parts) == 1:
        return op, set(), set()
    toks = [x.strip().split()[0] if x.strip() else "" for x in parts[1].split(",")]
    dst = _regs(toks[0]) if toks else set()
    src = set()
    for x in toks[1:]:
        src |= _regs(x)
    return op, dst, src


def _parse(lines):
    ins, labels = [], {}
    for line in lines:
        t = line.strip()
        if not t or t.startswith(";"):
            continue
        m = re.match(r"^(\.LBB\w+):", t)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if t.startswith("."):
            continue
        ins.append(t)
    return ins, labels


def _walk(ins, labels, k, dst, ws, depth, seen, found, origin):
    while k < len(ins) and depth < HORIZON:
        t = ins[k]
        op, d, s = _operands(t)
        if op == "s_nop":
            ws += int(t.split()[1]) + 1
            k += 1
            depth += 1
            continue
        if op.startswith("v_") and not op.startswith("v_mfma") and s & dst:
            if ws < MIN_WAIT_STATES:
                found.append((origin, k, t, ws))
            return
        if op.startswith("v_mfma") and (d & dst or s & dst):
            return
        if (op.startswith("v_") or "_load" in op or op.startswith("ds_read")) and d & dst:
            return
        if op == "s_endpgm":
            return
        m = re.match(r"s_(c?branch)\w*\s+(\.LBB\w+)", t)
        if m:
            target = labels.get(m.group(2))
            if target is not None and (target, ws) not in seen:
                seen.add((target, ws))
                _walk(ins, labels, target, dst, ws + 1, depth + 1, seen, found, origin)
            if m.group(1) == "branch":
                return
        ws += 1
        k += 1
        depth += 1


def short_mfma_reads(asm_lines):
    """(mfma index, read index, read, wait states) of every read closer than the minimum."""
    ins, labels = _parse(asm_lines)
    found = []
    for k, t in enumerate(ins):
        if t.startswith("v_mfma"):
            _, dst, _ = _operands(t)
            _walk(ins, labels, k + 1, dst, 0, 0, set(), found, k)
    return found


PLANTED = """
\tv_mfma_f32_16x16x32_bf16 v[62:65], v[62:65], v[136:139], v[150:153]
\ts_cbranch_scc1 .LBB0_2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
\tv_mov_b32_e32 v1, v2
.LBB0_2:
\tv_add_f32_e32 v50, v50, v62
\ts_endpgm
"""


def test_checker_finds_a_read_behind_a_branch():
    found = short_mfma_reads(PLANTED.splitlines())
    # The taken branch reaches the read after 1 wait state; the fall-through after 10.
    assert [f[3] for f in found] == [1]
    padded = PLANTED.replace("\ts_cbranch_scc1", "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_cbranch_scc1")
    assert short_mfma_reads(padded.splitlines()) == []


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="needs hipcc")
def test_compiled_kernels_read_mfma_results_after_enough_wait_states(tmp_path):
    out = tmp_path / "pd_kernels.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", "--offload-device-only", "-S",
           os.path.join(CSRC, "pd_kernels.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text()
    kernels = sorted(set(re.findall(r"^(_Z\w*kernel\w*):", text, re.M)))
    assert len(kernels) > 50
    bad = {}
    mfmas = 0
    for name in kernels:
        body = text[text.index(name + ":"):text.index(".Lfunc_end", text.index(name + ":"))]
        mfmas += body.count("v_mfma")
        found = short_mfma_reads(body.splitlines())
        if found:
            bad[name] = found[:3]
    assert mfmas > 1000
    assert not bad, bad
