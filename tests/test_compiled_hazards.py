"""Two hazards the hardware leaves to software, checked in the compiled kernels (CPU:
hipcc's gfx950 assembly of pd_kernels.hip with the library's flags).

MFMA results.  The hardware does not interlock a vector-ALU read of an MFMA's
destination, so the compiler inserts wait states; it has been seen to insert too few
when a branch separates the MFMA from the read (a read two wait states after the last
P V MFMA gave stale outputs of one-tile sequences).  Every control-flow path after each
v_mfma is followed for 40 instructions: every vector-ALU read of the MFMA's destination
must come at least MIN_WAIT_STATES wait states after it, the fewest the compiler places
on straight-line paths of these kernels.

LDS results.  An LDS read writes its destination registers when its data returns;
until an s_waitcnt lgkmcnt(N) has covered it, reading those registers gives stale
values and writing them is undone by the late return.  The compiler tracks its own LDS
reads, but the kernels also issue LDS reads from inline asm (so that no compiler wait
counts the LDS copies in flight), whose results only a wait the kernel places makes
safe.  Every control-flow path after each LDS read that returns data is followed until
a wait covers it (LDS operations complete in order, so lgkmcnt(N) covers a read that
has at least N later LDS operations behind it): no instruction may read or write its
destination registers before that.

Both checkers are pinned on small planted cases.
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
LDS_HORIZON = 3000  # instructions followed per path after an LDS read


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


def _branch(t):
    """('branch' | 'cbranch', target label) of a branch to a label, else None."""
    m = re.match(r"s_(c?branch)\w*\s+(\.LBB\w+)", t)
    return (m.group(1), m.group(2)) if m else None


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
        br = _branch(t)
        if br:
            target = labels.get(br[1])
            if target is not None and (target, ws) not in seen:
                seen.add((target, ws))
                _walk(ins, labels, target, dst, ws + 1, depth + 1, seen, found, origin)
            if br[0] == "branch":
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


def _lds_returns(op):
    """An LDS operation that writes vector registers when it completes."""
    return op.startswith("ds_") and any(
        x in op for x in ("read", "load", "permute", "swizzle", "_rtn", "append", "consume"))


def _reads_writes(t):
    """(op, registers written, registers read) of one instruction, for the LDS check."""
    parts = t.split(None, 1)
    op = parts[0]
    rest = parts[1] if len(parts) > 1 else ""
    regs = [_regs(x.strip().split()[0]) if x.strip() else set() for x in rest.split(",")]
    # Stores, LDS writes and LDS copies (buffer_load ... lds) only read registers.
    if ("store" in op or (op.startswith("ds_") and not _lds_returns(op))
            or (op.startswith("buffer_load") and rest.rstrip().endswith(" lds"))):
        return op, set(), set().union(*regs) if regs else set()
    if not regs:
        return op, set(), set()
    dst = regs[0]
    src = set().union(*regs[1:]) if len(regs) > 1 else set()
    # Forms that keep part of the destination read it too.
    if op.startswith(("v_writelane", "v_fmac", "v_mac")) or "dpp" in t:
        src = src | dst
    return op, dst, src


def _lds_walk(ins, labels, start, dst, origin, found):
    stack, seen = [(start, 0, 0)], set()
    while stack:
        k, later, depth = stack.pop()
        while k < len(ins) and depth < LDS_HORIZON:
            t = ins[k]
            op, d, s = _reads_writes(t)
            if op == "s_waitcnt":
                m = re.search(r"lgkmcnt\((\d+)\)", t)
                if m and int(m.group(1)) <= later:
                    break
            if s & dst or d & dst:
                found.append((origin, k, t, "read" if s & dst else "write"))
                break
            if op.startswith("ds_"):
                later = min(later + 1, 16)
            if op in ("s_endpgm", "s_setpc_b64"):
                break
            br = _branch(t)
            if br:
                target = labels.get(br[1])
                if target is not None and (target, later) not in seen:
                    seen.add((target, later))
                    stack.append((target, later, depth + 1))
                if br[0] == "branch":
                    break
            k += 1
            depth += 1
        else:
            if depth >= LDS_HORIZON:
                found.append((origin, k, "<horizon>", "horizon"))


def unwaited_lds_results(asm_lines):
    """(read index, use index, use, 'read' | 'write' | 'horizon') of every access to an
    LDS read's destination that no wait covers on some control-flow path."""
    ins, labels = _parse(asm_lines)
    found = []
    for k, t in enumerate(ins):
        op = t.split(None, 1)[0]
        if _lds_returns(op):
            _, dst, _ = _reads_writes(t)
            _lds_walk(ins, labels, k + 1, dst, k, found)
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


LDS_PLANTED = """
\tds_read_b128 v[10:13], v10
\tds_read_b32 v20, v21
\ts_cbranch_scc1 .LBB0_2
\tv_mov_b32_e32 v1, v2
\tWAIT
.LBB0_2:
\tv_add_f32_e32 v50, v50, v11
\ts_endpgm
"""


def _lds(text):
    return [(f[3], f[2]) for f in unwaited_lds_results(text.splitlines())]


def test_lds_checker_pins_waits_paths_and_counts():
    # The taken branch reaches the reads of v11 (and of nothing of v20) with no wait.
    assert _lds(LDS_PLANTED.replace("WAIT", "s_waitcnt lgkmcnt(0)")) == [
        ("read", "v_add_f32_e32 v50, v50, v11")]
    # A wait before the branch covers both paths; lgkmcnt(1) covers the first read
    # (one LDS read behind it) but not the second, whose result nothing reads.
    early = LDS_PLANTED.replace("\ts_cbranch_scc1", "\ts_waitcnt lgkmcnt(0)\n\ts_cbranch_scc1")
    assert _lds(early.replace("WAIT", "s_nop 0")) == []
    one = LDS_PLANTED.replace("\ts_cbranch_scc1", "\ts_waitcnt lgkmcnt(1)\n\ts_cbranch_scc1")
    assert _lds(one.replace("WAIT", "s_nop 0")) == []
    one_read = one.replace("\tds_read_b32 v20, v21\n", "").replace("WAIT", "s_nop 0")
    # Without the second read, lgkmcnt(1) covers nothing: both paths reach the use.
    assert _lds(one_read) == [("read", "v_add_f32_e32 v50, v50, v11")] * 2
    # Writing a pending read's destination is caught like a read, also through
    # vmcnt-only waits.
    overwrite = early.replace("\ts_waitcnt lgkmcnt(0)\n\ts_cbranch", "\ts_waitcnt vmcnt(0)\n"
                              "\tv_mov_b32_e32 v20, 0\n\ts_cbranch").replace("WAIT", "s_nop 0")
    assert ("write", "v_mov_b32_e32 v20, 0") in _lds(overwrite)
    # LDS writes and copies into LDS read their operands: a store of the result is a use.
    store = LDS_PLANTED.replace("\ts_cbranch_scc1 .LBB0_2\n", "\tds_write_b32 v30, v20\n")
    assert ("read", "ds_write_b32 v30, v20") in _lds(store.replace("WAIT", "s_nop 0"))


@pytest.fixture(scope="module")
def kernel_asm(tmp_path_factory):
    if not shutil.which(HIPCC) and not os.path.exists(HIPCC):
        pytest.skip("needs hipcc")
    out = tmp_path_factory.mktemp("asm") / "pd_kernels.s"
    cmd = [HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature",
           "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-kernarg-preload-count=16",
           f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}", "--offload-device-only", "-S",
           os.path.join(CSRC, "pd_kernels.hip"), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, timeout=600)
    text = out.read_text()
    kernels = sorted(set(re.findall(r"^(_Z\w*kernel\w*):", text, re.M)))
    assert len(kernels) > 50
    return {name: text[text.index(name + ":"):text.index(".Lfunc_end", text.index(name + ":"))]
            for name in kernels}


def test_compiled_kernels_read_mfma_results_after_enough_wait_states(kernel_asm):
    bad = {}
    mfmas = 0
    for name, body in kernel_asm.items():
        mfmas += body.count("v_mfma")
        found = short_mfma_reads(body.splitlines())
        if found:
            bad[name] = found[:3]
    assert mfmas > 1000
    assert not bad, bad


def test_compiled_kernels_wait_for_every_lds_read_before_its_registers(kernel_asm):
    bad = {}
    reads = asm_reads = 0
    for name, body in kernel_asm.items():
        lines = body.splitlines()
        reads += sum(1 for t in _parse(lines)[0] if _lds_returns(t.split(None, 1)[0]))
        asm_reads += len(re.findall(r";;#ASMSTART\s*\n\s*ds_read", body))
        found = unwaited_lds_results(lines)
        if found:
            bad[name] = found[:3]
    assert reads > 10000 and asm_reads > 1000, (reads, asm_reads)
    assert not bad, bad
