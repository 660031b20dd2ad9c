"""Host-only measurement policy (mirrors benchmark_protocol.py:4-19 of the reference).

A graph that unrolls ``unroll`` operator calls and is replayed ``replays``
times is charged elapsed / (replays * unroll) per operator; the convergence
check compares the 32- and 128-call unrolls.

Also the run-evidence helpers of the reference's tools (tools/_common.py:20-51
``fingerprint``, tools/benchmark_operator_v2.py:17-31 busy-GPU refusal) on ROCm
terms: ``amd-smi process --json`` lists the processes holding the GPU, and the
fingerprint records the ROCm release, device, CU count and the SHA-256 of the
kernel sources and library that were measured.
"""
import hashlib
import json
import math
import os
import platform
import subprocess

UNROLLS = (1, 8, 32, 128)
CONVERGENCE_LIMIT = .05


def interval_per_operator(elapsed_ms, replays, unroll):
    if not math.isfinite(elapsed_ms) or elapsed_ms <= 0:
        raise ValueError("positive finite elapsed interval required")
    if type(replays) is not int or replays < 1 or type(unroll) is not int or unroll < 1:
        raise ValueError("positive integer replay/unroll counts required")
    return elapsed_ms * 1000 / (replays * unroll)


def convergence_delta(t32, t128):
    if min(t32, t128) <= 0 or not all(map(math.isfinite, (t32, t128))):
        raise ValueError("positive finite timings required")
    return abs(t32 - t128) / t128


def resident_gpu_pids(run=subprocess.run):
    """PIDs that ``amd-smi process --json`` reports on the visible GPU(s).

    Raises RuntimeError when the tool fails, so an unknown state is never
    mistaken for an idle GPU.  Does not initialize the GPU in this process.
    """
    result = run(["amd-smi", "process", "--json"], capture_output=True, text=True, timeout=30)
    if result.returncode:
        raise RuntimeError(f"amd-smi process failed: {result.stderr.strip()[-400:]}")
    pids = set()

    def walk(node):
        if isinstance(node, dict):
            for key, value in node.items():
                if key.lower() == "pid" and isinstance(value, int):
                    pids.add(value)
                else:
                    walk(value)
        elif isinstance(node, list):
            for item in node:
                walk(item)

    text = result.stdout.strip()
    if text.startswith(("[", "{")):
        walk(json.loads(text))
    return pids


def require_idle_gpu(run=subprocess.run):
    """Refuse to benchmark a GPU other processes are using; call before any GPU work."""
    others = resident_gpu_pids(run) - {os.getpid()}
    if others:
        raise RuntimeError(f"Selected GPU has resident compute processes {sorted(others)}; "
                           "no benchmark launched")


def _sha256(path):
    try:
        with open(path, "rb") as f:
            return hashlib.sha256(f.read()).hexdigest()
    except OSError:
        return None


def fingerprint(torch=None):
    """Environment record of a measurement: software, device and measured sources."""
    here = os.path.dirname(os.path.abspath(__file__))
    csrc = os.path.join(os.path.dirname(here), "csrc")
    sources = sorted(f for f in os.listdir(csrc) if f.endswith((".hip", ".h", ".cpp"))) \
        if os.path.isdir(csrc) else []
    record = {
        "python": platform.python_version(),
        "host": platform.machine(),
        "rocm": None,
        "sources_sha256": {f: _sha256(os.path.join(csrc, f)) for f in sources},
        "library_sha256": _sha256(os.path.join(here, "libpaged_decode.so")),
    }
    try:
        with open("/opt/rocm/.info/version") as f:
            record["rocm"] = f.read().strip()
    except OSError:
        pass
    if torch is not None:
        record["torch"] = torch.__version__
        record["hip"] = getattr(torch.version, "hip", None)
        if torch.cuda.is_available():
            props = torch.cuda.get_device_properties(0)
            record["device"] = props.name
            record["gfx"] = getattr(props, "gcnArchName", None)
            record["compute_units"] = props.multi_processor_count
            record["memory_gb"] = round(props.total_memory / 2**30, 1)
    return record
