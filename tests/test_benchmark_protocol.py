"""Measurement arithmetic (reference tests/test_benchmark_protocol.py:5-14)."""
import pytest

from paged_decode.benchmark_protocol import convergence_delta, interval_per_operator


def test_graph_nodes_are_counted_as_logical_operators():
    # 1280 operators in 1.28ms is 1us/operator, not 128us/replay.
    assert interval_per_operator(1.28, 10, 128) == 1.
    assert interval_per_operator(1.28, 1280, 1) == 1.
    assert convergence_delta(10.4, 10.) == pytest.approx(.04)


@pytest.mark.parametrize("args", [(0., 10, 128), (float("nan"), 10, 128), (1., 0, 128),
                                  (1., 10, 0), (1., 10, True)])
def test_invalid_denominators_cannot_produce_latency(args):
    with pytest.raises(ValueError):
        interval_per_operator(*args)


@pytest.mark.parametrize("args", [(0., 1.), (1., float("inf")), (-1., 2.)])
def test_invalid_convergence_inputs(args):
    with pytest.raises(ValueError):
        convergence_delta(*args)


def test_busy_gpu_is_rejected_before_gpu_initialization(monkeypatch):
    # reference tests/test_benchmark_protocol.py:17-31, with amd-smi in place of nvidia-smi
    import json
    from types import SimpleNamespace
    from paged_decode import benchmark_protocol as bp

    listing = [{"gpu": 0, "process_list": [{"process_info": {"name": "other", "pid": 12345}}]}]
    calls = []

    def run(cmd, **kwargs):
        calls.append(cmd)
        return SimpleNamespace(returncode=0, stderr="", stdout=json.dumps(listing))

    with pytest.raises(RuntimeError, match="resident compute processes"):
        bp.require_idle_gpu(run)
    assert calls == [["amd-smi", "process", "--json"]]


def test_idle_gpu_and_unknown_state(monkeypatch):
    from types import SimpleNamespace
    from paged_decode import benchmark_protocol as bp
    idle = lambda cmd, **kw: SimpleNamespace(returncode=0, stderr="", stdout='[{"gpu": 0, "process_list": []}]')
    bp.require_idle_gpu(idle)
    assert bp.resident_gpu_pids(lambda cmd, **kw: SimpleNamespace(
        returncode=0, stderr="", stdout="No running processes detected")) == set()
    failed = lambda cmd, **kw: SimpleNamespace(returncode=1, stderr="driver not loaded", stdout="")
    with pytest.raises(RuntimeError, match="amd-smi process failed"):
        bp.require_idle_gpu(failed)


def test_fingerprint_records_sources_without_a_gpu():
    from paged_decode.benchmark_protocol import fingerprint
    record = fingerprint()
    assert "pd_kernels.hip" in record["sources_sha256"]
    assert all(v is None or len(v) == 64 for v in record["sources_sha256"].values())
