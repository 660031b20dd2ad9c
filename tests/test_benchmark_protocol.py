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
