"""Host-side checks of the paired timing report (paged_decode.evidence), CPU only."""
import json
import os

import pytest

from paged_decode import evidence


def rows_for(times, rounds, unrolls=(32, 128)):
    return [{"variant": v, "unroll": u, "round": r, "order": 0, "us_per_call": times[v](u, r)}
            for v in times for u in unrolls for r in range(rounds)]


def test_paired_ratios_and_convergence():
    times = {"a": lambda u, r: 10.0 + r, "b": lambda u, r: (5.0 + r / 2) * (1.1 if u == 32 else 1)}
    report = evidence.paired_report(rows_for(times, 3), ["a", "b"], "a", 3)
    b = report["variants"]["b"]
    assert b["over_baseline"]["raw"] == [0.5, 0.5, 0.5]
    assert b["us_per_call"]["128"]["median"] == 5.5
    assert b["unroll_relative_delta"] == pytest.approx(0.1)
    assert not b["converged"] and report["variants"]["a"]["converged"]
    assert report["nonconverged"] == ["b"]


@pytest.mark.parametrize("mutate,match", [
    (lambda rows: rows.pop(), "incomplete"),
    (lambda rows: rows.append(dict(rows[0])), "duplicate"),
    (lambda rows: rows[0].update(us_per_call=float("nan")), "positive"),
    (lambda rows: rows[0].update(us_per_call=0), "positive"),
    (lambda rows: rows[0].update(variant="c"), "unexpected")])
def test_incomplete_or_invalid_matrices_are_refused(mutate, match):
    rows = rows_for({"a": lambda u, r: 1.0, "b": lambda u, r: 2.0}, 2)
    mutate(rows)
    with pytest.raises(ValueError, match=match):
        evidence.paired_report(rows, ["a", "b"], "a", 2)


def test_records_are_created_once(tmp_path):
    path = tmp_path / "sub" / "record.json"
    evidence.write_json_exclusive(path, {"x": 1})
    assert json.loads(path.read_text()) == {"x": 1}
    with pytest.raises(FileExistsError):
        evidence.write_json_exclusive(path, {"x": 2})
    with pytest.raises(ValueError):
        evidence.write_json_exclusive(tmp_path / "nan.json", {"x": float("nan")})


def test_summarize():
    s = evidence.summarize([3, 1, 2, 10])
    assert (s["count"], s["median"], s["min"], s["max"], s["p95"]) == (4, 2.5, 1.0, 10.0, 10.0)
    assert evidence.summarize([])["median"] is None


def test_bench_ab_refuses_unknown_variants_before_any_gpu_work():
    """bench.py --ab names its workload's variants (current or NAME=PATH outside the
    headline) and refuses others before it allocates anything on a GPU."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--ab", "bogus",
                          "--ab-workload", "edge_d64"], capture_output=True, text=True,
                         timeout=300, cwd=root)
    assert res.returncode != 0
    assert "unknown A/B variant 'bogus'" in res.stderr


def test_bench_ab_decode_variant_belongs_to_the_matched_workloads():
    """The decode variant (pd_matched_decode without counters) is a matched-decode call:
    a paged-backend workload refuses it before any GPU work."""
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    res = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--ab", "decode",
                          "--ab-workload", "edge_d64"], capture_output=True, text=True,
                         timeout=300, cwd=root)
    assert res.returncode != 0
    assert "decode variant is for the shape and partitions workloads" in res.stderr
