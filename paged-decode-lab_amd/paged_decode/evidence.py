"""Paired timing reports: A/B comparisons of operator variants in one process.

The counterpart of the reference's evidence tooling (tools/_common.py:12-17
exclusive-create JSON records and ``summarize``; tools/report_fragment_resident.py:18-60
paired summaries).  Every variant is captured as one hipGraph per unroll (32 and
128 calls, the reference convention); each round replays every graph
``replays`` times in a seeded shuffled order, so slow drift of the device
(clocks, temperature) spreads over the variants instead of favouring one.
The report gives, per variant and unroll, the median, minimum and maximum of
the rounds, the 32- vs 128-call convergence (3% gate), and per-round paired
ratios against a baseline variant at unroll 128 (the ratio of two timings
taken in the same round, then summarized over rounds).

Variants are plain callables (one operator call each), so two builds of the
library can be compared in one process: load the second build with
``_native.load_library`` and pass it as ``library=`` in one variant's calls.
"""
import json
import math
import os
import random
import statistics

UNROLLS = (32, 128)
CONVERGENCE_GATE = 0.03


def write_json_exclusive(path, data):
    """Writes ``data`` as JSON to a file that must not exist yet (no silent overwrite of a
    record); NaN and infinity are refused."""
    text = json.dumps(data, ensure_ascii=False, indent=2, allow_nan=False) + "\n"
    parent = os.path.dirname(os.path.abspath(path))
    os.makedirs(parent, exist_ok=True)
    with open(path, "x", encoding="utf-8") as stream:
        stream.write(text)


def summarize(values):
    """count, median, nearest-rank p95, min, max (tools/_common.py of the reference)."""
    values = [float(v) for v in values]
    if not values:
        return {"count": 0, "median": None, "p95": None, "min": None, "max": None}
    ordered = sorted(values)
    return {"count": len(values), "median": statistics.median(values),
            "p95": ordered[math.ceil(0.95 * len(values)) - 1],
            "min": ordered[0], "max": ordered[-1]}


def _describe(values):
    return {"median": statistics.median(values), "min": min(values), "max": max(values),
            "raw": list(values)}


def _positive(value):
    if (not isinstance(value, (int, float)) or isinstance(value, bool)
            or not math.isfinite(value) or value <= 0):
        raise ValueError("positive finite timing required")
    return float(value)


def paired_timings(torch, variants, *, rounds=5, replays=20, unrolls=UNROLLS, seed=20261105,
                   warmup=3):
    """Times every variant (name -> callable making one operator call on the current
    stream) as graphs of each unroll.  Returns rows {variant, unroll, round, order,
    us_per_call}; ``rounds`` rounds, each in a seeded shuffled order."""
    stream = torch.cuda.Stream()
    graphs = {}
    for name, fn in variants.items():
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for _ in range(warmup):
                fn()
        torch.cuda.current_stream().wait_stream(stream)
        torch.cuda.synchronize()
        for unroll in unrolls:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(unroll):
                    fn()
            graph.replay()
            graphs[name, unroll] = graph
    torch.cuda.synchronize()
    rng = random.Random(seed)
    rows = []
    for r in range(rounds):
        order = list(graphs)
        rng.shuffle(order)
        for ordinal, (name, unroll) in enumerate(order):
            graph = graphs[name, unroll]
            for _ in range(3):
                graph.replay()
            torch.cuda.synchronize()
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(replays):
                graph.replay()
            end.record()
            end.synchronize()
            rows.append({"variant": name, "unroll": unroll, "round": r, "order": ordinal,
                         "us_per_call": start.elapsed_time(end) * 1000.0 / (replays * unroll)})
    return rows


def paired_report(rows, variants, baseline, rounds, unrolls=UNROLLS):
    """Checks that ``rows`` hold exactly one positive timing per (variant, unroll, round)
    and summarizes them: per-unroll times, convergence, and paired ratios to
    ``baseline`` at the largest unroll."""
    if baseline not in variants:
        raise ValueError("baseline must be one of the variants")
    expected = {(v, u, r) for v in variants for u in unrolls for r in range(rounds)}
    values = {}
    for row in rows:
        key = (row["variant"], row["unroll"], row["round"])
        if key not in expected or key in values:
            raise ValueError(f"unexpected or duplicate timing {key}")
        values[key] = _positive(row["us_per_call"])
    if set(values) != expected:
        raise ValueError("incomplete timing matrix")
    top, low = max(unrolls), min(unrolls)
    report = {"baseline": baseline, "rounds": rounds, "unrolls": list(unrolls), "variants": {}}
    for v in variants:
        times = {str(u): _describe([values[v, u, r] for r in range(rounds)]) for u in unrolls}
        delta = times[str(low)]["median"] / times[str(top)]["median"] - 1.0
        ratio = _describe([values[v, top, r] / values[baseline, top, r] for r in range(rounds)])
        report["variants"][v] = {"us_per_call": times, "unroll_relative_delta": delta,
                                 "converged": abs(delta) <= CONVERGENCE_GATE,
                                 "over_baseline": ratio}
    report["nonconverged"] = [v for v, x in report["variants"].items() if not x["converged"]]
    return report
