"""Parity gate for bf16 operator outputs against the CPU oracle.

An output element passes when it is within one bf16 ulp of the oracle's value,
or when |actual - oracle| <= A + ulp_bf16(|oracle| + A) + 2^-18, where A is
the oracle's rounding-ambiguity bound for that element (zero where none is
given).  At most 0.5% of all elements may be more than one ulp away, which
catches systematic protocol errors even where A is generous.

Why A.  The matched protocol rounds every probability p to bf16 before the PV
product (matched_splitkv.py:86).  The operator and the oracle compute the same
fp32 scores and exp2 with different rounding (MFMA vs BLAS summation order,
v_exp_f32 vs NumPy), so a p within a few float32 ulps of a bf16 rounding
midpoint can round up on one side and down on the other; that moves the
output by ulp_bf16(p) * |v| / denom times the split's merge weight.  Such
flips cannot be removed by any implementation that is not bit-identical in
its fp32 arithmetic.  oracle.matched.matched_decode_with_bounds returns A as
the sum of that quantity over every p within 128 float32 ulps of a midpoint.
The 2^-18 term covers float32 accumulation-order noise on outputs that are
close to zero.  Planted protocol mistakes (forward tile walk, no bf16(p)) fail
this gate (tests/test_oracle_matched.py::test_parity_gate_rejects_protocol_mistakes).
"""
import os

import numpy as np

from oracle.numerics import bf16_ulp_distance

NOISE_FLOOR = 2.0 ** -18
MAX_FRACTION_BEYOND_ONE_ULP = 5e-3


# (test id, label, statistics) of every check that passed, for the summary that
# conftest.py prints at the end of the run.
RECORDS = []


def record(where="", **stats):
    """Keeps the statistics of a passed check under the running test's id."""
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]
    RECORDS.append((test, where, stats))


def bf16_ulp_of(x):
    x = np.abs(np.asarray(x, dtype=np.float64))
    _, e = np.frexp(np.where(x > 0, x, 1.0))
    return np.where(x > 0, np.ldexp(1.0, e - 8), 0.0)


def parity_stats(actual, expected, ambiguity=None):
    actual = np.asarray(actual, dtype=np.float32)
    expected = np.asarray(expected, dtype=np.float32)
    amb = np.zeros(expected.shape) if ambiguity is None else np.asarray(ambiguity, np.float64)
    ulps = bf16_ulp_distance(actual, expected)
    diff = np.abs(actual.astype(np.float64) - expected.astype(np.float64))
    allowed = amb + bf16_ulp_of(np.abs(expected) + amb) + NOISE_FLOOR
    ok = (ulps <= 1) | (diff <= allowed)
    # ulp counts of outputs that cancel to near zero say nothing (a 1e-8 output
    # next to 1e-6 is thousands of ulps away), so the summary counts ulps only for
    # outputs of magnitude 2^-10 or more
    sizable = np.abs(expected) >= 2.0 ** -10
    return dict(ok=ok, max_ulps=int(ulps.max(initial=0)),
                max_ulps_sizable=int(np.where(sizable, ulps, 0).max(initial=0)),
                beyond_one_ulp=float((ulps > 1).mean()),
                one_ulp=float((ulps == 1).mean()),
                max_abs=float(diff.max(initial=0.0)),
                ambiguous_elements=float((amb > 0).mean()))


def assert_parity(actual, expected, where="", ambiguity=None):
    stats = parity_stats(actual, expected, ambiguity)
    ok = stats.pop("ok")
    summary = ", ".join(f"{k}={v:.3g}" for k, v in stats.items())
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        extra = "" if ambiguity is None else f", bound {float(np.asarray(ambiguity)[i]):.3g}"
        raise AssertionError(f"{where}: {int((~ok).sum())} of {ok.size} outputs outside the "
                             f"parity gate ({summary}); first at {i}: got {actual[i]!r}, "
                             f"oracle {expected[i]!r}{extra}")
    if stats["beyond_one_ulp"] > MAX_FRACTION_BEYOND_ONE_ULP:
        raise AssertionError(f"{where}: too many outputs beyond one bf16 ulp ({summary})")
    print(f"parity {where}: {summary}")
    record(where, max_ulps_sizable=stats["max_ulps_sizable"],
           beyond_one_ulp=stats["beyond_one_ulp"],
           one_ulp=stats["one_ulp"], max_abs_vs_oracle=stats["max_abs"])
    return stats
