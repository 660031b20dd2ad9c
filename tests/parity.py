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
the sum of that quantity over every p within AMBIGUITY_ULPS (32) float32 ulps of a
midpoint.
The 2^-18 term covers float32 accumulation-order noise on outputs that are
close to zero.  Planted protocol mistakes (forward tile walk, no bf16(p)) fail
this gate (tests/test_oracle_matched.py::test_parity_gate_rejects_protocol_mistakes).

Attribution.  Each passed check records its worst output beyond one ulp (most ulps,
then largest difference): its ulps, |difference|, the bound A at that element, the
allowance A + ulp + 2^-18 it met, the oracle value and, where the caller passes the
oracle's counts, the number of ambiguous p values behind its row; and the same for
the worst among outputs of magnitude 2^-10 or more.  An element with A = 0 passed on
the 2^-18 floor alone (an output that cancels to near zero).
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


def worst_beyond_one_ulp(ulps, diff, amb, allowed, expected, ambiguous_p=None, among=None):
    """The output beyond one ulp with the most ulps (ties: largest difference), among the
    outputs ``among`` selects (all by default), and what admitted it; None when every such
    output is within one ulp."""
    beyond = ulps > 1
    if among is not None:
        beyond = beyond & among
    if not beyond.any():
        return None
    where = np.argwhere(beyond)
    order = np.lexsort((diff[beyond], ulps[beyond]))
    i = tuple(int(x) for x in where[order[-1]])
    worst = dict(ulps=int(ulps[i]), abs_diff=float(diff[i]), bound=float(amb[i]),
                 allowed=float(allowed[i]), oracle=float(expected[i]), index=i)
    if ambiguous_p is not None:
        worst["ambiguous_p"] = int(np.asarray(ambiguous_p)[i[:-1]])
    return worst


def parity_stats(actual, expected, ambiguity=None, ambiguous_p=None):
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
                ambiguous_elements=float((amb > 0).mean()),
                worst=worst_beyond_one_ulp(ulps, diff, amb, allowed, expected, ambiguous_p),
                worst_sizable=worst_beyond_one_ulp(ulps, diff, amb, allowed, expected,
                                                   ambiguous_p, sizable))


def assert_parity(actual, expected, where="", ambiguity=None, ambiguous_p=None):
    stats = parity_stats(actual, expected, ambiguity, ambiguous_p)
    ok = stats.pop("ok")
    worst = stats.pop("worst")
    worst_sizable = stats.pop("worst_sizable")
    summary = ", ".join(f"{k}={v:.3g}" for k, v in stats.items())
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        extra = "" if ambiguity is None else f", bound {float(np.asarray(ambiguity)[i]):.3g}"
        raise AssertionError(f"{where}: {int((~ok).sum())} of {ok.size} outputs outside the "
                             f"parity gate ({summary}); first at {i}: got {actual[i]!r}, "
                             f"oracle {expected[i]!r}{extra}")
    if stats["beyond_one_ulp"] > MAX_FRACTION_BEYOND_ONE_ULP:
        raise AssertionError(f"{where}: too many outputs beyond one bf16 ulp ({summary})")
    print(f"parity {where}: {summary}" + (f"; worst beyond one ulp {worst}" if worst else ""))
    record(where, max_ulps_sizable=stats["max_ulps_sizable"],
           beyond_one_ulp=stats["beyond_one_ulp"],
           one_ulp=stats["one_ulp"], max_abs_vs_oracle=stats["max_abs"], worst=worst,
           worst_sizable=worst_sizable)
    return stats
