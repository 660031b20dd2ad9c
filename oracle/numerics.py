"""Scalar/array numerics shared by the oracle restatements (test infrastructure).

* ``bf16_round``: float32 -> bfloat16 round-to-nearest-even, returned as float32
  values.  The reference converts with Triton's ``.to(tl.bfloat16)`` and stores
  fp32 into bf16 pointers (matched_splitkv.py:86, kernels.py:41); both are RNE.
  Pinned by tests/test_oracle_numerics.py against torch's bf16 cast.
* ``fma32``: single-rounding float32 fused multiply-add, computed exactly in
  float64 and rounded once (products of two float32 fit in 48 bits).  Used where
  the reference calls ``tl.fma`` (matched_splitkv.py:80, 95, 125).
* ``ln32``: natural log as log2(x) * RN(ln 2) in float32, i.e. the change of base
  the reference's ``_fast_log`` performs (matched_splitkv.py:44-49).  The
  log2 approximation error of the reference's instruction is not modelled:
  parity unpinned below float32 rounding for that detail (it is far below the
  bf16 tolerance the outputs are checked at).
"""
import numpy as np

F32 = np.float32
LOG2E = 1.4426950408889634          # matched_splitkv.py:363 (double literal)
LN2_F32 = np.float32(np.log(2.0))   # ln 2 rounded to nearest float32


def f32(x):
    return np.asarray(x, dtype=np.float32)


def bf16_round(x):
    """Round float32 values to the nearest bfloat16 (ties to even); NaN stays NaN."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.nan
    return out.reshape(np.shape(x))


def bf16_bits(x):
    """uint16 bit pattern of float32 values rounded to bf16."""
    return (bf16_round(x).view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(bits):
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def fma32(a, b, c):
    """float32 fma(a, b, c) with a single rounding (exact product in float64)."""
    a64 = np.asarray(a, dtype=np.float32).astype(np.float64)
    b64 = np.asarray(b, dtype=np.float32).astype(np.float64)
    c64 = np.asarray(c, dtype=np.float32).astype(np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        return (a64 * b64 + c64).astype(np.float32)


def ln32(x):
    """ln(x) = log2(x) * RN(ln 2), float32 (change of base)."""
    with np.errstate(divide="ignore", invalid="ignore"):
        return (np.log2(np.asarray(x, dtype=np.float32)) * LN2_F32).astype(np.float32)


def exp2_32(x):
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        return np.exp2(np.asarray(x, dtype=np.float32)).astype(np.float32)


def exp32(x):
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        return np.exp(np.asarray(x, dtype=np.float32)).astype(np.float32)


def next_pow2(n):
    return 1 << (int(n) - 1).bit_length()


def bf16_ulp_distance(a, b):
    """Distance in bf16 units-in-the-last-place between two bf16-valued arrays.

    Uses the monotone integer mapping of the bf16 bit patterns, so +0 and -0 are
    0 apart and adjacent representable values are 1 apart.
    """
    def key(x):
        bits = bf16_bits(x).astype(np.int32)
        return np.where(bits & 0x8000, 0x8000 - bits, bits)
    return np.abs(key(a) - key(b))
