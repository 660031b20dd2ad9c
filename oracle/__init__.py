"""CPU oracle for the paged decode operator — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

This package restates, on the CPU, the algorithms of the reference repository
(lingjiekong04/paged-decode-lab) for the paged decode hot path, so the HIP
operator in ``paged_decode`` can be checked against it on identical inputs.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import anything from here, and only as the checker or as the
timed CPU baseline.  The product package never imports it: a missing HIP
extension raises instead of falling back to these functions.

Modules
-------
numerics   bf16 rounding, single-rounding f32 FMA, ln by change of base
reference  restates src/paged_decode/reference.py (NumPy CPU path, dense oracle)
splitk     restates src/paged_decode/kernels.py (_base, _split, _merge)
matched    restates src/paged_decode/matched_splitkv.py (normalized partial + LSE)
plan       restates src/paged_decode/splitkv_plan.py and src/paged_decode/spec.py

Pinning status of each function (what checks it besides its own formula) is in
each module's docstring.  Functions whose exact rounding cannot be pinned
without the reference's CUDA toolchain say "parity unpinned" for that detail.
"""
