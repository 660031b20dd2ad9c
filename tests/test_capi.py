"""The C-ABI library loads and exports every function include/paged_decode.h declares.

No kernel is launched here: the launcher calls below fail argument validation
before any HIP API call.
"""
import ctypes
import os
import re

import numpy as np
import pytest
import torch

from paged_decode import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                      "include", "paged_decode.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(pd_[a-z_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported_and_bound():
    lib = _native.lib()
    names = declared_functions()
    assert names == sorted(_native.SIGNATURES), names
    for name in names:
        assert getattr(lib, name) is not None
    assert lib.pd_abi_version() == 7


def test_error_reporting_and_validation_without_launching():
    lib = _native.lib()
    null = ctypes.c_void_p(0)
    # head_dim 80 is rejected before any device call.
    status = lib.pd_partition(null, 0, 0, null, null, null, 0, 1, null, null, null,
                              1, 4, 1, 80, 1, 64, 64, 0.1, null)
    assert status == _native.PD_EINVAL
    assert b"head_dim" in lib.pd_last_error()
    status = lib.pd_lse_merge(null, null, null, 1, 4, 256, 0, 1, null)
    assert status == _native.PD_EINVAL and b"splits" in lib.pd_last_error()
    status = lib.pd_base(null, 0, 0, null, null, null, 0, 1, null, null, 1, 4, 3, 64, 0.1, null)
    assert status == _native.PD_EINVAL and b"divisible" in lib.pd_last_error()
    status = lib.pd_ml_merge(null, null, null, null, 1, 4, 64, 0, null)
    assert status == _native.PD_EINVAL and b"partitions" in lib.pd_last_error()
    with pytest.raises(ValueError, match="head_dim"):
        _native.check(lib.pd_split_fixed(null, 0, 0, null, null, null, 0, 1, null, null, null,
                                         null, 1, 4, 1, 96, 1, 1024, 0.1, null))


def test_metadata_validation_on_host_copies():
    # reference tests/test_reference.py:54-57 cases, through the native check.
    for length, table in [(-1, [[0]]), (257, [[0]]), (1, [[-1]]), (1, [[2]])]:
        t = torch.tensor(table, dtype=torch.int32)
        lens = torch.tensor([length], dtype=torch.int32)
        with pytest.raises(ValueError):
            _native.validate_metadata(t, lens, 2, 256)
    good = torch.tensor([[1, -1], [0, 1]], dtype=torch.int32)
    _native.validate_metadata(good, torch.tensor([200, 300], dtype=torch.int32), 2, 512)
    # Padding entries beyond the live pages may be anything.
    _native.validate_metadata(torch.tensor([[1, 99]], dtype=torch.int32),
                              torch.tensor([256], dtype=torch.int32), 2, 512)


def test_validate_device_metadata_accepts_cpu_tensors_and_rejects_bad_rows():
    from paged_decode.runtime import validate_device_metadata
    table = torch.from_numpy(np.array([[0, 1], [2, -1]], dtype=np.int32))
    validate_device_metadata(table, torch.tensor([300, 5], dtype=torch.int32), 3, 512)
    with pytest.raises(ValueError, match="live page"):
        validate_device_metadata(table, torch.tensor([300, 300], dtype=torch.int32), 3, 512)
    with pytest.raises(ValueError, match="batch"):
        validate_device_metadata(table, torch.tensor([1], dtype=torch.int32), 3, 512)


def test_validate_device_metadata_rejects_non_integral_and_wide_values():
    # reference.py:14-15: float or bool metadata is rejected, not truncated.
    from paged_decode.runtime import validate_device_metadata
    table = torch.tensor([[0, 1]], dtype=torch.int32)
    with pytest.raises(ValueError, match="integral"):
        validate_device_metadata(table.float(), torch.tensor([300], dtype=torch.int32), 2, 512)
    with pytest.raises(ValueError, match="integral"):
        validate_device_metadata(table, torch.tensor([1.5]), 2, 512)
    with pytest.raises(ValueError, match="integral"):
        validate_device_metadata(table, torch.tensor([True]), 2, 512)
    # int64 values past int32 saturate instead of wrapping: 2^32 + 5 would wrap to 5.
    with pytest.raises(ValueError, match="capacity"):
        validate_device_metadata(table, torch.tensor([2 ** 32 + 5], dtype=torch.int64), 2, 512)
    with pytest.raises(ValueError, match="capacity"):
        validate_device_metadata(table, torch.tensor([-(2 ** 32) + 5], dtype=torch.int64), 2, 512)
    # A live page entry of 2^32 would wrap to page 0.
    wide = torch.tensor([[2 ** 32, 1]], dtype=torch.int64)
    with pytest.raises(ValueError, match="live page"):
        validate_device_metadata(wide, torch.tensor([300], dtype=torch.int64), 2, 512)
    validate_device_metadata(table.long(), torch.tensor([300], dtype=torch.int64), 2, 512)


def test_kv_writes_reject_host_tensors_before_launching():
    from paged_decode.kv_write import store_kvcache, write_pages
    key = torch.zeros((1, 2, 3, 64), dtype=torch.bfloat16)
    pages = torch.zeros((2, 256, 2, 64), dtype=torch.bfloat16)
    tables = torch.zeros((1, 2), dtype=torch.int32)
    positions = torch.arange(3, dtype=torch.int64)
    with pytest.raises(ValueError, match="CUDA device"):
        write_pages(key, key.clone(), pages, pages.clone(), tables, positions)
    rows = torch.zeros((3, 2, 64), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA device"):
        store_kvcache(rows, rows.clone(), pages, pages.clone(), torch.zeros(3, dtype=torch.int32))


def test_lse_merge_lane_count_is_validated():
    lib = _native.lib()
    null = ctypes.c_void_p(0)
    for lanes, splits in ((3, 36), (128, 128), (64, 8), (0, 4)):
        status = lib.pd_lse_merge(null, null, null, 1, 4, 256, splits, lanes, null)
        assert status == _native.PD_EINVAL and b"lse_lanes" in lib.pd_last_error(), (lanes, splits)


def test_noalloc_rejects_workspaces_past_its_static_scratch():
    # batch 64 x 32 heads x 32 splits x 257 floats = 67 MB > 16 MiB: rejected before any
    # device call (the scratch address is looked up only for calls that fit).
    lib = _native.lib()
    null = ctypes.c_void_p(0)
    status = lib.pd_matched_decode_noalloc(null, 0, 0, null, null, null, 0, 128, null, null,
                                           64, 32, 8, 256, 32, 1024, 64, 0.0625, null)
    assert status == _native.PD_EINVAL and b"static scratch" in lib.pd_last_error()


def test_matched_decode_without_counters_needs_an_output():
    # Without counters pd_matched_decode runs the partition and the merge (or, for a plan
    # of one split, the partition alone writing the output): a NULL output is refused
    # before any device call.
    lib = _native.lib()
    null = ctypes.c_void_p(0)
    status = lib.pd_matched_decode(null, 0, 0, null, null, null, 0, 9, null, null, null, null,
                                   null, 1, 16, 4, 256, 1, 2304, 64, 0.0625, null)
    assert status == _native.PD_EINVAL and b"invalid matched workspace" in lib.pd_last_error()
