"""DecodeSpec / engine-option contract (reference tests/test_reference.py:60-81)."""
import pytest

from paged_decode.spec import (BACKENDS, DecodeSpec, canonical_backend,
                               validate_engine_options)


def test_spec_and_memory():
    spec = DecodeSpec(32, 32, 8, 128, 8192)
    assert spec.partitions == 8
    assert spec.table_width == 32
    assert spec.split_workspace_bytes == 32 * 32 * 8 * 130 * 4


@pytest.mark.parametrize("kwargs", [{"head_dim": 80}, {"page_size": 16}, {"num_kv_heads": 3},
                                    {"max_batch": 0}, {"max_context_len": -1},
                                    {"max_batch": True}, {"num_heads": 4.0}])
def test_unsupported_geometry(kwargs):
    values = dict(max_batch=8, num_heads=4, num_kv_heads=2, head_dim=64, max_context_len=2048)
    values.update(kwargs)
    with pytest.raises(ValueError):
        DecodeSpec(**values)


@pytest.mark.parametrize("backend,tp,page", [("typo", 1, 256), ("triton_base", 2, 256),
                                            ("triton_splitk", 1, 512), ("hip_base", 2, 256),
                                            ("triton_tc", 1, 256)])
def test_engine_rejects_unsupported_options(backend, tp, page):
    with pytest.raises(ValueError):
        validate_engine_options(backend, tp, page, 32, 8192)


def test_engine_accepts_supported_options():
    for backend in BACKENDS:
        validate_engine_options(backend, 1, 256, 32, 8192)
    validate_engine_options("flash_attn", 4, 16, 1, 1)


def test_backend_aliases_name_the_same_kernels():
    assert canonical_backend("triton_base") == canonical_backend("hip_base") == "hip_base"
    assert canonical_backend("triton_splitk") == canonical_backend("hip_splitk") == "hip_splitk"
    for bad in ("flash_attn", "triton_tc", "triton_tc_splitk", "nope"):
        with pytest.raises(ValueError, match="unknown decode_backend"):
            canonical_backend(bad)
