"""ctypes binding of libpaged_decode.so (declared in include/paged_decode.h).

torch is imported before the library is opened so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
loaded: streams, graphs and device pointers are then shared with torch.

There is no fallback: if the library is missing, every entry point raises.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libpaged_decode.so")

PD_OK, PD_EINVAL, PD_ELAUNCH = 0, 1, 2

_i32, _i64, _dbl, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_double, ctypes.c_void_p


class Plan(ctypes.Structure):
    _fields_ = [("splits", _i32), ("tile_tokens", _i32), ("tokens_per_split", _i32),
                ("table_capacity_tokens", _i32), ("lse_lanes", _i32), ("sm_count", _i32),
                ("is_explicit", _i32)]


# Exported symbol -> argtypes.  Kept in the order of include/paged_decode.h.
SIGNATURES = {
    "pd_last_error": [],
    "pd_abi_version": [],
    "pd_make_plan": [_i32, _i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(Plan)],
    "pd_validate_metadata": [_vp, _i64, _i32, _vp, _i32, _i64, _i32],
    "pd_partition": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp,
                     _i32, _i32, _i32, _i32, _i32, _i32, _i32, _dbl, _vp],
    "pd_lse_merge": [_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _vp],
    "pd_matched_decode": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp,
                          _i32, _i32, _i32, _i32, _i32, _i32, _i32, _dbl, _vp],
    "pd_matched_decode_noalloc": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _vp, _vp,
                                  _i32, _i32, _i32, _i32, _i32, _i32, _i32, _dbl, _vp],
    "pd_base": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _i32, _i32, _i32, _i32,
                _dbl, _vp],
    "pd_split_fixed": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp,
                       _i32, _i32, _i32, _i32, _i32, _i32, _dbl, _vp],
    "pd_ml_merge": [_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _vp],
    "pd_split_decode": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _vp, _vp, _vp, _vp, _vp,
                        _i32, _i32, _i32, _i32, _i32, _i32, _dbl, _vp],
    "pd_plan_chunks": [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i32),
                       ctypes.POINTER(_i32)],
    "pd_chunk_rows": [_i32, _i32, _i32, _i32, _i32, ctypes.POINTER(_i64)],
    "pd_store_kv": [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i32, _vp],
    "pd_store_kv_pages": [_vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _vp, _i64, _vp, _i64,
                          _i32, _vp, _i32, _i32, _i32, _i32, _vp],
}

_lib = None


def load_library(path):
    """A ctypes handle of a libpaged_decode.so build at ``path``, with the signatures set.
    Every entry point below takes ``library=`` to run through such a handle instead of
    the package's own build (an A/B of two builds in one process)."""
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} is not built: run `make -C paged-decode-lab_amd/csrc` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    handle = ctypes.CDLL(path)
    for name, argtypes in SIGNATURES.items():
        try:
            fn = getattr(handle, name)
        except AttributeError:
            if path == LIB_PATH:
                raise
            continue  # an older build compared in an A/B run: calls to it raise
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "pd_last_error" else ctypes.c_int
    return handle


def lib():
    """The loaded library; raises RuntimeError when it has not been built."""
    global _lib
    if _lib is None:
        _lib = load_library(LIB_PATH)
    return _lib


def check(status, library=None):
    if status == PD_OK:
        return
    message = (library or lib()).pd_last_error().decode()
    if status == PD_EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def make_plan(max_batch, num_heads, num_kv_heads, head_dim, max_context_len, sm_count,
              num_splits):
    plan = Plan()
    check(lib().pd_make_plan(max_batch, num_heads, num_kv_heads, head_dim, max_context_len,
                             sm_count, num_splits, ctypes.byref(plan)))
    return plan


def validate_metadata(table, lengths, num_pages, max_context_len):
    """``table``/``lengths``: contiguous int32 CPU tensors."""
    check(lib().pd_validate_metadata(table.data_ptr(), table.stride(0) if table.dim() else 0,
                                     table.shape[1], lengths.data_ptr(), lengths.shape[0],
                                     num_pages, max_context_len))


# torch's raw lookup of the current stream returns the handle without building a Stream
# object (a few microseconds of host time per launch); current_stream is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device):
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def partition(q, k, v, tables, lengths, partials, lse, num_kv_heads, splits, tokens_per_split,
              tile_tokens, scale, library=None):
    b, h, d = q.shape
    L = library or lib()
    check(L.pd_partition(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                         tables.data_ptr(), tables.stride(0), tables.shape[1],
                         lengths.data_ptr(), partials.data_ptr(), lse.data_ptr(), b, h,
                         num_kv_heads, d, splits,
                         tokens_per_split, tile_tokens, scale, stream_handle(q.device)), L)


def matched_decode(q, k, v, tables, lengths, partials, lse, counters, out, num_kv_heads, splits,
                   tokens_per_split, tile_tokens, scale, library=None):
    """pd_matched_decode: the fused launch with ``counters``; without (None) the partition
    and the LSE merge, or the partition alone for a plan of one multi-tile split."""
    b, h, d = q.shape
    L = library or lib()
    check(L.pd_matched_decode(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                              v.data_ptr(), tables.data_ptr(), tables.stride(0),
                              tables.shape[1], lengths.data_ptr(), partials.data_ptr(),
                              lse.data_ptr(),
                              None if counters is None else counters.data_ptr(),
                              out.data_ptr(), b, h, num_kv_heads, d,
                              splits, tokens_per_split, tile_tokens, scale,
                              stream_handle(q.device)), L)


def matched_decode_noalloc(q, k, v, tables, lengths, out, num_kv_heads, splits,
                           tokens_per_split, tile_tokens, scale, library=None):
    """pd_matched_decode with the split workspace in the library's static device scratch."""
    b, h, d = q.shape
    L = library or lib()
    check(L.pd_matched_decode_noalloc(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(),
                                      v.data_ptr(), tables.data_ptr(), tables.stride(0),
                                      tables.shape[1], lengths.data_ptr(), out.data_ptr(), b,
                                      h, num_kv_heads, d, splits, tokens_per_split,
                                      tile_tokens, scale, stream_handle(q.device)), L)


def lse_merge(partials, lse, out, lse_lanes, library=None):
    b, h, splits, d = partials.shape
    L = library or lib()
    check(L.pd_lse_merge(partials.data_ptr(), lse.data_ptr(), out.data_ptr(), b, h, d, splits,
                         lse_lanes, stream_handle(partials.device)), L)


def base(q, k, v, tables, lengths, out, num_kv_heads, scale, library=None):
    b, h, d = q.shape
    L = library or lib()
    check(L.pd_base(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                    tables.data_ptr(), tables.stride(0), tables.shape[1], lengths.data_ptr(),
                    out.data_ptr(),
                    b, h, num_kv_heads, d, scale, stream_handle(q.device)), L)


def split_fixed(q, k, v, tables, lengths, maxima, denoms, accums, num_kv_heads, partitions,
                partition_size, scale, library=None):
    b, h, d = q.shape
    L = library or lib()
    check(L.pd_split_fixed(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                           tables.data_ptr(), tables.stride(0), tables.shape[1],
                           lengths.data_ptr(), maxima.data_ptr(), denoms.data_ptr(),
                           accums.data_ptr(), b, h, num_kv_heads, d, partitions, partition_size,
                           scale, stream_handle(q.device)), L)


def ml_merge(maxima, denoms, accums, out, batch, library=None):
    _, h, parts, d = accums.shape
    L = library or lib()
    check(L.pd_ml_merge(maxima.data_ptr(), denoms.data_ptr(), accums.data_ptr(),
                        out.data_ptr(), batch, h, d, parts, stream_handle(out.device)), L)


def split_decode(q, k, v, tables, lengths, maxima, denoms, accums, out, num_kv_heads,
                 partitions, partition_size, scale, library=None):
    """pd_split_decode: the fixed-split partitions and their merge into ``out``."""
    b, h, d = q.shape
    L = library or lib()
    check(L.pd_split_decode(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(),
                            tables.data_ptr(), tables.stride(0), tables.shape[1],
                            lengths.data_ptr(), maxima.data_ptr(), denoms.data_ptr(),
                            accums.data_ptr(), out.data_ptr(), b, h, num_kv_heads, d,
                            partitions, partition_size, scale, stream_handle(q.device)), L)


def plan_chunks(batch, num_heads, num_kv_heads, head_dim, table_width, sm_count):
    """(chunks, chunk_tokens) of pd_plan_chunks: the small-batch split of the base and
    fixed-split protocols, chunks == 1 when the backend runs as it is."""
    chunks, tokens = _i32(0), _i32(0)
    check(lib().pd_plan_chunks(batch, num_heads, num_kv_heads, head_dim, table_width, sm_count,
                               ctypes.byref(chunks), ctypes.byref(tokens)))
    return chunks.value, tokens.value


def chunk_rows(max_batch, num_heads, num_kv_heads, head_dim, sm_count):
    """Chunk-workspace rows that serve every call of pd_plan_chunks (pd_chunk_rows)."""
    rows = _i64(0)
    check(lib().pd_chunk_rows(max_batch, num_heads, num_kv_heads, head_dim, sm_count,
                              ctypes.byref(rows)))
    return rows.value


def store_kv(key, value, k_cache, v_cache, slot_mapping):
    """key/value [N, Hkv, D] (rows 16-byte aligned); caches [..., Hkv, D] flat over slots."""
    n, hkv, d = key.shape
    check(lib().pd_store_kv(key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
                            k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(), n,
                            hkv * d, stream_handle(key.device)))


def store_kv_pages(key, value, k_pages, v_pages, tables, positions):
    """key/value [B, Hkv, S, D]; pages [P, 256, Hkv, D]; tables int32 [B, W]; positions int64 [S]."""
    b, hkv, steps, d = key.shape
    check(lib().pd_store_kv_pages(key.data_ptr(), key.stride(0), key.stride(1), key.stride(2),
                                  value.data_ptr(), value.stride(0), value.stride(1),
                                  value.stride(2), k_pages.data_ptr(), v_pages.data_ptr(),
                                  k_pages.shape[0], tables.data_ptr(), tables.stride(0),
                                  tables.shape[1],
                                  positions.data_ptr(), b, hkv, steps, d,
                                  stream_handle(key.device)))
