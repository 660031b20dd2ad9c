"""MI355X paged decode attention behind the paged-decode-lab Python API.

Modules mirror the reference package layout:
  spec               DecodeSpec, BACKENDS, validate_engine_options
  splitkv_plan       make_splitkv_plan, SplitKVPlan
  runtime            Resources, allocate_resources, paged_decode, validate_device_metadata
  matched_splitkv    MatchedResources, allocate_matched_resources, matched_decode
  benchmark_protocol interval_per_operator, convergence_delta
Device imports are lazy so the CPU-only specification imports without a GPU.
"""

from .spec import DecodeSpec

__all__ = ["DecodeSpec"]
