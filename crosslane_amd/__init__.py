"""crosslane_amd: MI355X-native routed-expert lane.

Python host-side mirror of the reference's expert-lane interface
(`WarmRedirect`, engine/strata/warm/runtime.hpp:10-16) over the C ABI in
include/crosslane.h (libcrosslane.so, built in-tree by crosslane_amd/_build.py).
There is no fallback path: if the HIP library is missing, importing the lane
raises.
"""
from .lane import (  # noqa: F401
    IQ1_M, IQ2_XS, IQ2_XXS, BLOCK_BYTES, Lane, XLError, codebook, generate_host, lib, pack_meta, pack_types,
    planar_bytes, repack, restore, shared_work_bytes,
)
