"""Host side of the data plane, mirroring the reference's xds package
(xds/__init__.py:3-5): pool facade, row allocator, derivation helpers and the
SIEVE coordinator, and the decode-step graph capture."""
from .graph import DecodeStepGraph
from .xds_offload import XdsOffloadCoordinator
from .xds_seg_pool import EmsPool, HostSegPool, RowAllocator, Segment, align, compute_ht_size, next_pow2

__all__ = ["DecodeStepGraph", "EmsPool", "HostSegPool", "RowAllocator", "Segment", "XdsOffloadCoordinator", "align",
           "compute_ht_size", "next_pow2"]
