"""kv_offload_proto_amd: MI355X-native decode-time KV data plane.

Hot path (gfx950 HIP kernels behind a C ABI, include/kvx/kvx.h):

* SIEVE miss detection over a per-request HBM hot buffer
  (reference: kvops/kernel/hisp_sieve_update.cpp, hisp_sieve_ht_init.cpp);
* miss-row gather from N host-pinned segments into the hot buffer and the
  prefill export back to the segments
  (reference: kvops/kernel/kvc_gather_rows.cpp, kvc_scatter_rows_alllayer.cpp).

Python surface: ``kvops_ext._kvops`` (the reference's launch module),
``xds.XdsOffloadCoordinator`` and ``xds.HostSegPool`` / ``xds.EmsPool``
(the reference's coordinator and pool facade).

torch is imported before the native module so libkvx.so binds to the HIP
runtime torch has already loaded (one runtime per process).
"""
import torch  # noqa: F401  (must precede the native module, see above)

from .kvops_ext import _kvops, install_alias  # noqa: E402

install_alias()

__all__ = ["_kvops", "install_alias"]
