"""kvops_ext: the launch extension package of the data plane.

``_kvops`` is the compiled module (kvops_pybind.cpp over libkvx.so) with the
reference's ``kvops_ext._kvops`` functions (kvops/kvops_ext/kvops_ext.cpp:373-401):
init, alloc_status, poll_status, import_seg, export_seg_alllayer, sieve_update,
sieve_ht_init, close -- plus import_all, host_alloc/host_free, read_overflow,
clear_overflow and last_sieve_variant.

Importing this package fails loudly when the native module has not been
built; there is no fallback implementation.
"""
import os
import sys

_HERE = os.path.dirname(os.path.abspath(__file__))

try:
    from . import _kvops  # noqa: F401
except ImportError as exc:  # pragma: no cover - exercised only on a broken install
    raise ImportError(
        "kvops_ext native module is not built ({}); run `python kv_offload_proto_amd/build.py`".format(exc)
    ) from exc


def lib_path():
    """Path of libkvx.so, the C-ABI library the module is linked against."""
    return os.path.join(_HERE, "libkvx.so")


def install_alias():
    """Register this package as top-level ``kvops_ext`` so code written against
    the reference (``import kvops_ext._kvops as _kvops``) imports it unchanged.
    An existing, different ``kvops_ext`` module is left alone."""
    pkg = sys.modules[__name__]
    cur = sys.modules.get("kvops_ext")
    if cur is None or cur is pkg:
        sys.modules["kvops_ext"] = pkg
        sys.modules["kvops_ext._kvops"] = _kvops
    return sys.modules["kvops_ext"] is pkg
