"""The drop-in boundary, checked without a GPU.

* libkvx.so loads and exports every function include/kvx/kvx.h declares.
* The ``kvops_ext._kvops`` module has the reference's functions with the same
  argument names, order and defaults (kvops/kvops_ext/kvops_ext.cpp:373-401).
* The launch-argument blocks have the reference's byte layout
  (kvops/kernel/kvc_args.h): against the sizes and offsets g++ gives for the
  reference header (literals below), and against the reference header itself
  where oracle/_ref/libkvref.so is built.
"""
import ctypes
import os
import re
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INCLUDE = os.path.join(ROOT, "include")
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libkvref.so")

# kvops_ext.cpp:376-400: name -> [(argument, default or None)]
REFERENCE_SURFACE = {
    "init": [("device_id", None), ("fatbin_path", None), ("rt_lib", "'libascendcl.so'")],
    "alloc_status": [("count", None)],
    "poll_status": [("status_addr", None), ("timeout_us", "-1")],
    "import_seg": [(a, None) for a in (
        "channel", "seg_base", "layer_offset_rows", "per_layer_seg_rows", "row_bytes", "topk_indices",
        "req_pool_indices", "req_host_base", "topk_device_slots", "is_miss", "num_real", "hot_row_base", "top_k",
        "max_num_reqs", "stripe_rows", "node_num", "my_node", "status")] + [("stream", "0"), ("block_dim", "1")],
    "export_seg_alllayer": [(a, None) for a in (
        "channel", "seg_base", "per_layer_seg_rows", "row_bytes", "row_lo", "row_cnt", "layer_num",
        "src_layer0_base", "src_layer_stride", "stripe_rows", "node_num", "my_node", "status")] +
    [("stream", "0"), ("block_dim", "1")],
    "sieve_update": [(a, None) for a in (
        "topk_indices", "req_pool_indices", "seq_lens", "prefill_lens", "device_buffer_tokens",
        "device_buffer_visited", "device_buffer_ht", "sieve_hand", "topk_device_slots", "is_miss", "num_real",
        "top_k", "device_buffer_size", "padded_buffer_size", "visited_stride_b", "max_num_reqs", "pool_size")] +
    [("stream", "0"), ("block_dim", "8")],
    "sieve_ht_init": [(a, None) for a in (
        "device_buffer_tokens", "device_buffer_ht", "prefill_lens", "req_start", "num_reqs", "layer_num",
        "pool_size", "device_buffer_size", "padded_buffer_size", "ht_size")] + [("stream", "0"), ("block_dim", "0")],
    "close": [],
}

# Arguments kvx appends after the reference's (keyword, with defaults).
EXTENSIONS = {"import_seg": [("hot_req_stride_rows", "0")]}


def _declared_symbols():
    text = open(os.path.join(INCLUDE, "kvx", "kvx.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(kvx_\w+)\s*\(", text)))


def _signature(fn):
    first = fn.__doc__.strip().split("\n")[0]
    inner = first[first.index("(") + 1:first.rindex(")")]
    args = []
    depth, cur = 0, ""
    for ch in inner + ",":
        if ch == "," and depth == 0:
            if cur.strip():
                args.append(cur.strip())
            cur = ""
            continue
        depth += ch in "([" and 1 or (ch in ")]" and -1 or 0)
        cur += ch
    out = []
    for a in args:
        name = a.split(":")[0].strip()
        default = a.split("=", 1)[1].strip() if "=" in a else None
        out.append((name, default))
    return out


def test_libkvx_exports_every_declared_symbol():
    import kv_offload_proto_amd  # noqa: F401  (loads torch's HIP runtime first)
    from kv_offload_proto_amd.kvops_ext import lib_path

    lib = ctypes.CDLL(lib_path())
    syms = _declared_symbols()
    assert len(syms) == 25, syms
    missing = [s for s in syms if not hasattr(lib, s)]
    assert missing == []


def test_kvops_surface_matches_reference():
    from kv_offload_proto_amd.kvops_ext import _kvops

    for name, want in REFERENCE_SURFACE.items():
        fn = getattr(_kvops, name)
        got = _signature(fn)
        assert got[:len(want)] == want, name
        assert got[len(want):] == EXTENSIONS.get(name, []), name


def test_kvops_alias_installs():
    import sys

    import kv_offload_proto_amd  # noqa: F401
    from kv_offload_proto_amd import kvops_ext

    assert kvops_ext.install_alias()
    import kvops_ext._kvops as alias  # the reference callers' import line

    assert alias is kvops_ext._kvops
    assert sys.modules["kvops_ext"] is kvops_ext


_ARGS_PROBE = r"""
#include <cstddef>
#include <cstdio>
#include "kvx/kvc_args.h"
int main() {
    const unsigned long long v[] = {
        sizeof(KvcGatherArgs), offsetof(KvcGatherArgs, segBase), offsetof(KvcGatherArgs, hotRowBase),
        offsetof(KvcGatherArgs, status), offsetof(KvcGatherArgs, layerOffsetRows), offsetof(KvcGatherArgs, myNode),
        offsetof(KvcGatherArgs, positionsPerCore), offsetof(KvcGatherArgs, hotReqStrideRows),
        sizeof(KvcScatterAllArgs), offsetof(KvcScatterAllArgs, srcLayerStride), offsetof(KvcScatterAllArgs, status),
        offsetof(KvcScatterAllArgs, rowLo), offsetof(KvcScatterAllArgs, myNode),
        sizeof(HispSieveUpdateArgs), offsetof(HispSieveUpdateArgs, sieveHand), offsetof(HispSieveUpdateArgs, numReal),
        offsetof(HispSieveUpdateArgs, topK), offsetof(HispSieveUpdateArgs, reqsPerCore),
        offsetof(HispSieveUpdateArgs, poolSize),
        sizeof(HispSieveHtInitArgs), offsetof(HispSieveHtInitArgs, reqStart), offsetof(HispSieveHtInitArgs, htSize),
        sizeof(KvxLaunch<KvcGatherArgs>), sizeof(KvxLaunch<KvcScatterAllArgs>),
        sizeof(KvxLaunch<HispSieveUpdateArgs>), sizeof(KvxLaunch<HispSieveHtInitArgs>)};
    for (unsigned i = 0; i < sizeof(v) / sizeof(v[0]); ++i) printf("%llu\n", v[i]);
    return 0;
}
"""

# g++ 11 on the reference's kvc_args.h: struct sizes 120/80/136/64, Gather
# status@72, layerOffsetRows@80, reserved@116, Sieve topK@96.  The order is
# the one kvref_args_layout (oracle/ref_shim.cpp) writes.
_SIZES = {0: 120, 3: 72, 4: 80, 7: 116, 8: 80, 13: 136, 16: 96, 19: 64}


@pytest.fixture(scope="module")
def args_layout(tmp_path_factory):
    d = tmp_path_factory.mktemp("args")
    src = d / "probe.cpp"
    src.write_text(_ARGS_PROBE)
    exe = d / "probe"
    subprocess.run(["g++", "-std=c++17", "-I", INCLUDE, "-o", str(exe), str(src)], check=True)
    return [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]


def test_args_layout_literals(args_layout):
    for i, want in _SIZES.items():
        assert args_layout[i] == want, i
    # a launch passes the block followed by the 8-byte tail slot
    assert args_layout[22:26] == [128, 88, 144, 72]


@pytest.mark.skipif(not os.path.exists(REF_LIB), reason="oracle/_ref not built (reference not mounted)")
def test_args_layout_matches_reference_header(args_layout):
    ref = ctypes.CDLL(REF_LIB)
    buf = (ctypes.c_uint64 * 64)()
    n = ref.kvref_args_layout(buf, 64)
    assert n == 22
    assert list(buf[:n]) == args_layout[:n]
