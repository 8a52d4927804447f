"""Placement of host segments on a NUMA node: the GPU's node as the platform
reports it, memory bound to a node (its pages on that node wherever the
system reports them: the runtime's pinned memory is a mapping of the GPU's
render node, whose pages the kernel does not report, so -1 is accepted), a
node the process may not use refused, the calling thread's memory policy
left as it was, and an import from segments placed on a node against the
oracle."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import read_words, to_dev
from kv_offload_proto_amd.kvops_ext import _kvops
from kv_offload_proto_amd.xds import HostSegPool
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SYS_GET_MEMPOLICY = 239  # x86_64
ROW = 1152


def _policy():
    """The calling thread's memory policy: (mode, node mask words)."""
    libc = ctypes.CDLL(None, use_errno=True)
    mode = ctypes.c_int(-1)
    mask = (ctypes.c_ulong * 16)()
    rc = libc.syscall(SYS_GET_MEMPOLICY, ctypes.byref(mode), mask, ctypes.c_ulong(1025), None, ctypes.c_ulong(0))
    assert rc == 0, ctypes.get_errno()
    return mode.value, list(mask)


def _allowed_nodes():
    """Nodes this process may place memory on (Mems_allowed_list)."""
    for line in open("/proc/self/status"):
        if line.startswith("Mems_allowed_list:"):
            nodes = set()
            for part in line.split(":", 1)[1].strip().split(","):
                a, _, b = part.partition("-")
                nodes.update(range(int(a), int(b or a) + 1))
            return nodes
    return {0}


def test_gpu_numa_node(kvops):
    node = _kvops.gpu_numa_node(0)
    print("gpu numa node", node, "allowed", sorted(_allowed_nodes()), flush=True)
    assert node == -1 or 0 <= node < 1024


def test_host_alloc_on_node(kvops):
    allowed = _allowed_nodes()
    before = _policy()
    node = min(allowed)
    addr, page_node = _kvops.host_alloc_node(8 << 20, False, node)
    try:
        assert page_node in (node, -1)
        assert _policy() == before
        # the memory is mapped for the device: a device write lands in it
        buf = (ctypes.c_uint8 * 4096).from_address(addr)
        src = torch.arange(4096, dtype=torch.int32, device="cuda").to(torch.uint8)
        _kvops.stream_copy(addr, src.data_ptr(), 4096, 0)
        torch.cuda.synchronize()
        assert bytes(buf) == bytes(src.cpu().numpy())
    finally:
        _kvops.host_free(addr)
    addr, page_node = _kvops.host_alloc_node(1 << 20, True, -1)  # no binding
    _kvops.host_free(addr)
    assert page_node == -1 or page_node in allowed
    outside = max(allowed) + 1
    if outside < 1024:
        with pytest.raises(RuntimeError, match="not available"):
            _kvops.host_alloc_node(1 << 20, False, outside)
        assert _policy() == before


@pytest.mark.parametrize("placement", ["node", "device"])
def test_import_from_placed_segments(kvops, placement):
    """Segments placed by the pool carry an import like any other: every hot
    byte and status word against the oracle."""
    node = min(_allowed_nodes()) if placement == "node" else "device"
    req, top_k, dbs, prefill, N, L = 4, 512, 256, 1024, 2, 1
    padded = (dbs + 15) // 16 * 16
    pool = HostSegPool(0, L, req * prefill, ROW, stripe_rows=1, node_num=N, placement=node)
    pool.create_pool()
    try:
        if placement == "node":
            assert pool.placement_node == node and all(n in (node, -1) for n in pool.segment_nodes)
        else:
            assert pool.placement_node == _kvops.gpu_numa_node(0)
        rng = np.random.default_rng(11)
        views = pool.segment_views()
        for v in views:
            v[...] = rng.integers(0, 256, size=v.shape, dtype=np.uint8)
        segs = [v.reshape(-1) for v in views]
        topk = rng.integers(0, prefill, size=(req, top_k)).astype(np.int32)
        slots = rng.integers(0, dbs, size=(req, top_k)).astype(np.int32)
        miss = (rng.random((req, top_k)) < 0.5).astype(np.int8)
        pool_idx = np.arange(req, dtype=np.int64)
        host_base = np.arange(req, dtype=np.int64) * prefill
        hot_np = np.zeros((req * padded, ROW), dtype=np.uint8)
        hot = torch.zeros((req * padded, ROW), dtype=torch.uint8, device="cuda")
        status = pool.batch_read_fused(0, to_dev(topk), to_dev(pool_idx), to_dev(host_base), to_dev(slots),
                                       to_dev(miss), to_dev(np.array([req], dtype=np.int32)), hot, req, top_k,
                                       block_dim=2, hot_req_stride_rows=padded)
        pool.wait(status, block_dim=2)
        torch.cuda.synchronize()
        for s in range(N):
            _, words = orc.gather_rows(segs, hot_np.reshape(-1), 0, ROW, topk, pool_idx, host_base, slots, miss, req,
                                       top_k, req, 1, N, s, hot_req_stride_rows=padded, block_dim=2)
            assert read_words(status + s * 64, 2) == [int(w) for w in words], s
        np.testing.assert_array_equal(hot.cpu().numpy(), hot_np)
    finally:
        pool.destroy(close_ext=False)
