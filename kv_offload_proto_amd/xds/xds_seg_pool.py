"""Host-segment pool: the reference's ``EmsPool`` surface over N pinned host segments.

Reference: xds/xds_ems_pool.py (EmsPool :109-241, RowAllocator :54-106,
helpers :25-51).  The EMS daemon, its TCP control plane and HCOMM channel
setup are replaced by N segments of pinned host memory on the same box, each
mapped into the GPU address space; ``channels[s]`` is the segment index.
Row ownership and the per-segment layout are unchanged
(``node = (row/S) % N``, ``segRow = (row/S) / N``,
segment = ``[layer 0 rows][layer 1 rows]...``, ``perLayerSegRows`` rows each).
"""
import ctypes
from typing import List, Optional

import numpy as np

from ..kvops_ext import _kvops


def _ptr(x) -> int:
    """Address of a tensor (``data_ptr()``) or an int address (xds_ems_pool.py:25-32)."""
    if isinstance(x, int):
        return x
    dp = getattr(x, "data_ptr", None)
    if dp is None:
        raise TypeError("expect tensor or int address, got {}".format(type(x)))
    return dp()


def next_pow2(v: int) -> int:
    """Smallest power of two >= v (>= 1)."""
    return 1 if v <= 1 else 1 << (int(v) - 1).bit_length()


def compute_ht_size(padded_buffer_size: int, top_k: int) -> int:
    """Hash-table entries: power of two >= 2*(padded+topK), at least 1024
    (kvops_ext.cpp:297-300, xds_ems_pool.py:42-47)."""
    return max(1024, next_pow2(2 * (padded_buffer_size + top_k)))


def align(v: int, a: int) -> int:
    return -(-v // a) * a


class RowAllocator:
    """Framework-side host row allocator (xds_ems_pool.py:54-106).

    ``alloc(n)`` returns the first free run of >= n rows when one exists (the
    contiguity contract ``src row = req_host_base + token`` relies on), else
    rows gathered from the front of the free list.  ``free`` merges adjacent
    runs.  Free runs are kept as a sorted list of [start, end) pairs.
    """

    def __init__(self, capacity: int):
        self.capacity = int(capacity)
        self._runs = [[0, self.capacity]] if self.capacity > 0 else []
        self._used = 0

    def alloc(self, n: int) -> List[int]:
        if n <= 0:
            raise ValueError("n must be > 0")
        if n > self.free_rows():
            raise MemoryError("allocator exhausted: free={} need={}".format(self.free_rows(), n))
        for run in self._runs:
            if run[1] - run[0] >= n:
                start = run[0]
                run[0] += n
                self._runs = [r for r in self._runs if r[1] > r[0]]
                self._used += n
                return list(range(start, start + n))
        rows: List[int] = []
        while len(rows) < n:
            run = self._runs[0]
            take = min(run[1] - run[0], n - len(rows))
            rows.extend(range(run[0], run[0] + take))
            run[0] += take
            if run[0] == run[1]:
                self._runs.pop(0)
        self._used += n
        return rows

    def free(self, rows: List[int]) -> None:
        if not rows:
            return
        for r in rows:
            if r < 0 or r >= self.capacity:
                raise ValueError("row out of range: {}".format(r))
        merged: List[List[int]] = []
        for s, e in sorted([list(r) for r in self._runs] + [[r, r + 1] for r in rows]):
            if merged and s <= merged[-1][1]:
                merged[-1][1] = max(merged[-1][1], e)
            else:
                merged.append([s, e])
        self._runs = merged
        self._used -= len(rows)

    def free_rows(self) -> int:
        return sum(e - s for s, e in self._runs)

    def used_rows(self) -> int:
        return self._used


class Segment:
    """One host segment (the reference's EMS segment record)."""

    def __init__(self, node_id: int, seg_base: int, size_bytes: int):
        self.node_id = node_id
        self.seg_base = seg_base
        self.size_bytes = size_bytes

    def view(self) -> np.ndarray:
        """uint8 numpy view of the whole segment (host memory, no copy)."""
        buf = (ctypes.c_uint8 * self.size_bytes).from_address(self.seg_base)
        return np.ctypeslib.as_array(buf)


class PoolInfo:
    def __init__(self, segments: List[Segment]):
        self.pool_id = 0
        self.node_num = len(segments)
        self.segments = segments


class HostSegPool:
    """N host-pinned segments + the batch read/write launches (EmsPool surface).

    ``coherent`` selects fine-grained (coherent) pinned memory; the default is
    coarse-grained, the faster mode for bulk GPU reads/writes over the link.

    ``placement`` chooses the NUMA node of the segments' pages: ``"device"``
    (default) binds them to the GPU's node when the platform reports one and
    leaves them unbound otherwise, ``"none"`` never binds, an int binds to
    that node.  The reference's daemon maps anonymous memory with no
    placement (ems/emsd/pool_mgr.cc:23-41); a segment far from the GPU's
    socket crosses the inter-socket link on every import.  After
    ``create_pool``, ``placement_node`` is the node bound (-1: none) and
    ``segment_nodes`` the node each segment's first page landed on (-1:
    unknown).
    """

    def __init__(self, device_id: int, layer_num: int, layer_rows: int, row_bytes: int, stripe_rows: int = 1,
                 node_num: int = 2, coherent: bool = False, placement="device"):
        if layer_num < 1 or layer_rows < 1 or row_bytes <= 0 or row_bytes % 128 != 0:
            raise ValueError("invalid pool dims: L={} rows={} rowBytes={}".format(layer_num, layer_rows, row_bytes))
        if node_num < 1 or node_num > 64:
            raise ValueError("node_num must be in [1, 64], got {}".format(node_num))
        if stripe_rows < 1:
            raise ValueError("stripe_rows must be >= 1")
        if not (placement in ("device", "none") or (isinstance(placement, int) and not isinstance(placement, bool)
                                                     and 0 <= placement < 1024)):
            raise ValueError("placement must be 'device', 'none' or a node in [0, 1024), got {!r}".format(placement))
        self.device_id = device_id
        self.layer_num = layer_num
        self.layer_rows = layer_rows
        self.row_bytes = row_bytes
        self.stripe_rows = stripe_rows
        self.coherent = coherent
        self.placement = placement
        self.placement_node = -1
        self.segment_nodes: List[int] = []
        self._node_num_cfg = node_num
        self.pool: Optional[PoolInfo] = None
        self.node_num = 0
        self.per_layer_seg_rows = 0
        self.channels: List[int] = []
        self._status_base = 0
        self._status_count = 0
        self._status_cursor = 0

    # ---- lifecycle (xds_ems_pool.py:141-180, :187-198) ----
    def create_pool(self, hbm_pool_base: int = 0, hbm_pool_size: int = 0, fatbin_path: str = "",
                    ems_size_bytes: Optional[int] = None) -> None:
        """Allocate the N segments, init the launch extension, allocate the 8N-slot status ring.
        hbm_pool_base/size (HCOMM memory registration in the reference) are not needed."""
        n = self._node_num_cfg
        self.node_num = n
        self.per_layer_seg_rows = -(-self.layer_rows // n)
        seg_bytes = self.layer_num * self.per_layer_seg_rows * self.row_bytes
        if ems_size_bytes is not None and ems_size_bytes < self.layer_num * self.layer_rows * self.row_bytes:
            raise ValueError("ems_size_bytes smaller than layer_num*layer_rows*row_bytes")
        if self.placement == "none":
            node = -1
        elif self.placement == "device":
            node = _kvops.gpu_numa_node(self.device_id)
        else:
            node = self.placement
        segs, nodes = [], []
        try:
            for s in range(n):
                addr, page_node = _kvops.host_alloc_node(seg_bytes, self.coherent, node)
                segs.append(Segment(s, addr, seg_bytes))
                nodes.append(page_node)
        except Exception:
            for sg in segs:
                _kvops.host_free(sg.seg_base)
            raise
        self.pool = PoolInfo(segs)
        self.placement_node = node
        self.segment_nodes = nodes
        self.channels = list(range(n))
        try:
            _kvops.init(self.device_id, fatbin_path)
        except RuntimeError as exc:
            if "already inited" not in str(exc):
                raise
        self._status_count = 8 * n
        self._status_base = _kvops.alloc_status(self._status_count)
        self._status_cursor = 0

    def next_status(self) -> int:
        """Base of the next status block: node s of a call writes slot base +
        s*64, so the cursor steps by node_num slots (the reference steps by one,
        xds_ems_pool.py:182-185, so consecutive calls share slots and the last
        blocks of its ring run past the allocation)."""
        addr = self._status_base + self._status_cursor * 64
        self._status_cursor = (self._status_cursor + self.node_num) % self._status_count
        return addr

    def destroy(self, close_ext: bool = True) -> None:
        if self.pool is not None:
            for sg in self.pool.segments:
                _kvops.host_free(sg.seg_base)
            self.pool = None
        if close_ext:
            _kvops.close()

    def make_allocator(self) -> RowAllocator:
        return RowAllocator(self.layer_rows)

    def segment_views(self) -> List[np.ndarray]:
        """Per-segment uint8 views shaped [layer_num, per_layer_seg_rows, row_bytes]."""
        if self.pool is None:
            raise RuntimeError("pool not created")
        shape = (self.layer_num, self.per_layer_seg_rows, self.row_bytes)
        return [sg.view().reshape(shape) for sg in self.pool.segments]

    # ---- batch read: one import per segment (xds_ems_pool.py:204-217) ----
    def batch_read(self, layer_id: int, topk_indices, req_pool_indices, req_host_base, topk_device_slots, is_miss,
                   num_real, hot_row_base, max_num_reqs: int, top_k: int, stream: int = 0, block_dim: int = 1,
                   hot_req_stride_rows: int = 0) -> int:
        if self.pool is None:
            raise RuntimeError("pool not created")
        status = self.next_status()
        layer_offset = layer_id * self.per_layer_seg_rows
        for s in range(self.node_num):
            seg = self.pool.segments[s]
            _kvops.import_seg(self.channels[s], seg.seg_base, layer_offset, self.per_layer_seg_rows, self.row_bytes,
                              _ptr(topk_indices), _ptr(req_pool_indices), _ptr(req_host_base),
                              _ptr(topk_device_slots), _ptr(is_miss), _ptr(num_real), _ptr(hot_row_base), top_k,
                              max_num_reqs, self.stripe_rows, self.node_num, s, status, stream, block_dim,
                              hot_req_stride_rows)
        return status

    def batch_read_fused(self, layer_id: int, topk_indices, req_pool_indices, req_host_base, topk_device_slots,
                         is_miss, num_real, hot_row_base, max_num_reqs: int, top_k: int, stream: int = 0,
                         block_dim: int = 1, hot_req_stride_rows: int = 0) -> int:
        """All N segments in one launch sequence; same result and status words as batch_read."""
        if self.pool is None:
            raise RuntimeError("pool not created")
        status = self.next_status()
        _kvops.import_all([sg.seg_base for sg in self.pool.segments], layer_id * self.per_layer_seg_rows,
                          self.per_layer_seg_rows, self.row_bytes, _ptr(topk_indices), _ptr(req_pool_indices),
                          _ptr(req_host_base), _ptr(topk_device_slots), _ptr(is_miss), _ptr(num_real),
                          _ptr(hot_row_base), top_k, max_num_reqs, self.stripe_rows, status, stream, block_dim,
                          hot_req_stride_rows)
        return status

    # ---- batch write: prefill export of all layers (xds_ems_pool.py:220-230) ----
    def batch_write_alllayers(self, row_lo: int, row_cnt: int, src_layer0_base, src_layer_stride: int,
                              stream: int = 0, block_dim: int = 1) -> int:
        if self.pool is None:
            raise RuntimeError("pool not created")
        status = self.next_status()
        for s in range(self.node_num):
            seg = self.pool.segments[s]
            _kvops.export_seg_alllayer(self.channels[s], seg.seg_base, self.per_layer_seg_rows, self.row_bytes,
                                       row_lo, row_cnt, self.layer_num, _ptr(src_layer0_base), src_layer_stride,
                                       self.stripe_rows, self.node_num, s, status, stream, block_dim)
        return status

    # ---- decode-incremental export of one layer (the reference design's
    # MemPoolHost.batch_export_rows, doc/kv_offload_design.md:353-354) ----
    def batch_export_rows(self, layer_id: int, src_layer_base, indices_host, num_real, max_rows: int,
                          stream: int = 0, block_dim: int = 1) -> int:
        """Entry i < num_real writes the row at src_layer_base + i*row_bytes to
        host row indices_host[i] (int64) of layer layer_id, one export per
        segment sharing a status slot like batch_read."""
        if self.pool is None:
            raise RuntimeError("pool not created")
        status = self.next_status()
        for s in range(self.node_num):
            seg = self.pool.segments[s]
            _kvops.export_rows(self.channels[s], seg.seg_base, layer_id, self.per_layer_seg_rows, self.row_bytes,
                               _ptr(src_layer_base), _ptr(indices_host), 0, _ptr(num_real), max_rows,
                               self.stripe_rows, self.node_num, s, status, stream, block_dim)
        return status

    def batch_export_rows_fused(self, layer_id: int, src_layer_base, indices_host, num_real, max_rows: int,
                                stream: int = 0, block_dim: int = 1) -> int:
        """All N segments in one launch pair; same result and status words as
        batch_export_rows."""
        if self.pool is None:
            raise RuntimeError("pool not created")
        status = self.next_status()
        _kvops.export_rows_all([sg.seg_base for sg in self.pool.segments], layer_id, self.per_layer_seg_rows,
                               self.row_bytes, _ptr(src_layer_base), _ptr(indices_host), 0, _ptr(num_real), max_rows,
                               self.stripe_rows, status, stream, block_dim)
        return status

    # ---- completion (xds_ems_pool.py:233-241) ----
    def wait(self, status: int, timeout_us: int = 60_000_000, block_dim: int = 1) -> None:
        for s in range(self.node_num):
            for b in range(max(block_dim, 1)):
                rc = _kvops.poll_status(status + s * 64 + b * 8, timeout_us)
                if rc != 0:
                    raise RuntimeError("kv op failed on node {} block {}: errCode=0x{:x}".format(
                        s, b, rc & 0xFFFFFFFF))


class EmsPool(HostSegPool):
    """The reference constructor signature (xds_ems_pool.py:115-118).  The EMS
    master address, ACL/HCOMM library names, rootinfo path and timeout have no
    meaning for local segments and are accepted and ignored; the segment count
    is ``node_num``."""

    def __init__(self, master_ip: str, master_port: int, device_id: int, layer_num: int, layer_rows: int,
                 row_bytes: int, stripe_rows: int = 1, acl_lib: str = "libascendcl.so", hcomm_lib: str = "libhcomm.so",
                 rootinfo_path: str = "/etc/hccl_rootinfo.json", timeout_sec: float = 120.0, node_num: int = 2,
                 coherent: bool = False, placement="device"):
        super().__init__(device_id, layer_num, layer_rows, row_bytes, stripe_rows=stripe_rows, node_num=node_num,
                         coherent=coherent, placement=placement)
        self.master = (master_ip, master_port)
