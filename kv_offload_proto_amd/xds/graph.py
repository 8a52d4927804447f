"""Decode-step capture: the SIEVE update and the fused miss import of a list of
layers, recorded once into a HIP graph and replayed every decode step.

The reference's design asks for the import to be stream-capturable with no
host synchronisation, replays equal to the eager path and at least 1000
replays without leaks (``doc/kv_offload_design.md:29,84,93-94``), and its
kernels read the batch size on the device so a capture at the maximum batch
serves smaller ones (``hisp_sieve_update.cpp:71-78`` writes dummy rows past
``num_real`` "for graph replay"; ``kvc_gather_rows.cpp:17-21``).  The
launches here qualify: every per-step input (topK rows, request pool indices,
sequence lengths, ``num_real``) is read from device memory, the import's
winner-tag epoch is a device counter that the last copy workgroup advances,
and the import's first kernel clears its status words on the device, so a
replay does exactly the work of the eager calls.

Rules for the caller:

* the captured tensors are fixed: write new inputs into them in place (the
  topK buffers, the coordinator's ``_req_pool_indices`` / ``_seq_lens``,
  ``num_real`` through :meth:`set_num_real`) -- never rebind them;
* :meth:`capture` records on a stream of its own (or the one given), whose
  library scratch it first sizes with ``reserve_scratch`` so that nothing is
  allocated during the capture; the graph's launches keep that stream's
  scratch, so replays of one graph must not overlap each other or eager
  launches on the capture stream;
* :meth:`replay` clears the host-visible status words before launching, and
  :meth:`wait` polls them like ``EmsPool.wait``.
"""
import ctypes
from typing import List, Optional, Sequence

import torch

from ..kvops_ext import _kvops


def _ptr(x) -> int:
    return x if isinstance(x, int) else x.data_ptr()


class DecodeStepGraph:
    def __init__(self, coord, pool, layers: Sequence[int], topk: Sequence[torch.Tensor], hot: Sequence,
                 hot_req_stride_rows: int = 0, block_dim: int = 1, sieve_block_dim: int = 8,
                 capture_stream: Optional[torch.cuda.Stream] = None):
        if len(layers) != len(topk) or len(layers) != len(hot):
            raise ValueError("layers, topk and hot must have one entry per layer")
        if pool.pool is None:
            raise RuntimeError("pool not created")
        self.coord = coord
        self.pool = pool
        self.layers: List[int] = list(layers)
        self.topk = list(topk)
        self.hot = list(hot)
        self.stride = hot_req_stride_rows
        self.block_dim = max(1, block_dim)
        self.sieve_block_dim = sieve_block_dim
        # one status block of node_num slots per captured layer
        self.n_slots = pool.node_num * len(self.layers)
        self.status_base = _kvops.alloc_status(self.n_slots)
        self.graph = None
        self.capture_stream = capture_stream

    def status_of(self, i: int) -> int:
        """Status address of the i-th captured layer (node s at +s*64)."""
        return self.status_base + i * self.pool.node_num * 64

    def _run(self):
        c, p = self.coord, self.pool
        stream = torch.cuda.current_stream().cuda_stream
        for i, (layer, tk, hot) in enumerate(zip(self.layers, self.topk, self.hot)):
            c.sieve_update(layer, tk, block_dim=self.sieve_block_dim, stream=stream)
            _kvops.import_all([sg.seg_base for sg in p.pool.segments], layer * p.per_layer_seg_rows,
                              p.per_layer_seg_rows, p.row_bytes, _ptr(tk), _ptr(c._req_pool_indices),
                              _ptr(c.req_host_base), _ptr(c.top_k_device_slots), _ptr(c.is_miss),
                              _ptr(c.num_real), _ptr(hot), c.top_k, c.max_num_reqs, p.stripe_rows, self.status_of(i),
                              stream, self.block_dim, self.stride)

    def capture(self) -> None:
        c = self.coord
        if c._req_pool_indices is None:
            raise RuntimeError("set_batch must be called before capture")
        if self.capture_stream is None:
            self.capture_stream = torch.cuda.Stream(device=c.device)  # default priority
        _kvops.reserve_scratch(self.capture_stream.cuda_stream, c.max_num_reqs, c.top_k, self.stride, 0, 0,
                               c.device_buffer_size)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.capture_stream):
            self._run()
        torch.cuda.synchronize()

    def set_num_real(self, n: int) -> None:
        """Batch rows of the next replays (at most max_num_reqs; rows past it
        get slot -1 / miss 0 and import nothing)."""
        if n < 0 or n > self.coord.max_num_reqs:
            raise ValueError("num_real must be in [0, max_num_reqs]")
        self.coord.num_real.fill_(n)

    def replay(self, clear_status: bool = True) -> None:
        """Launch the captured step.  With clear_status the host zeroes the
        status words first, so that :meth:`wait` cannot see the previous
        replay's completion; the previous replay must then have completed
        (waited for).  Back-to-back replays that nobody polls may skip it:
        the import's first kernel clears the words on the device too."""
        if self.graph is None:
            raise RuntimeError("capture() first")
        if clear_status:
            ctypes.memset(self.status_base, 0, self.n_slots * 64)
        self.graph.replay()

    def wait(self, timeout_us: int = 60_000_000) -> None:
        for i in range(len(self.layers)):
            base = self.status_of(i)
            for s in range(self.pool.node_num):
                for b in range(self.block_dim):
                    rc = _kvops.poll_status(base + s * 64 + b * 8, timeout_us)
                    if rc != 0:
                        raise RuntimeError("kv op failed on layer {} node {} block {}: errCode=0x{:x}".format(
                            self.layers[i], s, b, rc & 0xFFFFFFFF))
