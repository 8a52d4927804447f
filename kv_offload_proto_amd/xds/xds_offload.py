"""XdsOffloadCoordinator: per-layer SIEVE state, admission and the decode-step update.

Reference: xds/xds_offload.py:20-106 (same constructor, attributes and methods).
State tensors per layer and pool row (reference :43-53):

* ``device_buffer_tokens``  int32 [L, pool, padded]  slot -> token (-1 empty)
* ``device_buffer_visited`` uint8 [L, pool, visStrideB] visited bitmap
* ``device_buffer_ht``      int16 [L, pool, htSize]  token -> slot+1 table
* ``sieve_hand``            int32 [L, pool, 16]      hand in element 0

Differences from the reference: admission first resets the pool row's tokens
to -1 (the reference leaves stale tokens past ``init_n``), and launches go on
torch's current stream unless a stream is given.  Nothing here reads device
memory back to the host.
"""
from typing import Optional

import torch

from ..kvops_ext import _kvops
from .xds_seg_pool import align, compute_ht_size


def _stream_handle(stream) -> int:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


class XdsOffloadCoordinator:
    def __init__(self, device, layer_num: int, pool_size: int, device_buffer_size: int, top_k: int,
                 max_num_reqs: int, max_context_len: int):
        self.device = torch.device(device)
        self.layer_num = layer_num
        self.pool_size = pool_size
        self.device_buffer_size = device_buffer_size
        self.top_k = top_k
        self.max_num_reqs = max_num_reqs
        self.max_context_len = max_context_len

        self.padded_buffer_size = align(device_buffer_size, 16)
        self.visited_stride_b = align((self.padded_buffer_size + 7) // 8, 64)
        self.ht_size = compute_ht_size(self.padded_buffer_size, top_k)

        p, padded, L = pool_size, self.padded_buffer_size, layer_num
        dev = self.device
        self.device_buffer_tokens = torch.full((L, p, padded), -1, dtype=torch.int32, device=dev)
        self.device_buffer_visited = torch.zeros((L, p, self.visited_stride_b), dtype=torch.uint8, device=dev)
        self.device_buffer_ht = torch.zeros((L, p, self.ht_size), dtype=torch.int16, device=dev)
        self.sieve_hand = torch.zeros((L, p, 16), dtype=torch.int32, device=dev)
        self.prefill_lens = torch.zeros(p, dtype=torch.int32, device=dev)
        self.req_host_base = torch.zeros(max_num_reqs, dtype=torch.int64, device=dev)
        self.top_k_device_slots = torch.zeros((max_num_reqs, top_k), dtype=torch.int32, device=dev)
        self.is_miss = torch.zeros((max_num_reqs, top_k), dtype=torch.int8, device=dev)
        self.num_real = torch.zeros(1, dtype=torch.int32, device=dev)
        self._req_pool_indices: Optional[torch.Tensor] = None
        self._seq_lens: Optional[torch.Tensor] = None

    # ---- admission (xds_offload.py:56-77) ----
    def admit_request(self, req_batch_idx: int, req_pool_idx: int, prefill_len: int, host_base_row: int,
                      stream=None) -> None:
        """Identity layout (slot s holds token s for s < min(prefill, dbs)) in
        every layer, then rebuild the pool row's hash table in every layer."""
        if req_pool_idx < 0 or req_pool_idx >= self.pool_size:
            raise ValueError("req_pool_idx out of range: {}".format(req_pool_idx))
        if req_batch_idx < 0 or req_batch_idx >= self.max_num_reqs:
            raise ValueError("req_batch_idx out of range: {}".format(req_batch_idx))
        init_n = min(prefill_len, self.device_buffer_size)
        row = self.device_buffer_tokens[:, req_pool_idx, :]
        row.fill_(-1)
        row[:, :init_n] = torch.arange(init_n, dtype=torch.int32, device=self.device)
        self.device_buffer_visited[:, req_pool_idx, :].zero_()
        self.sieve_hand[:, req_pool_idx, :].zero_()
        self.prefill_lens[req_pool_idx] = prefill_len
        self.req_host_base[req_batch_idx] = host_base_row
        _kvops.sieve_ht_init(self.device_buffer_tokens.data_ptr(), self.device_buffer_ht.data_ptr(),
                             self.prefill_lens.data_ptr(), req_pool_idx, 1, self.layer_num, self.pool_size,
                             self.device_buffer_size, self.padded_buffer_size, self.ht_size,
                             _stream_handle(stream), self.layer_num)

    def set_batch(self, req_pool_indices: torch.Tensor, seq_lens: torch.Tensor) -> None:
        """Batch context of the next decode steps (xds_offload.py:79-87)."""
        if req_pool_indices.dtype != torch.int64:
            raise ValueError("req_pool_indices must be int64")
        if seq_lens.dtype != torch.int32:
            seq_lens = seq_lens.to(torch.int32)
        self._req_pool_indices = req_pool_indices
        self._seq_lens = seq_lens
        self.num_real[0] = req_pool_indices.shape[0]

    # ---- decode step (xds_offload.py:90-101) ----
    def sieve_update(self, layer_id: int, topk_indices: torch.Tensor, block_dim: int = 8, stream=None) -> None:
        if topk_indices.dtype != torch.int32:
            raise ValueError("topk_indices must be int32")
        if self._req_pool_indices is None:
            raise RuntimeError("set_batch must be called before sieve_update")
        _kvops.sieve_update(topk_indices.data_ptr(), self._req_pool_indices.data_ptr(),
                            self._seq_lens.data_ptr(), self.prefill_lens.data_ptr(),
                            self.device_buffer_tokens[layer_id].data_ptr(),
                            self.device_buffer_visited[layer_id].data_ptr(),
                            self.device_buffer_ht[layer_id].data_ptr(),
                            self.sieve_hand[layer_id].data_ptr(), self.top_k_device_slots.data_ptr(),
                            self.is_miss.data_ptr(), self.num_real.data_ptr(), self.top_k,
                            self.device_buffer_size, self.padded_buffer_size, self.visited_stride_b,
                            self.max_num_reqs, self.pool_size, _stream_handle(stream), block_dim)

    def miss_count(self) -> torch.Tensor:
        """Device-side count of misses of the last update (padding rows are 0)."""
        return self.is_miss.sum()
