"""Helpers shared by the GPU parity tests: mirror an oracle SieveState on the
device and compare the two after every launch."""
import numpy as np
import torch


def to_dev(a, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.view(dtype)
    return t.to("cuda")


class DevSieve:
    """Device copy of an oracle SieveState (ht stored as int16 like the coordinator)."""

    def __init__(self, st):
        self.st = st
        self.tokens = to_dev(st.tokens)
        self.vis = to_dev(st.vis)
        self.ht = to_dev(st.ht.view(np.int16))
        self.hand = to_dev(st.hand)
        self.prefill = to_dev(st.prefill_lens)

    def update(self, kv, layer, topk, req_pool, seq_lens, num_real, max_num_reqs, top_k, block_dim=8):
        topk_d = to_dev(np.ascontiguousarray(topk, dtype=np.int32))
        pool_d = to_dev(np.asarray(req_pool, dtype=np.int64))
        seq_d = to_dev(np.asarray(seq_lens, dtype=np.int32))
        nr = to_dev(np.array([num_real], dtype=np.int32))
        slots = torch.full((max_num_reqs, top_k), 12345, dtype=torch.int32, device="cuda")
        miss = torch.full((max_num_reqs, top_k), 7, dtype=torch.int8, device="cuda")
        st = self.st
        kv.sieve_update(topk_d.data_ptr(), pool_d.data_ptr(), seq_d.data_ptr(), self.prefill.data_ptr(),
                        self.tokens[layer].data_ptr(), self.vis[layer].data_ptr(), self.ht[layer].data_ptr(),
                        self.hand[layer].data_ptr(), slots.data_ptr(), miss.data_ptr(), nr.data_ptr(), top_k, st.dbs,
                        st.padded, st.vis_stride, max_num_reqs, st.pool_size, 0, block_dim)
        torch.cuda.synchronize()
        return slots.cpu().numpy(), miss.cpu().numpy(), (topk_d, pool_d, seq_d, nr, slots, miss)

    def assert_state_equal(self, layer=None, check_ht=True):
        st = self.st
        sl = slice(None) if layer is None else slice(layer, layer + 1)
        np.testing.assert_array_equal(self.tokens.cpu().numpy()[sl], st.tokens[sl])
        np.testing.assert_array_equal(self.vis.cpu().numpy()[sl], st.vis[sl])
        # element 0 is the hand; element 1 may carry the parallel kernel's
        # canonical-state flag (elements 1..15 are unused by the reference)
        np.testing.assert_array_equal(self.hand.cpu().numpy()[sl][..., 0], st.hand[sl][..., 0])
        if check_ht:
            np.testing.assert_array_equal(self.ht.cpu().numpy().view(np.uint16)[sl], st.ht[sl])


def read_words(addr, n):
    """n status words (uint64) at a host-visible status address."""
    import ctypes

    return [int(x) for x in (ctypes.c_uint64 * n).from_address(addr)]
