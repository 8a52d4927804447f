"""Decode-step graph capture (SIEVE update + fused import of every layer):
each replay must leave the state, outputs, hot rows and status words that the
oracle computes for the same inputs, and the same as the eager calls, for
full batches and padded ones (num_real below the captured maximum), and 1000
replays must not grow device memory (doc/kv_offload_design.md:84,94,477)."""
import ctypes

import numpy as np
import pytest
import torch

from kv_offload_proto_amd.kvops_ext import _kvops
from kv_offload_proto_amd.xds import DecodeStepGraph, HostSegPool, XdsOffloadCoordinator, streams
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROW = 1152


def _words(addr, n):
    return [int(x) for x in (ctypes.c_uint64 * n).from_address(addr)]


def _coord(L, req, dbs, top_k, prefill):
    c = XdsOffloadCoordinator("cuda", L, req, dbs, top_k, req, prefill)
    for r in range(req):
        c.admit_request(r, r, prefill, r * prefill)
    c.set_batch(torch.arange(req, dtype=torch.int64, device="cuda"),
                torch.full((req,), prefill, dtype=torch.int32, device="cuda"))
    return c


def _state(c):
    return [t.cpu().numpy() for t in (c.device_buffer_tokens, c.device_buffer_visited, c.device_buffer_ht,
                                      c.sieve_hand[..., 0], c.top_k_device_slots, c.is_miss)]


@pytest.mark.parametrize("L,req,prefill,top_k,dbs,N", [
    (3, 8, 1024, 256, 512, 2),       # generic parallel kernel
    (2, 4, 8192, 2048, 4096, 4),     # DSA-decode row shape (fixed-count kernel)
    (1, 2, 40000, 2048, 20000, 2),   # a 65536-cell table kept in HBM (batch kernel, reserved scratch)
])
def test_graph_replay_matches_eager(kvops, L, req, prefill, top_k, dbs, N):
    print("graph replay case", L, req, prefill, top_k, dbs, N, flush=True)
    pool = HostSegPool(0, L, req * prefill, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        g0 = torch.Generator(device="cuda")
        g0.manual_seed(5)
        src = torch.randint(0, 256, (L, req * prefill, ROW), dtype=torch.uint8, device="cuda", generator=g0)
        pool.wait(pool.batch_write_alllayers(0, req * prefill, src, req * prefill * ROW))
        ce, cg = _coord(L, req, dbs, top_k, prefill), _coord(L, req, dbs, top_k, prefill)
        padded = ce.padded_buffer_size
        hot_e = torch.zeros((L, req * padded, ROW), dtype=torch.uint8, device="cuda")
        hot_g = torch.zeros_like(hot_e)
        bufs = [torch.zeros((req, top_k), dtype=torch.int32, device="cuda") for _ in range(L)]
        graph = DecodeStepGraph(cg, pool, list(range(L)), bufs, [hot_g[l] for l in range(L)],
                                hot_req_stride_rows=padded)
        graph.capture()
        # capture ran nothing on the state
        for a, b in zip(_state(ce)[:4], _state(cg)[:4]):
            np.testing.assert_array_equal(a, b)
        st_e = _kvops.alloc_status(N)
        # the oracle twin: same admission, same batches, same num_real
        orc_st = orc.SieveState(L, req, dbs, top_k)
        for r in range(req):
            orc_st.admit(r, prefill)
        hot_o = np.zeros((L, req * padded, ROW), dtype=np.uint8)
        segs = [v.reshape(-1) for v in pool.segment_views()]
        plsr = pool.per_layer_seg_rows
        pool_idx, seq = np.arange(req, dtype=np.int64), np.full(req, prefill, dtype=np.int32)
        rng = np.random.default_rng(17)
        for step, nr in enumerate([req, req, req // 2 + 1, req, 1, 0, req]):
            batches = []
            for l in range(L):
                toks = ce.device_buffer_tokens[l, :, :dbs].cpu().numpy()
                batches.append(streams.state_batch(rng, toks, prefill, top_k, 0.3, zipf_s=1.1))
            # eager
            ce.num_real.fill_(nr)
            for l in range(L):
                tk = torch.from_numpy(batches[l]).cuda()
                ce.sieve_update(l, tk)
                _kvops.import_all([sg.seg_base for sg in pool.pool.segments], l * pool.per_layer_seg_rows,
                                  pool.per_layer_seg_rows, ROW, tk.data_ptr(), ce._req_pool_indices.data_ptr(),
                                  ce.req_host_base.data_ptr(), ce.top_k_device_slots.data_ptr(),
                                  ce.is_miss.data_ptr(), ce.num_real.data_ptr(), hot_e[l].data_ptr(), top_k, req,
                                  1, st_e, torch.cuda.current_stream().cuda_stream, 1, padded)
                pool.wait(st_e)
                if l == L - 1:
                    words_e = [_words(st_e + s * 64, 1) for s in range(N)]
            # graph: new inputs in place, one replay
            for l in range(L):
                bufs[l].copy_(torch.from_numpy(batches[l]))
            graph.set_num_real(nr)
            graph.replay()
            graph.wait()
            torch.cuda.synchronize()
            words_g = [_words(graph.status_of(L - 1) + s * 64, 1) for s in range(N)]
            assert words_g == words_e, (step, words_g, words_e)
            for name, a, b in zip(["tokens", "visited", "ht", "hand", "slots", "is_miss"], _state(ce), _state(cg)):
                np.testing.assert_array_equal(a, b, err_msg="step {} num_real {} {}".format(step, nr, name))
            assert torch.equal(hot_e, hot_g), (step, nr)
            # the oracle, layer by layer in the captured order
            for l in range(L):
                o_slots, o_miss = orc_st.update(l, batches[l], pool_idx, seq, nr, max_num_reqs=req)
                for s_ in range(N):
                    _, w = orc.gather_rows(segs, hot_o[l].reshape(-1), l * plsr, ROW, batches[l], pool_idx,
                                           pool_idx * prefill, o_slots, o_miss, nr, top_k, req, 1, N, s_,
                                           hot_req_stride_rows=padded)
                    assert _words(graph.status_of(l) + s_ * 64, 1) == [int(x) for x in w], (step, nr, l, s_)
            gs = _state(cg)
            for name, a, b in zip(["tokens", "visited", "ht", "hand"], gs[:4],
                                  [orc_st.tokens, orc_st.vis, orc_st.ht.view(np.int16), orc_st.hand[..., 0]]):
                np.testing.assert_array_equal(a, b, err_msg="oracle: step {} num_real {} {}".format(step, nr, name))
            np.testing.assert_array_equal(gs[4], o_slots, err_msg="oracle slots, step {}".format(step))
            np.testing.assert_array_equal(gs[5], o_miss, err_msg="oracle is_miss, step {}".format(step))
            assert torch.equal(hot_g, torch.from_numpy(hot_o).cuda()), ("oracle hot rows", step, nr)
    finally:
        pool.destroy(close_ext=False)


def test_graph_many_replays_no_growth(kvops):
    """1000 replays of a captured step: device memory does not grow and the
    state keeps matching an eager twin (same inputs every replay)."""
    L, req, prefill, top_k, dbs, N = 1, 4, 512, 64, 128, 2
    print("graph replay x1000", flush=True)
    pool = HostSegPool(0, L, req * prefill, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        cg = _coord(L, req, dbs, top_k, prefill)
        padded = cg.padded_buffer_size
        hot = torch.zeros((L, req * padded, ROW), dtype=torch.uint8, device="cuda")
        buf = torch.zeros((req, top_k), dtype=torch.int32, device="cuda")
        rng = np.random.default_rng(3)
        buf.copy_(torch.from_numpy(streams.state_batch(rng, cg.device_buffer_tokens[0, :, :dbs].cpu().numpy(),
                                                       prefill, top_k, 0.5)))
        graph = DecodeStepGraph(cg, pool, [0], [buf], [hot[0]], hot_req_stride_rows=padded)
        graph.capture()
        graph.replay()
        graph.wait()
        torch.cuda.synchronize()
        m0 = torch.cuda.memory_allocated()
        free0 = torch.cuda.mem_get_info()[0]
        for i in range(1000):
            graph.replay(clear_status=False)
            if i % 250 == 249:
                torch.cuda.synchronize()
                print("replays", i + 1, flush=True)
        graph.replay()
        graph.wait()
        torch.cuda.synchronize()
        assert torch.cuda.memory_allocated() == m0
        assert torch.cuda.mem_get_info()[0] >= free0 - (64 << 20)
        # an eager twin fed the same batch 1002 times reaches the same state
        ce = _coord(L, req, dbs, top_k, prefill)
        for _ in range(1002):
            ce.sieve_update(0, buf)
        torch.cuda.synchronize()
        for a, b in zip(_state(ce), _state(cg)):
            np.testing.assert_array_equal(a, b)
    finally:
        pool.destroy(close_ext=False)
