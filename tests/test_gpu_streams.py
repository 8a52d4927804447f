"""Launches on several streams and the per-stream scratch of the row movers.

The reference's launches carry no device state (kvops/kvops_ext/kvops_ext.cpp:7)
and callers may launch on different streams; here every stream has its own
scratch set, so an import on one stream and a decode-incremental export on
another, in flight together, both match the oracle.  A captured graph keeps
the scratch of its capture stream: growing that stream's scratch afterwards
must not free what the graph's launches use.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import read_words
from kv_offload_proto_amd.kvops_ext import _kvops
from kv_offload_proto_amd.xds import DecodeStepGraph, HostSegPool, XdsOffloadCoordinator, streams
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROW = 1152


def _setup(L, req, prefill, dbs, top_k, N, seed):
    rows = req * prefill
    pool = HostSegPool(0, L, rows, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    src = torch.randint(0, 256, (L, rows, ROW), dtype=torch.uint8, device="cuda", generator=g)
    pool.wait(pool.batch_write_alllayers(0, rows, src, rows * ROW))
    torch.cuda.synchronize()
    coord = XdsOffloadCoordinator("cuda", L, req, dbs, top_k, req, prefill)
    st = orc.SieveState(L, req, dbs, top_k)
    for r in range(req):
        coord.admit_request(r, r, prefill, r * prefill)
        st.admit(r, prefill)
    coord.set_batch(torch.arange(req, dtype=torch.int64, device="cuda"),
                    torch.full((req,), prefill, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    return pool, src, coord, st


def test_import_and_export_rows_on_two_streams(kvops):
    """SIEVE + fused import of layer 0 on stream A while a fused
    decode-incremental export into layer 1 runs on stream B; both results
    (hot rows, segment rows, status words) equal the oracle's."""
    L, req, prefill, dbs, top_k, N = 2, 64, 8192, 4096, 2048, 4
    print("two streams", L, req, prefill, dbs, top_k, N, flush=True)
    pool, src, coord, st = _setup(L, req, prefill, dbs, top_k, N, 31)
    try:
        rng = np.random.default_rng(8)
        views = pool.segment_views()
        segs = [v.reshape(-1) for v in views]
        plsr = pool.per_layer_seg_rows
        padded = coord.padded_buffer_size
        # the export's inputs: 4096 rows of new bytes for host rows of layer 1
        E = 4096
        idx = rng.integers(0, req * prefill, size=E).astype(np.int64)
        new_rows = rng.integers(0, 256, size=(E, ROW), dtype=np.uint8)
        idx_d = torch.from_numpy(idx).cuda()
        rows_d = torch.from_numpy(new_rows).cuda()
        nr_d = torch.tensor([E], dtype=torch.int32, device="cuda")
        # the import's inputs
        batch = streams.state_batch(rng, st.tokens[0, :, :dbs], prefill, top_k, 0.2, zipf_s=1.1)
        topk_d = torch.from_numpy(batch).cuda()
        hot = torch.zeros((req * padded, ROW), dtype=torch.uint8, device="cuda")
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        torch.cuda.synchronize()
        for rep in range(3):
            with torch.cuda.stream(sa):
                coord.sieve_update(0, topk_d, stream=sa.cuda_stream)
                st_imp = pool.batch_read_fused(0, topk_d, coord._req_pool_indices, coord.req_host_base,
                                               coord.top_k_device_slots, coord.is_miss, coord.num_real, hot, req,
                                               top_k, stream=sa.cuda_stream, block_dim=2, hot_req_stride_rows=padded)
            with torch.cuda.stream(sb):
                st_exp = pool.batch_export_rows_fused(1, rows_d, idx_d, nr_d, E, stream=sb.cuda_stream, block_dim=3)
            torch.cuda.synchronize()
            if rep == 0:
                e_slots, e_miss = st.update(0, batch, np.arange(req), np.full(req, prefill), req)
                hot_np = np.zeros((req * padded, ROW), dtype=np.uint8)
                imp_words = []
                for s in range(N):
                    _, w = orc.gather_rows(segs, hot_np.reshape(-1), 0, ROW, batch, np.arange(req),
                                           np.arange(req) * prefill, e_slots, e_miss, req, top_k, req, 1, N, s,
                                           hot_req_stride_rows=padded, block_dim=2)
                    imp_words.append([int(x) for x in w])
                seg_exp = [segs[s].copy() for s in range(N)]
                exp_words = []
                for s in range(N):
                    _, w = orc.export_rows(seg_exp[s], new_rows.reshape(-1), idx, E, E, 1, plsr, ROW, 1, N, s, 3)
                    exp_words.append([int(x) for x in w])
                np.testing.assert_array_equal(coord.top_k_device_slots.cpu().numpy(), e_slots)
                np.testing.assert_array_equal(coord.is_miss.cpu().numpy(), e_miss)
                assert torch.equal(hot, torch.from_numpy(hot_np).cuda())
                for s in range(N):
                    assert read_words(st_imp + s * 64, 2) == imp_words[s], s
                    assert read_words(st_exp + s * 64, 3) == exp_words[s], s
                    np.testing.assert_array_equal(segs[s], seg_exp[s], err_msg="segment {}".format(s))
                # the later repetitions re-run the same SIEVE batch (all hits
                # now) and the same export: each must still report its own
                # launch's status words
                batch2 = batch
            else:
                e_slots, e_miss = st.update(0, batch2, np.arange(req), np.full(req, prefill), req)
                np.testing.assert_array_equal(coord.top_k_device_slots.cpu().numpy(), e_slots)
                np.testing.assert_array_equal(coord.is_miss.cpu().numpy(), e_miss)
                for s in range(N):
                    _, w = orc.gather_rows(segs, hot_np.reshape(-1), 0, ROW, batch2, np.arange(req),
                                           np.arange(req) * prefill, e_slots, e_miss, req, top_k, req, 1, N, s,
                                           hot_req_stride_rows=padded, block_dim=2)
                    assert read_words(st_imp + s * 64, 2) == [int(x) for x in w], (rep, s)
                    assert read_words(st_exp + s * 64, 3) == exp_words[s], (rep, s)
                assert torch.equal(hot, torch.from_numpy(hot_np).cuda())
        assert _kvops.scratch_bytes(sa.cuda_stream) > 0 and _kvops.scratch_bytes(sb.cuda_stream) > 0
    finally:
        pool.destroy(close_ext=False)


def test_scratch_growth_after_capture(kvops):
    """Capture a decode step, then grow the capture stream's scratch with an
    export whose winner table is larger than the reserved one, then replay:
    the graph still uses its own (kept) buffers and matches the oracle."""
    # reserved winner table: (8 - 1) * 4096 + 65536 = 94208 entries; the
    # export's: 4 segments x 32768 rows = 131072
    L, req, prefill, dbs, top_k, N = 1, 8, 16384, 4096, 2048, 4
    print("scratch growth after capture", flush=True)
    pool, src, coord, st = _setup(L, req, prefill, dbs, top_k, N, 32)
    try:
        padded = coord.padded_buffer_size
        segs = [v.reshape(-1) for v in pool.segment_views()]
        hot = torch.zeros((req * padded, ROW), dtype=torch.uint8, device="cuda")
        hot_np = np.zeros((req * padded, ROW), dtype=np.uint8)
        buf = torch.zeros((req, top_k), dtype=torch.int32, device="cuda")
        graph = DecodeStepGraph(coord, pool, [0], [buf], [hot], hot_req_stride_rows=padded)
        graph.capture()
        cs = graph.capture_stream
        before = _kvops.scratch_bytes(cs.cuda_stream)
        # an eager export on the capture stream whose winner table (all four
        # segments' rows of a layer) exceeds what the capture reserved
        E = 64
        idx_d = torch.arange(E, dtype=torch.int64, device="cuda") * 7
        rows_d = src[0].index_select(0, idx_d).contiguous()
        nr_d = torch.tensor([E], dtype=torch.int32, device="cuda")
        with torch.cuda.stream(cs):
            stx = pool.batch_export_rows_fused(0, rows_d, idx_d, nr_d, E, stream=cs.cuda_stream)
        torch.cuda.synchronize()
        pool.wait(stx)
        assert _kvops.scratch_bytes(cs.cuda_stream) > before
        rng = np.random.default_rng(5)
        for step in range(3):
            batch = streams.state_batch(rng, st.tokens[0, :, :dbs], prefill, top_k, 0.2, zipf_s=1.1)
            buf.copy_(torch.from_numpy(batch))
            graph.replay()
            graph.wait()
            torch.cuda.synchronize()
            e_slots, e_miss = st.update(0, batch, np.arange(req), np.full(req, prefill), req)
            for s in range(N):
                _, w = orc.gather_rows(segs, hot_np.reshape(-1), 0, ROW, batch, np.arange(req),
                                       np.arange(req) * prefill, e_slots, e_miss, req, top_k, req, 1, N, s,
                                       hot_req_stride_rows=padded)
                assert read_words(graph.status_of(0) + s * 64, 1) == [int(x) for x in w], (step, s)
            np.testing.assert_array_equal(coord.top_k_device_slots.cpu().numpy(), e_slots)
            np.testing.assert_array_equal(coord.is_miss.cpu().numpy(), e_miss)
            np.testing.assert_array_equal(coord.device_buffer_tokens[0].cpu().numpy(), st.tokens[0])
            assert torch.equal(hot, torch.from_numpy(hot_np).cuda()), step
    finally:
        pool.destroy(close_ext=False)


def test_capture_without_reserve_is_refused(kvops):
    """A launch that would have to create or grow its stream's scratch during
    capture raises (nothing is allocated inside the capture)."""
    L, req, prefill, dbs, top_k, N = 1, 4, 256, 64, 64, 2
    pool, src, coord, st = _setup(L, req, prefill, dbs, top_k, N, 33)
    try:
        hot = torch.zeros((req * coord.padded_buffer_size, ROW), dtype=torch.uint8, device="cuda")
        topk_d = torch.zeros((req, top_k), dtype=torch.int32, device="cuda")
        s = torch.cuda.Stream()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with pytest.raises(RuntimeError, match="cannot grow during stream capture"):
            with torch.cuda.graph(g, stream=s):
                pool.batch_read_fused(0, topk_d, coord._req_pool_indices, coord.req_host_base,
                                      coord.top_k_device_slots, coord.is_miss, coord.num_real, hot, req, top_k,
                                      stream=s.cuda_stream)
        torch.cuda.synchronize()
        assert _kvops.scratch_bytes(s.cuda_stream) == 0
    finally:
        pool.destroy(close_ext=False)
