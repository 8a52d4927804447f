"""GPU parity of the row movers against the C oracle: prefill export into the
host segments, miss import into the hot buffer (per segment and fused), and
the status words of both."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import DevSieve, to_dev
from kv_offload_proto_amd.xds import HostSegPool, streams
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DONE = 1 << 32
ROW = 1152


def _src(layers, rows, row_bytes, seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return torch.randint(0, 256, (layers, rows, row_bytes), dtype=torch.uint8, device="cuda", generator=g)


@pytest.mark.parametrize("layers,layer_rows,N,S,row_lo,row_cnt,block_dim", [
    (2, 2048, 2, 1, 0, 2048, 1),
    (3, 1000, 3, 1, 17, 900, 2),
    (2, 4096, 4, 64, 0, 4096, 1),     # striped: rows of a stripe alias one segment row
    (2, 1500, 4, 64, 10, 1337, 3),    # partial first and last stripes
    (1, 777, 1, 5, 0, 777, 8),
])
def test_export_parity(kvops, layers, layer_rows, N, S, row_lo, row_cnt, block_dim):
    row_bytes = 1152
    pool = HostSegPool(0, layers, layer_rows, row_bytes, stripe_rows=S, node_num=N)
    pool.create_pool()
    try:
        segs = pool.segment_views()
        for v in segs:
            v[...] = 0xAB
        src = _src(layers, layer_rows, row_bytes, 1234 + layer_rows)
        st = pool.batch_write_alllayers(row_lo, row_cnt, src, layer_rows * row_bytes, block_dim=block_dim)
        pool.wait(st, block_dim=block_dim)
        torch.cuda.synchronize()
        src_np = src.cpu().numpy()
        plsr = pool.per_layer_seg_rows
        for s in range(N):
            exp = np.full(layers * plsr * row_bytes, 0xAB, dtype=np.uint8)
            q = orc.export_alllayer(exp, src_np.reshape(-1), layer_rows * row_bytes, plsr, row_bytes, row_lo, row_cnt,
                                    layers, S, N, s)
            np.testing.assert_array_equal(segs[s].reshape(-1), exp, err_msg="segment {}".format(s))
            words = _read_words(st + s * 64, block_dim)
            assert words[0] == (q << 40) | DONE
            assert all(w == DONE for w in words[1:])
    finally:
        pool.destroy(close_ext=False)


def _read_words(addr, n):
    buf = (ctypes.c_uint64 * n).from_address(addr)
    return [int(x) for x in buf]


@pytest.mark.parametrize("stride_mode", ["reference", "per_request", "overlap"])
@pytest.mark.parametrize("fused", [False, True])
def test_gather_parity_after_sieve(kvops, stride_mode, fused):
    """config-1 shapes: SIEVE on the GPU, then import; the hot buffer must equal
    the oracle's byte for byte after every step (last-position-wins rule when
    destinations collide: within a request when a step's sweep reuses a slot,
    across requests with stride 0 (every request on the same rows) and with a
    stride of 24 rows (request b's slots 24.. are request b+1's rows))."""
    req, prefill, top_k, dbs, L, N = 8, 256, 64, 64, 2, 2
    row_bytes = 1152
    layer_rows = req * prefill
    pool = HostSegPool(0, L, layer_rows, row_bytes, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        src = _src(L, layer_rows, row_bytes, 99)
        stt = pool.batch_write_alllayers(0, layer_rows, src, layer_rows * row_bytes)
        pool.wait(stt)
        st = orc.SieveState(L, req, dbs, top_k)
        for r in range(req):
            st.admit(r, prefill)
        dev = DevSieve(st)
        padded = st.padded
        stride = {"reference": 0, "per_request": padded, "overlap": 24}[stride_mode]
        hot_rows = (req - 1) * stride + padded
        hot = torch.zeros((L, hot_rows, row_bytes), dtype=torch.uint8, device="cuda")
        hot_np = np.zeros((L, hot_rows, row_bytes), dtype=np.uint8)
        host_base = np.arange(req, dtype=np.int64) * prefill
        host_base_d = to_dev(host_base)
        segs = [v.reshape(-1) for v in pool.segment_views()]
        rng = np.random.default_rng(42)
        req_pool = np.arange(req)
        seq = np.full(req, prefill)
        plsr = pool.per_layer_seg_rows
        for step in range(8):
            layer = step % L
            batch = streams.state_batch(rng, st.tokens[layer, :, :dbs], prefill, top_k, 0.5)
            e_slots, e_miss = st.update(layer, batch, req_pool, seq, req)
            g_slots, g_miss, keep = dev.update(kvops, layer, batch, req_pool, seq, req, req, top_k)
            np.testing.assert_array_equal(g_slots, e_slots)
            np.testing.assert_array_equal(g_miss, e_miss)
            topk_d, pool_d, seq_d, nr, slots_d, miss_d = keep
            if fused:
                status = pool.batch_read_fused(layer, topk_d, pool_d, host_base_d, slots_d, miss_d, nr, hot[layer],
                                               req, top_k, block_dim=2, hot_req_stride_rows=stride)
            else:
                status = pool.batch_read(layer, topk_d, pool_d, host_base_d, slots_d, miss_d, nr, hot[layer], req,
                                         top_k, block_dim=2, hot_req_stride_rows=stride)
            pool.wait(status, block_dim=2)
            torch.cuda.synchronize()
            for s in range(N):
                _, words = orc.gather_rows(segs, hot_np[layer].reshape(-1), layer * plsr, row_bytes, batch, req_pool,
                                           host_base, e_slots, e_miss, req, top_k, req, 1, N, s,
                                           hot_req_stride_rows=stride, block_dim=2)
                assert _read_words(status + s * 64, 2) == [int(w) for w in words], (step, s)
            np.testing.assert_array_equal(hot.cpu().numpy(), hot_np, err_msg="step {}".format(step))
    finally:
        pool.destroy(close_ext=False)


@pytest.mark.parametrize("req,top_k,num_real,S,N,stride_mode,fused,block_dim", [
    (3, 1500, 2, 1, 2, "padded", True, 3),    # 4500 positions: 18 chunks, the last one partial
    (3, 1500, 3, 64, 4, "zero", False, 2),    # stride 0: requests collide on hot rows
    (5, 4096, 5, 1, 3, "padded", True, 8),    # 80 chunks over the 64 workgroups
    (2, 2049, 1, 1, 1, "zero", True, 1),      # 4098 positions: just past the one-launch form
    (3, 1500, 3, 1, 2, "wide", True, 2),      # stride 70000: winner rows spaced 65536 apart
])
def test_gather_large_batch_parity(kvops, req, top_k, num_real, S, N, stride_mode, fused, block_dim):
    """The large-batch import (winner tags, then workgroups claiming chunks of
    positions) against the oracle on constructed inputs: duplicate and
    colliding destinations (the last valid miss wins), invalid tokens and
    slots, a request without a pool row, num_real below max_num_reqs, partial
    chunks; every hot byte and every node's status words."""
    print("large import case", req, top_k, num_real, S, N, stride_mode, fused, block_dim, flush=True)
    L, layer, prefill, dbs = 2, 1, 4096, 2048
    padded = (dbs + 15) // 16 * 16
    layer_rows = req * prefill
    pool = HostSegPool(0, L, layer_rows, ROW, stripe_rows=S, node_num=N)
    pool.create_pool()
    try:
        rng = np.random.default_rng(req * 100 + top_k + S + N)
        views = pool.segment_views()
        for v in views:
            v[...] = rng.integers(0, 256, size=v.shape, dtype=np.uint8)
        segs = [v.reshape(-1) for v in views]
        topk = rng.integers(0, prefill, size=(req, top_k)).astype(np.int32)
        topk[rng.random((req, top_k)) < 0.03] = -1
        slots = rng.integers(0, dbs, size=(req, top_k)).astype(np.int32)
        slots[rng.random((req, top_k)) < 0.02] = -1
        miss = (rng.random((req, top_k)) < 0.5).astype(np.int8)
        pool_idx = np.arange(req, dtype=np.int64)
        if req >= 3:
            pool_idx[1] = -1
        host_base = np.arange(req, dtype=np.int64) * prefill
        stride = {"padded": padded, "zero": 0, "wide": 70000}[stride_mode]
        hot_rows = (req - 1) * stride + padded  # the last request's slots end the buffer
        hot_np = rng.integers(0, 256, size=(hot_rows, ROW), dtype=np.uint8)
        hot = torch.from_numpy(hot_np.copy()).cuda()
        args = (layer, to_dev(topk), to_dev(pool_idx), to_dev(host_base), to_dev(slots), to_dev(miss),
                to_dev(np.array([num_real], dtype=np.int32)), hot, req, top_k)
        read = pool.batch_read_fused if fused else pool.batch_read
        status = read(*args, block_dim=block_dim, hot_req_stride_rows=stride)
        pool.wait(status, block_dim=block_dim)
        torch.cuda.synchronize()
        plsr = pool.per_layer_seg_rows
        for s in range(N):
            _, words = orc.gather_rows(segs, hot_np.reshape(-1), layer * plsr, ROW, topk, pool_idx, host_base, slots,
                                       miss, num_real, top_k, req, S, N, s, hot_req_stride_rows=stride,
                                       block_dim=block_dim)
            assert _read_words(status + s * 64, block_dim) == [int(w) for w in words], s
        np.testing.assert_array_equal(hot.cpu().numpy(), hot_np)
    finally:
        pool.destroy(close_ext=False)


@pytest.mark.parametrize("req,top_k,dbs,stride_mode,fused,block_dim", [
    (12, 20, 16, "padded", True, 2),     # a workgroup's 32 positions straddle two requests
    (40, 7, 8, "padded", False, 3),      # ... and five
    (10, 48, 32, "half", True, 1),       # stride 16 < slots in use: neighbouring requests share rows
    (6, 100, 64, "zero", False, 2),      # stride 0: every request on the same rows
    (1, 4096, 4096, "padded", True, 8),  # the largest one-launch call: one request of 4096 positions
])
def test_gather_small_batch_winners(kvops, req, top_k, dbs, stride_mode, fused, block_dim):
    """The one-launch import (max_num_reqs * top_k <= 4096) against the oracle
    on constructed inputs with many misses on one destination row: within a
    request (the winner decided in LDS from the workgroup's own requests,
    whose positions may straddle workgroups) and across requests (a stride
    below the slots in use: device-scope tags of every position); invalid
    tokens and slots, a request without a pool row; every hot byte and every
    node's status words."""
    print("small import case", req, top_k, dbs, stride_mode, fused, block_dim, flush=True)
    L, layer, prefill, S, N = 2, 1, 512, 1, 2
    padded = (dbs + 15) // 16 * 16
    layer_rows = req * prefill
    pool = HostSegPool(0, L, layer_rows, ROW, stripe_rows=S, node_num=N)
    pool.create_pool()
    try:
        rng = np.random.default_rng(req * 1000 + top_k + dbs)
        views = pool.segment_views()
        for v in views:
            v[...] = rng.integers(0, 256, size=v.shape, dtype=np.uint8)
        segs = [v.reshape(-1) for v in views]
        topk = rng.integers(0, prefill, size=(req, top_k)).astype(np.int32)
        topk[rng.random((req, top_k)) < 0.03] = -1
        slots = rng.integers(0, dbs, size=(req, top_k)).astype(np.int32)
        slots[rng.random((req, top_k)) < 0.02] = -1
        miss = (rng.random((req, top_k)) < 0.6).astype(np.int8)
        pool_idx = np.arange(req, dtype=np.int64)
        if req >= 3:
            pool_idx[2] = -1
        host_base = np.arange(req, dtype=np.int64) * prefill
        stride = {"padded": padded, "zero": 0, "half": padded // 2}[stride_mode]
        hot_rows = (req - 1) * stride + padded
        hot_np = rng.integers(0, 256, size=(hot_rows, ROW), dtype=np.uint8)
        hot = torch.from_numpy(hot_np.copy()).cuda()
        args = (layer, to_dev(topk), to_dev(pool_idx), to_dev(host_base), to_dev(slots), to_dev(miss),
                to_dev(np.array([req], dtype=np.int32)), hot, req, top_k)
        read = pool.batch_read_fused if fused else pool.batch_read
        status = read(*args, block_dim=block_dim, hot_req_stride_rows=stride)
        pool.wait(status, block_dim=block_dim)
        torch.cuda.synchronize()
        plsr = pool.per_layer_seg_rows
        for s in range(N):
            _, words = orc.gather_rows(segs, hot_np.reshape(-1), layer * plsr, ROW, topk, pool_idx, host_base, slots,
                                       miss, req, top_k, req, S, N, s, hot_req_stride_rows=stride,
                                       block_dim=block_dim)
            assert _read_words(status + s * 64, block_dim) == [int(w) for w in words], s
        np.testing.assert_array_equal(hot.cpu().numpy(), hot_np)
    finally:
        pool.destroy(close_ext=False)


@pytest.mark.parametrize("top_k", [1000, 3000])   # 3 x 1000 positions: one-launch form; 3 x 3000: two launches
@pytest.mark.parametrize("fused", [False, True])    # import_seg per segment, or import_all
def test_gather_rows_past_layer_region(kvops, top_k, fused):
    """Host rows whose segment row lies past the layer region (host base +
    token >= N * per_layer_seg_rows): the reference would read the next
    layer's region, or past the segment's end for the last layer
    (kvc_gather_rows.cpp:69-81).  Here such a row is not read, it still counts
    as queued and still competes for its destination, and its block's status
    word carries 0x200 + (p & 0xFF) + (1 << 16) for the lowest such position
    p; the oracle applies the same rule.  Every hot byte and status word."""
    print("past-region case", top_k, fused, flush=True)
    req, L, prefill, dbs, N, block_dim = 3, 2, 4096, 2048, 2, 3
    padded = dbs
    layer_rows = req * prefill
    pool = HostSegPool(0, L, layer_rows, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        plsr = pool.per_layer_seg_rows
        assert plsr * N == layer_rows
        rng = np.random.default_rng(top_k + fused)
        views = pool.segment_views()
        for v in views:
            v[...] = rng.integers(0, 256, size=v.shape, dtype=np.uint8)
        segs = [v.reshape(-1) for v in views]
        # request 2's run starts 1000 rows before the end of the layer, so its
        # tokens >= 1000 name rows past the region of either layer
        host_base = np.array([0, prefill, layer_rows - 1000], dtype=np.int64)
        topk = rng.integers(0, prefill, size=(req, top_k)).astype(np.int32)
        slots = rng.integers(0, dbs, size=(req, top_k)).astype(np.int32)
        miss = (rng.random((req, top_k)) < 0.6).astype(np.int8)
        pool_idx = np.arange(req, dtype=np.int64)
        outside = (miss[2] != 0) & (host_base[2] + topk[2] >= layer_rows)
        assert outside.sum() > 100
        for layer in (0, L - 1):
            hot_np = rng.integers(0, 256, size=(req * padded, ROW), dtype=np.uint8)
            hot = torch.from_numpy(hot_np.copy()).cuda()
            args = (layer, to_dev(topk), to_dev(pool_idx), to_dev(host_base), to_dev(slots), to_dev(miss),
                    to_dev(np.array([req], dtype=np.int32)), hot, req, top_k)
            read = pool.batch_read_fused if fused else pool.batch_read
            status = read(*args, block_dim=block_dim, hot_req_stride_rows=padded)
            # the blocks that report the rows past the region fail the wait
            with pytest.raises(RuntimeError, match="kv op failed on node"):
                pool.wait(status, block_dim=block_dim)
            torch.cuda.synchronize()
            errs = 0
            for s in range(N):
                _, words = orc.gather_rows(segs, hot_np.reshape(-1), layer * plsr, ROW, topk, pool_idx, host_base,
                                           slots, miss, req, top_k, req, 1, N, s, hot_req_stride_rows=padded,
                                           block_dim=block_dim, per_layer_seg_rows=plsr)
                got = _read_words(status + s * 64, block_dim)
                assert got == [int(w) for w in words], (layer, s, [hex(w) for w in got], [hex(w) for w in words])
                errs += sum(1 for w in words if int(w) & 0xFFFFFFFF)
            assert errs >= 1, "no block reported the rows past the region"
            np.testing.assert_array_equal(hot.cpu().numpy(), hot_np, err_msg="layer {}".format(layer))
    finally:
        pool.destroy(close_ext=False)


def test_status_poll_and_timeout(kvops):
    st = kvops.alloc_status(4)
    # nothing launched: the slot stays pending and the poll times out
    assert kvops.poll_status(st, 2000) == -0x2000
    # not a status address
    assert kvops.poll_status(12345, 10) == -0x1000


def test_status_poll_device_memory(kvops):
    """A status word in device memory (the reference polls any status
    address, kvops_ext.cpp:198-218): pending times out, a done word returns
    its err field, an unaligned address is refused."""
    import torch

    words = torch.zeros(16, dtype=torch.int64, device="cuda")
    addr = words.data_ptr()
    assert kvops.poll_status(addr, 2000) == -0x2000
    words[1] = (1 << 32) | (5 << 40) | 0x203  # done, 5 rows queued, err 0x203
    torch.cuda.synchronize()
    assert kvops.poll_status(addr + 8, 1000) == 0x203
    assert kvops.poll_status(addr + 4, 10) == -0x1000


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("S,N,block_dim,max_rows,num_real", [(1, 2, 1, 64, 64), (1, 3, 3, 500, 377), (64, 4, 2, 256, 256),
                                                             (4, 2, 8, 1000, 999), (1, 1, 1, 40, 0),
                                                             (1, 2, 2, 3000, 2900), (1, 2, 4, 5000, 4999)])
def test_export_rows_parity(kvops, S, N, block_dim, max_rows, num_real, fused):
    """Decode-incremental export of one layer into every segment against the
    oracle: host rows with duplicates (last entry wins), negative rows and rows
    outside the layer region (reported, not written), num_real below the
    capacity; all segment bytes and every node's status words.  Up to 4096
    entries the export is one launch, above it two (the 5000-entry case); the
    one launch decides winners in LDS up to 1024 entries and by device-scope
    tags above (the 2900-entry case)."""
    print("export_rows case", S, N, block_dim, max_rows, num_real, fused, flush=True)
    L, layer_rows = 3, 4096
    pool = HostSegPool(0, L, layer_rows, ROW, stripe_rows=S, node_num=N)
    pool.create_pool()
    try:
        plsr = pool.per_layer_seg_rows
        views = pool.segment_views()
        rng = np.random.default_rng(S * 1000 + N * 10 + block_dim)
        # non-zero starting content so untouched rows are checked too
        for v in views:
            v[...] = rng.integers(0, 256, size=v.shape, dtype=np.uint8)
        expect = [v.copy().reshape(-1) for v in views]
        idx = rng.integers(0, layer_rows, size=max_rows).astype(np.int64)
        dup = rng.integers(0, max_rows, size=max_rows // 4)
        idx[dup] = idx[rng.integers(0, max_rows, size=dup.size)]
        idx[rng.integers(0, max_rows, size=max_rows // 16)] = -1
        idx[rng.integers(0, max_rows, size=max_rows // 32)] = layer_rows * S * N + 7  # beyond the layer region
        src = rng.integers(0, 256, size=(max_rows, ROW), dtype=np.uint8)
        src_d = torch.from_numpy(src).cuda()
        idx_d = to_dev(idx)
        nr_d = to_dev(np.array([num_real], dtype=np.int32))
        layer = 1
        export = pool.batch_export_rows_fused if fused else pool.batch_export_rows
        status = export(layer, src_d, idx_d, nr_d, max_rows, block_dim=block_dim)
        torch.cuda.synchronize()  # (the status words carry error codes here, so no pool.wait)
        for s in range(N):
            _, words = orc.export_rows(expect[s], src.reshape(-1), idx, num_real, max_rows, layer, plsr, ROW, S, N, s,
                                       block_dim)
            got = _read_words(status + s * 64, block_dim)
            assert got == [int(w) for w in words], (s, got, [int(w) for w in words])
            np.testing.assert_array_equal(views[s].reshape(-1), expect[s], err_msg="segment {}".format(s))
    finally:
        pool.destroy(close_ext=False)


def test_status_ring_blocks(kvops):
    """next_status hands out disjoint blocks of node_num slots inside the ring;
    a call whose status block would run past its alloc_status block is
    rejected before anything is launched."""
    N = 3
    pool = HostSegPool(0, 1, 64, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        base, count = pool._status_base, pool._status_count
        blocks = [pool.next_status() for _ in range(30)]
        for addr in blocks:
            assert base <= addr and addr + N * 64 <= base + count * 64
        assert len(set(blocks[:count // N])) == count // N
        idx = to_dev(np.array([-1], dtype=np.int64))
        nr = to_dev(np.array([1], dtype=np.int32))
        src = torch.zeros((1, ROW), dtype=torch.uint8, device="cuda")
        seg = pool.pool.segments[N - 1].seg_base
        with pytest.raises(RuntimeError, match="past the end"):
            kvops.export_rows(0, seg, 0, pool.per_layer_seg_rows, ROW, src.data_ptr(), idx.data_ptr(), 0,
                              nr.data_ptr(), 1, 1, N, N - 1, base + (count - 1) * 64, 0, 1)
        kvops.export_rows(0, seg, 0, pool.per_layer_seg_rows, ROW, src.data_ptr(), idx.data_ptr(), 0, nr.data_ptr(),
                          1, 1, N, N - 1, base, 0, 1)
        torch.cuda.synchronize()
        assert _read_words(base + (N - 1) * 64, 1) == [DONE]
    finally:
        pool.destroy(close_ext=False)
