"""kvx_import_all_noalloc (the import with a fixed scratch array per GPU,
for callers that cannot allocate) against kvx_import_all, both called
through the C ABI: every hot-buffer byte and every status word equal, and
equal to the oracle's, on two calls in a row with the second one smaller;
a call beyond the fixed scratch's limits fails before anything runs."""
import ctypes

import numpy as np
import pytest
import torch

from gpu_helpers import read_words
from kv_offload_proto_amd.kvops_ext import lib_path
from kv_offload_proto_amd.xds import HostSegPool, XdsOffloadCoordinator, streams
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ROW = 1152
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
IMPORT_ARGS = [ctypes.POINTER(_u64), _u32, _u32, _u32, _u64, _u64, _u64, _u64, _u64, _u64, _u64, _u32, _u32, _u32,
               _u32, _u64, _u64, _u32, _u32]


def _lib():
    lib = ctypes.CDLL(lib_path())
    for name in ("kvx_import_all", "kvx_import_all_noalloc"):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = IMPORT_ARGS
    lib.kvx_last_error.restype = ctypes.c_char_p
    return lib


def _call(lib, name, pool, layer, topk, coord, nr, hot, top_k, max_num_reqs, status, stride):
    bases = (_u64 * pool.node_num)(*[sg.seg_base for sg in pool.pool.segments])
    rc = getattr(lib, name)(bases, layer * pool.per_layer_seg_rows, pool.per_layer_seg_rows, ROW, topk.data_ptr(),
                            coord._req_pool_indices.data_ptr(), coord.req_host_base.data_ptr(),
                            coord.top_k_device_slots.data_ptr(), coord.is_miss.data_ptr(), nr.data_ptr(),
                            hot.data_ptr(), top_k, max_num_reqs, pool.stripe_rows, pool.node_num, status,
                            torch.cuda.current_stream().cuda_stream, 2, stride)
    return rc


def test_import_all_noalloc_matches_import_all(kvops):
    L, R, prefill, dbs, top_k, N = 1, 16, 8192, 4096, 2048, 4
    print("no-alloc import", R, prefill, dbs, top_k, N, flush=True)
    lib = _lib()
    rows = R * prefill
    pool = HostSegPool(0, L, rows, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        g = torch.Generator(device="cuda")
        g.manual_seed(41)
        src = torch.randint(0, 256, (L, rows, ROW), dtype=torch.uint8, device="cuda", generator=g)
        pool.wait(pool.batch_write_alllayers(0, rows, src, rows * ROW))
        coord = XdsOffloadCoordinator("cuda", L, R, dbs, top_k, R, prefill)
        st = orc.SieveState(L, R, dbs, top_k)
        for r in range(R):
            coord.admit_request(r, r, prefill, r * prefill)
            st.admit(r, prefill)
        coord.set_batch(torch.arange(R, dtype=torch.int64, device="cuda"),
                        torch.full((R,), prefill, dtype=torch.int32, device="cuda"))
        padded = coord.padded_buffer_size
        segs = [v.reshape(-1) for v in pool.segment_views()]
        hot_a = torch.zeros((R * padded, ROW), dtype=torch.uint8, device="cuda")
        hot_b = torch.zeros_like(hot_a)
        hot_o = np.zeros((R * padded, ROW), dtype=np.uint8)
        sa, sb = kvops.alloc_status(N), kvops.alloc_status(N)
        rng = np.random.default_rng(12)
        # call 1: every row of the batch; call 2: a smaller batch (5 rows
        # allocated, 4 of them real) on the state the first call left; call
        # 3: 2 rows x 2048 positions, the one-launch form of small batches
        for call, (mnr, nreal) in enumerate([(R, R), (5, 4), (2, 2)]):
            batch = streams.state_batch(rng, st.tokens[0, :, :dbs], prefill, top_k, 0.2, zipf_s=1.1)
            batch[mnr:] = -1
            topk_d = torch.from_numpy(batch).cuda()
            nr = torch.tensor([nreal], dtype=torch.int32, device="cuda")
            coord.num_real.fill_(nreal)
            coord.sieve_update(0, topk_d)
            e_slots, e_miss = st.update(0, batch, np.arange(R), np.full(R, prefill), nreal, max_num_reqs=R)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(coord.top_k_device_slots.cpu().numpy(), e_slots)
            assert _call(lib, "kvx_import_all", pool, 0, topk_d, coord, nr, hot_a, top_k, mnr, sa, padded) == 0, \
                lib.kvx_last_error()
            assert _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_b, top_k, mnr, sb,
                         padded) == 0, lib.kvx_last_error()
            pool.wait(sa, block_dim=2)
            pool.wait(sb, block_dim=2)
            torch.cuda.synchronize()
            for s in range(N):
                _, w = orc.gather_rows(segs, hot_o.reshape(-1), 0, ROW, batch, np.arange(R), np.arange(R) * prefill,
                                       e_slots, e_miss, nreal, top_k, mnr, 1, N, s, hot_req_stride_rows=padded,
                                       block_dim=2)
                want = [int(x) for x in w]
                assert read_words(sa + s * 64, 2) == want, (call, s)
                assert read_words(sb + s * 64, 2) == want, (call, s)
            assert torch.equal(hot_a, hot_b), call
            assert torch.equal(hot_b, torch.from_numpy(hot_o).cuda()), call
        # beyond the fixed scratch: more winner rows than its 2228224 (checked before any launch)
        before = hot_b.clone()
        big = (2228224 - 65536) // min(padded, 65536) + 2
        rc = _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_b, top_k, big, sb, padded)
        assert rc != 0 and b"must fit the fixed scratch" in lib.kvx_last_error()
        torch.cuda.synchronize()
        assert torch.equal(before, hot_b)
    finally:
        pool.destroy(close_ext=False)


def test_import_all_noalloc_fresh_stream_graph_and_overlap(kvops):
    """The property the entry point exists for: calls on a stream the library
    has never seen leave that stream without scratch (scratch_bytes 0), and a
    call captured in a HIP graph (where any allocation is refused) replays
    with the results of import_all.  Calls on two streams that may overlap
    are refused: the fixed scratch is shared by every call on the GPU."""
    L, R, prefill, dbs, top_k, N = 1, 8, 4096, 2048, 1024, 2
    print("no-alloc fresh stream / graph / overlap", R, top_k, N, flush=True)
    lib = _lib()
    rows = R * prefill
    pool = HostSegPool(0, L, rows, ROW, stripe_rows=1, node_num=N)
    pool.create_pool()
    try:
        g = torch.Generator(device="cuda")
        g.manual_seed(43)
        src = torch.randint(0, 256, (L, rows, ROW), dtype=torch.uint8, device="cuda", generator=g)
        pool.wait(pool.batch_write_alllayers(0, rows, src, rows * ROW))
        coord = XdsOffloadCoordinator("cuda", L, R, dbs, top_k, R, prefill)
        st = orc.SieveState(L, R, dbs, top_k)
        for r in range(R):
            coord.admit_request(r, r, prefill, r * prefill)
            st.admit(r, prefill)
        coord.set_batch(torch.arange(R, dtype=torch.int64, device="cuda"),
                        torch.full((R,), prefill, dtype=torch.int32, device="cuda"))
        padded = coord.padded_buffer_size
        batch = streams.state_batch(np.random.default_rng(14), st.tokens[0, :, :dbs], prefill, top_k, 0.3)
        topk_d = torch.from_numpy(batch).cuda()
        nr = torch.tensor([R], dtype=torch.int32, device="cuda")
        coord.sieve_update(0, topk_d)
        torch.cuda.synchronize()
        hot_a = torch.zeros((R * padded, ROW), dtype=torch.uint8, device="cuda")
        sa = kvops.alloc_status(N)
        assert _call(lib, "kvx_import_all", pool, 0, topk_d, coord, nr, hot_a, top_k, R, sa, padded) == 0
        pool.wait(sa, block_dim=2)
        torch.cuda.synchronize()
        want_words = [read_words(sa + s * 64, 2) for s in range(N)]

        # a stream the library has never used: no scratch before or after
        fresh = torch.cuda.Stream()
        assert kvops.scratch_bytes(fresh.cuda_stream) == 0
        hot_b = torch.zeros_like(hot_a)
        sb = kvops.alloc_status(N)
        with torch.cuda.stream(fresh):
            assert _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_b, top_k, R, sb,
                         padded) == 0, lib.kvx_last_error()
        fresh.synchronize()
        assert kvops.scratch_bytes(fresh.cuda_stream) == 0
        assert torch.equal(hot_a, hot_b)
        assert [read_words(sb + s * 64, 2) for s in range(N)] == want_words

        # captured in a graph on another fresh stream, replayed three times
        cap = torch.cuda.Stream()
        hot_c = torch.zeros_like(hot_a)
        sc = kvops.alloc_status(N)
        graph = torch.cuda.CUDAGraph()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            assert _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_c, top_k, R, sc,
                         padded) == 0, lib.kvx_last_error()
        assert kvops.scratch_bytes(cap.cuda_stream) == 0
        for rep in range(3):
            hot_c.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(hot_a, hot_c), rep
            assert [read_words(sc + s * 64, 2) for s in range(N)] == want_words, rep
        del graph

        # overlap: a call queued behind a long kernel on one stream, then a
        # call on another stream while the first may still run
        s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
        hot_d = torch.zeros_like(hot_a)
        sd = kvops.alloc_status(N)
        torch.cuda.synchronize()
        with torch.cuda.stream(s1):
            torch.cuda._sleep(200_000_000)  # a bounded spin on the GPU (~0.1 s)
            assert _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_d, top_k, R, sd,
                         padded) == 0, lib.kvx_last_error()
        with torch.cuda.stream(s2):
            rc = _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_b, top_k, R, sb, padded)
        assert rc != 0 and b"another stream" in lib.kvx_last_error()
        s1.synchronize()
        with torch.cuda.stream(s2):
            assert _call(lib, "kvx_import_all_noalloc", pool, 0, topk_d, coord, nr, hot_b, top_k, R, sb,
                         padded) == 0, lib.kvx_last_error()
        torch.cuda.synchronize()
        assert torch.equal(hot_a, hot_d) and torch.equal(hot_a, hot_b)
    finally:
        pool.destroy(close_ext=False)
