"""The oracle's row movers (kvc_gather_rows.cpp:12-96,
kvc_scatter_rows_alllayer.cpp:11-67) against what the memcpy semantics fix.

Every host row carries a fingerprint of (layer, global row) in its first
eight bytes and a row-unique pattern after, so a row copied from the wrong
segment, layer or segment row, a dropped row and a wrong winner all show up.
The independent model walks positions forward and lets a later position
overwrite an earlier one (the reference's single-block order); the oracle
walks backward and keeps the first destination it sees.  The status words
are checked against the count the reference queues per block
(kvc_gather_rows.cpp:60-94): valid miss positions owned by the segment.
"""
import numpy as np
import pytest

from oracle import oracle as orc

ROW_BYTES = 128


def _fingerprint(layer, row):
    return (np.uint64(layer) << np.uint64(40)) | np.uint64(row + 1)


def _make_segments(rng, layer_num, layer_rows, S, N):
    """Host segments holding every (layer, global row) at its mapped place;
    returns (segments, plsr).  With S > 1 the last row of a stripe is the one
    a segment row holds (the export's winner rule)."""
    plsr = -(-layer_rows // N)
    if S > 1:
        plsr = -(-layer_rows // (S * N)) + 1
    elif S == 0:
        plsr = layer_rows
    segs = [np.zeros(layer_num * plsr * ROW_BYTES, dtype=np.uint8) for _ in range(N)]
    for l in range(layer_num):
        for row in range(layer_rows):
            node = (row // S) % N if S else 0
            seg_row = (row // S) // N if S else row
            off = (l * plsr + seg_row) * ROW_BYTES
            body = np.frombuffer(_fingerprint(l, row).tobytes(), dtype=np.uint8)
            segs[node][off:off + 8] = body
            segs[node][off + 8:off + ROW_BYTES] = rng.integers(0, 256, ROW_BYTES - 8, dtype=np.uint8)
    return segs, plsr


def _gather_case(rng, S, N, stride, block_dim):
    layer_num, reqs, top_k, prefill = 3, 5, 24, 40
    layer_rows = reqs * prefill
    segs, plsr = _make_segments(rng, layer_num, layer_rows, S, N)
    max_num_reqs = reqs + 1
    num_real = int(rng.integers(0, max_num_reqs + 2))
    topk = rng.integers(-2, prefill, size=(max_num_reqs, top_k)).astype(np.int32)
    slots = rng.integers(-1, 12, size=(max_num_reqs, top_k)).astype(np.int32)  # many collisions
    is_miss = (rng.random((max_num_reqs, top_k)) < 0.6).astype(np.int8)
    req_pool = rng.permutation(max_num_reqs).astype(np.int64) - 1  # one row has pool -1
    host_base = (rng.permutation(max_num_reqs) % reqs).astype(np.int64) * prefill
    layer = int(rng.integers(0, layer_num))
    hot_rows = 12 + (max_num_reqs - 1) * stride
    return dict(segs=segs, plsr=plsr, layer=layer, topk=topk, slots=slots, is_miss=is_miss, req_pool=req_pool,
                host_base=host_base, num_real=num_real, top_k=top_k, max_num_reqs=max_num_reqs, S=S, N=N,
                stride=stride, block_dim=block_dim, hot_rows=hot_rows)


def _model_gather(c, my_node, plsr=None):
    """Forward walk: later positions overwrite earlier ones.  With plsr, a
    row whose segment row is >= plsr is not read: it still claims its
    destination (so the destination keeps its old bytes if it is the last
    claim) and still counts as queued, and the first such position of a
    block sets that block's error field."""
    hot = {}
    first_err = {}
    counts = np.zeros(c["block_dim"], dtype=np.int64)
    numr = max(0, min(c["num_real"], c["max_num_reqs"]))
    total = numr * c["top_k"]
    ppc = -(-c["max_num_reqs"] * c["top_k"] // c["block_dim"])
    for p in range(total):
        b, k = divmod(p, c["top_k"])
        t, slot = int(c["topk"][b, k]), int(c["slots"][b, k])
        if not c["is_miss"][b, k] or t < 0 or slot < 0 or c["req_pool"][b] < 0:
            continue
        row = int(c["host_base"][b]) + t
        node = (row // c["S"]) % c["N"] if c["S"] else 0
        seg_row = (row // c["S"]) // c["N"] if c["S"] else row
        inside = plsr is None or seg_row < plsr
        dst = slot + b * c["stride"]
        hot[dst] = (node, row, inside)
        if node == my_node:
            counts[p // ppc] += 1
            if not inside:
                first_err.setdefault(p // ppc, p)
    words = []
    for b in range(c["block_dim"]):
        if b * ppc >= total:
            words.append(1 << 32)
        else:
            err = (0x200 + (first_err[b] & 0xFF) + (1 << 16)) if b in first_err else 0
            words.append((int(counts[b]) << 40) | (1 << 32) | err)
    return {d: r for d, (n, r, ok) in hot.items() if n == my_node and ok}, words


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("S,N,stride,block_dim", [(1, 2, 0, 1), (1, 4, 12, 3), (64, 2, 12, 8), (0, 3, 0, 2),
                                                   (3, 3, 12, 1)])
def test_gather_rows_against_forward_model(seed, S, N, stride, block_dim):
    rng = np.random.default_rng(1000 * seed + 7 * N + S)
    c = _gather_case(rng, S, N, stride, block_dim)
    sentinel = np.uint8(0xA5)
    union = np.full(c["hot_rows"] * ROW_BYTES, sentinel, dtype=np.uint8)
    owners = {}
    for my in range(N):
        hot = np.full(c["hot_rows"] * ROW_BYTES, sentinel, dtype=np.uint8)
        n, words = orc.gather_rows(c["segs"], hot, c["layer"] * c["plsr"], ROW_BYTES, c["topk"], c["req_pool"],
                                   c["host_base"], c["slots"], c["is_miss"], c["num_real"], c["top_k"],
                                   c["max_num_reqs"], S, N, my, hot_req_stride_rows=c["stride"],
                                   block_dim=block_dim)
        want, want_words = _model_gather(c, my)
        assert list(words) == want_words
        assert n == len(want)
        for dst in range(c["hot_rows"]):
            got = hot[dst * ROW_BYTES:(dst + 1) * ROW_BYTES]
            if dst in want:
                row = want[dst]
                node = (row // S) % N if S else 0
                seg_row = (row // S) // N if S else row
                off = (c["layer"] * c["plsr"] + seg_row) * ROW_BYTES
                np.testing.assert_array_equal(got, c["segs"][node][off:off + ROW_BYTES])
                if S <= 1:
                    assert got[:8].view(np.uint64)[0] == _fingerprint(c["layer"], row)
                assert dst not in owners
                owners[dst] = my
                union[dst * ROW_BYTES:(dst + 1) * ROW_BYTES] = got
            else:
                assert (got == sentinel).all()
    # after all N segments every destination holds its winning position's row
    assert set(owners) == set(_model_gather_all(c))


def _model_gather_all(c):
    dests = set()
    for my in range(c["N"]):
        dests |= set(_model_gather(c, my)[0])
    return dests


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("S,N,stride,block_dim", [(1, 2, 0, 1), (1, 4, 12, 3), (64, 2, 12, 8), (3, 3, 12, 2)])
def test_gather_rows_past_layer_region(seed, S, N, stride, block_dim):
    """Host rows past the layer region (segment row >= plsr, reachable when a
    request's host base sits near the end of the layer's rows): not read,
    counted as queued, still the winner of their destination, and the lowest
    such position of each block reported in the 0x200 band."""
    rng = np.random.default_rng(500 + 100 * seed + 7 * N + S)
    c = _gather_case(rng, S, N, stride, block_dim)
    edge = N * c["plsr"] * max(S, 1)  # the first global row past the region
    c["host_base"] = c["host_base"] + (edge - 60)
    c["num_real"] = c["max_num_reqs"]
    errs = 0
    for my in range(N):
        hot = np.full(c["hot_rows"] * ROW_BYTES, 0xA5, dtype=np.uint8)
        n, words = orc.gather_rows(c["segs"], hot, c["layer"] * c["plsr"], ROW_BYTES, c["topk"], c["req_pool"],
                                   c["host_base"], c["slots"], c["is_miss"], c["num_real"], c["top_k"],
                                   c["max_num_reqs"], S, N, my, hot_req_stride_rows=c["stride"],
                                   block_dim=block_dim, per_layer_seg_rows=c["plsr"])
        want, want_words = _model_gather(c, my, plsr=c["plsr"])
        assert list(words) == want_words
        assert n == len(want)
        errs += sum(1 for w in want_words if w & 0xFFFFFFFF)
        for dst in range(c["hot_rows"]):
            got = hot[dst * ROW_BYTES:(dst + 1) * ROW_BYTES]
            if dst in want:
                row = want[dst]
                node = (row // S) % N if S else 0
                seg_row = (row // S) // N if S else row
                off = (c["layer"] * c["plsr"] + seg_row) * ROW_BYTES
                np.testing.assert_array_equal(got, c["segs"][node][off:off + ROW_BYTES])
            else:
                assert (got == 0xA5).all()
    assert errs > 0


def test_gather_empty_slice_words():
    """num_real == 0: nothing copied, every block reports done with 0 queued."""
    rng = np.random.default_rng(3)
    c = _gather_case(rng, 1, 2, 0, 4)
    c["num_real"] = 0
    hot = np.zeros(c["hot_rows"] * ROW_BYTES, dtype=np.uint8)
    n, words = orc.gather_rows(c["segs"], hot, 0, ROW_BYTES, c["topk"], c["req_pool"], c["host_base"], c["slots"],
                               c["is_miss"], 0, c["top_k"], c["max_num_reqs"], 1, 2, 0, block_dim=4)
    assert n == 0 and list(words) == [1 << 32] * 4 and not hot.any()


@pytest.mark.parametrize("S,N,lo,cnt", [(1, 2, 0, 60), (1, 4, 13, 47), (8, 2, 5, 70), (0, 1, 0, 30), (3, 3, 1, 58)])
def test_export_round_trip(S, N, lo, cnt):
    """export every node, then read each row back through the mapping: with
    S <= 1 every row comes back; with S > 1 a segment row holds the highest
    exported row of its stripe.  queued = rows owned by the node per layer."""
    rng = np.random.default_rng(S * 100 + N * 10 + lo)
    layer_num, layer_rows = 3, 80
    stride = layer_rows * ROW_BYTES + 256
    src = rng.integers(0, 256, layer_num * stride, dtype=np.uint8)
    plsr = -(-layer_rows // N) if S <= 1 else -(-layer_rows // (S * N)) + 1
    segs = []
    for my in range(N):
        seg = np.zeros(layer_num * plsr * ROW_BYTES, dtype=np.uint8)
        q = orc.export_alllayer(seg, src, stride, plsr, ROW_BYTES, lo, cnt, layer_num, S, N, my)
        owned = [r for r in range(lo, lo + cnt) if ((r // S) % N if S else 0) == my]
        assert q == layer_num * len(owned)
        segs.append(seg)
    for l in range(layer_num):
        last = {}
        for r in range(lo, lo + cnt):
            node = (r // S) % N if S else 0
            seg_row = (r // S) // N if S else r
            last[(node, seg_row)] = r
        for (node, seg_row), r in last.items():
            off = (l * plsr + seg_row) * ROW_BYTES
            np.testing.assert_array_equal(segs[node][off:off + ROW_BYTES],
                                          src[l * stride + r * ROW_BYTES:l * stride + (r + 1) * ROW_BYTES])
        # untouched segment rows stay zero
        for node in range(N):
            for seg_row in range(plsr):
                if (node, seg_row) not in last:
                    off = (l * plsr + seg_row) * ROW_BYTES
                    assert not segs[node][off:off + ROW_BYTES].any()


# ---- decode-incremental export (the design's export_rows) ----

@pytest.mark.parametrize("S,N,row_lo,row_cnt,block_dim", [(1, 2, 0, 300, 1), (1, 3, 17, 250, 3), (64, 4, 0, 1024, 2),
                                                           (5, 2, 3, 97, 1)])
def test_export_rows_contiguous_equals_alllayer(S, N, row_lo, row_cnt, block_dim):
    """A contiguous index list [row_lo, row_lo+row_cnt) with entry i sourced
    from row row_lo+i leaves every segment exactly as the all-layer export of
    that range does for one layer (both resolve a stripe's shared segment row
    to its highest row), and the owned counts agree with its queued count."""
    rng = np.random.default_rng(S * 100 + N)
    layer_rows = row_lo + row_cnt + 64
    plsr = -(-layer_rows // N) if S == 1 else -(-layer_rows // (S * N)) + 1
    src = rng.integers(0, 256, size=layer_rows * ROW_BYTES, dtype=np.uint8)
    idx = np.arange(row_lo, row_lo + row_cnt, dtype=np.int64)
    for my in range(N):
        seg_a = np.zeros(plsr * ROW_BYTES, dtype=np.uint8)
        seg_b = np.zeros(plsr * ROW_BYTES, dtype=np.uint8)
        queued = orc.export_alllayer(seg_a, src, layer_rows * ROW_BYTES, plsr, ROW_BYTES, row_lo, row_cnt, 1, S, N, my)
        n, words = orc.export_rows(seg_b, np.ascontiguousarray(src[row_lo * ROW_BYTES:]), idx, row_cnt, row_cnt, 0,
                                   plsr, ROW_BYTES, S, N, my, block_dim)
        np.testing.assert_array_equal(seg_a, seg_b)
        assert sum(int(w) >> 40 for w in words) == queued
        assert all((int(w) >> 32) & 0xFF == 1 and int(w) & 0xFFFFFFFF == 0 for w in words)


def test_export_rows_last_entry_wins_and_errors():
    """Entries naming one host row leave the last one's bytes; negative rows,
    rows of other nodes and entries past num_real write nothing; a row whose
    segment row is outside the layer region is reported with the import's
    error code for the lowest such entry of its status block."""
    S, N, plsr, layers = 1, 2, 40, 3
    src = np.repeat(np.arange(1, 11, dtype=np.uint8), ROW_BYTES)  # entry i's row is all (i+1)
    idx = np.array([4, 6, 4, -1, 5, 200, 4, 9, 202, 6], dtype=np.int64)
    seg = np.zeros(layers * plsr * ROW_BYTES, dtype=np.uint8)
    n, words = orc.export_rows(seg, src, idx, 9, 10, 1, plsr, ROW_BYTES, S, N, 0, 2)
    rows = seg.reshape(layers, plsr, ROW_BYTES)
    # node 0 owns even rows: 4 -> segment row 2 (entries 0, 2, 6: last is 6), 6 -> row 3 (entry 1; entry 9 is
    # past num_real), 200 -> row 100 >= plsr (entry 5, error), 202 -> row 101 (entry 8, error)
    assert (rows[1, 2] == 7).all() and (rows[1, 3] == 2).all()
    assert n == 4
    written = {2, 3}
    for r in range(plsr):
        if r not in written:
            assert (rows[1, r] == 0).all(), r
    assert (rows[0] == 0).all() and (rows[2] == 0).all()
    # status blocks of 5 entries: [0,5) owns entries 0,1,2 ; [5,9) owns 5,6,8 with the first error at 5
    assert int(words[0]) == (3 << 40) | (1 << 32)
    assert int(words[1]) == (3 << 40) | (1 << 32) | (0x200 + 5 + (1 << 16))


@pytest.mark.parametrize("threads", [1, 3, 16])
@pytest.mark.parametrize("S,N,stride", [(1, 2, 0), (1, 4, 12), (64, 2, 12), (3, 3, 12)])
def test_stage_rows_scatter_equals_gather(threads, S, N, stride):
    """The CPU pipeline's staging step: scattering the staged rows to their
    hot rows gives what orc_gather_rows gives over all segments (each
    destination staged once, with its winning row)."""
    rng = np.random.default_rng(77 + threads + S + N)
    c = _gather_case(rng, S, N, stride, 1)
    want = np.zeros(c["hot_rows"] * ROW_BYTES, dtype=np.uint8)
    for my in range(N):
        orc.gather_rows(c["segs"], want, c["layer"] * c["plsr"], ROW_BYTES, c["topk"], c["req_pool"], c["host_base"],
                        c["slots"], c["is_miss"], c["num_real"], c["top_k"], c["max_num_reqs"], S, N, my,
                        hot_req_stride_rows=stride)
    cap = c["max_num_reqs"] * c["top_k"]
    staging = np.zeros((cap, ROW_BYTES), dtype=np.uint8)
    dst = np.full(cap, -1, dtype=np.int64)
    n = orc.stage_rows(c["segs"], staging, dst, c["layer"] * c["plsr"], ROW_BYTES, c["topk"], c["req_pool"],
                       c["host_base"], c["slots"], c["is_miss"], c["num_real"], c["top_k"], c["max_num_reqs"], S, N,
                       stride, threads)
    assert n == len(set(dst[:n].tolist()))
    got = np.zeros_like(want).reshape(-1, ROW_BYTES)
    got[dst[:n]] = staging[:n]
    np.testing.assert_array_equal(got.reshape(-1), want)
