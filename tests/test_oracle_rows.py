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


def _model_gather(c, my_node):
    """Forward walk: later positions overwrite earlier ones."""
    hot = {}
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
        dst = slot + b * c["stride"]
        hot[dst] = (node, row)
        if node == my_node:
            counts[p // ppc] += 1
    words = []
    for b in range(c["block_dim"]):
        if b * ppc >= total:
            words.append(1 << 32)
        else:
            words.append((int(counts[b]) << 40) | (1 << 32))
    return {d: r for d, (n, r) in hot.items() if n == my_node}, words


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
