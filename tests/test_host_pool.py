"""Host-side pieces of the segment pool and the synthetic streams, on the CPU.

The allocator and derivation cases follow the reference's
test/test_allocator.py:16-93 (the contiguity contract src = host_base + token
that the gather relies on, fragment merge, exhaustion, range checks); the
literals come from tests/golden/reference_kats.json.
"""
import json
import os

import numpy as np
import pytest

from kv_offload_proto_amd.xds import streams
from kv_offload_proto_amd.xds.configs import CONFIGS
from kv_offload_proto_amd.xds.xds_seg_pool import RowAllocator, align, compute_ht_size, next_pow2
from oracle import oracle as orc

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def test_allocator_contiguous_contract():
    c = KATS["allocator"]["contiguous"]
    a = RowAllocator(c["capacity"])
    r0 = a.alloc(c["first"][1] - c["first"][0])
    r1 = a.alloc(c["second"][1] - c["second"][0])
    assert r0 == list(range(*c["first"])) and r1 == list(range(*c["second"]))
    a.free(r0)
    assert a.alloc(c["reuse"][1]) == list(range(*c["reuse"]))
    a.free(r1)
    assert a.used_rows() == c["reuse"][1]


def test_allocator_fragments_exhaustion_ranges():
    a = RowAllocator(10)
    rows = [a.alloc(1)[0] for _ in range(10)]
    assert rows == list(range(10))
    for r in rows[:5]:
        a.free([r])
    assert a.free_rows() == 5
    assert sorted(a.alloc(5)) == [0, 1, 2, 3, 4]
    with pytest.raises(MemoryError):
        RowAllocator(4).alloc(5)
    with pytest.raises(ValueError):
        RowAllocator(4).free([99])
    b = RowAllocator(64)
    blocks = [b.alloc(16) for _ in range(4)]
    for blk in blocks:
        b.free(blk)
    assert b.used_rows() == 0 and b.free_rows() == 64


def test_allocator_scattered_fallback():
    """No free run is long enough: rows come from the front of the free list."""
    a = RowAllocator(12)
    rows = a.alloc(12)
    a.free(rows[0:2])
    a.free(rows[5:7])
    a.free(rows[10:12])
    got = a.alloc(5)
    assert got == [0, 1, 5, 6, 10]
    assert a.free_rows() == 1


def test_derive_helpers_literals():
    d = KATS["derive"]
    for v, a, want in d["align"]:
        assert align(v, a) == want
    for v, want in d["next_pow2"]:
        assert next_pow2(v) == want
    for padded, top_k, want in d["ht_size"]:
        assert compute_ht_size(padded, top_k) == want == orc.ht_size(padded, top_k)
    for padded, top_k in d["ht_size_props"]:
        ht = compute_ht_size(padded, top_k)
        assert ht & (ht - 1) == 0 and ht >= 2 * (padded + top_k) and ht >= 1024
    for padded, want in d["visited_stride"]:
        assert orc.vis_stride_of(padded) == want == align((padded + 7) // 8, 64)


def test_ref_batch_shape_and_split():
    """xds_decode.py:211-222: per request n_hit positions in [0, min(prefill, dbs))
    and n_miss distinct positions in [dbs, prefill), shuffled over the batch."""
    cfg = CONFIGS[0]
    rng = np.random.default_rng(cfg.seed)
    b = streams.ref_batch(rng, cfg.req_num, cfg.top_k, cfg.prefill, cfg.dbs, cfg.miss_ratio)
    assert b.shape == (cfg.req_num, cfg.top_k) and b.dtype == np.int32
    assert ((b >= 0) & (b < cfg.prefill)).all()
    assert int((b >= cfg.dbs).sum()) == cfg.req_num * int(cfg.top_k * cfg.miss_ratio)
    rng2 = np.random.default_rng(cfg.seed)
    np.testing.assert_array_equal(b, streams.ref_batch(rng2, cfg.req_num, cfg.top_k, cfg.prefill, cfg.dbs,
                                                       cfg.miss_ratio))


def test_state_batch_miss_fraction():
    """The state-driven stream draws distinct positions with about miss_ratio
    of them not resident."""
    cfg = CONFIGS[2]
    st = orc.SieveState(1, 8, cfg.dbs, cfg.top_k)
    for r in range(8):
        st.admit(r, cfg.prefill)
    rng = np.random.default_rng(1)
    b = streams.state_batch(rng, st.tokens[0, :, :cfg.dbs], cfg.prefill, cfg.top_k, cfg.miss_ratio,
                            zipf_s=cfg.zipf_s)
    assert b.shape == (8, cfg.top_k)
    for r in range(8):
        assert len(np.unique(b[r])) == cfg.top_k
        assert ((b[r] >= 0) & (b[r] < cfg.prefill)).all()
        resident = np.isin(b[r], st.tokens[0, r, :cfg.dbs])
        assert abs((~resident).mean() - cfg.miss_ratio) < 0.03


def test_adversarial_pool_collides():
    cfg = CONFIGS[4]
    pool = streams.adversarial_pool(cfg.prefill, cfg.adversarial_hash_below)
    h = (pool.astype(np.uint64) * np.uint64(2654435761) % np.uint64(1 << 32)) >> np.uint64(16)
    assert (h < cfg.adversarial_hash_below).all()
    # every position with a hash below the bound is in the pool
    t = np.arange(cfg.prefill, dtype=np.uint64)
    all_h = (t * np.uint64(2654435761) % np.uint64(1 << 32)) >> np.uint64(16)
    assert len(pool) == int((all_h < cfg.adversarial_hash_below).sum()) == 81922
    # more candidates than a full buffer plus one step's misses: the pool
    # never runs dry, whatever the buffer holds
    assert len(pool) > cfg.dbs + cfg.miss_ratio * cfg.top_k


def test_adversarial_stream_misses_every_step():
    """The slot-limit stress stream keeps its 90% misses step after step (the
    oracle's state drives the draw): over 7,000 misses per request on each of
    the first three steps."""
    from oracle import oracle as orc

    cfg = CONFIGS[4]
    pool = streams.adversarial_pool(cfg.prefill, cfg.adversarial_hash_below)
    st = orc.SieveState(1, cfg.req_num, cfg.dbs, cfg.top_k)
    for r in range(cfg.req_num):
        st.admit(r, cfg.prefill)
    rng = np.random.default_rng(cfg.seed)
    for _ in range(3):
        batch = streams.state_batch(rng, st.tokens[0, :, :cfg.dbs], cfg.prefill, cfg.top_k, cfg.miss_ratio,
                                    miss_pool=pool)
        _, miss = st.update(0, batch, np.arange(cfg.req_num), np.full(cfg.req_num, cfg.prefill), cfg.req_num,
                            threads=4)
        assert miss.sum(axis=1).min() >= 7000


@pytest.mark.parametrize("bad", ["gpu", -1, 1024, 1.0, True, None])
def test_pool_placement_argument(bad):
    """placement is 'device', 'none' or a node number below 1024; anything
    else is refused when the pool is configured, before any memory is taken."""
    from kv_offload_proto_amd.xds.xds_seg_pool import HostSegPool

    for ok in ("device", "none", 0, 3):
        assert HostSegPool(0, 1, 64, 1152, placement=ok).placement == ok
    with pytest.raises(ValueError, match="placement"):
        HostSegPool(0, 1, 64, 1152, placement=bad)
