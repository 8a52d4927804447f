"""Brute force: the C oracle against the independent ring-CLOCK model
(tests/sieve_model.py) on random small batches, including every defensive
case of hisp_sieve_update.cpp (padding rows, bad pool rows, dirty hands,
invalid and decode-extension positions, duplicates, wrap-around sweeps)."""
import numpy as np
import pytest

from oracle import oracle as orc
from sieve_model import RingClock, model_batch


def _vis_bits(vis_row, dbs):
    return [(int(vis_row[s >> 3]) >> (s & 7)) & 1 for s in range(dbs)]


@pytest.mark.parametrize("seed", range(40))
def test_oracle_matches_model(seed):
    rng = np.random.default_rng(1000 + seed)
    dbs = int(rng.integers(1, 40))
    top_k = int(rng.integers(1, 24))
    pool = 4
    max_reqs = 5
    st = orc.SieveState(1, pool, dbs, top_k)
    prefills = [int(rng.integers(1, 3 * dbs + 4)) for _ in range(pool)]
    for r in range(pool):
        st.admit(r, prefills[r])
    # occasionally start from a dirty hand (kernel clamps it back to 0)
    if rng.random() < 0.3:
        st.hand[0, int(rng.integers(pool)), 0] = int(rng.choice([-5, dbs, dbs + 7]))
    models = {r: RingClock(dbs, st.padded, st.tokens[0, r].tolist(), _vis_bits(st.vis[0, r], dbs),
                           int(st.hand[0, r, 0])) for r in range(pool)}
    for step in range(6):
        rows = list(rng.permutation(pool))[: int(rng.integers(1, pool + 1))]
        req_pool = rows + [-1] * (max_reqs - len(rows))
        if rng.random() < 0.3:
            req_pool[int(rng.integers(max_reqs))] = int(rng.choice([-3, pool, pool + 5]))
        # distinct valid pool rows only (callers must not repeat a pool row)
        seen = set()
        for i, p in enumerate(req_pool):
            if 0 <= p < pool:
                if p in seen:
                    req_pool[i] = -1
                seen.add(p)
        num_real = int(rng.integers(0, max_reqs + 3))
        seq_lens = []
        for b in range(max_reqs):
            p = req_pool[b]
            pf = prefills[p] if 0 <= p < pool else 10
            seq_lens.append(int(pf + rng.integers(-2, 5)))
        topk = np.empty((max_reqs, top_k), dtype=np.int32)
        for b in range(max_reqs):
            hi = max(seq_lens[b] + 3, 2)
            topk[b] = rng.integers(-2, hi, size=top_k)
            if rng.random() < 0.3 and top_k > 1:  # duplicates inside a row
                topk[b, -1] = topk[b, 0]
        slots, miss = st.update(0, topk, req_pool, seq_lens, num_real, max_num_reqs=max_reqs)
        m_slots, m_miss = model_batch(models, topk.tolist(), req_pool, seq_lens, st.prefill_lens.tolist(), num_real,
                                      pool, dbs, st.padded)
        assert slots.tolist() == m_slots, (seed, step)
        assert miss.tolist() == m_miss, (seed, step)
        for r in range(pool):
            tok = st.tokens[0, r]
            ring = [t if t is not None else -1 for t in models[r].ring]
            assert tok[:dbs].tolist() == ring
            assert np.all(tok[dbs:] == -1)
            assert _vis_bits(st.vis[0, r], dbs) == [int(b) for b in models[r].ref]
            touched = any(req_pool[b] == r for b in range(min(num_real, max_reqs)))
            if touched:
                assert int(st.hand[0, r, 0]) == models[r].hand
            # table <-> tokens consistent
            ht = st.ht[0, r]
            assert int((ht != 0).sum()) == int((tok[:dbs] >= 0).sum())
            for s in range(dbs):
                if tok[s] >= 0:
                    assert orc.ht_find(ht, tok, int(tok[s])) == s
    assert orc.get_error() == 0


def test_ring_clock_invariants_long_run():
    """Misses always land in [0, dbs), hits point at a slot holding the token,
    the hand stays in range, and the resident set never exceeds dbs."""
    rng = np.random.default_rng(5)
    dbs, top_k, prefill = 48, 32, 400
    st = orc.SieveState(1, 1, dbs, top_k)
    st.admit(0, prefill)
    for _ in range(60):
        topk = rng.integers(0, prefill, size=(1, top_k)).astype(np.int32)
        slots, miss = st.update(0, topk, [0], [prefill], 1)
        tok = st.tokens[0, 0]
        for k in range(top_k):
            s = int(slots[0, k])
            assert 0 <= s < dbs
            # the token at that position now owns the slot unless a later miss in
            # this same batch reused it
            if not any(int(slots[0, j]) == s and miss[0, j] for j in range(k + 1, top_k)):
                assert tok[s] == topk[0, k]
        assert 0 <= st.hand[0, 0, 0] < dbs
        assert (tok[:dbs] >= 0).sum() <= dbs
