"""The oracle's hash table (Knuth multiplicative hash, linear probing,
Algorithm R deletion; reference hisp_kernel_common.h:23-112) against
properties fixed by the mathematics, by brute force on small tables."""
import numpy as np
import pytest

from oracle import oracle as orc


def _home(t, size):
    return orc.ht_hash(t) & (size - 1)


def test_hash_closed_form():
    for t in [0, 1, 2, 3, 100, 65535, 131071, 2**31 - 1]:
        assert orc.ht_hash(t) == ((t * 2654435761) & 0xFFFFFFFF) >> 16
    # negative tokens are never hashed by the kernels; the cast is uint32 wrap
    assert orc.ht_hash(-1) == ((0xFFFFFFFF * 2654435761) & 0xFFFFFFFF) >> 16


def _check_table(ht, tok, live):
    """Every live token is found at its own slot; nothing else is in the table;
    each entry sits in the probe run from its home (no empty cell between)."""
    size = ht.size
    assert int((ht != 0).sum()) == len(live)
    for t, s in live.items():
        assert orc.ht_find(ht, tok, t) == s
    for i in range(size):
        e = int(ht[i])
        if e == 0:
            continue
        h = _home(int(tok[e - 1]), size)
        j = h
        while j != i:
            assert ht[j] != 0, "empty cell between home and entry"
            j = (j + 1) % size


@pytest.mark.parametrize("seed", range(12))
def test_random_insert_erase_history_independent(seed):
    """Algorithm R leaves the table exactly as inserting the live keys in their
    insertion order would; a dropped move or a wrong wrap test breaks it."""
    rng = np.random.default_rng(seed)
    size = int(rng.choice([8, 16, 32]))
    slots = size  # token storage, one slot per potential live key
    tok = np.full(slots, -1, dtype=np.int32)
    ht = np.zeros(size, dtype=np.uint16)
    live = {}  # token -> slot
    order = []
    free_slots = list(range(slots))
    universe = rng.choice(5000, size=3 * size, replace=False)
    for _ in range(200):
        if live and (rng.random() < 0.45 or len(live) >= size - 1):
            t = int(rng.choice(list(live)))
            orc.ht_erase(ht, tok, t)
            s = live.pop(t)
            order.remove(t)
            tok[s] = -1
            free_slots.append(s)
        else:
            cands = [int(u) for u in universe if int(u) not in live]
            t = cands[int(rng.integers(len(cands)))]
            s = free_slots.pop(0)
            orc.ht_insert(ht, tok, t, s)
            tok[s] = t
            live[t] = s
            order.append(t)
        _check_table(ht, tok, live)
        rebuilt = np.zeros(size, dtype=np.uint16)
        for t in order:
            orc.ht_insert(rebuilt, tok, t, live[t])
        assert np.array_equal(rebuilt, ht)
    assert orc.get_error() == 0


def test_insert_keeps_first_slot_for_duplicate():
    tok = np.array([5, 5, 7, -1], dtype=np.int32)
    ht = np.zeros(1024, dtype=np.uint16)
    orc.ht_insert(ht, tok, 5, 0)
    orc.ht_insert(ht, tok, 5, 1)
    assert (ht != 0).sum() == 1
    assert orc.ht_find(ht, tok, 5) == 0


def test_erase_wraps_around_table_end():
    size = 8
    # pick three tokens homed at the last cell so their run wraps to 0, 1
    toks = [t for t in range(20000) if _home(t, size) == size - 1][:3]
    tok = np.array(toks + [-1], dtype=np.int32)
    ht = np.zeros(size, dtype=np.uint16)
    for s, t in enumerate(toks):
        orc.ht_insert(ht, tok, t, s)
    assert ht[size - 1] == 1 and ht[0] == 2 and ht[1] == 3
    orc.ht_erase(ht, tok, toks[0])
    assert ht[size - 1] == 2 and ht[0] == 3 and ht[1] == 0
    assert orc.ht_find(ht, tok, toks[2]) == 2


def test_ht_init_equals_insert_replay():
    rng = np.random.default_rng(3)
    layers, pool, dbs = 2, 3, 40
    padded = orc.padded_of(dbs)
    size = orc.ht_size(padded, 8)
    tokens = np.full((layers, pool, padded), -1, dtype=np.int32)
    for l in range(layers):
        for r in range(pool):
            n = int(rng.integers(0, dbs + 1))
            tokens[l, r, :n] = rng.choice(1000, size=n, replace=False)
            tokens[l, r, dbs:] = 999999  # beyond dbs: never inserted
    ht = np.full((layers, pool, size), 77, dtype=np.uint16)
    orc.sieve_ht_init(tokens, ht, 1, 2, layers, pool, dbs, padded, size)
    for l in range(layers):
        assert np.all(ht[l, 0] == 77)  # row outside [reqStart, reqStart+numReqs) untouched
        for r in (1, 2):
            ref = np.zeros(size, dtype=np.uint16)
            for s in range(dbs):
                if tokens[l, r, s] >= 0:
                    orc.ht_insert(ref, tokens[l, r], int(tokens[l, r, s]), s)
            assert np.array_equal(ht[l, r], ref)


def test_derivations_match_reference_literals():
    import json, os
    d = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "reference_kats.json")))["derive"]
    for padded, topk, expect in d["ht_size"]:
        assert orc.ht_size(padded, topk) == expect
    for padded, topk in d["ht_size_props"]:
        h = orc.ht_size(padded, topk)
        assert h & (h - 1) == 0 and h >= 2 * (padded + topk) and h >= 1024
    for padded, expect in d["visited_stride"]:
        assert orc.vis_stride_of(padded) == expect
    # reqsPerCore: kvops_ext.cpp:307-312 (64/gcd alignment)
    assert orc.reqs_per_core(8, 8, 64) == 1
    assert orc.reqs_per_core(64, 8, 2048) == 8
    assert orc.reqs_per_core(8, 8, 6) == 32  # gcd(6,64)=2 -> align 32
    assert orc.reqs_per_core(3, 8, 7) == 64
