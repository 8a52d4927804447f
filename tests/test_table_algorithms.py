"""CPU checks of the two table algorithms the GPU kernels are built on.

* Batch deletion (the HBM SIEVE kernel's phase 4, csrc/sieve_batch.hip): one
  left-to-right pass per cluster, each surviving entry moving into the
  leftmost hole at or after its home, leaves the same table as sequential
  Algorithm R deletions (hisp_kernel_common.h:64-94) in any order, which is
  also the table of inserting the survivors in their insertion order; and so
  does the kernel's windowed form of the pass (events found one at a time,
  holes in a few queue lanes or a set, a window's writes after it).
* Parallel admission build (kvx_sieve_ht_init_par, csrc/sieve.hip): keys
  bucketed by home with later duplicates dropped, the used cells from the
  backlog recursion (the ring's fixed point entering cell 0), then each
  cluster's keys in slot order; equal to the oracle's sequential inserts
  (hisp_sieve_ht_init.cpp:14-60).

* Batched admission build for tables larger than LDS (kvx_sieve_ht_init_wave,
  csrc/sieve.hip): with distinct tokens, 64 keys at a time; keys whose
  backlog is zero take their own first free cell at once, the rest sweep the
  free cells in increasing order, earliest slot first; a batch whose probes
  could wrap past the table's end inserts its keys one by one.  Equal to the
  oracle's sequential inserts.

These pin the algorithms (brute force over small tables); the kernels
themselves are compared with the oracle in the GPU tests.
"""
import random

import numpy as np
import pytest

from oracle import oracle as orc


def _knuth_home(k, H):
    return ((k * 2654435761) & 0xFFFFFFFF) >> 16 & (H - 1)


def _insert(T, k, hf):
    H = len(T)
    i = hf(k)
    while T[i] is not None:
        if T[i] == k:
            return
        i = (i + 1) % H
    T[i] = k


def _erase(T, k, hf):
    """Algorithm R: backward-shift deletion."""
    H = len(T)
    i = hf(k)
    while T[i] != k:
        assert T[i] is not None
        i = (i + 1) % H
    T[i] = None
    j = i
    while True:
        j = (j + 1) % H
        if T[j] is None:
            return
        h = hf(T[j])
        inside = (i < h <= j) if i <= j else (h > i or h <= j)  # home cyclically in (i, j]
        if not inside:
            T[i], T[j] = T[j], None
            i = j


def _batch_delete(T, D, hf):
    """One pass from an empty cell: deleted cells become holes; every other
    entry moves into the leftmost hole at or after its home (its cell then
    becomes a hole); an empty cell ends the cluster and its holes."""
    H = len(T)
    T = list(T)
    start = next(c for c in range(H) if T[c] is None)
    holes = []  # offsets from start, increasing
    for off in range(1, H + 1):
        c = (start + off) % H
        if T[c] is None:
            holes = []
            continue
        if T[c] in D:
            T[c] = None
            holes.append(off)
            continue
        hoff = (hf(T[c]) - start) % H
        at = next((i for i, ho in enumerate(holes) if ho >= hoff), None)
        if at is not None:
            ho = holes.pop(at)
            T[(start + ho) % H], T[c] = T[c], None
            holes.append(off)
    return T


def _batch_delete_windows(T, D, hf, rng, cap=64):
    """The pass as the kernel runs it: windows of 1-64 cells; in each, the
    events (a deleted cell, or an entry whose home is at or before the last
    event) are found one at a time, each mover taking the leftmost hole at or
    after its home, and the window's cells are written after it: each mover's
    entry at its hole, each event cell no mover of the window took emptied.
    The holes sit in `cap` queue lanes, filled in increasing order and packed
    when the lanes run out; with `cap` holes the cluster's holes move to a
    set for the rest of it.  Returns the table and the number of clusters
    that needed the set."""
    H = len(T)
    T = list(T)
    start = next(c for c in range(H) if T[c] is None)
    lanes, big, R, spills = [None] * cap, None, -1, 0  # queue lanes (None: empty); big: the set
    qend = 0
    off = 1
    while off <= H:
        hi = min(off + rng.randint(1, 64), H + 1)
        end, moves, events = None, [], []
        for o in range(off, hi):
            c = (start + o) % H
            if o == H or T[c] is None:
                end = o  # the cluster ends here
                break
            if T[c] in D:
                pass
            else:
                hoff = (hf(T[c]) - start) % H
                if not (R >= 0 and hoff <= R):
                    continue
                if big is None:
                    at = next(i for i in range(qend) if lanes[i] is not None and lanes[i] >= hoff)
                    hole, lanes[at] = lanes[at], None
                else:
                    hole = min(x for x in big if x >= hoff)
                    big.remove(hole)
                assert hole < o
                moves.append((o, hole))
            events.append(o)
            R = o
            if big is None and qend == cap:
                held = [x for x in lanes if x is not None]
                if len(held) < cap:
                    lanes = held + [None] * (cap - len(held))
                    qend = len(held)
                else:
                    big, spills = set(held), spills + 1
            if big is None:
                lanes[qend] = o
                qend += 1
            else:
                big.add(o)
        vals = {o: T[(start + o) % H] for o in events}
        taken = {h for _, h in moves}
        for o, h in moves:
            T[(start + h) % H] = vals[o]
        for o in events:
            if o not in taken:
                T[(start + o) % H] = None
        if end is not None:
            lanes, qend, big, R = [None] * cap, 0, None, -1
            off = end + 1
        else:
            off = hi
    return T, spills


@pytest.mark.parametrize("seed", range(4))
def test_batch_deletion_equals_algorithm_r(seed):
    rng = random.Random(seed)
    for trial in range(600):
        H = rng.choice([16, 32, 64, 128])
        n = rng.randint(1, H - 1)
        skew = rng.choice([None, 3, 8])  # None: the Knuth hash; else a few homes (long clusters)
        if skew is None:
            def hf(k, H=H):
                return _knuth_home(k, H)
        else:
            def hf(k, H=H, s=skew):
                return (k * 7 % s + H - 2) % H  # homes next to the end: clusters wrap
        keys = rng.sample(range(100000), n)
        T = [None] * H
        for k in keys:
            _insert(T, k, hf)
        D = set(rng.sample(keys, rng.randint(0, n)))
        order = list(D)
        rng.shuffle(order)
        seq = list(T)
        for k in order:
            _erase(seq, k, hf)
        fcfs = [None] * H
        for k in keys:
            if k not in D:
                _insert(fcfs, k, hf)
        assert seq == fcfs, (seed, trial)
        assert _batch_delete(T, D, hf) == seq, (seed, trial, H, keys, sorted(D))
        for cap in (1, 2, 4, 64):
            got, _ = _batch_delete_windows(T, D, hf, rng, cap)
            assert got == seq, (seed, trial, H, cap, keys, sorted(D))


def test_windowed_deletion_spills_and_packs_the_hole_lanes():
    """Long clusters with many deletions: the hole lanes are packed and, once
    full, spill to the set; the table still equals Algorithm R's."""
    rng = random.Random(7)
    H = 4096
    def hf(k):
        return (k * 7) % 2048
    keys = rng.sample(range(1, 10 ** 6), 2000)
    T = [None] * H
    for k in keys:
        _insert(T, k, hf)
    for nd, cap in ((5, 4), (300, 8), (300, 64)):
        D = set(rng.sample(keys, nd))
        seq = list(T)
        for k in D:
            _erase(seq, k, hf)
        got, spills = _batch_delete_windows(T, D, hf, rng, cap)
        assert got == seq, (nd, cap)
        if nd > 10 * cap:
            assert spills > 0, (nd, cap)


def _parallel_build(tok, dbs, H, lanes=256):
    mask = H - 1
    lists = [[] for _ in range(H)]
    for s in range(dbs):
        t = int(tok[s])
        if t >= 0:
            lists[_knuth_home(t, H)].append(s)
    for h in range(H):  # slot order, later duplicates of a token dropped
        keep, seen = [], set()
        for s in sorted(lists[h]):
            if int(tok[s]) not in seen:
                seen.add(int(tok[s]))
                keep.append(s)
        lists[h] = keep
    n = [len(x) for x in lists]
    per = H // lanes
    maps = []
    for k in range(lanes):  # each lane's segment as x -> max(P, x + Q)
        P = Q = 0
        for c in range(k * per, (k + 1) * per):
            P, Q = max(0, P + n[c] - 1), Q + n[c] - 1
        maps.append((P, Q))
    P = Q = 0
    for p, q in maps:  # composed in cell order
        P, Q = max(p, P + q), Q + q
    assert Q < 0
    x = P  # the fixed point: the backlog entering cell 0
    used = []
    for c in range(H):
        used.append(x + n[c] >= 1)
        x = max(0, x + n[c] - 1)
    assert x == P
    ht = [0] * H
    for c in range(H):
        if used[c] and not used[(c - 1) & mask]:
            homes, e = [], c
            while used[e & mask]:
                homes.append(e & mask)
                e += 1
            for s in sorted(s for h in homes for s in lists[h]):
                y = _knuth_home(int(tok[s]), H)
                while ht[y] != 0:
                    y = (y + 1) & mask
                ht[y] = s + 1
    return np.array(ht, dtype=np.uint16)


@pytest.mark.parametrize("mode", ["unique", "dups", "few_homes", "wrap"])
def test_parallel_table_build_equals_sequential_inserts(mode):
    rng = np.random.default_rng(len(mode))
    for trial in range(6):
        dbs = int(rng.choice([1, 64, 300, 1000]))
        padded = (dbs + 15) // 16 * 16
        top_k = int(rng.integers(1, 256))
        H = orc.ht_size(padded, top_k)
        tok = np.full(padded, -1, dtype=np.int32)
        n = int(rng.integers(0, dbs + 1))
        if mode == "unique":
            vals = rng.choice(1 << 22, size=n, replace=False)
        elif mode == "dups":
            vals = rng.integers(-3, max(4, n // 3), size=n)
        else:
            t = np.arange(0, 1 << 21, dtype=np.int64)
            h = ((t * 2654435761) & 0xFFFFFFFF) >> 16 & (H - 1)
            cand = t[np.isin(h, rng.choice(H, size=4, replace=False))] if mode == "few_homes" else t[h >= H - 24]
            vals = rng.choice(cand, size=min(n, len(cand)), replace=False)
        tok[rng.choice(dbs, size=len(vals), replace=False)] = vals
        want = np.zeros((1, 1, H), dtype=np.uint16)
        orc.sieve_ht_init(tok.reshape(1, 1, padded).copy(), want, 0, 1, 1, 1, dbs, padded, H)
        np.testing.assert_array_equal(_parallel_build(tok, dbs, H), want[0, 0], err_msg="{} {}".format(mode, trial))


def _batch_sweep_build(tok, dbs, H, batch=64, cap=4):
    """Distinct tokens only (the kernel checks that first).  Per batch: each
    key's first free cell t (table before the batch); with the keys in order
    of t, the backlog b_k = max(0, b_{k-1} + 1 - D_k), D_k = free cells in
    [t_{k-1}, t_k) counted up to cap (a smaller count only overstates b); keys
    with b = 0 take their own t; the others sweep the free cells in
    increasing order, each cell going to the earliest waiting key whose t is
    at or before it (a jump goes to the first free cell at or after the next
    key's t).  With at least as many free cells as keys at or after the last
    t, nothing runs past the table's end; otherwise, or when a probe wraps,
    the keys go in one by one."""
    used = [False] * H
    ht = [0] * H

    def first_free(x):
        for c in range(x, H):
            if not used[c]:
                return c
        return -1

    def place(c, s):
        assert not used[c]
        used[c], ht[c] = True, s + 1

    for b0 in range(0, dbs, batch):
        keys = [(s, _knuth_home(int(tok[s]), H)) for s in range(b0, min(b0 + batch, dbs)) if int(tok[s]) >= 0]
        if not keys:
            continue
        targets = [first_free(h) for _, h in keys]
        n = len(keys)
        one_by_one = any(t < 0 for t in targets)
        if not one_by_one:
            one_by_one = sum(1 for c in range(max(targets), H) if not used[c]) < n
        if one_by_one:
            for s, h in keys:
                c = first_free(h)
                place(c if c >= 0 else first_free(0), s)
            continue
        order = sorted(range(n), key=lambda i: (targets[i], i))
        st = [targets[i] for i in order]
        backlog = [0]
        for r in range(1, n):
            d = 0
            if st[r] > st[r - 1]:
                d, x = 1, st[r - 1]
                while d < cap:
                    x = first_free(x + 1)
                    if x < 0 or x >= st[r]:
                        break
                    d += 1
            backlog.append(max(0, backlog[-1] + 1 - d))
        for r in range(n):
            if backlog[r] == 0:
                place(st[r], keys[order[r]][0])
        cong = [r for r in range(n) if backlog[r] > 0]
        waiting, ready, nxt = {order[r] for r in cong}, set(), 0
        c = first_free(st[cong[0]]) if cong else 0
        while waiting:
            while nxt < len(cong) and st[cong[nxt]] <= c:
                ready.add(order[cong[nxt]])
                nxt += 1
            if not ready:
                c = first_free(st[cong[nxt]])
                continue
            i = min(ready)  # the earliest slot
            ready.discard(i)
            waiting.discard(i)
            place(c, keys[i][0])
            if ready:
                c = first_free(c + 1)
    return np.array(ht, dtype=np.uint16)


@pytest.mark.parametrize("mode", ["spread", "few_homes", "wrap", "dense"])
def test_batched_sweep_build_equals_sequential_inserts(mode):
    rng = np.random.default_rng(100 + len(mode))
    for trial in range(8):
        H = int(rng.choice([64, 256, 1024]))
        dbs = int(rng.integers(1, H - 1))
        tok = np.full(dbs, -1, dtype=np.int32)
        n = int(rng.integers(0, dbs + 1))
        t = np.arange(0, 1 << 20, dtype=np.int64)
        h = ((t * 2654435761) & 0xFFFFFFFF) >> 16 & (H - 1)
        if mode == "spread":
            cand = t
        elif mode == "few_homes":
            cand = t[np.isin(h, rng.choice(H, size=3, replace=False))]
        elif mode == "wrap":
            cand = t[h >= H - max(4, H // 16)]
        else:
            cand = t[h < H // 4]
        vals = rng.choice(cand, size=min(n, len(cand)), replace=False)
        tok[rng.choice(dbs, size=len(vals), replace=False)] = vals
        want = np.zeros((1, 1, H), dtype=np.uint16)
        orc.sieve_ht_init(tok.reshape(1, 1, dbs).copy(), want, 0, 1, 1, 1, dbs, dbs, H)
        for batch, cap in ((64, 4), (8, 1), (4, 4)):
            np.testing.assert_array_equal(_batch_sweep_build(tok, dbs, H, batch, cap), want[0, 0],
                                          err_msg="{} {} {} {}".format(mode, trial, batch, cap))


# ---- the batch SIEVE kernel's in-order decision when the hand wraps -------
def _round_decide(ring, vis, hand0, batch, seq_len, prefill):
    """The one-wave decision loop of kvx_sieve_update_batch (csrc/sieve_batch.hip),
    64 positions a round.  A token's state is (slot, whether the step had
    evicted that slot when the token was found or placed there); it is
    resident while that has not changed.  Within a round the evictions are a
    list: a token found at the round's start stays while the round has not
    evicted its slot; one placed in the round stays while the round has
    evicted its slot once.  Returns (outputs [(slot, miss)], visited, hand,
    evicted, misses [(position, slot)], again): `again` is a slot evicted a
    second time, which the kernel does not decide (it runs the in-order
    recurrence instead) and which cannot happen while topK < dbs."""
    dbs, K = len(ring), len(batch)
    where = {t: s for s, t in enumerate(ring) if t is not None}
    code, first = [None] * K, {}
    for k, t in enumerate(batch):
        if t < 0 or t >= seq_len:
            code[k] = ("inv",)
        elif t >= prefill:
            code[k] = ("ext",)
        elif t in first:
            code[k] = ("dup", first[t])
        else:
            first[t] = k
            code[k] = ("st", where[t], 0) if t in where else ("not",)
    first_miss = min([k for k in range(K) if code[k][0] == "not"], default=K)
    vis = list(vis)
    out = [(0, 0)] * K
    for k in range(first_miss):  # all hits, applied in parallel
        c = code[k]
        if c[0] in ("inv", "ext"):
            continue
        s = c[1] if c[0] == "st" else code[c[1]][1]
        out[k] = (s, 0)
        vis[s] = True
    evicted = [0] * dbs
    hand = hand0 if 0 <= hand0 < dbs else 0
    misses, again = [], False
    k0 = first_miss & ~63
    while k0 < K:
        lanes = range(k0, min(k0 + 64, K))
        st = {}
        for k in lanes:
            c = code[k]
            if c[0] in ("inv", "ext"):
                continue
            f, s = (c[1], code[c[1]]) if c[0] == "dup" else (k, c)
            st[k] = [f, 0, None, False] if s[0] == "not" else [f, s[1], 0 if evicted[s[1]] == s[2] else None, False]
        ev = []
        for j in lanes:
            if j not in st:
                continue
            f, s, need, _ = st[j]
            if need is not None and ev.count(s) == need:
                vis[s] = True
                out[j] = (s, 0)
                continue
            while vis[hand]:
                vis[hand] = False
                hand = (hand + 1) % dbs
            h = hand
            vis[h] = True
            ev.append(h)
            out[j] = (h, 1)
            misses.append((j, h))
            for q in st.values():
                if q[0] == f:
                    q[1:] = [h, 1, True]
            hand = (h + 1) % dbs
        for f, s, need, rel in st.values():
            if rel:
                code[f] = ("st", s, 1)
        for h in ev:
            again |= evicted[h] != 0
            evicted[h] = 1
        k0 += 64
    return out, vis, hand, evicted, misses, again


@pytest.mark.parametrize("seed", range(3))
def test_wrapping_step_decisions_and_table(seed):
    """The decision loop against the ring-clock model (sieve_model.py, written
    from the policy) on steps whose hand passes slots twice (a full turn of
    clearing, then evictions of slots hit earlier in the step), and the table
    the rebuild is handed (deleted: the initial tokens of the evicted slots;
    new keys: the misses in position order) against the step's inserts and
    Algorithm R deletions replayed in order."""
    from tests.sieve_model import RingClock

    rng = random.Random(seed)
    seen = {"passed_twice": 0, "hit_then_evicted": 0, "evicted_then_again": 0, "wide_decided": 0,
            "wide_again": 0}
    for trial in range(400):
        storm = trial % 3 == 0  # misses on a nearly all-visited ring, repeats of the step's hits
        dbs = rng.choice([20, 33, 64, 65, 70, 130])
        wide = trial % 5 == 1   # topK >= dbs: a slot may be evicted twice
        K = rng.randint(dbs, 2 * dbs) if wide else (dbs - 1 if storm else rng.randint(1, dbs - 1))
        prefill = 3 * dbs if storm else rng.choice([dbs // 2, dbs, 3 * dbs])
        seq_len = prefill + rng.randint(0, 5)
        toks = rng.sample(range(prefill), min(prefill, dbs - rng.randint(0, 3)))
        ring = toks + [None] * (dbs - len(toks))
        rng.shuffle(ring)
        p_vis = 0.97 if storm else rng.choice([0.5, 0.95, 1.0])
        vis = [t is not None and rng.random() < p_vis for t in ring]
        hand0 = rng.choice([rng.randrange(dbs), dbs - 1, -1])
        pool = [t for t in ring if t is not None]
        batch = []
        for _ in range(K):
            u = rng.random()
            if u < (0.3 if storm else 0.15) and batch:
                batch.append(rng.choice(batch))              # a repeat within the step
            elif u < 0.35 and pool:
                batch.append(rng.choice(pool))               # a resident token
            elif u < 0.4 and not storm:
                batch.append(rng.choice([-1, seq_len, prefill]))  # invalid or decode-extension
            else:
                batch.append(rng.randrange(prefill))
        out, vis_g, hand_g, evicted, misses, again = _round_decide(ring, vis, hand0, batch, seq_len, prefill)
        if wide:
            seen["wide_again" if again else "wide_decided"] += 1
            if again:
                continue  # the kernel runs the in-order recurrence for this step
        assert not again, (seed, trial)
        rc = RingClock(dbs, dbs, [t if t is not None else -1 for t in ring], vis, hand0)
        want = [rc.access(t, seq_len, prefill) for t in batch]
        got = [(-1, 0) if batch[k] < 0 or batch[k] >= seq_len else
               ((dbs + batch[k] - prefill, 0) if batch[k] >= prefill else out[k]) for k in range(K)]
        assert got == want, (seed, trial)
        assert vis_g == rc.ref and hand_g == rc.hand, (seed, trial)
        final = list(ring)
        for k, s in misses:
            final[s] = batch[k]
        assert final == rc.ring, (seed, trial)
        # the table: the step replayed, against the initial survivors (slot
        # order) then the new keys (position order)
        H = 1 << max(4, (2 * dbs).bit_length())

        def hf(k, H=H):
            return _knuth_home(k, H)

        seq = [None] * H
        for t in ring:
            if t is not None:
                _insert(seq, t, hf)
        cur = list(ring)
        for k, s in misses:
            if cur[s] is not None:
                _erase(seq, cur[s], hf)
            cur[s] = batch[k]
            _insert(seq, batch[k], hf)
        fcfs = [None] * H
        for s, t in enumerate(ring):
            if t is not None and not evicted[s]:
                _insert(fcfs, t, hf)
        for k, _ in misses:
            _insert(fcfs, batch[k], hf)
        assert fcfs == seq, (seed, trial)
        # coverage: a slot hit in the step and evicted later; then the token again
        hits = {}
        for k, (s, m) in enumerate(out):
            if not m and 0 <= batch[k] < prefill and k < K:
                hits.setdefault(batch[k], k)
        evk = {s: k for k, s in misses}
        seen["passed_twice"] += any(hits.get(ring[s], K) < k for k, s in misses if ring[s] is not None)
        tw = [t for t, k1 in hits.items() if any(batch[k2] == t for k2, _ in misses if k2 > k1)]
        seen["hit_then_evicted"] += bool(tw)
        seen["evicted_then_again"] += any(sum(1 for k in range(K) if batch[k] == t and out[k][1] == 0 and
                                              k > max(k2 for k2, _ in misses if batch[k2] == t)) > 0 for t in tw)
        del evk
    assert all(v > 0 for v in seen.values()), seen


@pytest.mark.parametrize("seed", range(3))
def test_cell_order_rebuild_equals_the_replayed_step(seed):
    """The parallel table rebuild (csrc/sieve_table.hip): after a step that deletes the keys D of a table and then inserts the keys
    N in order, the table equals inserting, into an empty table, the
    surviving keys in the pre-step table's cell order read from an empty cell
    on, then N in order.  The pre-step tables come from random histories of
    inserts and Algorithm R deletions, with homes packed at the table's end
    so that clusters wrap."""
    rng = random.Random(100 + seed)
    for trial in range(400):
        H = rng.choice([16, 32, 64, 128])
        skew = rng.choice([None, 3, 8])
        if skew is None:
            def hf(k, H=H):
                return _knuth_home(k, H)
        else:
            def hf(k, H=H, s=skew):
                return (k * 7 % s + H - 3) % H
        T = [None] * H
        live = []
        for _ in range(rng.randint(1, 3 * H)):  # a history of inserts and deletions
            if live and (rng.random() < 0.4 or len(live) >= H - 2):
                k = live.pop(rng.randrange(len(live)))
                _erase(T, k, hf)
            else:
                k = rng.randrange(10 ** 6)
                if k in live:
                    continue
                _insert(T, k, hf)
                live.append(k)
        D = set(rng.sample(live, rng.randint(0, len(live))))
        room = H - 1 - (len(live) - len(D))
        N = [k for k in rng.sample(range(10 ** 6, 2 * 10 ** 6), rng.randint(0, max(0, room)))]
        seq = list(T)
        for k in rng.sample(sorted(D), len(D)):
            _erase(seq, k, hf)
        for k in N:
            _insert(seq, k, hf)
        e0 = T.index(None)
        order = [T[(e0 + 1 + i) % H] for i in range(H)]
        fcfs = [None] * H
        for k in order:
            if k is not None and k not in D:
                _insert(fcfs, k, hf)
        for k in N:
            _insert(fcfs, k, hf)
        assert fcfs == seq, (seed, trial)
