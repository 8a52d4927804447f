"""Synthetic topK streams for decode steps.

Two modes:

* ``ref_batch`` reproduces the reference driver's stream exactly
  (xds/xds_decode.py:211-222): per request, n_hit positions drawn with
  replacement from [0, min(prefill, dbs)) and n_miss distinct positions from
  [dbs, prefill), concatenated, then one in-place shuffle over the whole batch.
  The numpy Generator call order is the reference's, so a given seed gives the
  same batches.
* ``state_batch`` draws from the current SIEVE state: per request, about
  ``miss_ratio * topK`` distinct positions not resident in the hot buffer and
  the rest distinct resident positions, optionally with a Zipf recency bias
  (weight (rank+1)^-s over resident positions sorted newest first) and with
  misses restricted to a given candidate pool (the adversarial hash-collision
  set).
"""
import numpy as np


def ref_batch(rng, req_num, top_k, prefill, dbs, miss_ratio):
    hit_span = min(prefill, dbs)
    miss_span = max(prefill - dbs, 0)
    n_miss = int(top_k * miss_ratio) if miss_span > 0 else 0
    n_hit = top_k - n_miss
    batch = np.empty((req_num, top_k), dtype=np.int32)
    for r in range(req_num):
        hits = rng.integers(0, hit_span, size=n_hit) if n_hit > 0 else np.empty(0, dtype=np.int64)
        misses = (rng.choice(miss_span, size=n_miss, replace=False) + dbs) if n_miss > 0 else np.empty(0, np.int64)
        batch[r] = np.concatenate([hits, misses]).astype(np.int32)
    rng.shuffle(batch.ravel())
    return batch


def _top_order(key, n, width):
    """Column indices of the `width` largest keys per row, largest first
    (only the first n are guaranteed; the rest follow in descending order)."""
    if n <= 0:
        return np.zeros((key.shape[0], width), dtype=np.int64)
    part = np.argpartition(-key, n - 1, axis=1)[:, :width] if n < key.shape[1] else np.argsort(-key, axis=1)[:, :width]
    sub = np.take_along_axis(key, part, axis=1)
    return np.take_along_axis(part, np.argsort(-sub, axis=1, kind="stable"), axis=1)


def state_batch(rng, tokens_rows, prefill, top_k, miss_ratio, zipf_s=None, miss_pool=None):
    """tokens_rows: [req, >=dbs] int32 resident tokens per request (-1 = empty).

    Returns an int32 [req, top_k] batch of distinct positions per request:
    round(miss_ratio*top_k) non-resident positions (from miss_pool when given)
    and the rest resident ones, in random order.  Rows short of candidates are
    filled from the other class, then padded with -1.  Sampling without
    replacement uses one exponential key per candidate, uniform or weighted by
    (recency rank + 1)^-zipf_s, and keeps the largest keys (Efraimidis-Spirakis);
    all requests are drawn together.
    """
    tokens_rows = np.asarray(tokens_rows)
    req = tokens_rows.shape[0]
    rows = np.repeat(np.arange(req), tokens_rows.shape[1])
    toks = tokens_rows.reshape(-1)
    ok = (toks >= 0) & (toks < prefill)
    resident = np.zeros((req, prefill), dtype=bool)
    resident[rows[ok], toks[ok]] = True
    eligible = ~resident
    if miss_pool is not None:
        in_pool = np.zeros(prefill, dtype=bool)
        in_pool[np.asarray(miss_pool, dtype=np.int64)] = True
        eligible &= in_pool[None, :]
    n_res = resident.sum(axis=1)
    n_el = eligible.sum(axis=1)
    want_miss = int(round(top_k * miss_ratio))
    n_miss = np.minimum(want_miss, n_el)
    n_hit = np.minimum(top_k - n_miss, n_res)
    n_miss = np.minimum(top_k - n_hit, n_el)

    u = rng.random((2, req, prefill))
    with np.errstate(divide="ignore"):
        lu = np.log(u)
    # misses: uniform keys over eligible positions
    mkey = np.where(eligible, lu[0], -np.inf)
    # hits: keys over resident positions, optionally recency-weighted
    if zipf_s is None:
        hkey = np.where(resident, lu[1], -np.inf)
    else:
        rank = np.cumsum(resident[:, ::-1], axis=1)[:, ::-1] - 1  # 0 = newest resident position
        w = (np.maximum(rank, 0).astype(np.float64) + 1.0) ** (-float(zipf_s))
        hkey = np.where(resident, lu[1] / w, -np.inf)
    take = min(top_k, prefill)
    horder = _top_order(hkey, int(n_hit.max(initial=0)), take)
    morder = _top_order(mkey, int(n_miss.max(initial=0)), take)
    out = np.full((req, top_k), -1, dtype=np.int64)
    col = np.arange(top_k)
    hsel = col[None, :] < n_hit[:, None]
    msel = (col[None, :] >= n_hit[:, None]) & (col[None, :] < (n_hit + n_miss)[:, None])
    hpad = np.full((req, top_k), -1, dtype=np.int64)
    hpad[:, :take] = horder
    idx = np.clip(col[None, :] - n_hit[:, None], 0, top_k - 1)
    mtake = np.full((req, top_k), -1, dtype=np.int64)
    mtake[:, :take] = morder
    mpad = np.take_along_axis(mtake, idx, axis=1)
    out[hsel] = hpad[hsel]
    out[msel] = mpad[msel]
    out = rng.permuted(out, axis=1)
    return out.astype(np.int32)


def adversarial_pool(prefill, ht_bits_below):
    """Positions in [0, prefill) whose 16-bit Knuth hash is < ht_bits_below: their
    home buckets pack into one window of the table (long probe runs).  About
    prefill * ht_bits_below / 65536 positions."""
    t = np.arange(prefill, dtype=np.uint64)
    h = ((t * np.uint64(2654435761)) & np.uint64(0xFFFFFFFF)) >> np.uint64(16)
    return np.nonzero(h < ht_bits_below)[0].astype(np.int64)
