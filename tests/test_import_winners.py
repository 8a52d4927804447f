"""CPU check of the winner rule of the one-launch import (kvx_gather_small,
csrc/rows.hip).

The rule (kvc_gather_rows.cpp:69-81 copies in position order, so the last
miss on a destination row wins): a position takes part when it is a miss with
a valid token, slot 0 <= s < 65536 and a pool row; its destination is
d = b * span + s (b its request, span = min(stride, 65536)); the winner of a
destination is its largest position.  The kernel's workgroups own 32
positions each and decide them without device-scope tags when none of their
own participating positions has s >= span: then only the positions of the
same request can share a destination with a later position, and eight lanes
per position search the request's later positions in LDS.  Otherwise the
workgroup tags every position (the global rule).  Here that decomposition is
replayed and compared with the global rule by brute force, over strides that
keep requests apart, make neighbours share rows, or put every request on the
same rows, and top_k values whose requests straddle workgroups.
"""
import numpy as np
import pytest

SPAN = 32  # positions per workgroup (kSmallSpan)


def _inputs(rng, req, top_k, dbs):
    topk = rng.integers(-1, 50, size=req * top_k)
    slots = rng.integers(-1, dbs, size=req * top_k)
    slots[rng.random(req * top_k) < 0.01] = 70000  # outside the rule (>= 65536)
    miss = rng.random(req * top_k) < 0.6
    pool = np.where(rng.random(req) < 0.15, -1, np.arange(req))
    return topk, slots, miss, pool


def _part(p, topk, slots, miss, pool, top_k):
    """Slot of position p when it takes part in the winner rule, else -1."""
    s = int(slots[p])
    if not miss[p] or topk[p] < 0 or s < 0 or s >= 65536 or pool[p // top_k] < 0:
        return -1
    return s


def _global_winners(total, top_k, span, part):
    last = {}
    for p in range(total):
        s = part(p)
        if s >= 0:
            last[(p // top_k) * span + s] = p
    return {p for p in last.values()}


def _kernel_winners(total, top_k, span, part):
    """The one-launch import's decisions, workgroup by workgroup."""
    glob = _global_winners(total, top_k, span, part)
    won = set()
    for lo in range(0, total, SPAN):
        hi = min(lo + SPAN, total)
        own = [p for p in range(lo, hi) if part(p) >= 0]
        if any(part(p) >= span for p in own):
            won |= {p for p in own if p in glob}  # device-scope tags of every position
            continue
        for p in own:
            end = (p // top_k + 1) * top_k
            if not any(part(q) == part(p) for q in range(p + 1, end)):
                won.add(p)
    return won


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("req,top_k,dbs,stride", [
    (12, 20, 16, 16), (40, 7, 8, 8), (10, 48, 32, 16), (6, 100, 64, 0), (8, 64, 64, 64),
    (3, 33, 40, 70000), (5, 1, 4, 2), (1, 300, 50, 48),
    (12, 20, 17, 16), (20, 10, 9, 8),  # slots up to the span itself: only s == span reaches the next request
])
def test_small_import_winners_equal_global_rule(seed, req, top_k, dbs, stride):
    rng = np.random.default_rng(seed * 7919 + req * 131 + top_k)
    topk, slots, miss, pool = _inputs(rng, req, top_k, dbs)
    total = req * top_k
    span = min(stride, 65536)

    def part(p):
        return _part(p, topk, slots, miss, pool, top_k)

    assert _kernel_winners(total, top_k, span, part) == _global_winners(total, top_k, span, part)


def test_request_local_search_alone_misses_shared_rows():
    """The fallback is needed: with stride 0 (every request on the same rows)
    a search within each request keeps an earlier request's position that a
    later request overwrites."""
    top_k, span = 4, 0
    slots = np.array([3, 1, 2, 0, 3, 5, 6, 7])  # request 0's slot 3 is request 1's slot 3 too
    miss = np.ones(8, dtype=bool)
    topk = np.zeros(8, dtype=np.int64)
    pool = np.arange(2)

    def part(p):
        return _part(p, topk, slots, miss, pool, top_k)

    local = set()
    for p in range(8):
        end = (p // top_k + 1) * top_k
        if not any(part(q) == part(p) for q in range(p + 1, end)):
            local.add(p)
    glob = _global_winners(8, top_k, span, part)
    assert 0 in local and 0 not in glob
    assert _kernel_winners(8, top_k, span, part) == glob
