"""A small, independent model of the SIEVE (ring CLOCK) miss detector.

Written from the policy's statement, not from any implementation: a ring of
`dbs` slots, each holding a token (or nothing) and a reference bit; a hand.
  * a position outside [0, seq_len) is invalid: slot -1, not a miss;
  * a position >= prefill is a decode-extension token: slot padded + (pos - prefill);
  * a resident token is a hit: its slot, reference bit set;
  * otherwise a miss: starting at the hand, clear set reference bits while
    advancing (wrapping at dbs); the first clear slot is the victim; its old
    token is dropped, the new token takes the slot with its bit set, and the
    hand moves one past the victim.
Batch rows past num_real, or naming a pool row outside [0, pool), produce
(-1, 0) rows; a hand outside [0, dbs) restarts at 0.

It is used only to cross-check the C oracle by brute force on small inputs.
"""


class RingClock:
    def __init__(self, dbs, padded, tokens, visited_bits, hand):
        self.dbs = dbs
        self.padded = padded
        self.ring = [t if t >= 0 else None for t in tokens[:dbs]]
        self.ref = [bool(b) for b in visited_bits[:dbs]]
        self.where = {}
        for s, t in enumerate(self.ring):
            if t is not None and t not in self.where:
                self.where[t] = s
        self.hand = hand if 0 <= hand < dbs else 0

    def access(self, pos, seq_len, prefill):
        if pos < 0 or pos >= seq_len:
            return -1, 0
        if pos >= prefill:
            return self.padded + (pos - prefill), 0
        if pos in self.where:
            s = self.where[pos]
            self.ref[s] = True
            return s, 0
        while self.ref[self.hand]:
            self.ref[self.hand] = False
            self.hand = (self.hand + 1) % self.dbs
        victim = self.hand
        old = self.ring[victim]
        if old is not None and self.where.get(old) == victim:
            del self.where[old]
        self.ring[victim] = pos
        self.where[pos] = victim
        self.ref[victim] = True
        self.hand = (victim + 1) % self.dbs
        return victim, 1


def model_batch(state_rows, topk, req_pool, seq_lens, prefill_lens, num_real, pool_size, dbs, padded):
    """state_rows: dict pool_idx -> RingClock.  Returns (slots, miss) lists of rows."""
    n = len(topk)
    num_real = min(num_real, n)
    slots, miss = [], []
    for b in range(n):
        k = len(topk[b])
        if b >= num_real or not (0 <= req_pool[b] < pool_size):
            slots.append([-1] * k)
            miss.append([0] * k)
            continue
        rc = state_rows[req_pool[b]]
        rs, rm = [], []
        for pos in topk[b]:
            s, m = rc.access(int(pos), int(seq_lens[b]), int(prefill_lens[req_pool[b]]))
            rs.append(s)
            rm.append(m)
        slots.append(rs)
        miss.append(rm)
    return slots, miss
