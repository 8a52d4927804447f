// Device helpers shared by the SIEVE kernels: the state format of
// hisp_kernel_common.h (uint16 table entries = slot+1, Knuth hash, linear
// probing, Algorithm R deletion, visited bitmap) and the exact sequential
// recurrence of hisp_sieve_update.cpp:115-163.
#pragma once

#include "kvx_internal.h"

// v_writelane_b32: x with lane l (the same in the whole wave) replaced by v,
// whatever the exec mask.  The LLVM intrinsic, which this clang does not
// expose as a builtin.
extern "C" __device__ int32_t kvx_writelane_i32(int32_t v, int32_t l, int32_t x) __asm("llvm.amdgcn.writelane.i32");

namespace kvx {
namespace sieve {

struct Guard {
    uint64_t code = 0;
    uint32_t fpd = 0;  // change of the row's token fingerprint (slot_token_mix sum) by the replaced tokens
};

// Tables up to this many cells run the in-order recurrence on one lane (short
// probe runs); larger ones use a whole wave per probe, sweep and shift step.
constexpr int32_t kSmallTable = 4096;

// Value of x in lane l, l the same in the whole wave (a register read, no
// LDS round trip as a shuffle would take).
__device__ __forceinline__ int32_t lane_value(int32_t x, int32_t l) { return __builtin_amdgcn_readlane(x, l); }

// x, the same in every lane, as a wave-uniform value: the compiler then keeps
// it, and the loops and branches that depend on it, in scalar registers.
__device__ __forceinline__ int32_t uniform32(int32_t x) { return __builtin_amdgcn_readfirstlane(x); }
__device__ __forceinline__ uint64_t uniform64(uint64_t x)
{
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(x)));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int32_t>(x >> 32)));
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

// x with lane l set to v (a register write, no compare and select).
__device__ __forceinline__ int32_t lane_set(int32_t x, int32_t l, int32_t v) { return kvx_writelane_i32(v, l, x); }

// Token held by the slot an entry points at.  An entry past the tokens row
// can only come from a corrupted table; it reads as the empty token (-1)
// instead of touching memory outside the row.
__device__ __forceinline__ int32_t tok_at(const int32_t *tok, uint32_t e, int32_t ntok)
{
    return (static_cast<int32_t>(e) - 1 < ntok) ? tok[static_cast<int32_t>(e) - 1] : -1;
}

__device__ __forceinline__ int32_t ht_find(const uint16_t *ht, const int32_t *tok, int32_t ntok, int32_t token,
                                           int32_t mask, Guard &g)
{
    int32_t idx = static_cast<int32_t>(ht_hash(token)) & mask;
    for (int32_t n = 0; n <= mask; ++n) {
        const uint16_t e = ht[idx];
        if (e == 0) return -1;
        if (tok_at(tok, e, ntok) == token) return static_cast<int32_t>(e) - 1;
        idx = (idx + 1) & mask;
    }
    g.code = kOverflowProbe;
    return -1;
}

// Insert token -> slot; a present token keeps its first slot
// (hisp_kernel_common.h:46-61, :97-112).
__device__ __forceinline__ void ht_insert(uint16_t *ht, const int32_t *tok, int32_t ntok, int32_t token,
                                          int32_t slot, int32_t mask, Guard &g)
{
    int32_t idx = static_cast<int32_t>(ht_hash(token)) & mask;
    for (int32_t n = 0; n <= mask; ++n) {
        const uint16_t e = ht[idx];
        if (e == 0) {
            ht[idx] = static_cast<uint16_t>(slot + 1);
            return;
        }
        if (tok_at(tok, e, ntok) == token) return;
        idx = (idx + 1) & mask;
    }
    g.code = kOverflowProbe;
}

// Backward-shift erase, Knuth 6.4 Algorithm R (hisp_kernel_common.h:64-94).
__device__ __forceinline__ void ht_erase(uint16_t *ht, const int32_t *tok, int32_t ntok, int32_t token,
                                         int32_t mask, Guard &g)
{
    int32_t idx = static_cast<int32_t>(ht_hash(token)) & mask;
    int32_t n = 0;
    for (;; ++n) {
        if (n > mask) {
            g.code = kOverflowProbe;
            return;
        }
        const uint16_t e = ht[idx];
        if (e == 0) return;
        if (tok_at(tok, e, ntok) == token) break;
        idx = (idx + 1) & mask;
    }
    int32_t j = idx, i = idx;
    for (n = 0;; ++n) {
        if (n > mask) {
            g.code = kOverflowProbe;
            return;
        }
        i = (i + 1) & mask;
        const uint16_t e = ht[i];
        if (e == 0) break;
        const int32_t home = static_cast<int32_t>(ht_hash(tok_at(tok, e, ntok))) & mask;
        const bool move = (j < i) ? (home <= j || home > i) : (home <= j && home > i);
        if (move) {
            ht[j] = e;
            j = i;
        }
    }
    ht[j] = 0;
}

__device__ __forceinline__ int vis_get(const uint8_t *v, int32_t s) { return (v[s >> 3] >> (s & 7)) & 1; }
__device__ __forceinline__ void vis_set(uint8_t *v, int32_t s)
{
    v[s >> 3] = static_cast<uint8_t>(v[s >> 3] | (1u << (s & 7)));
}
__device__ __forceinline__ void vis_clear(uint8_t *v, int32_t s)
{
    v[s >> 3] = static_cast<uint8_t>(v[s >> 3] & ~(1u << (s & 7)));
}

__device__ __forceinline__ void report_overflow(uint64_t slot, uint64_t code)
{
    if (slot != 0 && code != 0) {
        atomicCAS(reinterpret_cast<unsigned long long *>(slot), 0ull, static_cast<unsigned long long>(code));
    }
}

// The per-position recurrence of hisp_sieve_update.cpp:115-163 for one batch
// row, run by a single lane.  Returns true when a miss modified tokens/ht.
__device__ bool sieve_row_sequential(const int32_t *rt, int32_t *rs, int8_t *rm, int32_t topK, int32_t seqLen,
                                     int32_t prefill, int32_t dbs, int32_t padded, int32_t mask, int32_t *tok,
                                     uint8_t *vis, uint16_t *ht, int32_t &hand, Guard &g)
{
    bool dirty = false;
    for (int32_t k = 0; k < topK; ++k) {
        const int32_t tp = rt[k];
        if (g.code != 0 || tp < 0 || tp >= seqLen) {  // past a bound violation the row reads as invalid
            rs[k] = -1;
            rm[k] = 0;
            continue;
        }
        if (tp >= prefill) {
            rs[k] = padded + (tp - prefill);
            rm[k] = 0;
            continue;
        }
        const int32_t hit = ht_find(ht, tok, padded, tp, mask, g);
        if (hit >= 0) {
            rs[k] = hit;
            rm[k] = 0;
            vis_set(vis, hit);
            continue;
        }
        int32_t h = hand;
        int32_t swept = 0;
        while (vis_get(vis, h) != 0) {
            vis_clear(vis, h);
            if (++h == dbs) h = 0;
            if (++swept > dbs) {
                g.code = kOverflowSweep;
                break;
            }
        }
        const int32_t old = tok[h];
        if (old >= 0) ht_erase(ht, tok, padded, old, mask, g);
        ht_insert(ht, tok, padded, tp, h, mask, g);
        g.fpd += slot_token_mix(static_cast<uint32_t>(h), tp) - slot_token_mix(static_cast<uint32_t>(h), old);
        dirty = true;
        rs[k] = h;
        rm[k] = 1;
        tok[h] = tp;
        vis_set(vis, h);
        hand = (h + 1 == dbs) ? 0 : h + 1;
    }
    return dirty;
}

// The same recurrence run by one whole wave on an LDS-staged row: each probe
// reads 64 consecutive cells and takes the first empty or matching one with a
// ballot, the hand sweep tests 64 visited bits at once, and Algorithm R's
// backward shift walks 64 cells per step, taking the moves in order.  Every
// lane of the wave calls it (uniform control flow); same results as
// sieve_row_sequential.
__device__ __forceinline__ int32_t wave_probe_lds(const uint16_t *ht, const int32_t *tok, int32_t ntok, int32_t idx,
                                                  int32_t token, int32_t mask, bool &found, uint32_t &entry, Guard &g)
{
    const int32_t lane = static_cast<int32_t>(__lane_id());
    for (int32_t base = 0; base <= mask; base += 64) {
        const int32_t c = (idx + base + lane) & mask;
        const uint16_t e = ht[c];
        const bool hitL = e != 0 && tok_at(tok, e, ntok) == token;
        const uint64_t hit = __ballot(hitL);
        const uint64_t any = hit | __ballot(e == 0);
        if (any != 0ull) {
            const int f = __builtin_ctzll(any);
            found = (hit >> f) & 1ull;
            entry = static_cast<uint32_t>(lane_value(static_cast<int>(e), f));
            return (idx + base + f) & mask;
        }
    }
    g.code = kOverflowProbe;
    found = false;
    return -1;
}

__device__ __forceinline__ void wave_shift_lds(uint16_t *ht, const int32_t *tok, int32_t ntok, int32_t j,
                                               int32_t mask, Guard &g)
{
    const int32_t lane = static_cast<int32_t>(__lane_id());
    const int32_t start = j;
    for (int32_t base = 1; base <= mask; base += 64) {
        const int32_t i = (start + base + lane) & mask;
        const uint16_t e = ht[i];
        const int32_t home = (e != 0) ? static_cast<int32_t>(ht_hash(tok_at(tok, e, ntok))) & mask : 0;
        uint64_t active = ~0ull;
        for (;;) {
            const bool mv = (j < i) ? (home <= j || home > i) : (home <= j && home > i);
            const uint64_t m = __ballot(e == 0 || mv) & active;
            if (m == 0ull) break;
            const int f = __builtin_ctzll(m);
            if (lane_value(static_cast<int>(e), f) == 0) {
                if (lane == 0) ht[j] = 0;
                return;
            }
            if (lane == f) ht[j] = e;
            j = lane_value(i, f);
            active = (f == 63) ? 0ull : (~0ull << (f + 1));
        }
    }
    g.code = kOverflowProbe;
}

__device__ bool sieve_row_wave(const int32_t *rt, int32_t *rs, int8_t *rm, int32_t topK, int32_t seqLen,
                               int32_t prefill, int32_t dbs, int32_t padded, int32_t mask, int32_t *tok, uint8_t *vis,
                               uint16_t *ht, int32_t &hand, Guard &g)
{
    const int32_t lane = static_cast<int32_t>(__lane_id());
    uint32_t *vis32 = reinterpret_cast<uint32_t *>(vis);
    const int32_t width = dbs < 64 ? dbs : 64;  // slots per sweep step (no slot twice in one step)
    bool dirty = false;
    for (int32_t k0 = 0; k0 < topK; k0 += 64) {
        const int32_t myT = (k0 + lane < topK) ? rt[k0 + lane] : 0;
        int32_t mySlot = -1, myMiss = 0;
        const int32_t kn = (topK - k0 < 64) ? topK - k0 : 64;
        for (int32_t kk = 0; kk < kn; ++kk) {
            const int32_t tp = lane_value(myT, kk);
            int32_t slot = -1, miss = 0;
            if (g.code != 0 || tp < 0 || tp >= seqLen) {  // past a bound violation the row reads as invalid
            } else if (tp >= prefill) {
                slot = padded + (tp - prefill);
            } else {
                const int32_t home = static_cast<int32_t>(ht_hash(tp)) & mask;
                bool found = false;
                uint32_t e = 0;
                const int32_t cell = wave_probe_lds(ht, tok, padded, home, tp, mask, found, e, g);
                if (cell < 0) {
                } else if (found) {
                    slot = static_cast<int32_t>(e) - 1;
                    if (lane == 0) vis_set(vis, slot);
                } else {
                    int32_t h = -1;
                    for (int32_t base = 0; base <= 2 * dbs && h < 0; base += width) {
                        const bool on = lane < width;
                        const int32_t s = (hand + base + lane) % dbs;
                        const bool v = on && vis_get(vis, s);
                        const uint64_t unv = __ballot(on && !v);
                        const int f = unv ? __builtin_ctzll(unv) : 64;
                        if (lane < f && v) atomicAnd(vis32 + (s >> 5), ~(1u << (s & 31)));
                        if (f < 64) h = lane_value(s, f);
                    }
                    if (h < 0) {
                        g.code = kOverflowSweep;
                    } else {
                        const int32_t old = tok[h];
                        g.fpd += slot_token_mix(static_cast<uint32_t>(h), tp) - slot_token_mix(static_cast<uint32_t>(h), old);
                        if (old >= 0) {
                            bool f2 = false;
                            uint32_t e2 = 0;
                            const int32_t c2 = wave_probe_lds(ht, tok, padded, static_cast<int32_t>(ht_hash(old)) & mask,
                                                              old, mask, f2, e2, g);
                            if (c2 >= 0 && f2) wave_shift_lds(ht, tok, padded, c2, mask, g);
                        }
                        bool f3 = false;
                        uint32_t e3 = 0;
                        const int32_t c3 = wave_probe_lds(ht, tok, padded, home, tp, mask, f3, e3, g);
                        if (c3 >= 0 && !f3 && lane == 0) ht[c3] = static_cast<uint16_t>(h + 1);
                        if (lane == 0) {
                            tok[h] = tp;
                            vis_set(vis, h);
                        }
                        dirty = true;
                        slot = h;
                        miss = 1;
                        hand = (h + 1 == dbs) ? 0 : h + 1;
                    }
                }
            }
            if (lane == kk) {
                mySlot = slot;
                myMiss = miss;
            }
        }
        if (lane < kn) {
            rs[k0 + lane] = mySlot;
            rm[k0 + lane] = static_cast<int8_t>(myMiss);
        }
    }
    return dirty;
}

// Copy n bytes (multiple of 16, both sides 16-byte aligned) with the block.
// The in-order recurrence of hisp_sieve_update.cpp:115-163 for a row of at
// most 64 slots whose table indexes exactly its non-negative tokens (each
// at its own slot), with one wave: slot s's token and the cell of its entry
// in lane s, the visited bits and the hand in scalar registers, and the home
// of every occupied cell in hmc (htSize entries of LDS scratch, plus 64 for
// the set-up).  A lookup is a ballot over the lanes (the slot holding the
// token is the one the table's probe finds), the sweep a few mask
// operations; an eviction reads one window of 64 cells (entries and homes)
// for the erase's shifts and one for the insert.  Updates tok, vis and ht in
// place; returns whether any slot changed.
__device__ bool sieve_row_regs(const int32_t *rt, int32_t *rs, int8_t *rm, int32_t topK, int32_t seqLen,
                               int32_t prefill, int32_t dbs, int32_t padded, int32_t mask, int32_t *tok, uint8_t *vis,
                               uint16_t *ht, uint16_t *hmc, int32_t &hand, Guard &g)
{
    const int32_t lane = static_cast<int32_t>(__lane_id());
    const bool mine = lane < dbs;
    int32_t tokR = mine ? tok[lane] : -1;
    const uint64_t all = dbs >= 64 ? ~0ull : ((1ull << dbs) - 1ull);
    uint64_t vm = __ballot(mine && ((vis[lane >> 3] >> (lane & 7)) & 1));
    // homes of the occupied cells; the cell of each slot's entry
    int32_t cellR = -1;
    {
        uint16_t *cellF = hmc + mask + 1;
        for (int32_t c = lane; c <= mask; c += 64) {
            const uint32_t e = ht[c];
            if (e - 1u < static_cast<uint32_t>(dbs)) {
                hmc[c] = static_cast<uint16_t>(ht_hash(tok[e - 1u]) & static_cast<uint32_t>(mask));
                cellF[e - 1u] = static_cast<uint16_t>(c);
            }
        }
        if (mine && tokR >= 0) cellR = cellF[lane];
    }
    int32_t hd = hand;
    bool dirty = false;
    for (int32_t k0 = 0; k0 < topK; k0 += 64) {
        const int32_t kn = (topK - k0 < 64) ? topK - k0 : 64;
        const int32_t myT = lane < kn ? rt[k0 + lane] : -1;
        int32_t mySlot = -1, myMiss = 0;
        for (int32_t kk = 0; kk < kn; ++kk) {
            const int32_t tp = lane_value(myT, kk);
            int32_t slot = -1, miss = 0;
            if (tp < 0 || tp >= seqLen) {
            } else if (tp >= prefill) {
                slot = padded + (tp - prefill);
            } else {
                const uint64_t hm = __ballot(mine && tokR == tp);
                if (hm != 0ull) {
                    slot = __builtin_ctzll(hm);
                    vm |= 1ull << slot;
                } else {
                    // sweep from the hand: visited slots passed are cleared
                    const uint64_t unv = ~vm & all, from = all & ~((1ull << hd) - 1ull);
                    int32_t h;
                    if (unv & from) {
                        h = __builtin_ctzll(unv & from);
                        vm &= ~(((1ull << h) - 1ull) & from);
                    } else if (unv) {
                        h = __builtin_ctzll(unv);
                        vm &= ~(from | ((1ull << h) - 1ull));
                    } else {  // every slot visited: a whole revolution clears them all
                        h = hd;
                        vm = 0ull;
                    }
                    if (lane_value(tokR, h) >= 0) {
                        // erase (Algorithm R): entries after the hole move into
                        // it unless their home lies cyclically in (hole, cell]
                        const int32_t c = lane_value(cellR, h);
                        int32_t j = c;
                        bool closed = false;
                        for (int32_t base = 1; base <= mask + 1; base += 64) {
                            const int32_t i = (c + base + lane) & mask;
                            const uint32_t e = ht[i];
                            const int32_t hme = hmc[i];
                            const uint64_t z = __ballot(e == 0u);
                            const int32_t lim = z ? __builtin_ctzll(z) : 64;
                            int32_t last = -1;
                            for (;;) {
                                const bool mv = lane < lim && lane > last &&
                                                ((j < i) ? (hme <= j || hme > i) : (hme <= j && hme > i));
                                const uint64_t cm = __ballot(mv);
                                if (cm == 0ull) break;
                                last = __builtin_ctzll(cm);
                                if (lane == last) {
                                    ht[j] = static_cast<uint16_t>(e);
                                    hmc[j] = static_cast<uint16_t>(hme);
                                }
                                if (lane == lane_value(static_cast<int32_t>(e), last) - 1) cellR = j;
                                j = lane_value(i, last);
                            }
                            if (z) {
                                closed = true;
                                break;
                            }
                        }
                        if (!closed) g.code = kOverflowProbe;
                        if (lane == 0) ht[j] = 0;
                    }
                    // insert: the first empty cell from the new token's home
                    const int32_t home = static_cast<int32_t>(ht_hash(tp)) & mask;
                    bool placed = false;
                    for (int32_t base = 0; base <= mask; base += 64) {
                        const int32_t i = (home + base + lane) & mask;
                        const uint64_t z = __ballot(ht[i] == 0u);
                        if (z) {
                            const int32_t f = __builtin_ctzll(z);
                            if (lane == f) {
                                ht[i] = static_cast<uint16_t>(h + 1);
                                hmc[i] = static_cast<uint16_t>(home);
                            }
                            if (lane == h) cellR = lane_value(i, f);
                            placed = true;
                            break;
                        }
                    }
                    if (!placed) g.code = kOverflowProbe;
                    g.fpd += slot_token_mix(static_cast<uint32_t>(h), tp) -
                             slot_token_mix(static_cast<uint32_t>(h), lane_value(tokR, h));
                    if (lane == h) tokR = tp;
                    vm |= 1ull << h;
                    hd = (h + 1 == dbs) ? 0 : h + 1;
                    slot = h;
                    miss = 1;
                    dirty = true;
                }
            }
            if (lane == kk) {
                mySlot = slot;
                myMiss = miss;
            }
        }
        if (lane < kn) {
            rs[k0 + lane] = mySlot;
            rm[k0 + lane] = static_cast<int8_t>(myMiss);
        }
    }
    if (mine) tok[lane] = tokR;
    if (lane < (dbs + 7) / 8) {  // the visited bytes of slots [0, dbs); bits past dbs keep their value
        const int32_t b0 = lane * 8;
        const uint32_t keep = (dbs - b0 >= 8) ? 0u : (0xFFu << (dbs - b0)) & 0xFFu;
        vis[lane] = static_cast<uint8_t>((vis[lane] & keep) | (static_cast<uint32_t>(vm >> b0) & 0xFFu & ~keep));
    }
    hand = hd;
    return dirty;
}

// The hit/miss decisions of the in-order recurrence (hisp_sieve_update.cpp:
// 115-163) for a row of at most 64 slots whose table indexes exactly its
// non-negative tokens, in one wave's registers and without the table: a
// lookup is a ballot over the slots' tokens (slot s in lane s), the sweep a
// few mask operations on the visited bits.  Writes the outputs; returns the
// number of misses (events) and, per lane s, the slot's final token and the
// event that placed it (-1: not evicted this step), with the visited bits of
// slots [0, dbs) and the hand.  The table is left to the caller: it loses
// the pre-step token of every evicted slot and gains the final tokens in
// event order (a token placed and evicted within the step leaves no trace).
__device__ int32_t sieve_row_regs_decide(const int32_t *rt, int32_t *rs, int8_t *rm, int32_t topK, int32_t seqLen,
                                         int32_t prefill, int32_t dbs, int32_t padded, const int32_t *tok,
                                         const uint8_t *vis, int32_t &hand, int32_t &tokFinal, int32_t &lastEv,
                                         uint64_t &visMask)
{
    const int32_t lane = static_cast<int32_t>(__lane_id());
    const bool mine = lane < dbs;
    // slot s's token in lane s; -1 past dbs, so a valid token (>= 0) matches
    // only a slot of the row
    int32_t tokR = mine ? tok[lane] : -1;
    const uint64_t all = dbs >= 64 ? ~0ull : ((1ull << dbs) - 1ull);
    uint64_t vm = __ballot(mine && ((vis[lane >> 3] >> (lane & 7)) & 1));
    int32_t hd = hand, ev = -1, nev = 0;
    for (int32_t k0 = 0; k0 < topK; k0 += 64) {
        const int32_t kn = __builtin_amdgcn_readfirstlane((topK - k0 < 64) ? topK - k0 : 64);
        const int32_t myT = lane < kn ? rt[k0 + lane] : -1;
        // invalid and decode-extension positions in parallel; the rest are
        // looked up one after another (their outcomes change the row)
        const bool valid = lane < kn && myT >= 0 && myT < seqLen;
        int32_t mySlot = (valid && myT >= prefill) ? padded + (myT - prefill) : -1;
        uint64_t missBits = 0;
        for (uint64_t m = __ballot(valid && myT < prefill); m != 0ull; m &= m - 1ull) {
            const int32_t kk = __builtin_ctzll(m);
            const int32_t tp = __builtin_amdgcn_readlane(myT, kk);
            const uint64_t hm = __ballot(tokR == tp);
            int32_t slot;
            if (hm != 0ull) {
                slot = __builtin_ctzll(hm);
                vm |= 1ull << slot;
            } else {
                const uint64_t unv = ~vm & all, from = all & ~((1ull << hd) - 1ull);
                int32_t h;
                if (unv & from) {
                    h = __builtin_ctzll(unv & from);
                    vm &= ~(((1ull << h) - 1ull) & from);
                } else if (unv) {
                    h = __builtin_ctzll(unv);
                    vm &= ~(from | ((1ull << h) - 1ull));
                } else {  // every slot visited: a whole revolution clears them all
                    h = hd;
                    vm = 0ull;
                }
                tokR = lane_set(tokR, h, tp);
                ev = lane_set(ev, h, nev);
                ++nev;
                vm |= 1ull << h;
                hd = (h + 1 == dbs) ? 0 : h + 1;
                slot = h;
                missBits |= 1ull << kk;
            }
            mySlot = lane_set(mySlot, kk, slot);
        }
        if (lane < kn) {
            rs[k0 + lane] = mySlot;
            rm[k0 + lane] = static_cast<int8_t>((missBits >> lane) & 1ull);
        }
    }
    tokFinal = tokR;
    lastEv = ev;
    visMask = vm;
    hand = hd;
    return nev;
}

__device__ __forceinline__ void block_copy16(void *dst, const void *src, uint32_t n)
{
    const uint4 *s = static_cast<const uint4 *>(src);
    uint4 *d = static_cast<uint4 *>(dst);
    for (uint32_t i = threadIdx.x; i < n / 16u; i += blockDim.x) d[i] = s[i];
}

__device__ __forceinline__ void write_dummy_row(int32_t *rs, int8_t *rm, int32_t topK)
{
    for (int32_t k = threadIdx.x; k < topK; k += blockDim.x) {
        rs[k] = -1;
        rm[k] = 0;
    }
}

}  // namespace sieve
}  // namespace kvx
