// The in-order SIEVE recurrence on a row whose state lives in HBM: the exact
// per-position steps of hisp_sieve_update.cpp:115-163, with every inner loop
// run 64 cells or slots at a time by one wave.  A probe reads 64 consecutive
// table cells and picks the first empty or matching one with a ballot, the
// hand sweep tests 64 visited bits at once, and Algorithm R's backward shift
// walks the cluster 64 cells per step, taking the moves in order with
// ballots.  Probes compare tokens through a shadow of the table (cell ->
// token of its entry, built by the whole workgroup first), so one probe step
// is two coalesced row reads instead of a chain of dependent slot lookups.
// Shared by the HBM-resident kernels (sieve_wave.hip, sieve_batch.hip).
#pragma once

#include "kvx_internal.h"
#include "sieve_common.h"

namespace kvx {
namespace sieve_hbm {

using namespace sieve;

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// HBM pointers carry the global address space, so accesses compile to
// global_* instructions: flat ones also count against the LDS wait counter,
// and these kernels interleave table accesses with LDS work.
#define KVX_GM __attribute__((address_space(1)))

struct Row {
    KVX_GM uint16_t *ht;
    KVX_GM int32_t *ct;  // shadow: token of the entry in each cell, -1 for empty
    KVX_GM int32_t *tok;
    KVX_GM uint32_t *vis32;
    int32_t mask, dbs, padded;
};

// Workgroup-scope fence: the wave's stores and atomics are complete and
// visible to its later loads (one CU, one L1).  Taken once per position and
// where a step reads what an earlier step of the same position wrote, not
// per move: a shift writes only cells behind the window it reads next.
__device__ __forceinline__ void wave_fence() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup"); }

__device__ __forceinline__ uint16_t ld16(const KVX_GM uint16_t *p) { return *p; }
__device__ __forceinline__ int32_t ld32(const KVX_GM int32_t *p) { return *p; }
__device__ __forceinline__ uint32_t ldu32(const KVX_GM uint32_t *p) { return *p; }
// relaxed device-scope atomics (atomicOr / atomicAnd) on global-space words
__device__ __forceinline__ uint32_t g_or(KVX_GM uint32_t *p, uint32_t v)
{
    return __hip_atomic_fetch_or(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t g_and(KVX_GM uint32_t *p, uint32_t v)
{
    return __hip_atomic_fetch_and(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// token of the slot an entry names (-1 past the tokens row), as tok_at
__device__ __forceinline__ int32_t g_tok_at(const KVX_GM int32_t *tok, uint32_t e, int32_t ntok)
{
    return (static_cast<int32_t>(e) - 1 < ntok) ? tok[static_cast<int32_t>(e) - 1] : -1;
}

constexpr int kBatch = 16;  // 64-cell windows loaded together (one memory round trip)

// First cell at or after idx (cyclic) that is empty or holds `token`
// (hisp_kernel_common.h:29-61); -1 after the whole table.  *entry receives
// the cell's entry.
static __device__ int32_t probe(const Row &r, int32_t idx, int32_t token, bool &found, uint32_t &entry, Guard &g)
{
    const uint32_t lane = lane_id();
    for (int32_t base = 0; base <= r.mask; base += 64 * kBatch) {
        uint16_t e[kBatch];
        int32_t t[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            const int32_t c = (idx + base + 64 * q + static_cast<int32_t>(lane)) & r.mask;
            e[q] = ld16(r.ht + c);
            t[q] = ld32(r.ct + c);
        }
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            const uint64_t hit = __ballot(e[q] != 0 && t[q] == token);
            const uint64_t any = hit | __ballot(e[q] == 0);
            if (any != 0ull) {
                const int f = __builtin_ctzll(any);
                found = (hit >> f) & 1ull;
                entry = static_cast<uint32_t>(lane_value(static_cast<int>(e[q]), f));
                return (idx + base + 64 * q + f) & r.mask;
            }
        }
    }
    g.code = kOverflowProbe;
    found = false;
    return -1;
}

// Algorithm R from the hole at cell j (hisp_kernel_common.h:64-94): an entry
// at i moves into the hole j unless its home lies cyclically in (j, i], and
// then i is the new hole.  Per 64-cell window the chain of movers is found
// first (each step is one ballot against the current hole, no memory
// access), then every mover writes its entry into the cell of the mover
// before it (the window's incoming hole for the first) at once.  Moves write
// only cells behind the window being scanned, so the windows ahead can be
// loaded before the moves are made.
static __device__ int32_t shift_from(const Row &r, int32_t j, Guard &g)
{
    const uint32_t lane = lane_id();
    const int32_t start = j;
    for (int32_t base = 1; base <= r.mask; base += 64 * kBatch) {
        uint16_t eb[kBatch];
        int32_t tb[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            const int32_t c = (start + base + 64 * q + static_cast<int32_t>(lane)) & r.mask;
            eb[q] = ld16(r.ht + c);
            tb[q] = ld32(r.ct + c);
        }
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            const int32_t w0 = (start + base + 64 * q) & r.mask;  // cell of lane 0
            const int32_t i = (w0 + static_cast<int32_t>(lane)) & r.mask;
            const uint16_t e = eb[q];
            const int32_t t = tb[q];
            const int32_t home = (e != 0) ? static_cast<int32_t>(ht_hash(t)) & r.mask : 0;
            const uint64_t empty = __ballot(e == 0);
            const int32_t jin = j;
            uint64_t movers = 0;
            bool stop = false;
            for (int from = 0; from < 64;) {
                const bool mv = (j < i) ? (home <= j || home > i) : (home <= j && home > i);
                const uint64_t m = __ballot(static_cast<int>(lane) >= from && (e == 0 || mv));
                if (m == 0ull) break;
                const int f = __builtin_ctzll(m);
                if ((empty >> f) & 1ull) {
                    stop = true;
                    break;
                }
                movers |= 1ull << f;
                j = (w0 + f) & r.mask;
                from = f + 1;
            }
            if ((movers >> lane) & 1ull) {
                const uint64_t below = movers & ((1ull << lane) - 1ull);
                const int32_t dst = below ? ((w0 + 63 - __builtin_clzll(below)) & r.mask) : jin;
                r.ht[dst] = e;
                r.ct[dst] = t;
            }
            if (stop) {
                if (lane == 0) {
                    r.ht[j] = 0;
                    r.ct[j] = -1;
                }
                wave_fence();
                return j;
            }
        }
    }
    g.code = kOverflowProbe;
    return -1;
}

// Table shadow of the row (token of each cell's entry, -1 for empty), built by
// every thread of the workgroup.
__device__ __forceinline__ void build_shadow(const Row &r)
{
    for (int32_t c = threadIdx.x; c <= r.mask; c += blockDim.x) {
        const uint16_t e = r.ht[c];
        r.ct[c] = (e != 0) ? g_tok_at(r.tok, e, r.padded) : -1;
    }
}

// The recurrence over every position of the row, run by one wave after the
// shadow is built: outputs rs/rm, state updated in place, the hand stored in
// gHand[0] and a bound violation reported to the tail slot.
static __device__ __forceinline__ void recurrence(const Row r, const KVX_GM int32_t *rt, KVX_GM int32_t *rs, KVX_GM int8_t *rm,
                                  int32_t K, int32_t seqLen, int32_t prefill, KVX_GM int32_t *gHand,
                                  uint64_t overflowSlot)
{
    const int32_t dbs = r.dbs;
    const int32_t padded = r.padded;
    const uint32_t lane = lane_id();
    int32_t hand = gHand[0];
    if (hand < 0 || hand >= dbs) hand = 0;  // hisp_sieve_update.cpp:108-111
    const int32_t width = dbs < 64 ? dbs : 64;  // slots per sweep step (no slot twice in one step)
    Guard g;
    for (int32_t k0 = 0; k0 < K; k0 += 64) {
        const int32_t myT = (k0 + static_cast<int32_t>(lane) < K) ? rt[k0 + lane] : 0;
        int32_t mySlot = -1;
        int32_t myMiss = 0;
        const int32_t kn = (K - k0 < 64) ? K - k0 : 64;
        for (int32_t kk = 0; kk < kn; ++kk) {
            const int32_t tp = lane_value(myT, kk);
            int32_t slot = -1;
            int32_t miss = 0;
            if (g.code != 0 || tp < 0 || tp >= seqLen) {  // past a bound violation the row reads as invalid
            } else if (tp >= prefill) {
                slot = padded + (tp - prefill);
            } else {
                const int32_t home = static_cast<int32_t>(ht_hash(tp)) & r.mask;
                bool found = false;
                uint32_t e = 0;
                const int32_t cell = probe(r, home, tp, found, e, g);
                if (cell < 0) {
                } else if (found) {
                    slot = static_cast<int32_t>(e) - 1;
                    if (lane == 0) g_or(r.vis32 + (slot >> 5), 1u << (slot & 31));
                    wave_fence();
                } else {
                    // the hand passes visited slots, clearing them, and stops at the first unvisited one
                    int32_t h = -1;
                    for (int32_t base = 0; base <= 2 * dbs && h < 0; base += width) {
                        const bool on = static_cast<int32_t>(lane) < width;
                        const int32_t s = (hand + base + static_cast<int32_t>(lane)) % dbs;
                        const bool v = on && ((ldu32(r.vis32 + (s >> 5)) >> (s & 31)) & 1u);
                        const uint64_t unv = __ballot(on && !v);
                        const int f = unv ? __builtin_ctzll(unv) : 64;
                        if (static_cast<int>(lane) < f && v) g_and(r.vis32 + (s >> 5), ~(1u << (s & 31)));
                        // a later window of this sweep reads cleared bits only after a full turn
                        if (base + 2 * width > (base / dbs + 1) * dbs) wave_fence();
                        if (f < 64) h = lane_value(s, f);
                    }
                    if (h < 0) {
                        g.code = kOverflowSweep;
                    } else {
                        // the first probe stopped at the first empty cell c1 after
                        // tp's home; an erase empties exactly one cell (its final
                        // hole), so tp goes there if it lies in [home, c1), else c1
                        int32_t c3 = cell;
                        const int32_t old = ld32(r.tok + h);
                        if (old >= 0) {  // erase the evicted token
                            bool f2 = false;
                            uint32_t e2 = 0;
                            const int32_t c2 = probe(r, static_cast<int32_t>(ht_hash(old)) & r.mask, old, f2, e2, g);
                            if (c2 >= 0 && f2) {
                                const int32_t hole = shift_from(r, c2, g);
                                if (hole >= 0 && ((hole - home) & r.mask) < ((cell - home) & r.mask)) c3 = hole;
                            }
                        }
                        if (c3 >= 0 && lane == 0) {
                            r.ht[c3] = static_cast<uint16_t>(h + 1);
                            r.ct[c3] = tp;
                        }
                        if (lane == 0) {
                            r.tok[h] = tp;
                            g_or(r.vis32 + (h >> 5), 1u << (h & 31));
                        }
                        wave_fence();
                        slot = h;
                        miss = 1;
                        hand = (h + 1 == dbs) ? 0 : h + 1;
                    }
                }
            }
            if (static_cast<int32_t>(lane) == kk) {
                mySlot = slot;
                myMiss = miss;
            }
        }
        if (static_cast<int32_t>(lane) < kn) {
            rs[k0 + lane] = mySlot;
            rm[k0 + lane] = static_cast<int8_t>(myMiss);
        }
    }
    if (lane == 0) {
        gHand[0] = hand;
        report_overflow(overflowSlot, g.code);
    }
}

}  // namespace sieve_hbm
}  // namespace kvx
