// SIEVE update for rows whose state does not fit LDS, decided in one pass
// and applied to the hash table in batch (variant 5).
//
// One 1024-lane workgroup per batch row, after two pre-passes of 64
// workgroups per row that do a flagged row's order-free work (counts, first
// occurrences, token bitmap, resident slots) in HBM scratch; the state
// stays in HBM.  The result
// equals the in-order recurrence of hisp_sieve_update.cpp:115-163 whenever
// the row's table is canonical (every live token findable at its own slot)
// and topK < dbs (then no slot is evicted twice in a step); otherwise the row
// runs that recurrence (sieve_hbm.h) instead.  Phases:
//
//  1. check: a token -> slot map of the row (HBM scratch: every launch leaves
//     the map and first-occurrence table zeroed) finds duplicate tokens; a
//     scan of the table checks that each occupied cell names a live slot, no
//     slot twice, every live slot once, and that no empty cell lies between
//     an entry's home and its cell (so a probe from the home reaches it).  A
//     row whose consistency flag (sieve_hand[row][1]) is set, which this
//     kernel and the LDS kernel set when they leave the row consistent, only
//     has its live tokens and entries counted, and its tokens' fingerprint
//     compared with the one written with the flag (sieve_hand[row][3]);
//  2. decide: each position's first occurrence in the batch and the initial
//     slot of its token are found in parallel first (for a flagged row whose
//     tokens lie below the table size the pre-passes mark the step's tokens
//     in a bitmap and find their slots in one pass over the slots instead of
//     a token map); up to the first miss every position is a hit, applied in
//     parallel; a step whose hand does not come back to where it started is
//     then decided in parallel (decide_parallel); otherwise one wave decides
//     in order, from LDS only: a token is resident at the slot it was last
//     found in or placed into unless the hand evicted that slot since (a
//     hand that turns the whole ring comes back to slots hit earlier in the
//     step), and a miss sweeps the visited bitmap from the hand;
//  3. outputs, tokens, visited bits and hand, in parallel, and the cells of
//     the evicted slots (a step without misses ends here);
//  4. deletion of the evicted tokens' cells: Algorithm R leaves a table as if
//     the deleted key had never been inserted, so all of the step's
//     deletions give the same table in any order; one left-to-right pass per
//     cluster that holds a deleted cell does them all: walking the cluster
//     from its first deleted cell, each entry moves into the leftmost hole at
//     or after its home, if any (its cell then becomes a hole).  The pass
//     runs 64 cells at a time on one wave: which entries move depends only
//     on the rightmost hole (an entry moves iff it is at or after its home),
//     found one event at a time with one ballot each.  While the cluster
//     holds at most 64 holes they sit in the wave's lanes (a mover's hole is
//     one more ballot); beyond that, in a three-level hole bitmap for the
//     rest of the cluster.  A window without deleted cells finds its events
//     in parallel; when its movers all take the hole their previous event
//     left it is applied at once, otherwise only the holes go in order.  A
//     window's moves are written after it, in parallel;
//  5. the step's new tokens go in in position order, each into the first
//     empty cell at or after its home (a three-level bitmap of empty cells):
//     with step 4 this is the table the in-order recurrence leaves, which
//     equals inserting the live tokens in the order they were inserted.  The
//     row's consistency flag is then set (cleared on the in-order path).
#include "kvx_internal.h"
#include "sieve_hbm.h"

namespace kvx {
namespace {

using namespace sieve_hbm;

constexpr int BT = kBatchThreads;
constexpr uint32_t kInvalid = 0xFFFFFFFFu;   // position: outside [0, seqLen)
constexpr uint32_t kExt = 0xFFFFFFFEu;       // position: at or past prefill
constexpr uint32_t kNotRes = 0xFFFFFFFDu;    // position: first occurrence, token not resident
constexpr uint32_t kDup = 0x80000000u;       // position: later occurrence of the position in the low bits
constexpr uint32_t kMissBit = 0x80000000u;   // slotOut: the position was a miss
constexpr int kCheckUnroll = 8;              // loads of table cells in flight per lane in the scans
constexpr int kMapUnroll = 8;                // token loads in flight per lane (slots or positions)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16 bytes: eight table cells
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));   // 16 bytes: four slots' tokens

struct BatchParams {
    KvxLaunch<HispSieveUpdateArgs> L;
    int32_t *shadow;   // [maxNumReqs][H] table shadow for the in-order fallback
    uint32_t *aux;     // [maxNumReqs][auxWords]: map [mapCap], first [mapCap], bits [mapCap/32], counts [4],
                       // resident slot + 1 per position [topK]
    uint64_t auxWords;
    uint32_t mapCap;
    BatchLayout lay;
    uint32_t *tbl;      // the rebuild's scratch [maxNumReqs][t.words], or null: a step with
                        // misses then applies its table changes here (phases 4, 5)
    TableLayout t;
};

__device__ __forceinline__ int bit_get(const uint64_t *b, uint32_t i) { return (b[i >> 6] >> (i & 63)) & 1; }

// A three-level bitmap over n bits (n a multiple of 64): l1 bit w is set iff
// l0 word w is nonzero, l2 bit v iff l1 word v is nonzero.  Searches read at
// most one word per level going up and one going down (plus the l2 words,
// 64 bits per 2^18 cells).  Uniform in the wave: every lane reads the same
// words; one lane writes (the wave's LDS operations complete in order, so
// its later reads see the writes).
struct Bits3 {
    uint64_t *l0, *l1, *l2;
    uint32_t n;
};

__device__ __forceinline__ uint64_t from_bit(uint32_t b) { return ~0ull << (b & 63u); }

// First set bit at or after i, or -1.
__device__ __forceinline__ int64_t next_set(const Bits3 &m, uint32_t i)
{
    if (i >= m.n) return -1;
    const uint32_t w = i >> 6;
    const uint64_t x0 = m.l0[w] & from_bit(i);
    if (x0) return (static_cast<int64_t>(w) << 6) + __builtin_ctzll(x0);
    const uint32_t nw = m.n >> 6, n1 = (nw + 63u) >> 6;
    const uint32_t s1 = w + 1u;  // l0 words after w
    if (s1 < nw && (s1 & 63u)) {
        const uint64_t x1 = m.l1[s1 >> 6] & from_bit(s1);
        if (x1) {
            const uint32_t w0 = ((s1 >> 6) << 6) + static_cast<uint32_t>(__builtin_ctzll(x1));
            return (static_cast<int64_t>(w0) << 6) + __builtin_ctzll(m.l0[w0]);
        }
    }
    uint32_t s2 = (s1 + 63u) >> 6;  // l1 words after the one searched
    while (s2 < n1) {
        const uint64_t x2 = m.l2[s2 >> 6] & from_bit(s2);
        if (x2) {
            const uint32_t w1 = ((s2 >> 6) << 6) + static_cast<uint32_t>(__builtin_ctzll(x2));
            const uint32_t w0 = (w1 << 6) + static_cast<uint32_t>(__builtin_ctzll(m.l1[w1]));
            return (static_cast<int64_t>(w0) << 6) + __builtin_ctzll(m.l0[w0]);
        }
        s2 = ((s2 >> 6) + 1u) << 6;
    }
    return -1;
}

__device__ __forceinline__ void set_bit3(const Bits3 &m, uint32_t i, bool writer)
{
    const uint32_t w = i >> 6, v = w >> 6;
    const uint64_t x0 = m.l0[w] | (1ull << (i & 63u));
    const uint64_t x1 = m.l1[v] | (1ull << (w & 63u));
    const uint64_t x2 = m.l2[v >> 6] | (1ull << (v & 63u));
    if (writer) {
        m.l0[w] = x0;
        m.l1[v] = x1;
        m.l2[v >> 6] = x2;
    }
}

__device__ __forceinline__ void clr_bit3(const Bits3 &m, uint32_t i, bool writer)
{
    const uint32_t w = i >> 6, v = w >> 6;
    const uint64_t x0 = m.l0[w] & ~(1ull << (i & 63u));
    if (writer) m.l0[w] = x0;
    if (x0) return;
    const uint64_t x1 = m.l1[v] & ~(1ull << (w & 63u));
    if (writer) m.l1[v] = x1;
    if (x1) return;
    const uint64_t x2 = m.l2[v >> 6] & ~(1ull << (v & 63u));
    if (writer) m.l2[v >> 6] = x2;
}

// The parts of a flagged row's check and decide that need no order, spread
// over kPreSplit workgroups per row ahead of the row's own workgroup: the
// positions' first occurrences (atomic max of K - k per token), the bitmap of
// the step's tokens, and the table's entries and last empty cell.  A row the
// batch kernel will not take in its bitmap form is left alone.
constexpr int kPreSplit = 64;
constexpr int kPreThreads = 256;
constexpr int kPreLoads = 2;  // a lane's first loads of tokens or cells, issued with the row header

// Uniform values the pre-passes read and no kernel of the launch writes
// before (num_real, the request index, lengths, the flag) load through the
// constant address space, as scalar loads.
#define KVX_CM __attribute__((address_space(4)))

// The batch row's header, first level: num_real, the request index and the
// length in one round trip (every bid < maxNumReqs has its entries, so they
// are read before num_real is known).  False for a padding row or a request
// index outside the pool.
__device__ __forceinline__ bool batch_row_head(const HispSieveUpdateArgs &a, int32_t bid, int64_t &reqIdx,
                                               int32_t &seqLen)
{
    int32_t numReal = *(KVX_CM const int32_t *)(a.numReal);
    reqIdx = ((KVX_CM const int64_t *)(a.reqPoolIndices))[bid];
    seqLen = ((KVX_CM const int32_t *)(a.seqLens))[bid];
    asm volatile("" : : "s"(reqIdx), "s"(seqLen));
    const int32_t maxNumReqs = static_cast<int32_t>(a.maxNumReqs);
    if (numReal > maxNumReqs) numReal = maxNumReqs;
    if (bid >= numReal) return false;
    return reqIdx >= 0 && reqIdx < static_cast<int32_t>(a.poolSize);
}

// Second level: the request's flag and prefill length.  True when the batch
// kernel takes the row in its bitmap form (flagged, tokens below the table size).
__device__ __forceinline__ bool batch_row_bitmap(const HispSieveUpdateArgs &a, int64_t reqIdx, int32_t &prefill,
                                                 uint32_t mapCap)
{
    const int32_t flag = ((KVX_CM const int32_t *)(a.sieveHand))[reqIdx * kHandStride + 1];
    prefill = ((KVX_CM const int32_t *)(a.prefillLens))[reqIdx];
    asm volatile("" : : "s"(flag), "s"(prefill));
    if (flag != kCanonFlag) return false;
    const int32_t mapLim = prefill < static_cast<int32_t>(mapCap) ? prefill : static_cast<int32_t>(mapCap);
    return mapLim <= static_cast<int32_t>(a.htSize);
}

__global__ __launch_bounds__(kPreThreads) void kvx_sieve_batch_pre(BatchParams P)
{
    const HispSieveUpdateArgs &a = P.L.a;
    const int32_t bid = blockIdx.y, part = blockIdx.x, tid = threadIdx.x;
    if (bid >= static_cast<int32_t>(a.maxNumReqs)) return;
    const int32_t K = static_cast<int32_t>(a.topK);
    const int32_t H = static_cast<int32_t>(a.htSize);
    // this part's positions and table cells (8 a 16-byte load)
    const int32_t k0 = static_cast<int32_t>((static_cast<int64_t>(K) * part) / kPreSplit);
    const int32_t k1 = static_cast<int32_t>((static_cast<int64_t>(K) * (part + 1)) / kPreSplit);
    const uint32_t nChunk = static_cast<uint32_t>(H) / 8u;
    const uint32_t c0 = static_cast<uint32_t>((static_cast<uint64_t>(nChunk) * part) / kPreSplit);
    const uint32_t c1 = static_cast<uint32_t>((static_cast<uint64_t>(nChunk) * (part + 1)) / kPreSplit);
    // the first tokens need only the batch row (topk_indices holds
    // maxNumReqs rows): in flight with the header
    const KVX_GM int32_t *rt = reinterpret_cast<const KVX_GM int32_t *>(a.topkIndices) + static_cast<int64_t>(bid) * K;
    int32_t tk[kPreLoads];
#pragma unroll
    for (int q = 0; q < kPreLoads; ++q) {
        const int32_t k = k0 + tid + q * kPreThreads;
        tk[q] = k < k1 ? rt[k] : -1;
    }
    int64_t reqIdx = 0;
    int32_t prefill = 0, seqLen = 0;
    if (!batch_row_head(a, bid, reqIdx, seqLen)) return;
    // the first cells need the request: in flight with the flag
    const KVX_GM u32x4 *t16 = reinterpret_cast<const KVX_GM u32x4 *>(
        reinterpret_cast<const KVX_GM uint16_t *>(a.deviceBufferHt) + reqIdx * H);
    u32x4 cv[kPreLoads];
#pragma unroll
    for (int q = 0; q < kPreLoads; ++q) {
        const uint32_t c = c0 + static_cast<uint32_t>(tid + q * kPreThreads);
        if (c < c1) cv[q] = t16[c];
    }
    if (!batch_row_bitmap(a, reqIdx, prefill, P.mapCap)) return;
    const int32_t mapLim = prefill < static_cast<int32_t>(P.mapCap) ? prefill : static_cast<int32_t>(P.mapCap);
    KVX_GM uint32_t *first = (KVX_GM uint32_t *)P.aux + static_cast<uint64_t>(bid) * P.auxWords + P.mapCap;
    KVX_GM uint32_t *bits = first + P.mapCap;
    KVX_GM uint32_t *counts = bits + P.mapCap / 32u;
    auto position = [&](int32_t k, int32_t t) {
        if (t >= 0 && t < seqLen && t < prefill && t < mapLim) {
            __hip_atomic_fetch_max(first + t, static_cast<uint32_t>(K - k), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_or(bits + (t >> 5), 1u << (t & 31), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
#pragma unroll
    for (int q = 0; q < kPreLoads; ++q) {
        const int32_t k = k0 + tid + q * kPreThreads;
        if (k < k1) position(k, tk[q]);
    }
    for (int32_t k = k0 + tid + kPreLoads * kPreThreads; k < k1; k += kPreThreads) position(k, rt[k]);
    uint32_t occ = 0, lastPlus1 = 0;
    auto cells = [&](uint32_t c, u32x4 v) {
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const uint32_t lo = w[h] & 0xFFFFu, hi = w[h] >> 16;
            occ += (lo != 0u) + (hi != 0u);
            if (lo == 0u) lastPlus1 = c * 8u + 2u * h + 1u;
            if (hi == 0u) lastPlus1 = c * 8u + 2u * h + 2u;
        }
    };
#pragma unroll
    for (int q = 0; q < kPreLoads; ++q) {
        const uint32_t c = c0 + static_cast<uint32_t>(tid + q * kPreThreads);
        if (c < c1) cells(c, cv[q]);
    }
    for (uint32_t c = c0 + static_cast<uint32_t>(tid + kPreLoads * kPreThreads); c < c1; c += kPreThreads) cells(c, t16[c]);
    // a wave's sums, then one atomic per wave
    for (int d = 32; d > 0; d >>= 1) {
        occ += __shfl_xor(occ, d);
        const uint32_t o = __shfl_xor(lastPlus1, d);
        lastPlus1 = o > lastPlus1 ? o : lastPlus1;
    }
    if ((tid & 63) == 0) {
        if (occ) __hip_atomic_fetch_add(counts, occ, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (lastPlus1) __hip_atomic_fetch_max(counts + 1, lastPlus1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The slots of such a row, after the pre-pass, spread the same way: live
// tokens counted, a token past the map flagged, and each position that is the
// first occurrence of a resident token given that token's slot (+ 1).
__global__ __launch_bounds__(kPreThreads) void kvx_sieve_batch_slots(BatchParams P)
{
    const HispSieveUpdateArgs &a = P.L.a;
    const int32_t bid = blockIdx.y, part = blockIdx.x, tid = threadIdx.x;
    if (bid >= static_cast<int32_t>(a.maxNumReqs)) return;
    int64_t reqIdx = 0;
    int32_t prefill = 0, seqLen = 0;
    if (!batch_row_head(a, bid, reqIdx, seqLen)) return;
    const int32_t K = static_cast<int32_t>(a.topK);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const KVX_GM i32x4 *t4 = reinterpret_cast<const KVX_GM i32x4 *>(
        reinterpret_cast<const KVX_GM int32_t *>(a.deviceBufferTokens) + reqIdx * static_cast<int32_t>(a.paddedBufferSize));
    const int32_t nQuad = (dbs + 3) / 4;  // the row holds padded >= dbs slots, padded a multiple of 16
    const int32_t q0 = static_cast<int32_t>((static_cast<int64_t>(nQuad) * part) / kPreSplit);
    const int32_t q1 = static_cast<int32_t>((static_cast<int64_t>(nQuad) * (part + 1)) / kPreSplit);
    // the first slots' tokens: in flight with the flag
    i32x4 tv[kPreLoads];
#pragma unroll
    for (int j = 0; j < kPreLoads; ++j) {
        const int32_t q = q0 + tid + j * kPreThreads;
        if (q < q1) tv[j] = t4[q];
    }
    if (!batch_row_bitmap(a, reqIdx, prefill, P.mapCap)) return;
    const int32_t mapLim = prefill < static_cast<int32_t>(P.mapCap) ? prefill : static_cast<int32_t>(P.mapCap);
    KVX_GM uint32_t *first = (KVX_GM uint32_t *)P.aux + static_cast<uint64_t>(bid) * P.auxWords + P.mapCap;
    const KVX_GM uint32_t *bits = first + P.mapCap;
    KVX_GM uint32_t *counts = first + P.mapCap + P.mapCap / 32u;
    KVX_GM uint32_t *resSlot = counts + kBatchCounts;
    uint32_t live = 0, bad = 0, fp = 0;
    auto quad = [&](int32_t q, i32x4 v) {
        const int32_t t4v[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const int32_t sl = 4 * q + h, t = t4v[h];
            if (sl >= dbs) continue;
            fp += slot_token_mix(static_cast<uint32_t>(sl), t);
            if (t < 0) continue;
            ++live;
            if (t >= mapLim) {
                bad = 1;
            } else if ((bits[t >> 5] >> (t & 31)) & 1u) {
                resSlot[K - static_cast<int32_t>(first[t])] = static_cast<uint32_t>(sl + 1);
            }
        }
    };
#pragma unroll
    for (int j = 0; j < kPreLoads; ++j) {
        const int32_t q = q0 + tid + j * kPreThreads;
        if (q < q1) quad(q, tv[j]);
    }
    for (int32_t q = q0 + tid + kPreLoads * kPreThreads; q < q1; q += kPreThreads) quad(q, t4[q]);
    for (int d = 32; d > 0; d >>= 1) {
        live += __shfl_xor(live, d);
        bad |= __shfl_xor(bad, d);
        fp += __shfl_xor(fp, d);
    }
    if ((tid & 63) == 0) {
        if (live) __hip_atomic_fetch_add(counts + 2, live, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (bad) __hip_atomic_fetch_or(counts + 3, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (fp) __hip_atomic_fetch_add(counts + 4, fp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---------------------------------------------------------------------------
// The step's decisions in parallel (rows whose hand does not wrap).
//
// Within a step the hand passes each slot at most once, so a slot's fate
// depends on its class (the decision of the in-order recurrence,
// hisp_sieve_update.cpp:115-163): visited before the step (passed: cleared,
// set again by a later hit); unvisited and not hit (evicted by whichever miss
// the hand serves when it arrives); unvisited with its first hit at position k
// (evicted iff the hand arrives while serving a miss before k; the hit at k is
// then itself a miss, a conversion).  Walking the ring from the hand, slot i
// of the last class is evicted iff a_i = cc_i - n_i - 1 >= D_i, with cc_i the
// misses of non-resident tokens before k_i, n_i the unvisited unhit slots
// before i and D_i the evicted slots of the same class before i with a later
// first hit.  a_i < 0: passed; a_i >= U_i (the same count over every earlier
// slot with a_j >= 0, a bound on D_i): evicted; the rest in ring order.  The
// misses, in position order, take the evicted slots in ring order.  The hand
// stops at the last one; a slot passed while serving miss r is visited at the
// end iff a hit on it comes after that miss.
// ---------------------------------------------------------------------------
constexpr uint32_t kPdMaxSM = 512;  // slots of the last class within reach (more: the in-order loop)

struct PdLds {
    uint32_t *code, *slotOut;
    uint64_t *visB, *evB;     // visited bits; evB: the step's hit slots, then its evicted slots
    unsigned char *regA;      // scratch (the deleted-cell bitmap's LDS, unused while deciding)
    uint32_t regABytes;
    unsigned char *regB;      // scratch (the walk's stage)
    uint32_t regBBytes;
};

__device__ __forceinline__ uint64_t low_bits(uint32_t n) { return n >= 64u ? ~0ull : ((1ull << n) - 1ull); }

// n <= 64 bits of an absolute slot bitmap from slot `start` (start + n <= dbs)
__device__ __forceinline__ uint64_t bits_at(const uint64_t *bm, uint32_t start, uint32_t n)
{
    if (n == 0u) return 0ull;
    const uint32_t w = start >> 6, o = start & 63u;
    uint64_t v = bm[w] >> o;
    if (o != 0u && o + n > 64u) v |= bm[w + 1u] << (64u - o);
    return v & low_bits(n);
}

// Ring word j: the 64 ring offsets [64j, 64j + 64) from the hand (slot
// (hand + offset) mod dbs), as bits of an absolute slot bitmap.
__device__ __forceinline__ uint64_t ring_word(const uint64_t *bm, uint32_t j, uint32_t hand, uint32_t dbs)
{
    const uint32_t r0 = j << 6;
    const uint32_t len = dbs - r0 < 64u ? dbs - r0 : 64u;
    const uint32_t s0 = hand + r0 < dbs ? hand + r0 : hand + r0 - dbs;
    const uint32_t n1 = dbs - s0 < len ? dbs - s0 : len;
    uint64_t v = bits_at(bm, s0, n1);
    if (len > n1) v |= bits_at(bm, 0u, len - n1) << n1;
    return v;
}

// Exclusive prefix sum of one value per thread of the block; total in *tot.
__device__ __forceinline__ uint32_t block_exscan(uint32_t v, uint32_t *tot, uint32_t *sPart)
{
    const uint32_t lane = static_cast<uint32_t>(__lane_id()), wave = threadIdx.x >> 6;
    uint32_t inc = v;
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(inc), d));
        if (lane >= static_cast<uint32_t>(d)) inc += o;
    }
    if (lane == 63u) sPart[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int w = 0; w < kBatchWaves; ++w) {
            const uint32_t x = sPart[w];
            sPart[w] = run;
            run += x;
        }
        sPart[kBatchWaves] = run;
    }
    __syncthreads();
    const uint32_t r = sPart[wave] + inc - v;
    *tot = sPart[kBatchWaves];
    __syncthreads();
    return r;
}

// Offset of the r-th set bit (r < popcount) of x.
__device__ __forceinline__ uint32_t select_bit(uint64_t x, uint32_t r)
{
    uint32_t base = 0;
    for (uint32_t w = 32; w >= 1; w >>= 1) {
        const uint64_t lo = x & low_bits(w);
        const uint32_t c = static_cast<uint32_t>(__builtin_popcountll(lo));
        if (r >= c) {
            r -= c;
            x >>= w;
            base += w;
        } else {
            x = lo;
        }
    }
    return base;
}

// All threads call it; true: the step is decided (slotOut from firstMiss on,
// visB, evB = evicted slots, *hand, *misses); false: nothing was changed and
// the in-order loop decides.
__device__ __forceinline__ bool decide_parallel(const PdLds L, int32_t K, int32_t dbs, int32_t hand0, int32_t firstMiss,
                                int32_t *outHand, int32_t *outMisses)
{
    __shared__ uint32_t sPart[kBatchWaves + 1];
    __shared__ uint32_t sRel, sNev, sEnd;
    const uint32_t tid = threadIdx.x, lane = static_cast<uint32_t>(__lane_id());
    const uint32_t D = static_cast<uint32_t>(dbs);
    const uint32_t hand = (hand0 < 0 || hand0 >= dbs) ? 0u : static_cast<uint32_t>(hand0);
    const uint32_t nR = (D + 63u) / 64u, nW = nR;  // ring words; absolute words of the slot bitmaps
    const uint32_t nP = (static_cast<uint32_t>(K) + 63u) / 64u;  // position words
    // scratch: ring masks and their prefix counts (A); the candidate list and
    // the position bitmaps (B)
    const uint32_t needA = nR * 8u * 2u + (nR + 1u) * 4u * 2u;
    const uint32_t needB = kPdMaxSM * 8u * 2u + nP * 8u * 2u + (nP + 1u) * 4u * 2u;
    if (needA > L.regABytes || needB > L.regBBytes || nP > static_cast<uint32_t>(BT)) return false;
    uint64_t *snR = reinterpret_cast<uint64_t *>(L.regA);       // ring: unvisited, unhit (then: evicted)
    uint64_t *relR = snR + nR;                                   // ring: candidate slots of the last class
    uint32_t *snPre = reinterpret_cast<uint32_t *>(relR + nR);
    uint32_t *relPre = snPre + nR + 1u;
    uint64_t *list0 = reinterpret_cast<uint64_t *>(L.regB);     // candidates, unordered: ring << 40 | k << 20 | a
    uint64_t *list = list0 + kPdMaxSM;                           // the same in ring order
    uint64_t *cB = list + kPdMaxSM;                               // positions: non-resident first occurrences
    uint64_t *eB = cB + nP;                                       // positions: every miss
    uint32_t *cPre = reinterpret_cast<uint32_t *>(eB + nP);
    uint32_t *ePre = cPre + nP + 1u;
    auto ringOf = [&](uint32_t s) { return s >= hand ? s - hand : s + D - hand; };
    auto slotOf = [&](uint32_t r) { return hand + r < D ? hand + r : hand + r - D; };
    auto below = [](uint32_t b) { return low_bits(b); };
    const uint32_t k0 = static_cast<uint32_t>(firstMiss);

    // 1. positions from the first miss: non-resident first occurrences; the
    // slots hit by resident first occurrences (evB, zero until now)
    for (uint32_t w = tid; w < nP; w += BT) {
        cB[w] = 0ull;
        eB[w] = 0ull;
    }
    if (tid == 0) {
        sRel = 0u;
        sNev = 0u;
    }
    __syncthreads();
    for (uint32_t k = k0 + tid; k < static_cast<uint32_t>(K); k += BT) {
        const uint32_t c = L.code[k];
        if (c == kNotRes) {
            atomicOr(reinterpret_cast<unsigned long long *>(cB + (k >> 6)), 1ull << (k & 63u));
        } else if (c != kInvalid && c != kExt && !(c & kDup)) {
            atomicOr(reinterpret_cast<unsigned long long *>(L.evB + (c >> 6)), 1ull << (c & 63u));
        }
    }
    __syncthreads();
    // 2. ring words: unvisited unhit slots, counted in ring order
    uint32_t mySn = 0;
    if (tid < nR) {
        const uint32_t len = D - (tid << 6) < 64u ? D - (tid << 6) : 64u;
        const uint64_t v = ring_word(L.visB, tid, hand, D), h = ring_word(L.evB, tid, hand, D);
        const uint64_t sn = ~v & ~h & low_bits(len);
        snR[tid] = sn;
        relR[tid] = 0ull;
        mySn = static_cast<uint32_t>(__builtin_popcountll(sn));
    }
    uint32_t totSN = 0;
    const uint32_t snEx = block_exscan(mySn, &totSN, sPart);
    if (tid < nR) snPre[tid] = snEx;
    uint32_t myC = tid < nP ? static_cast<uint32_t>(__builtin_popcountll(cB[tid])) : 0u;
    uint32_t M = 0;
    const uint32_t cEx = block_exscan(myC, &M, sPart);
    if (tid < nP) cPre[tid] = cEx;
    __syncthreads();
    // from here on a refusal clears the hit bits (evB starts the in-order loop empty)
    auto refuse = [&]() {
        for (uint32_t w = tid; w < nW; w += BT) L.evB[w] = 0ull;
        __syncthreads();
        return false;
    };
    // every non-resident first occurrence needs an unvisited unhit slot
    // within one turn of the ring (more: the hand wraps)
    if (totSN < M) return refuse();
    // 3. candidates of the last class within reach (a >= 0)
    for (uint32_t k = k0 + tid; k < static_cast<uint32_t>(K); k += BT) {
        const uint32_t c = L.code[k];
        if (c == kInvalid || c == kExt || c == kNotRes || (c & kDup)) continue;
        if ((L.visB[c >> 6] >> (c & 63u)) & 1ull) continue;  // visited: passed
        const uint32_t r = ringOf(c), j = r >> 6;
        const uint32_t n = snPre[j] + static_cast<uint32_t>(__builtin_popcountll(snR[j] & below(r & 63u)));
        const uint32_t cc = cPre[k >> 6] + static_cast<uint32_t>(__builtin_popcountll(cB[k >> 6] & below(k & 63u)));
        if (cc < n + 1u) continue;  // a < 0: the hand reaches it while serving a miss after k (or never)
        const uint32_t a = cc - n - 1u;
        const uint32_t at = atomicAdd(&sRel, 1u);
        if (at < kPdMaxSM) {
            list0[at] = (static_cast<uint64_t>(r) << 40) | (static_cast<uint64_t>(k) << 20) | a;
            atomicOr(reinterpret_cast<unsigned long long *>(relR + j), 1ull << (r & 63u));
        }
    }
    __syncthreads();
    const uint32_t nRel = sRel;
    if (nRel > kPdMaxSM) return refuse();
    uint32_t myRel = tid < nR ? static_cast<uint32_t>(__builtin_popcountll(relR[tid])) : 0u;
    uint32_t relTot = 0;
    const uint32_t relEx = block_exscan(myRel, &relTot, sPart);
    if (tid < nR) relPre[tid] = relEx;
    __syncthreads();
    if (tid < nRel) {
        const uint64_t e = list0[tid];
        const uint32_t r = static_cast<uint32_t>(e >> 40), j = r >> 6;
        list[relPre[j] + static_cast<uint32_t>(__builtin_popcountll(relR[j] & below(r & 63u)))] = e;
    }
    __syncthreads();
    // 4. decide them: evicted for sure, passed, or in ring order
    // state: 1 = evicted, 2 = undecided
    uint32_t st = 0, myK = 0, myA = 0;
    if (tid < nRel) {
        const uint64_t e = list[tid];
        myK = static_cast<uint32_t>(e >> 20) & 0xFFFFFu;
        myA = static_cast<uint32_t>(e) & 0xFFFFFu;
        uint32_t U = 0;
        for (uint32_t i = 0; i < tid; ++i) U += ((static_cast<uint32_t>(list[i] >> 20) & 0xFFFFFu) > myK) ? 1u : 0u;
        st = myA >= U ? 1u : 2u;
    }
    // the undecided ones in ring order by one wave; its lanes hold the list,
    // entry i in lane i % 64 of register i / 64
    {
        uint32_t *sState = reinterpret_cast<uint32_t *>(list0);  // (the unordered list is dead)
        if (tid < nRel) sState[tid] = st;
        __syncthreads();
        if (tid < 64) {
            constexpr int R = kPdMaxSM / 64;
            uint32_t ks[R], sts[R];
#pragma unroll
            for (int q = 0; q < R; ++q) {
                const uint32_t i = static_cast<uint32_t>(q) * 64u + lane;
                ks[q] = i < nRel ? (static_cast<uint32_t>(list[i] >> 20) & 0xFFFFFu) : 0u;
                sts[q] = i < nRel ? sState[i] : 0u;
            }
#pragma unroll
            for (int q = 0; q < R; ++q) {
                uint64_t und = __ballot(sts[q] == 2u);
                while (und) {
                    const uint32_t l = static_cast<uint32_t>(__builtin_ctzll(und));
                    und &= und - 1ull;
                    const uint32_t i = static_cast<uint32_t>(q) * 64u + l;
                    const uint32_t ki = static_cast<uint32_t>(__shfl(static_cast<int>(ks[q]), static_cast<int>(l)));
                    const uint32_t ai = static_cast<uint32_t>(list[i]) & 0xFFFFFu;
                    uint32_t Dn = 0;
#pragma unroll
                    for (int q2 = 0; q2 < R; ++q2) {
                        const uint32_t i2 = static_cast<uint32_t>(q2) * 64u + lane;
                        Dn += static_cast<uint32_t>(__builtin_popcountll(__ballot(i2 < i && sts[q2] == 1u && ks[q2] > ki)));
                    }
                    const uint32_t dec = ai >= Dn ? 1u : 0u;
                    if (lane == l) sts[q] = dec;
                }
            }
#pragma unroll
            for (int q = 0; q < R; ++q) {
                const uint32_t i = static_cast<uint32_t>(q) * 64u + lane;
                if (i < nRel) sState[i] = sts[q];
            }
        }
        __syncthreads();
        st = tid < nRel ? sState[tid] : 0u;
    }
    // 5. evictions in ring order: the unvisited unhit slots and the evicted
    // slots of the last class; the misses are the non-resident first
    // occurrences and the conversions, the hand stops at the last one
    if (st == 1u) {
        const uint32_t r = static_cast<uint32_t>(list[tid] >> 40);
        atomicOr(reinterpret_cast<unsigned long long *>(snR + (r >> 6)), 1ull << (r & 63u));
        atomicOr(reinterpret_cast<unsigned long long *>(eB + (myK >> 6)), 1ull << (myK & 63u));
        atomicAdd(&sNev, 1u);
    }
    __syncthreads();
    const uint32_t E = M + sNev;
    uint32_t myEv = tid < nR ? static_cast<uint32_t>(__builtin_popcountll(snR[tid])) : 0u;
    uint32_t evTot = 0;
    const uint32_t evEx = block_exscan(myEv, &evTot, sPart);
    if (tid < nR) {
        snPre[tid] = evEx;
        if (E > 0u && evEx <= E - 1u && E - 1u < evEx + myEv) sEnd = (tid << 6) + select_bit(snR[tid], E - 1u - evEx);
    }
    if (tid < nP) eB[tid] |= cB[tid];
    __syncthreads();
    if (evTot < E) return refuse();  // not reachable (the count of unhit slots was checked)
    const uint32_t endRing = sEnd;
    uint32_t myE = tid < nP ? static_cast<uint32_t>(__builtin_popcountll(eB[tid])) : 0u;
    uint32_t eTot = 0;
    const uint32_t eEx = block_exscan(myE, &eTot, sPart);
    if (tid < nP) ePre[tid] = eEx;
    __syncthreads();
    // 6. outputs: misses take the evicted slot of their rank; hits keep theirs
    auto evictedSlot = [&](uint32_t r) {  // the r-th eviction in ring order
        uint32_t lo = 0, hi = nR;  // the last word whose prefix is <= r
        while (hi - lo > 1u) {
            const uint32_t mid = (lo + hi) >> 1;
            if (snPre[mid] <= r) lo = mid; else hi = mid;
        }
        return slotOf((lo << 6) + select_bit(snR[lo], r - snPre[lo]));
    };
    // (kNotRes carries the kDup bit: later occurrences are c & kDup other than it)
    auto isDup = [](uint32_t c) { return c != kInvalid && c != kExt && c != kNotRes && (c & kDup); };
    for (uint32_t k = k0 + tid; k < static_cast<uint32_t>(K); k += BT) {
        const uint32_t c = L.code[k];
        if (c == kInvalid || c == kExt || isDup(c)) continue;
        if ((eB[k >> 6] >> (k & 63u)) & 1ull) {
            const uint32_t r = ePre[k >> 6] + static_cast<uint32_t>(__builtin_popcountll(eB[k >> 6] & below(k & 63u)));
            L.slotOut[k] = evictedSlot(r) | kMissBit;
        } else {
            L.slotOut[k] = c;
        }
    }
    __syncthreads();
    for (uint32_t k = k0 + tid; k < static_cast<uint32_t>(K); k += BT) {
        const uint32_t c = L.code[k];
        if (isDup(c)) L.slotOut[k] = L.slotOut[c & ~kDup] & 0xFFFFu;
    }
    // 7. visited bits: swept slots (ring offsets up to endRing) end cleared,
    // or set when evicted; the rest keep theirs; then the hits
    const uint32_t endSlot = slotOf(endRing);
    auto sweptMask = [&](uint32_t w) {  // slots of word w with ring offset <= endRing
        const uint32_t a0 = w << 6, a1 = a0 + 64u < D ? a0 + 64u : D;
        uint64_t m = 0;
        // the swept slots: [hand, hand + endRing] mod dbs, one or two runs
        const uint32_t e1 = hand + endRing;  // inclusive end, may pass dbs
        const uint32_t r1lo = hand, r1hi = e1 < D ? e1 + 1u : D;
        if (r1hi > a0 && r1lo < a1) {
            const uint32_t lo = r1lo > a0 ? r1lo : a0, hi = r1hi < a1 ? r1hi : a1;
            m |= low_bits(hi - lo) << (lo - a0);
        }
        if (e1 >= D) {
            const uint32_t r2hi = e1 - D + 1u;
            if (r2hi > a0) {
                const uint32_t hi = r2hi < a1 ? r2hi : a1;
                m |= low_bits(hi - a0);
            }
        }
        return m;
    };
    uint64_t nv = 0, ne = 0;
    if (tid < nW) {
        const uint32_t a0 = tid << 6, len = D - a0 < 64u ? D - a0 : 64u;
        const uint64_t v = L.visB[tid], h = L.evB[tid], sw = sweptMask(tid);
        const uint64_t sn = ~v & ~h & low_bits(len);
        nv = (v & ~sw) | (sn & sw);
        ne = sn & sw;
    }
    __syncthreads();
    if (tid < nW) {
        L.visB[tid] = nv;
        L.evB[tid] = ne;
    }
    __syncthreads();
    if (st == 1u) {
        const uint32_t s = slotOf(static_cast<uint32_t>(list[tid] >> 40));
        atomicOr(reinterpret_cast<unsigned long long *>(L.visB + (s >> 6)), 1ull << (s & 63u));
        atomicOr(reinterpret_cast<unsigned long long *>(L.evB + (s >> 6)), 1ull << (s & 63u));
    }
    __syncthreads();
    for (uint32_t k = k0 + tid; k < static_cast<uint32_t>(K); k += BT) {
        const uint32_t c = L.code[k];
        if (c == kInvalid || c == kExt || c == kNotRes) continue;
        const uint32_t so = L.slotOut[k];
        if (so & kMissBit) continue;
        const uint32_t s = so & 0xFFFFu;
        const uint32_t r = ringOf(s);
        bool set = true;
        if (r <= endRing) {
            if ((L.evB[s >> 6] >> (s & 63u)) & 1ull) continue;  // evicted: visited already
            // passed while serving the miss of rank rs: visited again iff this hit comes after it
            const uint32_t j = r >> 6;
            const uint32_t rs = snPre[j] + static_cast<uint32_t>(__builtin_popcountll(snR[j] & below(r & 63u)));
            const uint32_t before = ePre[k >> 6] + static_cast<uint32_t>(__builtin_popcountll(eB[k >> 6] & below(k & 63u)));
            set = before > rs;
        }
        if (set) atomicOr(reinterpret_cast<unsigned long long *>(L.visB + (s >> 6)), 1ull << (s & 63u));
    }
    __syncthreads();
    *outHand = static_cast<int32_t>(endSlot + 1u == D ? 0u : endSlot + 1u);
    *outMisses = static_cast<int32_t>(E);
    return true;
}

__global__ __launch_bounds__(BT) void kvx_sieve_update_batch(BatchParams P)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ int32_t sScan[BT];
    __shared__ int32_t sBad, sWrap, sLive, sOcc, sNamed, sNdel, sHand, sE0, sTableBad, sFirstMiss, sMisses;
    __shared__ uint32_t sFp, sFpD;  // the pre-step tokens' fingerprint; its change by the step's new tokens

    const HispSieveUpdateArgs &a = P.L.a;
    const int32_t K = static_cast<int32_t>(a.topK);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t visStrideB = static_cast<int32_t>(a.visitedStrideB);
    const int32_t maxNumReqs = static_cast<int32_t>(a.maxNumReqs);
    const int32_t H = static_cast<int32_t>(a.htSize);
    const uint32_t mask = static_cast<uint32_t>(H) - 1u;
    const int32_t bid = blockIdx.x;
    const int tid = threadIdx.x;
    const uint32_t lane = lane_id();
    if (bid >= maxNumReqs) return;

    KVX_GM int32_t *rs = reinterpret_cast<KVX_GM int32_t *>(a.topKDeviceSlots) + static_cast<int64_t>(bid) * K;
    KVX_GM int8_t *rm = reinterpret_cast<KVX_GM int8_t *>(a.isMiss) + static_cast<int64_t>(bid) * K;
    // no table rebuild pending for this row unless this launch hands it one
    KVX_GM uint32_t *tbl = (KVX_GM uint32_t *)P.tbl + static_cast<uint64_t>(bid) * P.t.words;
    if (P.tbl != nullptr && tid == 0) tbl[P.t.meta] = 0u;
    // a padding row (bid >= num_real, capped at maxNumReqs) or a request
    // index outside the pool gets the dummy outputs (hisp_sieve_update.cpp:31-34,80-87)
    int64_t reqIdx = 0;
    int32_t seqLen = 0;
    if (!batch_row_head(a, bid, reqIdx, seqLen)) {
        write_dummy_row((int32_t *)rs, (int8_t *)rm, K);
        return;
    }
    // the prefill length, the flag and the hand as scalar loads, issued
    // together.  This kernel writes the flag and the hand later (the
    // outputs, the end of the table update), and a load from the constant
    // address space may be issued again at any later use: the two words pass
    // through an opaque asm, so every use reads the registers loaded here.
    const int32_t prefill = ((KVX_CM const int32_t *)(a.prefillLens))[reqIdx];
    int32_t flagWord = ((KVX_CM const int32_t *)(a.sieveHand))[reqIdx * kHandStride + 1];
    int32_t hand0 = ((KVX_CM const int32_t *)(a.sieveHand))[reqIdx * kHandStride];  // phase 2 starts from it
    // the fingerprint of the tokens the flag was written with
    int32_t fpWord = ((KVX_CM const int32_t *)(a.sieveHand))[reqIdx * kHandStride + kFingerprintWord];
    asm volatile("" : "+s"(flagWord), "+s"(hand0), "+s"(fpWord));
    const KVX_GM int32_t *rt = reinterpret_cast<const KVX_GM int32_t *>(a.topkIndices) + static_cast<int64_t>(bid) * K;
    Row r;
    r.tok = reinterpret_cast<KVX_GM int32_t *>(a.deviceBufferTokens) + reqIdx * padded;
    r.vis32 = reinterpret_cast<KVX_GM uint32_t *>(a.deviceBufferVisited + static_cast<uint64_t>(reqIdx) * visStrideB);
    r.ht = reinterpret_cast<KVX_GM uint16_t *>(a.deviceBufferHt) + reqIdx * H;
    r.ct = (KVX_GM int32_t *)P.shadow + static_cast<int64_t>(bid) * H;
    r.mask = H - 1;
    r.dbs = dbs;
    r.padded = padded;
    KVX_GM int32_t *gHand = reinterpret_cast<KVX_GM int32_t *>(a.sieveHand) + reqIdx * kHandStride;
    KVX_GM uint64_t *vis64 = (KVX_GM uint64_t *)r.vis32;
    KVX_GM uint32_t *map = (KVX_GM uint32_t *)P.aux + static_cast<uint64_t>(bid) * P.auxWords;
    KVX_GM uint32_t *first = map + P.mapCap;
    KVX_GM uint32_t *gBits = first + P.mapCap;     // the step's tokens, from kvx_sieve_batch_pre
    KVX_GM uint32_t *gCounts = gBits + P.mapCap / 32u;
    KVX_GM uint32_t *gResSlot = gCounts + kBatchCounts;  // from kvx_sieve_batch_slots
    const int32_t mapLim = prefill < static_cast<int32_t>(P.mapCap) ? prefill : static_cast<int32_t>(P.mapCap);
    // loads that need only the batch row, issued before the flag is known:
    // the pre-passes' counts (thread 0) and phase 2's first group of tokens
    // and resident slots (the row's scratch always holds topK of them; used
    // only in the bitmap form)
    uint32_t pc[5] = {0u, 0u, 0u, 0u, 0u};
    if (tid == 0) {
#pragma unroll
        for (int q = 0; q < 5; ++q) pc[q] = gCounts[q];
    }
    int32_t tv0[kMapUnroll];
    uint32_t rv0[kMapUnroll];
#pragma unroll
    for (int q = 0; q < kMapUnroll; ++q) {
        const int32_t k = tid + q * BT;
        tv0[q] = k < K ? rt[k] : -1;
        rv0[q] = k < K ? gResSlot[k] : 0u;
    }
    // a row this kernel (or the LDS kernel) left consistent: the table scans
    // of the check are skipped, its live tokens and entries still counted
    const bool flagged = flagWord == kCanonFlag;
    // such a row, with its tokens below the table size, needs no map: the
    // step's tokens are marked in a bitmap over [0, mapLim) (the LDS of the
    // deleted-cell bits, unused until the outputs), and one pass over the
    // slots finds the resident ones
    const bool useBits = flagged && mapLim <= H;

    const BatchLayout &y = P.lay;
    uint64_t *visB = reinterpret_cast<uint64_t *>(lds + y.vis);
    uint64_t *evB = reinterpret_cast<uint64_t *>(lds + y.ev);
    uint64_t *delB = reinterpret_cast<uint64_t *>(lds + y.del);       // also the named-slot bits of phase 1
    uint32_t *slotOut = reinterpret_cast<uint32_t *>(lds + y.slot);
    uint32_t *code = reinterpret_cast<uint32_t *>(lds + y.uni);       // phase 2 ...
    uint64_t *bitL0 = reinterpret_cast<uint64_t *>(lds + y.uni);      // ... then holes (4), empty cells (5)
    uint64_t *bitL1 = reinterpret_cast<uint64_t *>(lds + y.uniL1);
    uint64_t *bitL2 = reinterpret_cast<uint64_t *>(lds + y.uniL2);
    const Bits3 bits{bitL0, bitL1, bitL2, static_cast<uint32_t>(H)};
    uint32_t *stage = reinterpret_cast<uint32_t *>(lds + y.stage);
    const uint32_t nVisW = (static_cast<uint32_t>(dbs) + 63u) / 64u;
    const uint32_t nCellW = static_cast<uint32_t>(H) / 64u;
    const uint32_t nL1 = (nCellW + 63u) / 64u;
    const uint32_t nL2 = (nL1 + 63u) / 64u;

#ifdef KVX_BATCH_STAMPS
    uint64_t stamp[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    stamp[0] = __builtin_amdgcn_s_memtime();
#define KVX_STAMP(i) stamp[i] = __builtin_amdgcn_s_memtime()
#else
#define KVX_STAMP(i) (void)0
#endif
    // ---- 1. check ------------------------------------------------------
    if (tid == 0) {
        sBad = 0;
        sWrap = 0;
        sLive = 0;
        sOcc = 0;
        sNamed = 0;
        sNdel = 0;
        sE0 = -1;
        sTableBad = 0;
        sFirstMiss = K;
        sMisses = 0;
        sFp = sFpD = 0u;
    }
    for (uint32_t w = tid; w < nVisW; w += BT) {
        visB[w] = vis64[w];
        evB[w] = 0ull;
    }
    for (uint32_t w = tid; w < nCellW; w += BT) delB[w] = 0ull;
    __syncthreads();
    if (!useBits) {
        // the map by plain stores; a token held by two slots is found when
        // the map is read back below (one of them reads the other's slot).
        // kMapUnroll slots' tokens are loaded before any is used (one memory
        // round trip per group, not per slot).
        int32_t live = 0, bad = 0;
        uint32_t fp = 0;
        for (int32_t s0 = tid; s0 < dbs; s0 += BT * kMapUnroll) {
            int32_t tv[kMapUnroll];
#pragma unroll
            for (int q = 0; q < kMapUnroll; ++q) {
                const int32_t s = s0 + q * BT;
                tv[q] = s < dbs ? r.tok[s] : -1;
            }
#pragma unroll
            for (int q = 0; q < kMapUnroll; ++q) {
                const int32_t t = tv[q];
                if (s0 + q * BT < dbs) fp += slot_token_mix(static_cast<uint32_t>(s0 + q * BT), t);
                if (t < 0) continue;
                ++live;
                if (t >= mapLim) {
                    bad = 1;
                } else {
                    map[t] = static_cast<uint32_t>(s0 + q * BT + 1);
                }
            }
        }
        if (live) atomicAdd(&sLive, live);
        if (bad) sBad = 1;
        for (int d = 32; d > 0; d >>= 1) fp += __shfl_xor(fp, d);
        if (lane == 0 && fp) atomicAdd(&sFp, fp);
    }
    // a flagged row whose tokens changed since the flag was written (an edit
    // in place) is checked in full like an unflagged one (in the bitmap form,
    // without a map, it takes the in-order recurrence instead, below)
    bool full = !flagged;
    if (flagged && !useBits) {
        __syncthreads();
        full = sFp != static_cast<uint32_t>(fpWord);
    }
    if (full) {
        __syncthreads();
        {
            int32_t bad = 0;
            for (int32_t s0 = tid; s0 < dbs; s0 += BT * kMapUnroll) {
                int32_t tv[kMapUnroll];
                uint32_t mv[kMapUnroll];
    #pragma unroll
                for (int q = 0; q < kMapUnroll; ++q) {
                    const int32_t s = s0 + q * BT;
                    tv[q] = s < dbs ? r.tok[s] : -1;
                }
    #pragma unroll
                for (int q = 0; q < kMapUnroll; ++q) {
                    const int32_t t = tv[q];
                    mv[q] = (t >= 0 && t < mapLim) ? map[t] : 0u;
                }
    #pragma unroll
                for (int q = 0; q < kMapUnroll; ++q) {
                    const int32_t t = tv[q];
                    if (t >= 0 && t < mapLim && mv[q] != static_cast<uint32_t>(s0 + q * BT + 1)) bad = 1;
                }
            }
            if (bad) sBad = 1;
        }
        // The table in one segment per wave, read 64 cells per load, four loads
        // in flight: first the last empty cell of each segment; then, with the
        // last empty cell before each segment (cyclic), every occupied cell.
        const uint32_t wave = static_cast<uint32_t>(tid) >> 6;
        const uint32_t segCells = static_cast<uint32_t>(H) / kBatchWaves;  // a multiple of 64
        const uint32_t seg0 = wave * segCells;
        {
            int32_t last = -1;
            for (uint32_t base = seg0; base < seg0 + segCells; base += 64u * kCheckUnroll) {
                uint16_t e[kCheckUnroll];
    #pragma unroll
                for (int q = 0; q < kCheckUnroll; ++q) {
                    const uint32_t c = base + 64u * q + lane;
                    e[q] = c < seg0 + segCells ? r.ht[c] : static_cast<uint16_t>(1);
                }
    #pragma unroll
                for (int q = 0; q < kCheckUnroll; ++q) {
                    const uint64_t em = __ballot(e[q] == 0);
                    if (em) last = static_cast<int32_t>(base + 64u * q + 63u - __builtin_clzll(em));
                }
            }
            if (lane == 0) sScan[wave] = last;
        }
        __syncthreads();
        {
            int32_t lastAll = -1, carry = -1;
            for (uint32_t w = 0; w < kBatchWaves; ++w) {
                const int32_t v = sScan[w];
                if (v >= 0) {
                    lastAll = v;
                    if (w < wave) carry = v;
                }
            }
            if (tid == 0) {
                sE0 = lastAll;
                if (lastAll < 0) sBad = 1;  // no empty cell: probes never stop
            }
            if (carry < 0) carry = lastAll;  // the probe runs wrap around the table end
            int32_t occ = 0, bad = 0;
            uint32_t *named = reinterpret_cast<uint32_t *>(delB);
            for (uint32_t base = seg0; base < seg0 + segCells; base += 64u * kCheckUnroll) {
                uint16_t e[kCheckUnroll];
                int32_t t[kCheckUnroll];
    #pragma unroll
                for (int q = 0; q < kCheckUnroll; ++q) {
                    const uint32_t c = base + 64u * q + lane;
                    e[q] = c < seg0 + segCells ? r.ht[c] : static_cast<uint16_t>(0);
                }
    #pragma unroll
                for (int q = 0; q < kCheckUnroll; ++q) {
                    const int32_t sl = static_cast<int32_t>(e[q]) - 1;
                    t[q] = (e[q] != 0 && sl < dbs) ? r.tok[sl] : -1;
                }
    #pragma unroll
                for (int q = 0; q < kCheckUnroll; ++q) {
                    const uint32_t c = base + 64u * q + lane;
                    const uint64_t em = __ballot(e[q] == 0 && c < seg0 + segCells);
                    // the last empty cell at or before this lane's cell
                    const uint64_t upTo = em & (lane == 63 ? ~0ull : ((2ull << lane) - 1ull));
                    const int32_t lastE = upTo ? static_cast<int32_t>(base + 64u * q + 63u - __builtin_clzll(upTo)) : carry;
                    if (em) carry = static_cast<int32_t>(base + 64u * q + 63u - __builtin_clzll(em));
                    if (e[q] == 0 || c >= seg0 + segCells) continue;
                    ++occ;
                    const int32_t sl = static_cast<int32_t>(e[q]) - 1;
                    if (sl >= dbs || t[q] < 0) {
                        bad = 1;  // an entry naming a slot past the buffer or an empty slot
                        continue;
                    }
                    atomicOr(named + (sl >> 5), 1u << (sl & 31));  // a slot named twice shows in the count below
                    const uint32_t home = ht_hash(t[q]) & mask;
                    // no empty cell in [home, c): the last empty cell before c is
                    // further from c than the home is
                    if (((c - static_cast<uint32_t>(lastE)) & mask) <= ((c - home) & mask)) bad = 1;
                }
            }
            if (occ) atomicAdd(&sOcc, occ);
            if (bad) sBad = 1;
        }
        __syncthreads();
        {
            // every occupied cell names a distinct live slot iff the named slots
            // number as many as the occupied cells (and as the live slots)
            const uint32_t *named = reinterpret_cast<const uint32_t *>(delB);
            int32_t cnt = 0;
            for (int32_t w = tid; w < (dbs + 31) / 32; w += BT) cnt += __builtin_popcount(named[w]);
            if (cnt) atomicAdd(&sNamed, cnt);
        }
    } else {
        // the entries counted and the last empty cell found, 8 cells a load
        // (counted by the pre-pass for a row in the bitmap form)
        int32_t occ = 0, last = -1;
        if (useBits && tid == 0) {
            occ = static_cast<int32_t>(pc[0]);
            last = static_cast<int32_t>(pc[1]) - 1;
            sLive = static_cast<int32_t>(pc[2]);
            sFp = pc[4];
            // a token past the map, or a live token without an entry (or the
            // reverse), or tokens changed since the flag was written: the
            // in-order recurrence instead
            if (pc[3] != 0u || pc[2] != pc[0] || pc[4] != static_cast<uint32_t>(fpWord)) sBad = 1;
        }
        const uint32_t nChunk = static_cast<uint32_t>(H) / 8u;
        const KVX_GM u32x4 *t16 = reinterpret_cast<const KVX_GM u32x4 *>(r.ht);
        for (uint32_t c0 = tid; c0 < nChunk && !useBits; c0 += BT * kCheckUnroll) {
            u32x4 v[kCheckUnroll];
#pragma unroll
            for (int q = 0; q < kCheckUnroll; ++q) {
                const uint32_t c = c0 + static_cast<uint32_t>(q) * BT;
                if (c < nChunk) v[q] = t16[c];
            }
#pragma unroll
            for (int q = 0; q < kCheckUnroll; ++q) {
                if (c0 + static_cast<uint32_t>(q) * BT >= nChunk) continue;
                const uint32_t c = (c0 + static_cast<uint32_t>(q) * BT) * 8u;
                const uint32_t w[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                    const uint32_t lo = w[h] & 0xFFFFu, hi = w[h] >> 16;
                    occ += (lo != 0u) + (hi != 0u);
                    if (lo == 0u) last = static_cast<int32_t>(c + 2u * h);
                    if (hi == 0u) last = static_cast<int32_t>(c + 2u * h + 1u);
                }
            }
        }
        if (occ) atomicAdd(&sOcc, occ);
        if (last >= 0) atomicMax(&sE0, last);
        __syncthreads();
        if (tid == 0) {
            sNamed = sOcc;
            if (sE0 < 0) sBad = 1;  // no empty cell: probes never stop
        }
    }
    __syncthreads();
    // (the bitmap form's counts were compared above)
    const bool canonical = sBad == 0 && (useBits || (sOcc == sLive && sNamed == sOcc));

    KVX_STAMP(1);
    // ---- 2. decide -----------------------------------------------------
    if (canonical) {
        for (int32_t k0 = tid; k0 < K; k0 += BT * kMapUnroll) {
            int32_t tv[kMapUnroll];  // loads in flight together
            uint32_t rv[kMapUnroll];
            if (k0 == tid) {  // the group loaded at the start
#pragma unroll
                for (int q = 0; q < kMapUnroll; ++q) {
                    tv[q] = tv0[q];
                    rv[q] = useBits ? rv0[q] : 0u;
                }
            } else {
#pragma unroll
                for (int q = 0; q < kMapUnroll; ++q) {
                    tv[q] = k0 + q * BT < K ? rt[k0 + q * BT] : -1;
                    rv[q] = (useBits && k0 + q * BT < K) ? gResSlot[k0 + q * BT] : 0u;
                }
            }
#pragma unroll
            for (int q = 0; q < kMapUnroll; ++q) {
                const int32_t k = k0 + q * BT;
                if (k >= K) continue;
                const int32_t t = tv[q];
                uint32_t c = kInvalid;
                if (t >= 0 && t < seqLen) {
                    c = kExt;
                    if (t < prefill) {
                        c = kNotRes;
                        if (useBits) {
                            // the pre-passes found the first occurrences and their slots
                            if (rv[q] != 0u) c = rv[q] - 1u;
                        } else if (t < mapLim) {
                            __hip_atomic_fetch_max(first + t, static_cast<uint32_t>(K - k), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
                        }
                    }
                }
                code[k] = c;
                slotOut[k] = 0u;  // positions that change nothing read as hits of slot 0 without the miss bit
            }
        }
        __syncthreads();
        for (int32_t k = tid; k < K; k += BT) {
            if (code[k] != kNotRes) continue;
            const int32_t t = rt[k];
            if (t >= mapLim) {
                sBad = 1;  // a token the map cannot hold: decided in order instead
                continue;
            }
            const int32_t f = K - static_cast<int32_t>(first[t]);
            if (f < k) {
                code[k] = kDup | static_cast<uint32_t>(f);
            } else {
                // a first occurrence still unresolved: with the bitmap, not
                // resident; otherwise the map says
                const uint32_t s0 = useBits ? 0u : map[t];
                if (s0 != 0u) {
                    code[k] = s0 - 1u;
                } else {
                    atomicMin(&sFirstMiss, k);  // a first occurrence not resident: a miss
                }
            }
        }
        __syncthreads();
        // Up to the first miss every position is a hit (no slot has been
        // evicted yet): applied in parallel, a later occurrence taking its
        // first occurrence's slot, which is a resident one before the miss.
        const int32_t firstMiss = sFirstMiss;
        for (int32_t k = tid; k < firstMiss; k += BT) {
            const uint32_t c = code[k];
            if (c == kInvalid || c == kExt) continue;
            const uint32_t sl = (c & kDup) ? code[c & ~kDup] : c;
            slotOut[k] = sl;
            atomicOr(reinterpret_cast<unsigned long long *>(visB + (sl >> 6)), 1ull << (sl & 63));
        }
        __syncthreads();
    }
    bool decided = false;
    if (canonical && sBad == 0 && sFirstMiss < K) {
        const PdLds pl{code, slotOut, visB, evB, reinterpret_cast<unsigned char *>(delB), nCellW * 8u,
                       reinterpret_cast<unsigned char *>(stage), kBatchStage * 4u};
        int32_t ph = 0, pm = 0;
        decided = decide_parallel(pl, K, dbs, hand0, sFirstMiss, &ph, &pm);
        if (decided && tid == 0) {
            sHand = ph;
            sWrap = 0;
            sMisses = pm;
        }
    }
    if (canonical && sBad == 0 && !decided && tid < 64) {
        // One wave, 64 positions per round, in position order, from LDS only.
        // The hand may pass a slot twice in a step (a full turn clearing
        // visited bits, then evictions from where it started), so a token hit
        // earlier in the step can be evicted: a token's state is the slot it
        // was last found in or placed into, and whether the step had evicted
        // that slot then; it is resident while that has not changed.  No slot
        // is evicted twice when topK < dbs: between two evictions of a slot
        // the hand passes every slot twice, the second time clearing only
        // bits set after the first (by a placement, or a hit), so the
        // positions in between number at least dbs.  (With topK >= dbs a
        // second eviction is possible: the round that makes one finds the
        // slot's eviction bit already set, and the row takes the in-order
        // recurrence instead.)  code[f] of a first
        // occurrence f holds its token's state (slot | evicted << 16) from the
        // round that last changed it (a resident token's initial slot to begin
        // with).  Per round, what each position needs from LDS is read at
        // once: its first occurrence and that token's state, resident or not
        // at the round's start.  The positions are then decided one at a time
        // in scalar registers: the hand, the visited word it sweeps, the
        // round's evictions (in lanes; a token found at the round's start
        // stays while the round has not evicted its slot) and results (in
        // lanes).  A hit's visited bit goes to that word, or to LDS with an
        // atomic OR when it lies elsewhere; the wave's LDS operations
        // complete in order, so a word the sweep loads later holds it.
        int32_t hand = hand0;
        if (hand < 0 || hand >= dbs) hand = 0;  // hisp_sieve_update.cpp:108-111
        int32_t passed = 0, nMiss = 0;
        bool bail = false;  // a slot evicted twice: decided in order instead
        const int32_t passLimit = dbs + 2 * K;
        const uint32_t lastW = nVisW - 1u;
        const uint64_t lastMask = (dbs & 63) ? ((1ull << (dbs & 63)) - 1ull) : ~0ull;
        uint32_t cwIdx = static_cast<uint32_t>(hand) >> 6;  // the visited word held in registers
        uint64_t cwVal = uniform64(visB[cwIdx]);
        constexpr uint32_t kGone = 0xFFu;  // a lane's token not resident
        // from the round of the first miss (the positions before it, applied
        // again, change nothing)
        for (int32_t k0 = sFirstMiss & ~63; k0 < K && !bail; k0 += 64) {
            const int32_t k = k0 + static_cast<int32_t>(lane);
            const uint32_t c = k < K ? code[k] : kInvalid;
            const bool work = c != kInvalid && c != kExt;
            // the lane's first occurrence, its token's slot, and the number of
            // the round's evictions of that slot at which the token is there
            uint32_t myF = 0xFFFFFFFFu, mySlot = 0u, myNeed = kGone;
            bool myRel = false;  // placed in this round
            if (work) {
                uint32_t st = c;
                myF = static_cast<uint32_t>(k);
                if (c != kNotRes && (c & kDup)) {
                    myF = c & ~kDup;
                    st = code[myF];
                }
                if (st != kNotRes) {
                    mySlot = st & 0xFFFFu;
                    myNeed = static_cast<uint32_t>(bit_get(evB, mySlot)) == (st >> 16) ? 0u : kGone;
                }
            }
            uint64_t pend = __ballot(work);
            uint32_t result = 0u;             // lane j: position k0 + j's slot (| kMissBit)
            uint32_t evRound = 0xFFFFFFFFu;   // lane i: the round's i-th eviction
            int32_t nEv = 0;
            while (pend) {
                const int j = __builtin_ctzll(pend);
                pend &= pend - 1ull;
                const uint32_t sj = static_cast<uint32_t>(lane_value(static_cast<int32_t>(mySlot), j));
                const uint32_t nd = static_cast<uint32_t>(lane_value(static_cast<int32_t>(myNeed), j));
                if (nd != kGone && static_cast<uint32_t>(__builtin_popcountll(__ballot(evRound == sj))) == nd) {
                    if ((sj >> 6) == cwIdx) {
                        cwVal |= 1ull << (sj & 63u);
                    } else if (lane == 0) {
                        atomicOr(reinterpret_cast<unsigned long long *>(visB + (sj >> 6)), 1ull << (sj & 63u));
                    }
                    result = static_cast<uint32_t>(lane_set(static_cast<int32_t>(result), j, static_cast<int32_t>(sj)));
                    continue;
                }
                // the miss: the hand passes visited slots, clearing them, and
                // stops at the first unvisited one
                int32_t h = -1;
                while (h < 0) {
                    const uint32_t wi = static_cast<uint32_t>(hand) >> 6;
                    if (wi != cwIdx) {
                        if (lane == 0) visB[cwIdx] = cwVal;
                        cwIdx = wi;
                        cwVal = uniform64(visB[wi]);
                    }
                    const uint32_t b = static_cast<uint32_t>(hand) & 63u;
                    const uint64_t inRing = wi == lastW ? lastMask : ~0ull;
                    const uint64_t unv = ~cwVal & inRing & (~0ull << b);
                    if (unv) {
                        const uint32_t f = static_cast<uint32_t>(__builtin_ctzll(unv));
                        const uint64_t cleared = ((1ull << f) - 1ull) & (~0ull << b);  // visited bits passed
                        passed += static_cast<int32_t>(f - b) + 1;
                        h = static_cast<int32_t>((wi << 6) + f);
                        cwVal = (cwVal & ~cleared) | (1ull << f);
                    } else {
                        const uint64_t cleared = inRing & (~0ull << b);
                        passed += static_cast<int32_t>(__builtin_popcountll(cleared));
                        cwVal &= ~cleared;
                        hand = wi == lastW ? 0 : static_cast<int32_t>((wi + 1u) << 6);
                    }
                    if (passed > passLimit) {  // past the travel bound (dbs + 2 topK): not reachable
                        bail = true;
                        break;
                    }
                }
                if (bail) break;
                evRound = static_cast<uint32_t>(lane_set(static_cast<int32_t>(evRound), nEv, h));
                ++nEv;
                result = static_cast<uint32_t>(lane_set(static_cast<int32_t>(result), j, h | static_cast<int32_t>(kMissBit)));
                // every occurrence of the token now finds it in h, which the
                // round has evicted once
                const uint32_t fj = static_cast<uint32_t>(lane_value(static_cast<int32_t>(myF), j));
                if (myF == fj) {
                    mySlot = static_cast<uint32_t>(h);
                    myNeed = 1u;
                    myRel = true;
                }
                ++nMiss;
                hand = h + 1 == dbs ? 0 : h + 1;
            }
            if (bail) break;
            if (work) {
                slotOut[k] = result;
                if (myRel) code[myF] = mySlot | (1u << 16);
            }
            // the round's evictions; a slot evicted before (not reachable)
            // sends the row to the in-order recurrence
            bool again = false;
            if (static_cast<int32_t>(lane) < nEv) {
                const unsigned long long bit = 1ull << (evRound & 63u);
                again = (atomicOr(reinterpret_cast<unsigned long long *>(evB + (evRound >> 6)), bit) & bit) != 0ull;
            }
            bail = bail || __ballot(again) != 0ull;
        }
        if (lane == 0) {
            visB[cwIdx] = cwVal;
            sHand = hand;
            sWrap = bail ? 1 : 0;
            sMisses = nMiss;
        }
    }
    __syncthreads();
    KVX_STAMP(2);
    const bool fast = canonical && sBad == 0 && sWrap == 0;

    // the map and first-occurrence scratch are left zeroed (tokens still the
    // initial ones here)
    for (int32_t s0 = tid; s0 < dbs && !useBits; s0 += BT * kMapUnroll) {
        int32_t tv[kMapUnroll];
#pragma unroll
        for (int q = 0; q < kMapUnroll; ++q) {
            const int32_t s = s0 + q * BT;
            tv[q] = s < dbs ? r.tok[s] : -1;
        }
#pragma unroll
        for (int q = 0; q < kMapUnroll; ++q) {
            if (tv[q] >= 0 && tv[q] < mapLim) map[tv[q]] = 0u;
        }
    }
#pragma unroll
    for (int q = 0; q < kMapUnroll; ++q) {  // the first group's tokens are still in registers
        const int32_t t = tv0[q];
        if (t >= 0 && t < seqLen && t < prefill && t < mapLim) first[t] = 0u;
    }
    for (int32_t k = tid + kMapUnroll * BT; k < K; k += BT) {
        const int32_t t = rt[k];
        if (t >= 0 && t < seqLen && t < prefill && t < mapLim) first[t] = 0u;
    }
    if (useBits) {
        for (int32_t w = tid; w < (mapLim + 31) / 32; w += BT) gBits[w] = 0u;
        for (int32_t k = tid; k < K; k += BT) gResSlot[k] = 0u;
        if (tid < static_cast<int>(kBatchCounts)) gCounts[tid] = 0u;
    }
    __syncthreads();  // the cleanup read the initial tokens; phase 3 replaces some
    KVX_STAMP(3);
    if (!fast) {
        // the in-order recurrence on the untouched row, which the next launch
        // checks in full
        if (tid == 0) gHand[1] = 0;
        build_shadow(r);
        __threadfence_block();
        __syncthreads();
        if (tid < 64) recurrence(r, rt, rs, rm, K, seqLen, prefill, gHand, P.L.overflowSlot);
        return;
    }

    // ---- 3. outputs, visited bits, hand; cells of the evicted slots -------
    for (int32_t k = tid; k < K; k += BT) {
        const uint32_t c = code[k];
        int32_t slot = -1;
        int8_t miss = 0;
        if (c == kExt) {
            slot = padded + (rt[k] - prefill);
        } else if (c != kInvalid) {
            const uint32_t s = slotOut[k];
            slot = static_cast<int32_t>(s & 0xFFFFu);
            miss = (s & kMissBit) ? 1 : 0;
        }
        rs[k] = slot;
        rm[k] = miss;
    }
    for (uint32_t w = tid; w < nVisW; w += BT) vis64[w] = visB[w];
    if (tid == 0) gHand[0] = sHand;
    for (uint32_t w = tid; w < nCellW; w += BT) delB[w] = 0ull;
    __syncthreads();  // code[] is dead from here on (its LDS becomes the bitmaps)
    if (P.tbl != nullptr && sMisses > 0) {
        // The table's deletions and inserts go to the rebuild kernels: the
        // step's evicted slots, its new keys in event order with their homes
        // (zeroed per-home counts for them to fill), then the new tokens.
        const uint32_t HH = static_cast<uint32_t>(H) < 65536u ? static_cast<uint32_t>(H) : 65536u;
        KVX_GM uint64_t *ev64 = (KVX_GM uint64_t *)(tbl + P.t.evict);
        for (uint32_t w = tid; w < nVisW; w += BT) ev64[w] = evB[w];
        for (uint32_t i = tid; i < HH; i += BT) tbl[P.t.hist + i] = 0u;
        // the misses' ranks in position order: a contiguous run of positions per thread
        const int32_t per = (K + BT - 1) / BT;
        const int32_t k0 = tid * per, k1 = k0 + per < K ? k0 + per : K;
        int32_t cnt = 0;
        for (int32_t k = k0; k < k1; ++k) cnt += (slotOut[k] & kMissBit) ? 1 : 0;
        int32_t inc = cnt;
        for (int d = 1; d < 64; d <<= 1) {
            const int32_t o = __shfl_up(inc, d);
            if (static_cast<int>(lane) >= d) inc += o;
        }
        if (lane == 63) sScan[tid >> 6] = inc;
        __syncthreads();
        if (tid == 0) {
            int32_t run = 0;
            for (int w = 0; w < kBatchWaves; ++w) {
                const int32_t v = sScan[w];
                sScan[w] = run;
                run += v;
            }
        }
        __syncthreads();
        int32_t rank = sScan[tid >> 6] + inc - cnt;
        KVX_GM uint32_t *newk = tbl + P.t.newk;
        // 8 positions at a time: their tokens and their slots' old tokens
        // are loaded before any store (each evicted slot is named once)
        uint32_t fpd = 0;
        for (int32_t kb = k0; kb < k1; kb += 8) {
            uint32_t so[8];
            int32_t tk[8], old[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int32_t k = kb + q;
                so[q] = k < k1 ? slotOut[k] : 0u;
                tk[q] = (so[q] & kMissBit) ? rt[k] : 0;
                old[q] = (so[q] & kMissBit) ? r.tok[so[q] & 0xFFFFu] : 0;
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (!(so[q] & kMissBit)) continue;
                const uint32_t sl = so[q] & 0xFFFFu;
                newk[rank++] = ((ht_hash(tk[q]) & mask) << 16) | (sl + 1u);
                r.tok[sl] = tk[q];
                fpd += slot_token_mix(sl, tk[q]) - slot_token_mix(sl, old[q]);
            }
        }
        for (int d = 32; d > 0; d >>= 1) fpd += __shfl_xor(fpd, d);
        if (lane == 0 && fpd) atomicAdd(&sFpD, fpd);
        __syncthreads();
        if (tid == 0) {
            tbl[P.t.meta + 1] = static_cast<uint32_t>(sMisses);
            tbl[P.t.meta] = 1u;
            gHand[1] = kCanonFlag;  // the rebuild leaves the table consistent
            gHand[kFingerprintWord] = static_cast<int32_t>(sFp + sFpD);
        }
#ifdef KVX_BATCH_STAMPS
        KVX_STAMP(4);
        if (tid == 0)
            printf("stamps bid %d misses %d: check %llu decide %llu cleanup %llu handoff %llu\n", bid, sMisses,
                   (unsigned long long)(stamp[1] - stamp[0]), (unsigned long long)(stamp[2] - stamp[1]),
                   (unsigned long long)(stamp[3] - stamp[2]), (unsigned long long)(stamp[4] - stamp[3]));
#endif
        return;
    }
    if (sMisses > 0) {
        // the cells whose entries name an evicted slot, 8 cells a load
        int32_t nd = 0;
        const uint32_t nChunk = static_cast<uint32_t>(H) / 8u;
        const KVX_GM u32x4 *t16 = reinterpret_cast<const KVX_GM u32x4 *>(r.ht);
        for (uint32_t c0 = tid; c0 < nChunk; c0 += BT * kCheckUnroll) {
            u32x4 v[kCheckUnroll];
#pragma unroll
            for (int q = 0; q < kCheckUnroll; ++q) {
                const uint32_t c = c0 + static_cast<uint32_t>(q) * BT;
                if (c < nChunk) v[q] = t16[c];
            }
#pragma unroll
            for (int q = 0; q < kCheckUnroll; ++q) {
                if (c0 + static_cast<uint32_t>(q) * BT >= nChunk) continue;
                const uint32_t cb = (c0 + static_cast<uint32_t>(q) * BT) * 8u;
                const uint32_t w[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
                uint32_t m = 0u;  // the load's deleted cells
#pragma unroll
                for (int h = 0; h < 8; ++h) {
                    const uint32_t e = (w[h >> 1] >> (16 * (h & 1))) & 0xFFFFu;
                    if (e != 0u && e - 1u < static_cast<uint32_t>(dbs) && bit_get(evB, e - 1u)) m |= 1u << h;
                }
                if (m) {
                    atomicOr(reinterpret_cast<unsigned long long *>(delB + (cb >> 6)),
                             static_cast<unsigned long long>(m) << (cb & 63u));
                    nd += __builtin_popcount(m);
                }
            }
        }
        if (nd) atomicAdd(&sNdel, nd);
    }
    // the new tokens (each evicted slot gets one), 8 positions a thread at a
    // time: their tokens and their slots' old tokens loaded before any store
    {
        uint32_t fpd = 0;
        for (int32_t kb = tid; kb < K; kb += BT * 8) {
            uint32_t so[8];
            int32_t tk[8], old[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int32_t k = kb + q * BT;
                so[q] = k < K ? slotOut[k] : 0u;
                tk[q] = (so[q] & kMissBit) ? rt[k] : 0;
                old[q] = (so[q] & kMissBit) ? r.tok[so[q] & 0xFFFFu] : 0;
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                if (!(so[q] & kMissBit)) continue;
                const uint32_t sl = so[q] & 0xFFFFu;
                r.tok[sl] = tk[q];
                fpd += slot_token_mix(sl, tk[q]) - slot_token_mix(sl, old[q]);
            }
        }
        for (int d = 32; d > 0; d >>= 1) fpd += __shfl_xor(fpd, d);
        if (lane == 0 && fpd) atomicAdd(&sFpD, fpd);
    }
    for (uint32_t w = tid; w < nCellW; w += BT) bitL0[w] = 0ull;  // holes, in offsets from sE0
    for (uint32_t w = tid; w < nL1; w += BT) bitL1[w] = 0ull;
    for (uint32_t w = tid; w < nL2; w += BT) bitL2[w] = 0ull;
    __syncthreads();

    KVX_STAMP(4);
    // ---- 4. the deletions, one pass per cluster with a deleted cell ------
    // Offsets count cells from the empty cell sE0, so no cluster crosses 0.
    // The walk's state lives in LDS and only wave 0 changes it; every wave
    // stages the next chunk of cells.
    __shared__ uint32_t sCur, sClusterLo;
    __shared__ int32_t sLeft, sR;
    // The cluster's holes while they number at most 64: offsets in wave 0's
    // lanes, increasing with the lane (qmask: the lanes holding one; qend: the
    // next lane to fill); sQ packs them when the lanes run out.
    __shared__ uint32_t sQ[64];
    uint32_t qv = 0u, qend = 0u;
    uint64_t qmask = 0ull;
    bool big = false;   // the cluster's holes are in the three-level bitmap instead
    const uint32_t e0 = static_cast<uint32_t>(sE0);
    if (tid == 0) {
        sCur = 1;
        sLeft = sNdel;
        sR = -1;
        sClusterLo = 0;
    }
    for (;;) {
        // every wave reads the walk state before wave 0 changes it again
        __syncthreads();
        const bool go = sLeft > 0 || sR >= 0;
        const bool between = sR < 0;
        __syncthreads();
        if (!go) break;
        if (between && tid < 64) {
            // between clusters: skip to the next deleted cell (offset order)
            uint32_t off = sCur;
            uint32_t found = 0xFFFFFFFFu;
            while (off < static_cast<uint32_t>(H)) {
                const uint32_t cell = (e0 + off) & mask;
                uint64_t m = delB[cell >> 6] & (~0ull << (cell & 63));
                uint32_t span = 64u - (cell & 63);
                const uint32_t toEnd = static_cast<uint32_t>(H) - off;
                if (span > toEnd) {
                    m &= (1ull << ((cell & 63) + toEnd)) - 1ull;
                    span = toEnd;
                }
                if (m) {
                    found = off + static_cast<uint32_t>(__builtin_ctzll(m)) - (cell & 63);
                    break;
                }
                off += span;
            }
            if (lane == 0) {
                if (found == 0xFFFFFFFFu) {
                    sLeft = 0;  // cannot happen while deletions are left
                } else {
                    sCur = found;
                    sClusterLo = found;
                }
            }
        }
        __syncthreads();
        // wave 0 changes the state only after the staging barrier below
        if (sLeft <= 0 && sR < 0) break;
        // stage cells [chunk, chunk + kBatchStage) of the walk: entry | home << 16
        const uint32_t chunk = static_cast<uint32_t>(uniform32(static_cast<int32_t>(sCur)));
        const uint32_t chunkEnd = chunk + kBatchStage < static_cast<uint32_t>(H) ? chunk + kBatchStage
                                                                                : static_cast<uint32_t>(H);
        for (uint32_t i = tid; i < kBatchStage; i += BT) {
            const uint32_t off = chunk + i;
            uint32_t v = 0u;
            if (off < chunkEnd) {
                const uint32_t cell = (e0 + off) & mask;
                const uint32_t e = r.ht[cell];
                // the entry's home from its token (a slot past the buffer only
                // in a corrupted table: home 0)
                const uint32_t sl = e - 1u;
                const int32_t tk = (e != 0u && sl < static_cast<uint32_t>(dbs)) ? r.tok[sl] : 0;
                v = e ? (e | ((ht_hash(tk) & mask) << 16)) : 0u;
            }
            stage[i] = v;
        }
        __syncthreads();
        if (tid < 64) {
            const bool wr = lane == 0;
            bool bad = false;
            // the walk state in scalar registers (LDS values reach the wave in
            // vector registers)
            int32_t R = uniform32(sR);
            uint32_t clusterLo = static_cast<uint32_t>(uniform32(static_cast<int32_t>(sClusterLo)));
            int32_t left = uniform32(sLeft);
            uint32_t w0 = chunk;
            // wave 0's own state: uniform in the wave (the compiler cannot see
            // that past the branch on the thread index)
            qmask = uniform64(qmask);
            qend = static_cast<uint32_t>(uniform32(static_cast<int32_t>(qend)));
            big = uniform32(big ? 1 : 0) != 0;
            while ((left > 0 || R >= 0) && w0 < chunkEnd && !bad) {
                if (R < 0) {
                    // between clusters: the next deleted cell inside the chunk
                    uint32_t off = w0;
                    uint32_t found = 0xFFFFFFFFu;
                    while (off < chunkEnd) {
                        const uint32_t cell = (e0 + off) & mask;
                        uint64_t m = delB[cell >> 6] & (~0ull << (cell & 63));
                        uint32_t span = 64u - (cell & 63);
                        if (span > chunkEnd - off) {
                            m &= (1ull << ((cell & 63) + (chunkEnd - off))) - 1ull;
                            span = chunkEnd - off;
                        }
                        if (m) {
                            found = off + static_cast<uint32_t>(__builtin_ctzll(m)) - (cell & 63);
                            break;
                        }
                        off += span;
                    }
                    if (found == 0xFFFFFFFFu) {
                        w0 = chunkEnd;
                        break;
                    }
                    w0 = found;
                    clusterLo = found;
                }
                // one window of up to 64 cells from w0 (not past the chunk)
                const uint32_t off = w0 + lane;
                const bool inChunk = off < chunkEnd;
                const uint32_t v = inChunk ? stage[off - chunk] : 0u;
                const uint32_t cell = (e0 + off) & mask;
                const uint32_t e = v & 0xFFFFu;
                const bool occ = inChunk && e != 0u;
                const bool del = occ && bit_get(delB, cell);
                const uint32_t homeOff = ((v >> 16) - e0) & mask;
                const uint64_t inMask = __ballot(inChunk);
                // offset H is the empty cell e0 again: every cluster ends by then
                const uint64_t emptyM = __ballot((inChunk && !occ) || off >= static_cast<uint32_t>(H));
                const int f = emptyM ? __builtin_ctzll(emptyM) : 64;  // the cluster ends inside the window
                const uint64_t active = (f < 64 ? ((1ull << f) - 1ull) : ~0ull) & inMask;
                const uint64_t D = __ballot(del) & active;
                const uint64_t S = __ballot(occ && !del) & active;  // entries that stay unless they move
                // The events in cell order: a deleted cell, or an entry whose
                // home is at or before the rightmost hole (the last event).  A
                // deletion makes a hole; a mover takes the leftmost hole at or
                // after its home and leaves a hole.  Each event is found with one
                // ballot; the moves are recorded per lane and written after the
                // window.
                const uint64_t below = (1ull << lane) - 1ull;
                uint64_t rem = active, E = 0ull, Mv = 0ull, taken = 0ull;
                uint32_t tgt = 0u;
                if (!big && R >= 0 && D == 0ull) {
                    // A window without deletions: the events are found in
                    // parallel (each lane's previous event from the events so
                    // far, grown to a fixpoint: an entry is an event iff its
                    // home is at or before the previous event, so the set only
                    // grows and each round adds the first one missing).  If no
                    // mover's home reaches an older hole, each takes the hole
                    // its previous event left (the rightmost one), all at once.
                    const uint64_t older = qmask & ~(1ull << (qend - 1u));  // lane qend-1 holds R
                    const int32_t R2 = older ? lane_value(static_cast<int32_t>(qv), 63 - __builtin_clzll(older)) : -1;
                    uint64_t Ef = 0ull;
                    uint32_t prev = static_cast<uint32_t>(R);
                    for (int it = 0; it <= 64; ++it) {
                        const uint64_t bl = Ef & below;
                        prev = bl ? w0 + 63u - static_cast<uint32_t>(__builtin_clzll(bl)) : static_cast<uint32_t>(R);
                        const uint64_t E2 = uniform64(Ef | (__ballot(homeOff <= prev) & S));
                        if (E2 == Ef) break;
                        Ef = E2;
                    }
                    const bool olderReached = __ballot(((Ef >> lane) & 1ull) && R2 >= 0 &&
                                                       static_cast<int32_t>(homeOff) <= R2) != 0ull;
                    if (!olderReached) {
                        if (Ef) {
                            const int last = 63 - __builtin_clzll(Ef);
                            E = Mv = Ef;
                            taken = Ef & ~(1ull << last);  // each event's cell is taken by the next one
                            tgt = prev;
                            R = static_cast<int32_t>(w0 + static_cast<uint32_t>(last));
                            qv = static_cast<uint32_t>(lane_set(static_cast<int32_t>(qv), static_cast<int32_t>(qend - 1u), R));
                        }
                        rem = 0ull;  // nothing left for the one-at-a-time loop
                    } else if (qend + static_cast<uint32_t>(__builtin_popcountll(Ef)) <= 64u) {
                        // the events are known; only the holes go in order: each
                        // mover takes the leftmost hole at or after its home from
                        // the lanes and its cell joins them
                        for (uint64_t ev = Ef; ev; ev &= ev - 1ull) {
                            const int j = __builtin_ctzll(ev);
                            const uint32_t h = static_cast<uint32_t>(lane_value(static_cast<int32_t>(homeOff), j));
                            const uint64_t m = uniform64(__ballot(qv >= h) & qmask);
                            if (!m) {
                                bad = true;  // the rightmost hole is at or after the home: only a broken invariant
                                break;
                            }
                            const int t = __builtin_ctzll(m);
                            const uint32_t hole = static_cast<uint32_t>(lane_value(static_cast<int32_t>(qv), t));
                            qmask &= ~(1ull << t);
                            tgt = static_cast<uint32_t>(lane_set(static_cast<int32_t>(tgt), j, static_cast<int32_t>(hole)));
                            if (hole >= w0) taken |= 1ull << (hole - w0);
                            const uint32_t offJ = w0 + static_cast<uint32_t>(j);
                            qv = static_cast<uint32_t>(lane_set(static_cast<int32_t>(qv), static_cast<int32_t>(qend),
                                                                static_cast<int32_t>(offJ)));
                            qmask |= 1ull << qend;
                            ++qend;
                            Mv |= 1ull << j;
                            E |= 1ull << j;
                            R = static_cast<int32_t>(offJ);
                        }
                        rem = 0ull;
                    }
                }
                for (;;) {
                    const uint64_t reach = R >= 0 ? __ballot(homeOff <= static_cast<uint32_t>(R)) & S : 0ull;
                    const uint64_t cand = uniform64((D | reach) & rem);
                    if (!cand) break;
                    const int j = __builtin_ctzll(cand);
                    rem &= ~((2ull << j) - 1ull);
                    const uint32_t offJ = w0 + static_cast<uint32_t>(j);
                    if ((D >> j) & 1ull) {
                        --left;
                    } else {
                        const uint32_t h = static_cast<uint32_t>(lane_value(static_cast<int32_t>(homeOff), j));
                        uint32_t hole = 0xFFFFFFFFu;  // none
                        if (__builtin_expect(!big, 1)) {
                            const uint64_t m = __ballot(qv >= h) & qmask;
                            if (m) {
                                const int t = __builtin_ctzll(m);
                                hole = static_cast<uint32_t>(lane_value(static_cast<int32_t>(qv), t));
                                qmask &= ~(1ull << t);
                            }
                        } else {
                            // (a scalar like the lanes' hole, so both stay in scalar registers)
                            const int32_t x = uniform32(static_cast<int32_t>(next_set(bits, h)));
                            if (x >= 0 && static_cast<uint32_t>(x) < offJ) {
                                hole = static_cast<uint32_t>(x);
                                clr_bit3(bits, hole, wr);
                            }
                        }
                        if (hole >= offJ) {
                            bad = true;  // not reachable by the move rule; reported, nothing written
                            break;
                        }
                        tgt = static_cast<uint32_t>(lane_set(static_cast<int32_t>(tgt), j, static_cast<int32_t>(hole)));
                        Mv |= 1ull << j;
                        if (hole >= w0) taken |= 1ull << (hole - w0);
                    }
                    E |= 1ull << j;
                    R = static_cast<int32_t>(offJ);
                    // offJ is a hole now
                    if (__builtin_expect(!big && qend < 64u, 1)) {
                        qv = static_cast<uint32_t>(lane_set(static_cast<int32_t>(qv), static_cast<int32_t>(qend),
                                                            static_cast<int32_t>(offJ)));
                        qmask |= 1ull << qend;
                        ++qend;
                        continue;
                    }
                    if (!big) {
                        // the queue's lanes are used up: pack the holes to the
                        // front, or with 64 holes keep the rest of the cluster's
                        // holes in the bitmap
                        const uint32_t n = static_cast<uint32_t>(__builtin_popcountll(qmask));
                        if (n < 64u) {
                            if ((qmask >> lane) & 1ull) sQ[__builtin_popcountll(qmask & below)] = qv;
                            qv = sQ[lane];
                            qmask = n ? (~0ull >> (64u - n)) : 0ull;
                            qv = static_cast<uint32_t>(lane_set(static_cast<int32_t>(qv), static_cast<int32_t>(n),
                                                                static_cast<int32_t>(offJ)));
                            qmask |= 1ull << n;
                            qend = n + 1u;
                            continue;
                        }
                        // every lane holds a hole (an offset below H)
                        const uint32_t w = qv >> 6, v1 = w >> 6;
                        atomicOr(reinterpret_cast<unsigned long long *>(bitL0 + w), 1ull << (qv & 63u));
                        atomicOr(reinterpret_cast<unsigned long long *>(bitL1 + v1), 1ull << (w & 63u));
                        atomicOr(reinterpret_cast<unsigned long long *>(bitL2 + (v1 >> 6)), 1ull << (v1 & 63u));
                        big = true;
                    }
                    set_bit3(bits, offJ, wr);
                }
                if ((Mv >> lane) & 1ull) r.ht[(e0 + tgt) & mask] = static_cast<uint16_t>(e);
                if (((E & ~taken) >> lane) & 1ull) r.ht[cell] = 0;  // a hole no mover of the window took
                if (f < 64) {
                    // the cluster ends at w0 + f: its remaining holes stay empty
                    const uint32_t hi = w0 + static_cast<uint32_t>(f);
                    const uint32_t top = hi < static_cast<uint32_t>(H) ? hi : static_cast<uint32_t>(H) - 1u;
                    if (big) {
                        for (uint32_t w = (clusterLo >> 6) + lane; w <= (top >> 6); w += 64) bitL0[w] = 0ull;
                        for (uint32_t w = (clusterLo >> 12) + lane; w <= (top >> 12); w += 64) bitL1[w] = 0ull;
                        for (uint32_t w = (clusterLo >> 18) + lane; w <= (top >> 18); w += 64) bitL2[w] = 0ull;
                    }
                    R = -1;
                    qmask = 0ull;
                    qend = 0u;
                    big = false;
                    w0 = hi + 1u;
                } else {
                    w0 = w0 + 64u < chunkEnd ? w0 + 64u : chunkEnd;  // the next window starts inside the stage
                }
            }
            if (bad) {
                // a broken invariant: stop the walk (the row's table is left
                // partly updated) and report it in the tail slot
                R = -1;
                left = 0;
                if (wr) report_overflow(P.L.overflowSlot, kOverflowProbe);
                sTableBad = 1;
            }
            if (wr) {
                sCur = w0;
                sR = R;
                sClusterLo = clusterLo;
                sLeft = left;
            }
        }
    }
    __threadfence_block();
    __syncthreads();

    KVX_STAMP(5);
    // ---- 5. the new tokens, in position order ----------------------------
    if (sMisses == 0) {
        if (tid == 0) {  // nothing to insert
            gHand[1] = sTableBad ? 0 : kCanonFlag;
            gHand[kFingerprintWord] = static_cast<int32_t>(sFp);
        }
        return;
    }
    for (uint32_t w = tid; w < nCellW; w += BT) {
        // the empty cells of 64 cells, 8 cells a load
        uint64_t m = 0ull;
        const KVX_GM u32x4 *t16 = reinterpret_cast<const KVX_GM u32x4 *>(r.ht + (w << 6));
        u32x4 v[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) v[q] = t16[q];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint32_t x[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                if ((x[h] & 0xFFFFu) == 0u) m |= 1ull << (8 * q + 2 * h);
                if ((x[h] >> 16) == 0u) m |= 1ull << (8 * q + 2 * h + 1);
            }
        }
        bitL0[w] = m;
    }
    __syncthreads();
    for (uint32_t w = tid; w < nL1; w += BT) {
        uint64_t sm = 0ull;
        for (uint32_t q = 0; q < 64 && (w << 6) + q < nCellW; ++q) {
            if (bitL0[(w << 6) + q]) sm |= 1ull << q;
        }
        bitL1[w] = sm;
    }
    __syncthreads();
    for (uint32_t w = tid; w < nL2; w += BT) {
        uint64_t sm = 0ull;
        for (uint32_t q = 0; q < 64 && (w << 6) + q < nL1; ++q) {
            if (bitL1[(w << 6) + q]) sm |= 1ull << q;
        }
        bitL2[w] = sm;
    }
    __syncthreads();
    if (tid < 64) {
        const bool wr = lane == 0;
        for (int32_t k0 = 0; k0 < K; k0 += 64) {
            const int32_t k = k0 + static_cast<int32_t>(lane);
            const bool in = k < K;
            const uint32_t s = in ? slotOut[k] : 0u;
            const bool miss = (s & kMissBit) != 0u;
            const int32_t t = miss ? rt[k] : 0;
            uint64_t mm = __ballot(miss);
            while (mm) {
                const int i = __builtin_ctzll(mm);
                mm &= mm - 1ull;
                const int32_t ti = lane_value(t, i);
                const uint32_t si = static_cast<uint32_t>(lane_value(static_cast<int32_t>(s), i)) & 0xFFFFu;
                const uint32_t home = ht_hash(ti) & mask;
                int64_t x = next_set(bits, home);
                if (x < 0) x = next_set(bits, 0u);
                if (x < 0) {
                    if (wr) report_overflow(P.L.overflowSlot, kOverflowProbe);  // a full table: not reachable
                    sTableBad = 1;
                    continue;
                }
                clr_bit3(bits, static_cast<uint32_t>(x), wr);
                if (wr) r.ht[x] = static_cast<uint16_t>(si + 1u);
            }
        }
        // the row's table is consistent with its tokens unless a bound broke
        if (wr) {
            gHand[1] = sTableBad ? 0 : kCanonFlag;
            gHand[kFingerprintWord] = static_cast<int32_t>(sFp + sFpD);
        }
#ifdef KVX_BATCH_STAMPS
        KVX_STAMP(6);
        if (tid == 0)
            printf("stamps bid %d misses %d ndel %d: check %llu decide %llu cleanup %llu outputs %llu deletions %llu "
                   "inserts %llu\n",
                   bid, sMisses, sNdel, (unsigned long long)(stamp[1] - stamp[0]),
                   (unsigned long long)(stamp[2] - stamp[1]), (unsigned long long)(stamp[3] - stamp[2]),
                   (unsigned long long)(stamp[4] - stamp[3]), (unsigned long long)(stamp[5] - stamp[4]),
                   (unsigned long long)(stamp[6] - stamp[5]));
#endif
    }
}

}  // namespace

hipError_t sieve_batch_set_lds_limit(size_t bytes)
{
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update_batch),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_sieve_update_batch(const HispSieveUpdateArgs &a, uint64_t overflowSlot, int32_t *shadow,
                                     uint32_t *aux, uint32_t *tbl, hipStream_t stream)
{
    BatchParams P{};
    P.L = KvxLaunch<HispSieveUpdateArgs>{a, overflowSlot};
    P.shadow = shadow;
    P.aux = aux;
    P.mapCap = kBatchMapCap;
    P.auxWords = batch_aux_words(a.htSize);
    P.lay = batch_layout(a.deviceBufferSize, a.htSize, a.topK);
    P.tbl = tbl;
    P.t = table_layout(a.htSize);
    hipLaunchKernelGGL(kvx_sieve_batch_pre, dim3(kPreSplit, a.maxNumReqs), dim3(kPreThreads), 0, stream, P);
    hipLaunchKernelGGL(kvx_sieve_batch_slots, dim3(kPreSplit, a.maxNumReqs), dim3(kPreThreads), 0, stream, P);
    hipLaunchKernelGGL(kvx_sieve_update_batch, dim3(a.maxNumReqs), dim3(BT), P.lay.total, stream, P);
    if (tbl != nullptr) {
        const hipError_t err = hipGetLastError();
        if (err != hipSuccess) return err;
        return launch_sieve_table_rebuild(a, overflowSlot, tbl, stream);
    }
    return hipGetLastError();
}

}  // namespace kvx
