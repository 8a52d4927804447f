// SIEVE (ring CLOCK) update, parallel decomposition for gfx950.
//
// Same results as the sequential recurrence of hisp_sieve_update.cpp:115-163
// (slots, is_miss, tokens, visited bitmap, hand and the hash table's exact
// layout), computed by one 1024-lane workgroup per batch row with the state
// row staged in LDS.
//
// Events are the positions that need a slot: the first occurrence of each
// token that is not resident (a candidate miss), and every hit whose token
// the hand evicted earlier in the same step (a conversion).  Within one step
// the hand passes each slot at most once (a wrap falls back), so a slot's fate
// depends only on its class:
//   S0  visited before the step: passed;
//   SN  not visited and not hit this step: evicted by the event the hand
//       serves when it arrives;
//   SM  not visited, first hit at position k: evicted iff the hand arrives
//       while serving an event earlier than k (then the hit at k converts).
// With j(u) = the number of evictions before ring offset u, the hand reaches
// u while serving event j(u), and an SM slot is evicted iff more than j(u)
// events precede k.  Events before k are the candidates before k (a prefix
// count) plus the conversions made so far, so only the SM slots need a
// sequential pass, and it touches nothing but counters.  Everything else --
// classification, dedup, the event sequence, marks, outputs, visited bits --
// is prefix sums and scatters.
//
// Phases:
//   stage    tokens/table/visited/topK row into LDS; table consistency check
//   classify hit / candidate / invalid / decode-extension per position; the
//            first hit time of every slot (LDS min)
//   dedup    provisional table entries padded+1+k, smallest k wins
//   compact  candidate prefix counts per position
//   ring     classes per ring offset from the hand, SM list with its counts
//   decide   one wave: SM slots in ring order, 64 at a time, speculating that
//            none is evicted and correcting at each eviction
//   events   the merged event sequence (a prefix scan over positions)
//   marks    per ring offset: evicted at event p / passed at event p
//   outputs  slots, is_miss, visited bits
//   table    erase the evicted tokens (Algorithm R deletions commute when
//            each cluster is done right to left), insert the new tokens with
//            a tentative parallel placement (the occupied cells do not depend
//            on order) and redo, in event order, every final cluster that
//            holds more than one new token.  Linear probing with Algorithm R
//            leaves the table equal to inserting the live keys in insertion
//            order, so the result is the sequential table byte for byte.
//
// Preconditions, checked in the kernel: the table indexes exactly the
// non-negative tokens of slots [0, dbs) (each found at its own slot),
// padded + 1 + topK <= 65535, topK < 16383, no hand wrap within the step.
// Otherwise the row is restaged from HBM and the sequential recurrence runs.
#include "kvx_internal.h"
#include "sieve_common.h"

namespace kvx {
namespace {

using namespace sieve;

constexpr int NT = kFastThreads;
constexpr int NWAVES = NT / 64;

constexpr uint32_t CLS_INV = 0u, CLS_EXT = 1u, CLS_HIT = 2u, CLS_CAND = 3u;
constexpr uint16_t VT_NONE = 0xFFFF, VT_EVICTED = 0x8000, VT_PASSED = 0x4000, VT_NOCONV = 0x3FFF;
// sieve_hand[row][1]: set when this kernel left the row's table consistent
constexpr int32_t kCanonFlag = 0x4B565843;

// Phase timestamps for profiling builds (-DKVX_SIEVE_PHASE_STAMPS): thread 0
// of each workgroup records clock64() at phase boundaries into kvx_dbg_stamps.
#ifdef KVX_SIEVE_PHASE_STAMPS
__device__ unsigned long long kvx_dbg_stamps[1024][16];
#define STAMP(i)                                                        \
    do {                                                                \
        if (tid == 0 && bid < 1024) kvx_dbg_stamps[bid][i] = clock64(); \
    } while (0)
__device__ unsigned long long kvx_dbg_sub[1024][16];
#define SUBSTAMP(i)                                                   \
    do {                                                              \
        if (tid == 0 && bid < 1024) kvx_dbg_sub[bid][i] = clock64();  \
    } while (0)
#else
#define STAMP(i) \
    do {         \
    } while (0)
#define SUBSTAMP(i) \
    do {            \
    } while (0)
#endif

struct Misc {
    int32_t nTok, nEnt, bad, ovf, late;
    int32_t M, nSM, T, nConv, N, nUnd, nRest, uEnd, nTakes, nMulti;
    uint32_t wt0[NWAVES];
    uint32_t wt1[NWAVES];
};

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t lanes_below(uint64_t m, uint32_t lane)
{
    return static_cast<uint32_t>(__popcll(m & ((1ull << lane) - 1ull)));
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += static_cast<uint32_t>(__shfl_xor(static_cast<int>(v), o));
    return v;
}

// Exclusive prefix over the workgroup of per-thread values whose set bits all
// lie in `bits` (small counts: one ballot per bit), in thread order.  Returns
// the prefix and the total.  `wt` is read after the call returns: the next
// use of the same `wt` must come after another barrier.
__device__ __forceinline__ uint32_t block_exscan(uint32_t v, uint32_t bits, uint32_t *wt, uint32_t &total)
{
    const uint32_t lane = lane_id();
    const int wave = static_cast<int>(threadIdx.x >> 6);
    uint32_t pre = 0, tot = 0;
    while (bits != 0u) {
        const int b = __builtin_ctz(bits);
        bits &= bits - 1u;
        const uint64_t bal = __ballot((v >> b) & 1u);
        pre += lanes_below(bal, lane) << b;
        tot += static_cast<uint32_t>(__popcll(bal)) << b;
    }
    if (lane == 0) wt[wave] = tot;
    __syncthreads();
    uint32_t off = 0, all = 0;
#pragma unroll
    for (int w = 0; w < NWAVES; ++w) {
        const uint32_t c = wt[w];
        off += (w < wave) ? c : 0u;
        all += c;
    }
    total = all;
    return off + pre;
}

// Bit mask covering the values 0..n.
__host__ __device__ __forceinline__ uint32_t bits_for(uint32_t n)
{
    uint32_t m = 1u;
    while (m < n + 1u && m != 0x80000000u) m = (m << 1) | 1u;
    return m;
}

// 16-bit LDS min via a CAS on the containing word.
__device__ __forceinline__ void lds_min16(uint32_t *w32, uint32_t i, uint16_t v)
{
    uint32_t *w = w32 + (i >> 1);
    const uint32_t sh = (i & 1u) * 16u;
    uint32_t old = *reinterpret_cast<volatile uint32_t *>(w);
    for (;;) {
        const uint32_t cur = (old >> sh) & 0xFFFFu;
        if (cur <= v) return;
        const uint32_t nw = (old & ~(0xFFFFu << sh)) | (static_cast<uint32_t>(v) << sh);
        const uint32_t prev = atomicCAS(w, old, nw);
        if (prev == old) return;
        old = prev;
    }
}

// Claim the first empty cell at or after `idx` with value v (16-bit cells,
// CAS on words).  Returns the cell, or -1 after a whole-table probe.
__device__ __forceinline__ int32_t lds_claim16(uint32_t *w32, int32_t idx, int32_t mask, uint16_t v)
{
    for (int32_t n = 0; n <= mask; ++n) {
        uint32_t *w = w32 + (idx >> 1);
        const uint32_t sh = (static_cast<uint32_t>(idx) & 1u) * 16u;
        uint32_t old = *reinterpret_cast<volatile uint32_t *>(w);
        for (;;) {
            if (((old >> sh) & 0xFFFFu) != 0u) break;
            const uint32_t prev = atomicCAS(w, old, old | (static_cast<uint32_t>(v) << sh));
            if (prev == old) return idx;
            old = prev;
        }
        idx = (idx + 1) & mask;
    }
    return -1;
}

__device__ __forceinline__ bool bit_get(const uint32_t *b, uint32_t i) { return (b[i >> 5] >> (i & 31u)) & 1u; }

// Algorithm R deletion of the entry at cell c (homes from the tokens row, or
// from the per-slot token hashes in the compact form).
template <bool kC>
__device__ void rdel_at(uint16_t *ht, const void *tokv, int32_t ntok, int32_t c, int32_t mask, Guard &g)
{
    int32_t j = c, i = c;
    for (int32_t n = 0;; ++n) {
        if (n > mask) {
            g.code = kOverflowProbe;
            return;
        }
        i = (i + 1) & mask;
        const uint16_t e = ht[i];
        if (e == 0) break;
        int32_t home;
        if constexpr (kC) {
            const uint16_t *hv = static_cast<const uint16_t *>(tokv);
            home = static_cast<int32_t>((static_cast<int32_t>(e) - 1 < ntok) ? hv[e - 1u] : ht_hash(-1)) & mask;
        } else {
            home = static_cast<int32_t>(ht_hash(tok_at(static_cast<const int32_t *>(tokv), e, ntok))) & mask;
        }
        const bool move = (j < i) ? (home <= j || home > i) : (home <= j && home > i);
        if (move) {
            ht[j] = e;
            j = i;
        }
    }
    ht[j] = 0;
}

// Copy n bytes (multiple of 16) with the workgroup, four 16-byte chunks in
// flight per lane.
__device__ __forceinline__ void wg_copy16(void *dst, const void *src, uint32_t n)
{
    const uint4 *s = static_cast<const uint4 *>(src);
    uint4 *d = static_cast<uint4 *>(dst);
    const uint32_t n16 = n / 16u;
    uint32_t i = threadIdx.x;
    for (; i + 3u * NT < n16; i += 4u * NT) {
        const uint4 a = s[i];
        const uint4 b = s[i + NT];
        const uint4 c = s[i + 2u * NT];
        const uint4 e = s[i + 3u * NT];
        d[i] = a;
        d[i + NT] = b;
        d[i + 2u * NT] = c;
        d[i + 3u * NT] = e;
    }
    for (; i < n16; i += NT) d[i] = s[i];
}

__device__ __forceinline__ int32_t ring_slot(int32_t hand0, int32_t u, int32_t dbs)
{
    const int32_t s = hand0 + u;
    return s >= dbs ? s - dbs : s;
}

template <bool kC>
__global__ __launch_bounds__(NT) void kvx_sieve_update_fast(KvxLaunch<HispSieveUpdateArgs> L)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ Misc ms;
    const HispSieveUpdateArgs &a = L.a;
    const int32_t K = static_cast<int32_t>(a.topK);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t visStrideB = static_cast<int32_t>(a.visitedStrideB);
    const int32_t maxNumReqs = static_cast<int32_t>(a.maxNumReqs);
    const int32_t H = static_cast<int32_t>(a.htSize);
    const int32_t mask = H - 1;
    const int32_t poolSize = static_cast<int32_t>(a.poolSize);
    const int32_t bid = blockIdx.x;
    const int32_t tid = threadIdx.x;
    const uint32_t lane = lane_id();
    const int32_t wave = tid >> 6;
    if (bid >= maxNumReqs) return;

    int32_t numReal = *reinterpret_cast<const int32_t *>(a.numReal);
    if (numReal > maxNumReqs) numReal = maxNumReqs;  // hisp_sieve_update.cpp:31-34
    int32_t *rs = reinterpret_cast<int32_t *>(a.topKDeviceSlots) + static_cast<int64_t>(bid) * K;
    int8_t *rm = reinterpret_cast<int8_t *>(a.isMiss) + static_cast<int64_t>(bid) * K;
    if (bid >= numReal) {
        write_dummy_row(rs, rm, K);
        return;
    }
    const int64_t reqIdx = reinterpret_cast<const int64_t *>(a.reqPoolIndices)[bid];
    if (reqIdx < 0 || reqIdx >= poolSize) {
        write_dummy_row(rs, rm, K);
        return;
    }
    const int32_t seqLen = reinterpret_cast<const int32_t *>(a.seqLens)[bid];
    const int32_t prefill = reinterpret_cast<const int32_t *>(a.prefillLens)[reqIdx];
    const int32_t *rt = reinterpret_cast<const int32_t *>(a.topkIndices) + static_cast<int64_t>(bid) * K;
    int32_t *gTok = reinterpret_cast<int32_t *>(a.deviceBufferTokens) + reqIdx * padded;
    uint8_t *gVis = reinterpret_cast<uint8_t *>(a.deviceBufferVisited) + reqIdx * visStrideB;
    uint16_t *gHt = reinterpret_cast<uint16_t *>(a.deviceBufferHt) + reqIdx * H;
    int32_t *gHand = reinterpret_cast<int32_t *>(a.sieveHand) + reqIdx * kHandStride;

    const FastLayout lay = fast_layout(padded, H, K, visStrideB, kC);
    int32_t *tok = reinterpret_cast<int32_t *>(smem + lay.tok);    // full form: tokens
    uint16_t *hv = reinterpret_cast<uint16_t *>(smem + lay.tok);   // compact form: token hashes
    // token of slot s equals t (th = its hash); the compact form checks the
    // hash in LDS and confirms with the HBM row
    auto tok_is = [&](uint32_t s, int32_t t, uint32_t th) -> bool {
        if constexpr (kC) return hv[s] == th && gTok[s] == t;
        else return tok[s] == t;
    };
    auto tok_hash = [&](uint32_t s) -> uint32_t {
        if constexpr (kC) return hv[s];
        else return ht_hash(tok[s]);
    };
    uint16_t *ht = reinterpret_cast<uint16_t *>(smem + lay.ht);
    uint32_t *ht32 = reinterpret_cast<uint32_t *>(smem + lay.ht);
    uint8_t *vis = smem + lay.vis;
    uint32_t *vis32 = reinterpret_cast<uint32_t *>(smem + lay.vis);
    int32_t *ptok = reinterpret_cast<int32_t *>(smem + lay.ptok);
    uint32_t *pinf = reinterpret_cast<uint32_t *>(smem + lay.pinf);
    uint16_t *vt = reinterpret_cast<uint16_t *>(smem + lay.vt);
    uint32_t *vt32 = reinterpret_cast<uint32_t *>(smem + lay.vt);
    uint16_t *candPre = reinterpret_cast<uint16_t *>(smem + lay.candPre);
    uint16_t *evslot = reinterpret_cast<uint16_t *>(smem + lay.evslot);
    uint16_t *evold = reinterpret_cast<uint16_t *>(smem + lay.evold);
    uint16_t *smKp = reinterpret_cast<uint16_t *>(smem + lay.cvlist);  // k of SM slots that can be evicted, else 0
    uint16_t *eseq = reinterpret_cast<uint16_t *>(smem + lay.eseq);
    uint16_t *tb = reinterpret_cast<uint16_t *>(smem + lay.tb);
    uint32_t *smA = reinterpret_cast<uint32_t *>(smem + lay.smA);  // ring offset | k << 16
    uint32_t *smB = reinterpret_cast<uint32_t *>(smem + lay.smB);  // SN before | candidates before k << 16
    uint32_t *kst = reinterpret_cast<uint32_t *>(smem + lay.kst);
    uint32_t *vset = reinterpret_cast<uint32_t *>(smem + lay.vset);
    uint32_t *ber = reinterpret_cast<uint32_t *>(smem + lay.ber);
    uint32_t *bg = reinterpret_cast<uint32_t *>(smem + lay.bg);
    uint32_t *bm = reinterpret_cast<uint32_t *>(smem + lay.bm);
    uint32_t *bnew = reinterpret_cast<uint32_t *>(smem + lay.bnew);
    // direct token -> slot map for rows whose prefill fits the LDS left over
    // (after the layout): 0 = not resident, slot+1 when resident,
    // padded+1+k for a candidate's first position k
    const int32_t invCap = static_cast<int32_t>(a.reserved >> 8);
    const bool direct = !kC && prefill > 0 && prefill <= invCap;
    uint16_t *inv = reinterpret_cast<uint16_t *>(smem + lay.total);
    uint32_t *inv32 = reinterpret_cast<uint32_t *>(smem + lay.total);
    // reuse of regions whose earlier contents are dead by then
    uint32_t *pcell = smA;                                             // dedup: provisional cell per position
    uint16_t *posSM = evslot;                                          // decide: SM index + 1 per first-hit position
    uint32_t *undl = kst;                                              // decide: undecided SM indices
    uint32_t *ecell = smA;                                             // table: erase cell (| leader bit) per event
    uint32_t *ntokv = smB;                                             // table: new token per event
    uint64_t *mlist = reinterpret_cast<uint64_t *>(smem + lay.ptok);  // multi-cluster keys
    uint64_t *msort = reinterpret_cast<uint64_t *>(smem + lay.smA);   // the same, sorted

    // ---- stage the state row and the topK row; count live tokens and table entries
    STAMP(0);
    int32_t hand0 = gHand[0];
    if (hand0 < 0 || hand0 >= dbs) hand0 = 0;  // hisp_sieve_update.cpp:108-111
    const bool flagged = gHand[1] == kCanonFlag;
    {
        const int32_t nt = padded >> 2, nh = H >> 3, nv = visStrideB >> 4;  // 16-byte chunks
        const int32_t nAll = nt + nh + nv;
        const uint4 *sT = reinterpret_cast<const uint4 *>(gTok);
        const uint4 *sH = reinterpret_cast<const uint4 *>(gHt);
        const uint4 *sV = reinterpret_cast<const uint4 *>(gVis);
        uint32_t nTok = 0, nEnt = 0;
        int32_t t0 = 0, t1 = 0;
        const bool h0 = tid < K, h1 = tid + NT < K;
        if (h0) t0 = rt[tid];
        if (h1) t1 = rt[tid + NT];
        for (int32_t c0 = tid; c0 < nAll; c0 += 4 * NT) {
            uint4 v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int32_t c = c0 + j * NT;
                if (c < nt) v[j] = sT[c];
                else if (c < nt + nh) v[j] = sH[c - nt];
                else if (c < nAll) v[j] = sV[c - nt - nh];
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int32_t c = c0 + j * NT;
                if (c < nt) {
                    if constexpr (kC) {
                        const uint32_t a0 = ht_hash(static_cast<int32_t>(v[j].x)), a1 = ht_hash(static_cast<int32_t>(v[j].y));
                        const uint32_t a2 = ht_hash(static_cast<int32_t>(v[j].z)), a3 = ht_hash(static_cast<int32_t>(v[j].w));
                        reinterpret_cast<uint2 *>(hv)[c] = make_uint2(a0 | (a1 << 16), a2 | (a3 << 16));
                    } else {
                        reinterpret_cast<uint4 *>(tok)[c] = v[j];
                    }
                    const int32_t s0 = c * 4;
                    nTok += (s0 < dbs && static_cast<int32_t>(v[j].x) >= 0) + (s0 + 1 < dbs && static_cast<int32_t>(v[j].y) >= 0) +
                            (s0 + 2 < dbs && static_cast<int32_t>(v[j].z) >= 0) + (s0 + 3 < dbs && static_cast<int32_t>(v[j].w) >= 0);
                } else if (c < nt + nh) {
                    reinterpret_cast<uint4 *>(ht)[c - nt] = v[j];
                    const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) nEnt += ((w4[q] & 0xFFFFu) != 0u) + ((w4[q] >> 16) != 0u);
                } else if (c < nAll) {
                    reinterpret_cast<uint4 *>(vis)[c - nt - nh] = v[j];
                }
            }
        }
        SUBSTAMP(4);
        if (h0) ptok[tid] = t0;
        if (h1) ptok[tid + NT] = t1;
        for (int32_t k = tid + 2 * NT; k < K; k += NT) ptok[k] = rt[k];
        // vset (and in the full form ber, bg, bm, bnew) are contiguous
        const int32_t nz = (visStrideB >> 2) + (kC ? 0 : 4 * (H >> 5));
        for (int32_t i = tid; i < nz; i += NT) vset[i] = 0u;
        for (int32_t k = tid; k < K; k += NT) evslot[k] = 0;  // SM index + 1 by first-hit position
        if (direct) {
            for (int32_t i = tid; i < (prefill + 1) >> 1; i += NT) inv32[i] = 0u;
        }
        nTok = wave_sum(nTok);
        nEnt = wave_sum(nEnt);
        if (tid == 0) {
            ms.nTok = ms.nEnt = ms.bad = ms.ovf = ms.late = 0;
            ms.M = ms.nSM = ms.T = ms.nConv = ms.N = ms.nUnd = ms.nRest = ms.uEnd = ms.nTakes = ms.nMulti = 0;
        }
        __syncthreads();
        if (lane == 0) {
            atomicAdd(&ms.nTok, static_cast<int32_t>(nTok));
            atomicAdd(&ms.nEnt, static_cast<int32_t>(nEnt));
        }
    }
    STAMP(1);

    // ---- consistency: the table indexes exactly the non-negative tokens of
    // [0, dbs), each at its own slot.  A row this kernel wrote last carries
    // the flag, and then only the counts are checked.
    for (int32_t s = tid; s < dbs; s += NT) {
        vt[s] = vis_get(vis, s) ? 0 : VT_NONE;
        if (direct) {
            const int32_t t = tok[s];
            if (t >= 0 && t < prefill) inv[t] = static_cast<uint16_t>(s + 1);
        }
    }
    if (!flagged) {
        Guard g;
        bool bad = false;
        for (int32_t s = tid; s < dbs; s += NT) {
            const int32_t t = kC ? gTok[s] : tok[s];
            if (t < 0) continue;
            const uint32_t th = ht_hash(t);
            int32_t idx = static_cast<int32_t>(th) & mask, found = -1;
            for (int32_t n = 0; n <= mask; ++n) {
                const uint16_t e = ht[idx];
                if (e == 0) break;
                if (static_cast<int32_t>(e) - 1 < padded && tok_is(e - 1u, t, th)) {
                    found = static_cast<int32_t>(e) - 1;
                    break;
                }
                idx = (idx + 1) & mask;
            }
            if (found != s) bad = true;
        }
        if (__ballot(bad || g.code != 0) != 0ull && lane == 0) atomicOr(&ms.bad, 1);
    }
    __syncthreads();
    const bool canonical = ms.bad == 0 && ms.nTok == ms.nEnt;
    bool fast = canonical;
    STAMP(2);

    if (fast) {
        // ---- classify every position and deduplicate the candidates in one
        // probe: a hit stops at its entry (provisional entries only fill empty
        // cells, never the probe path of a resident token); a miss stops at
        // its token's provisional entry padded+1+k (smallest k wins) or claims
        // the first empty cell with one
        {
            Guard g;
            for (int32_t k = tid; k < K; k += NT) {
                const int32_t t = ptok[k];
                uint32_t inf;
                if (t < 0 || t >= seqLen) {
                    inf = CLS_INV << 30;
                } else if (t >= prefill) {
                    inf = CLS_EXT << 30;
                } else if (direct) {
                    const uint32_t v = static_cast<uint32_t>(padded + 1 + k);
                    uint32_t *w = inv32 + (t >> 1);
                    const uint32_t sh = (static_cast<uint32_t>(t) & 1u) * 16u;
                    uint32_t old = *reinterpret_cast<volatile uint32_t *>(w);
                    const uint32_t e0 = (old >> sh) & 0xFFFFu;
                    if (e0 != 0u && e0 <= static_cast<uint32_t>(padded)) {
                        inf = (CLS_HIT << 30) | (e0 - 1u);
                        lds_min16(vt32, e0 - 1u, static_cast<uint16_t>(k + 1));
                    } else {
                        inf = CLS_CAND << 30;
                        for (;;) {  // keep the smallest position of the token
                            const uint32_t cur = (old >> sh) & 0xFFFFu;
                            if (cur != 0u && cur <= v) break;
                            const uint32_t prev = atomicCAS(w, old, (old & ~(0xFFFFu << sh)) | (v << sh));
                            if (prev == old) break;
                            old = prev;
                        }
                    }
                } else {
                    const uint32_t v = static_cast<uint32_t>(padded + 1 + k);
                    const uint32_t th = ht_hash(t);
                    int32_t idx = static_cast<int32_t>(th) & mask;
                    inf = 0xFFFFFFFFu;
                    for (int32_t n = 0; n <= mask; ++n) {
                        uint32_t *w = ht32 + (idx >> 1);
                        const uint32_t sh = (static_cast<uint32_t>(idx) & 1u) * 16u;
                        uint32_t old = *reinterpret_cast<volatile uint32_t *>(w);
                        bool next = false;
                        for (;;) {
                            const uint32_t cur = (old >> sh) & 0xFFFFu;
                            if (cur == 0u) {
                                const uint32_t prev = atomicCAS(w, old, old | (v << sh));
                                if (prev == old) {
                                    inf = CLS_CAND << 30;
                                    pcell[k] = static_cast<uint32_t>(idx);
                                    break;
                                }
                                old = prev;
                            } else if (cur <= static_cast<uint32_t>(padded)) {
                                if (tok_is(cur - 1u, t, th)) {
                                    inf = (CLS_HIT << 30) | (cur - 1u);
                                    lds_min16(vt32, cur - 1u, static_cast<uint16_t>(k + 1));
                                } else {
                                    next = true;
                                }
                                break;
                            } else if (ptok[cur - static_cast<uint32_t>(padded) - 1u] == t) {
                                pcell[k] = static_cast<uint32_t>(idx);
                                inf = CLS_CAND << 30;
                                if (v >= cur) break;
                                const uint32_t prev = atomicCAS(w, old, (old & ~(0xFFFFu << sh)) | (v << sh));
                                if (prev == old) break;
                                old = prev;
                            } else {
                                next = true;
                                break;
                            }
                        }
                        if (!next) break;
                        idx = (idx + 1) & mask;
                    }
                    if (inf == 0xFFFFFFFFu) {
                        g.code = kOverflowProbe;
                        inf = CLS_INV << 30;
                    }
                }
                pinf[k] = inf;
            }
            if (g.code) atomicOr(&ms.ovf, 1);
        }
        SUBSTAMP(3);
        __syncthreads();
        STAMP(3);
        // the first occurrence of each candidate token: its cell's final value
        // (with the direct map, read in the compaction pass below)
        if (!direct) {
            for (int32_t k = tid; k < K; k += NT) {
                if ((pinf[k] >> 30) != CLS_CAND) continue;
                const uint32_t e = ht[pcell[k]];
                pinf[k] = (CLS_CAND << 30) | (e - static_cast<uint32_t>(padded) - 1u);
            }
            __syncthreads();
        }
        STAMP(4);
        // ---- candidate prefix counts per position (contiguous chunk per
        // lane); first occurrences drop their provisional entries
        {
            const int32_t P = (K + NT - 1) / NT;
            const int32_t k0 = tid * P;
            uint32_t cnt = 0, fl = 0;
            for (int32_t i = 0; i < P; ++i) {
                const int32_t k = k0 + i;
                if (k < K) {
                    uint32_t inf = pinf[k];
                    if (direct && (inf >> 30) == CLS_CAND) {
                        inf = (CLS_CAND << 30) | (static_cast<uint32_t>(inv[ptok[k]]) - static_cast<uint32_t>(padded) - 1u);
                        pinf[k] = inf;
                    }
                    const uint32_t f = ((inf >> 30) == CLS_CAND && (inf & 0xFFFFu) == static_cast<uint32_t>(k)) ? 1u : 0u;
                    if (f && !direct) ht[pcell[k]] = 0;
                    fl |= f << i;
                    cnt += f;
                }
            }
            uint32_t M;
            uint32_t pre = block_exscan(cnt, bits_for(static_cast<uint32_t>(P)), ms.wt0, M);
            for (int32_t i = 0; i < P; ++i) {
                const int32_t k = k0 + i;
                if (k < K) {
                    candPre[k] = static_cast<uint16_t>(pre);
                    pre += (fl >> i) & 1u;
                }
            }
            if (tid == 0) {
                candPre[K] = static_cast<uint16_t>(M);
                ms.M = static_cast<int32_t>(M);
            }
        }
        if (ms.ovf) fast = false;
    }

    // ---- ring classes per offset from the hand (contiguous chunk per lane)
    const int32_t Q = (dbs + NT - 1) / NT;
    const int32_t u0 = tid * Q;
    uint64_t snM = 0, smM = 0;
    uint32_t preSN = 0, preSM = 0;
    if (fast) {
        __syncthreads();  // candPre complete
        STAMP(5);
        for (int32_t j = 0; j < Q; ++j) {
            const int32_t u = u0 + j;
            if (u >= dbs) break;
            const uint16_t v = vt[ring_slot(hand0, u, dbs)];
            if (v == VT_NONE) snM |= 1ull << j;
            else if (v != 0) smM |= 1ull << j;
        }
        SUBSTAMP(0);
        const uint32_t cSN = static_cast<uint32_t>(__popcll(snM)), cSM = static_cast<uint32_t>(__popcll(smM));
        const uint32_t qb = bits_for(static_cast<uint32_t>(Q));
        uint32_t tot;
        const uint32_t pre = block_exscan(cSN | (cSM << 16), qb | (qb << 16), ms.wt1, tot);
        SUBSTAMP(1);
        preSN = pre & 0xFFFFu;
        preSM = pre >> 16;
        uint32_t nsn = preSN, nsm = preSM;
        for (int32_t j = 0; j < Q; ++j) {
            const int32_t u = u0 + j;
            if (u >= dbs) break;
            if ((snM >> j) & 1ull) {
                ++nsn;
            } else if ((smM >> j) & 1ull) {
                const uint32_t k = static_cast<uint32_t>(vt[ring_slot(hand0, u, dbs)]) - 1u;
                const uint32_t cc = candPre[k];
                smA[nsm] = static_cast<uint32_t>(u) | (k << 16);
                smB[nsm] = nsn | (cc << 16);
                smKp[nsm] = (cc > nsn) ? static_cast<uint16_t>(k) : static_cast<uint16_t>(0);
                posSM[k] = static_cast<uint16_t>(nsm + 1u);
                ++nsm;
            }
        }
        if (tid == 0) ms.nSM = static_cast<int32_t>(tot >> 16);
        SUBSTAMP(2);
        __syncthreads();
        STAMP(6);

        // ---- decide the SM slots.  In ring order, slot i (k_i, need0_i = SN
        // slots before it, cc_i = candidates before k_i) is evicted iff the
        // events before k_i outnumber the event being served on arrival:
        //   cc_i + #{evicted j < i: k_j < k_i} > need0_i + #{evicted j < i},
        // i.e. a_i = cc_i - need0_i - 1 >= D_i = #{evicted j < i: k_j > k_i}.
        // a_i < 0: passed.  a_i >= U_i = #{j < i: a_j >= 0, k_j > k_i} (a
        // bound on D_i): evicted.  The rest (rare) are settled in ring order
        // by one wave.  A slot with need0_i >= M lies past the walk's end.
        {
            const int32_t nSM = ms.nSM, M = ms.M;
            for (int32_t i = tid; i < nSM; i += NT) {
                const uint32_t eb = smB[i];
                const int32_t need0 = static_cast<int32_t>(eb & 0xFFFFu);
                const int32_t ai = static_cast<int32_t>(eb >> 16) - need0 - 1;
                uint16_t dec = 0;  // 0 passed, 1 evicted, 2 undecided
                if (need0 < M && ai >= 0) {
                    const uint32_t ki = smA[i] >> 16;
                    int32_t U = 0;
                    int32_t j = 0;
                    for (; j + 8 <= i; j += 8) {
                        uint32_t kk[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) kk[q] = smKp[j + q];
#pragma unroll
                        for (int q = 0; q < 8; ++q) U += (kk[q] > ki) ? 1 : 0;
                    }
                    for (; j < i; ++j) U += (static_cast<uint32_t>(smKp[j]) > ki) ? 1 : 0;
                    dec = (ai >= U) ? 1 : 2;
                    if (dec == 2) undl[atomicAdd(&ms.nUnd, 1)] = static_cast<uint32_t>(i);
                }
                tb[i] = dec;
            }
        }
        SUBSTAMP(5);
        __syncthreads();
        STAMP(7);
        // undecided slots, one wave each: count the evictions already settled
        // before them (L) and the undecided ones before them with a larger k
        // (X); with X == 0, D = L exactly.  A concurrent settle of j < i reads
        // either as undecided (counted in X) or settled (counted exactly):
        // both are safe.
        {
            const int32_t nUnd = ms.nUnd;
            for (int32_t e = wave; e < nUnd; e += NWAVES) {
                const int32_t i = static_cast<int32_t>(undl[e]);
                const uint32_t ki = smA[i] >> 16;
                uint32_t lx = 0;
                for (int32_t j = static_cast<int32_t>(lane); j < i; j += 64) {
                    const uint16_t dj = tb[j];
                    if (dj != 0 && (smA[j] >> 16) > ki) lx += (dj == 1) ? 1u : 0x10000u;
                }
                lx = wave_sum(lx);
                if (lane == 0) {
                    if ((lx >> 16) == 0u) {
                        const uint32_t eb = smB[i];
                        const int32_t ai = static_cast<int32_t>(eb >> 16) - static_cast<int32_t>(eb & 0xFFFFu) - 1;
                        tb[i] = (ai >= static_cast<int32_t>(lx & 0xFFFFu)) ? 1 : 0;
                    } else {
                        atomicAdd(&ms.nRest, 1);
                    }
                }
            }
        }
        SUBSTAMP(6);
        __syncthreads();
        SUBSTAMP(7);
        if (ms.nRest > 0 && wave == 0) {  // the rest, in ring order
            const int32_t nSM = ms.nSM;
            for (int32_t c = 0; c < nSM; c += 64) {
                uint64_t und = __ballot(c + static_cast<int32_t>(lane) < nSM && tb[c + lane] == 2);
                while (und != 0ull) {
                    const int f = __builtin_ctzll(und);
                    und &= und - 1ull;
                    const int32_t i = c + f;
                    const uint32_t ki = smA[i] >> 16;
                    const uint32_t eb = smB[i];
                    const int32_t ai = static_cast<int32_t>(eb >> 16) - static_cast<int32_t>(eb & 0xFFFFu) - 1;
                    uint32_t d = 0;
                    for (int32_t j = static_cast<int32_t>(lane); j < i; j += 64) {
                        d += (tb[j] == 1 && (smA[j] >> 16) > ki) ? 1u : 0u;
                    }
                    d = wave_sum(d);
                    if (lane == 0) tb[i] = (ai >= static_cast<int32_t>(d)) ? 1 : 0;
                }
            }
        }
        __syncthreads();
        // ---- one scan for both the eviction prefix over the SM list and the
        // event sequence over positions (candidates' first occurrences and
        // conversions -- first hits of evicted SM slots -- in position order)
        {
            const int32_t nSM = ms.nSM;
            const int32_t Ps = (nSM + NT - 1) / NT, i0 = tid * Ps;
            const int32_t Pk = (K + NT - 1) / NT, k0 = tid * Pk;
            uint32_t cs = 0, fs = 0, ce = 0, fe = 0;
            for (int32_t q = 0; q < Ps; ++q) {
                const int32_t i = i0 + q;
                if (i < nSM && tb[i] == 1) {
                    fs |= 1u << q;
                    ++cs;
                    const uint32_t ea = smA[i];
                    evold[ea >> 16] = static_cast<uint16_t>(ring_slot(hand0, static_cast<int32_t>(ea & 0xFFFFu), dbs));
                }
            }
            for (int32_t q = 0; q < Pk; ++q) {
                const int32_t k = k0 + q;
                if (k < K) {
                    const uint32_t inf = pinf[k];
                    const uint32_t c = inf >> 30;
                    bool f = c == CLS_CAND && (inf & 0xFFFFu) == static_cast<uint32_t>(k);
                    if (c == CLS_HIT) {
                        const uint32_t sm = posSM[k];
                        f = sm != 0u && tb[sm - 1u] == 1;
                    }
                    if (f) {
                        fe |= 1u << q;
                        ++ce;
                    }
                }
            }
            const uint32_t bs = bits_for(static_cast<uint32_t>(Ps)), be = bits_for(static_cast<uint32_t>(Pk));
            uint32_t tot;
            const uint32_t pre = block_exscan(cs | (ce << 16), bs | (be << 16), ms.wt0, tot);
            uint32_t ps = pre & 0xFFFFu, pe = pre >> 16;
            for (int32_t q = 0; q < Ps; ++q) {
                const int32_t i = i0 + q;
                if (i < nSM) {
                    const uint32_t tk = (fs >> q) & 1u;
                    tb[i] = static_cast<uint16_t>(ps | (tk << 15));
                    ps += tk;
                }
            }
            for (int32_t q = 0; q < Pk; ++q) {
                if ((fe >> q) & 1u) eseq[pe++] = static_cast<uint16_t>(k0 + q);
            }
            const int32_t T = static_cast<int32_t>(tot & 0xFFFFu);
            if (tid == 0) {
                tb[nSM] = static_cast<uint16_t>(T);
                ms.T = T;
                ms.nConv = T;
                ms.N = ms.M + T;
                if (static_cast<int32_t>(tot >> 16) != ms.M + T) ms.ovf = 1;
            }
        }
        __syncthreads();
        STAMP(8);
        // ---- marks per ring offset: evicted by event p, or passed while serving event p
        {
            const int32_t N = ms.N;
            uint32_t nsn2 = preSN, nsm2 = preSM, ntk = 0;
            for (int32_t j = 0; j < Q; ++j) {
                const int32_t u = u0 + j;
                if (u >= dbs) break;
                const int32_t s = ring_slot(hand0, u, dbs);
                const bool isSN = (snM >> j) & 1ull, isSM = (smM >> j) & 1ull;
                const uint32_t tbv = tb[nsm2];
                const int32_t r = static_cast<int32_t>(nsn2 + (tbv & 0x7FFFu));
                if (r < N) {
                    const uint32_t p = eseq[r];
                    if (isSN || (isSM && (tbv & 0x8000u))) {
                        evslot[p] = static_cast<uint16_t>(s);
                        vt[s] = isSM ? static_cast<uint16_t>(VT_EVICTED | (vt[s] - 1u))
                                     : static_cast<uint16_t>(VT_EVICTED | VT_NOCONV);
                        ++ntk;
                        if (r == N - 1) ms.uEnd = u + 1;
                    } else {
                        vt[s] = static_cast<uint16_t>(VT_PASSED | p);
                    }
                }
                nsn2 += isSN ? 1u : 0u;
                nsm2 += isSM ? 1u : 0u;
            }
            ntk = wave_sum(ntk);
            if (lane == 0 && ntk) atomicAdd(&ms.nTakes, static_cast<int32_t>(ntk));
        }
        __syncthreads();
        STAMP(9);
        if (ms.nTakes != ms.N || ms.ovf) fast = false;  // the hand would wrap within the step
    }

    if (fast) {
        const int32_t N = ms.N, uEnd = ms.uEnd;
        Guard g;
        // ---- outputs; visited bits set this step (into vset); the cell of
        // each evicted token and each event's new token (conversions
        // re-insert a pre-step token)
        for (int32_t k = tid; k < K; k += NT) {
            const uint32_t inf = pinf[k];
            const uint32_t cls = inf >> 30;
            int32_t slot = -1;
            int8_t miss = 0;
            if (cls == CLS_EXT) {
                slot = padded + (ptok[k] - prefill);
            } else if (cls == CLS_HIT) {
                const uint32_t s0 = inf & 0xFFFFu;
                const uint16_t v = vt[s0];
                if (v & VT_EVICTED) {  // evicted before its first hit: converted at time c
                    const uint32_t c = v & VT_NOCONV;
                    slot = evslot[c];
                    miss = (static_cast<uint32_t>(k) == c) ? 1 : 0;
                } else {
                    slot = static_cast<int32_t>(s0);
                    if (!(v & VT_PASSED) || static_cast<uint32_t>(k) > (v & VT_NOCONV)) {
                        atomicOr(vset + (s0 >> 5), 1u << (s0 & 31u));
                    }
                }
            } else if (cls == CLS_CAND) {
                const uint32_t k1 = inf & 0xFFFFu;
                slot = evslot[k1];
                miss = (k1 == static_cast<uint32_t>(k)) ? 1 : 0;
            }
            rs[k] = slot;
            rm[k] = miss;
        }
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t p = eseq[i];
            const uint32_t s = evslot[p];
            atomicOr(vset + (s >> 5), 1u << (s & 31u));
            const int32_t old = kC ? gTok[s] : tok[s];
            uint32_t cell = 0xFFFFFFFFu;
            if (old >= 0) {
                int32_t idx = static_cast<int32_t>(ht_hash(old)) & mask;
                for (int32_t n = 0; n <= mask; ++n) {
                    if (ht[idx] == s + 1u) {
                        cell = static_cast<uint32_t>(idx);
                        break;
                    }
                    idx = (idx + 1) & mask;
                }
                if (cell == 0xFFFFFFFFu) g.code = kOverflowProbe;
                else if (!kC) atomicOr(ber + (cell >> 5), 1u << (cell & 31u));
            }
            ecell[i] = cell;
            const uint32_t src = evold[p];
            ntokv[i] = static_cast<uint32_t>((pinf[p] >> 30) == CLS_CAND ? ptok[p] : (kC ? gTok[src] : tok[src]));
        }
        __syncthreads();
        if constexpr (kC) {  // the bitmaps share vt's memory: clear them now that vt is read
            for (int32_t i = tid; i < 4 * (H >> 5); i += NT) ber[i] = 0u;
            __syncthreads();
            for (int32_t i = tid; i < N; i += NT) {
                const uint32_t cell = ecell[i];
                if (cell != 0xFFFFFFFFu) atomicOr(ber + (cell >> 5), 1u << (cell & 31u));
            }
            __syncthreads();
        }
        STAMP(10);
        // ---- table: erase the evicted tokens; the rightmost marked cell of a
        // cluster leads it and deletes right to left
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t c = ecell[i];
            if (c == 0xFFFFFFFFu) continue;
            bool ld = true;
            int32_t x = (static_cast<int32_t>(c) + 1) & mask;
            for (int32_t n = 0; n < H && ht[x] != 0; ++n, x = (x + 1) & mask) {
                if (bit_get(ber, x)) {
                    ld = false;
                    break;
                }
            }
            if (ld) ecell[i] = c | 0x80000000u;
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t e = ecell[i];
            if (e == 0xFFFFFFFFu || !(e & 0x80000000u)) continue;
            const int32_t c = static_cast<int32_t>(e & 0x7FFFFFFFu);
            rdel_at<kC>(ht, smem + lay.tok, padded, c, mask, g);
            int32_t x = (c - 1) & mask;
            for (int32_t n = 0; n < H && ht[x] != 0; ++n, x = (x - 1) & mask) {
                if (bit_get(ber, x)) rdel_at<kC>(ht, smem + lay.tok, padded, x, mask, g);
            }
        }
        __syncthreads();
        STAMP(11);
        // ---- new tokens; tentative placement (the final occupied cells do not depend on order)
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t s = evslot[eseq[i]];
            const int32_t t = static_cast<int32_t>(ntokv[i]);
            if constexpr (kC) {
                hv[s] = static_cast<uint16_t>(ht_hash(t));
                gTok[s] = t;
            } else {
                tok[s] = t;
            }
            const int32_t c = lds_claim16(ht32, static_cast<int32_t>(ht_hash(t)) & mask, mask,
                                          static_cast<uint16_t>(s + 1u));
            if (c < 0) g.code = kOverflowProbe;
            else atomicOr(bnew + (c >> 5), 1u << (c & 31));
        }
        __syncthreads();
        // final cluster of each new key (its start); clusters with two or more new keys are redone
        for (int32_t i = tid; i < N; i += NT) {
            int32_t st = static_cast<int32_t>(ht_hash(static_cast<int32_t>(ntokv[i]))) & mask;
            for (int32_t n = 0; n < H && ht[(st - 1) & mask] != 0; ++n) st = (st - 1) & mask;
            kst[i] = static_cast<uint32_t>(st);
            const uint32_t bit = 1u << (st & 31);
            const uint32_t old = atomicOr(bg + (st >> 5), bit);
            if (old & bit) atomicOr(bm + (st >> 5), bit);
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t st = kst[i];
            if (bit_get(bm, st)) {
                const uint32_t p = eseq[i];
                const int32_t q = atomicAdd(&ms.nMulti, 1);
                mlist[q] = (static_cast<uint64_t>(st) << 32) | (static_cast<uint64_t>(p) << 16) | evslot[p];
            }
        }
        __syncthreads();
        STAMP(12);
        const int32_t nMulti = ms.nMulti;
        if (nMulti > 0) {
            for (int32_t q = tid; q < nMulti; q += NT) {  // sort by (cluster start, event time)
                const uint64_t key = mlist[q];
                int32_t r = 0;
                for (int32_t j = 0; j < nMulti; ++j) r += (mlist[j] < key) ? 1 : 0;
                msort[r] = key;
            }
            __syncthreads();
            for (int32_t q = tid; q < nMulti; q += NT) {  // the first key of each cluster redoes it in time order
                const uint64_t key = msort[q];
                const uint32_t st = static_cast<uint32_t>(key >> 32);
                if (q > 0 && static_cast<uint32_t>(msort[q - 1] >> 32) == st) continue;
                int32_t end = static_cast<int32_t>(st);
                for (int32_t n = 0; n < H && ht[end] != 0; ++n) end = (end + 1) & mask;
                for (int32_t x = static_cast<int32_t>(st); x != end; x = (x + 1) & mask) {
                    if (bit_get(bnew, static_cast<uint32_t>(x))) ht[x] = 0;
                }
                for (int32_t r = q; r < nMulti && static_cast<uint32_t>(msort[r] >> 32) == st; ++r) {
                    const uint32_t s = static_cast<uint32_t>(msort[r] & 0xFFFFu);
                    int32_t idx = static_cast<int32_t>(tok_hash(s)) & mask;
                    for (int32_t n = 0; n < H && ht[idx] != 0; ++n) idx = (idx + 1) & mask;
                    ht[idx] = static_cast<uint16_t>(s + 1u);
                }
            }
        }
        if (g.code) atomicOr(&ms.late, 1);
        __syncthreads();
        STAMP(13);
        if (!ms.late) {
            // ---- write back; visited = (staged bits minus the ring range the
            // hand passed) | bits set this step
            const int32_t e0 = hand0 + uEnd;  // passed slots: [hand0, e0) then [0, e0 - dbs)
            for (int32_t w = tid; w < (visStrideB >> 2); w += NT) {
                const int32_t lo = w * 32;
                uint32_t clr = 0;
                if (uEnd > 0) {
                    const int32_t a0 = max(lo, hand0), a1 = min(lo + 32, min(e0, dbs));
                    if (a1 > a0) clr |= (a1 - a0 == 32 ? 0xFFFFFFFFu : ((1u << (a1 - a0)) - 1u)) << (a0 - lo);
                    const int32_t b1 = min(lo + 32, e0 - dbs);
                    if (b1 > lo) clr |= (b1 - lo == 32 ? 0xFFFFFFFFu : ((1u << (b1 - lo)) - 1u));
                }
                reinterpret_cast<uint32_t *>(gVis)[w] = (vis32[w] & ~clr) | vset[w];
            }
            if (N > 0) {
                if constexpr (!kC) wg_copy16(gTok, tok, static_cast<uint32_t>(padded) * 4u);  // compact: written in place
                wg_copy16(gHt, ht, static_cast<uint32_t>(H) * 2u);
            }
            if (tid == 0) {
                int32_t hd = hand0;
                if (N > 0) {
                    hd = hand0 + uEnd;
                    while (hd >= dbs) hd -= dbs;
                }
                gHand[0] = hd;
                gHand[1] = kCanonFlag;
            }
            STAMP(14);
            return;
        }
        if constexpr (kC) {
            // the compact form has already written the new tokens to HBM; a
            // late bound violation only comes from a corrupted table
            if (tid == 0) report_overflow(L.overflowSlot, kOverflowProbe);
            return;
        }
        fast = false;
    }

    // ---- fallback: restage the pre-step row from HBM (nothing has been
    // written back) and run the sequential recurrence on it
    __syncthreads();
    int32_t *tokF = reinterpret_cast<int32_t *>(smem);
    uint16_t *htF = reinterpret_cast<uint16_t *>(smem + static_cast<size_t>(padded) * 4u);
    uint8_t *visF = smem + static_cast<size_t>(padded) * 4u + static_cast<size_t>(H) * 2u;
    wg_copy16(tokF, gTok, static_cast<uint32_t>(padded) * 4u);
    wg_copy16(htF, gHt, static_cast<uint32_t>(H) * 2u);
    wg_copy16(visF, gVis, static_cast<uint32_t>(visStrideB));
    __syncthreads();
    __shared__ int32_t s_dirty;
    if (wave == 0) {  // the in-order recurrence: one lane for small tables, else 64 cells/slots per step
        int32_t hand = hand0;
        Guard g;
        bool dirty = false;
        if (H <= kSmallTable) {
            if (lane == 0) dirty = sieve_row_sequential(rt, rs, rm, K, seqLen, prefill, dbs, padded, mask, tokF, visF, htF, hand, g);
        } else {
            dirty = sieve_row_wave(rt, rs, rm, K, seqLen, prefill, dbs, padded, mask, tokF, visF, htF, hand, g);
        }
        if (lane == 0) {
            gHand[0] = hand;
            gHand[1] = (canonical && g.code == 0) ? kCanonFlag : 0;
            s_dirty = dirty ? 1 : 0;
            report_overflow(L.overflowSlot, g.code);
        }
    }
    __syncthreads();
    wg_copy16(gVis, visF, static_cast<uint32_t>(visStrideB));
    if (s_dirty) {
        wg_copy16(gTok, tokF, static_cast<uint32_t>(padded) * 4u);
        wg_copy16(gHt, htF, static_cast<uint32_t>(H) * 2u);
    }
}

}  // namespace

hipError_t sieve_fast_set_lds_limit(size_t bytes)
{
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update_fast<false>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update_fast<true>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_sieve_update_fast(const HispSieveUpdateArgs &a, uint64_t overflowSlot, size_t ldsBytes, bool compact,
                                    hipStream_t stream)
{
    KvxLaunch<HispSieveUpdateArgs> L{a, overflowSlot};
    if (compact) {
        hipLaunchKernelGGL(kvx_sieve_update_fast<true>, dim3(a.maxNumReqs), dim3(NT), ldsBytes, stream, L);
    } else {
        hipLaunchKernelGGL(kvx_sieve_update_fast<false>, dim3(a.maxNumReqs), dim3(NT), ldsBytes, stream, L);
    }
    return hipGetLastError();
}

}  // namespace kvx

#ifdef KVX_SIEVE_PHASE_STAMPS
extern "C" int kvx_dbg_read_sub(unsigned long long *out, int rows)
{
    if (rows > 1024) rows = 1024;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(kvx::kvx_dbg_sub), sizeof(unsigned long long) * 16 * rows, 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}

extern "C" int kvx_dbg_read_stamps(unsigned long long *out, int rows)
{
    if (rows > 1024) rows = 1024;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(kvx::kvx_dbg_stamps), sizeof(unsigned long long) * 16 * rows, 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif
