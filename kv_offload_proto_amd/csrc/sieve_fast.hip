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
// Phases (one barrier each unless noted):
//   stage    tokens/table/visited/topK row into LDS, per-slot visited flags,
//            the table's occupancy bitmap and (when the prefill fits) a
//            direct token -> slot map; table consistency check (first step)
//   classify hit / candidate / invalid / decode-extension per position; the
//            first hit time of every slot (LDS min); candidate dedup (smallest
//            position per token) through the direct map or provisional
//            table entries
//   scan     ballots of the candidates' first occurrences and a prefix scan
//            of the ring classes; the SM slots before the M-th SN slot
//   decide   per SM slot, bounds that settle almost all of them in parallel;
//            the rest in ring order
//   events   eviction prefix over the SM slots and the event sequence in
//            position order, both from ballot masks
//   marks    per ring offset: evicted at event p / passed at event p; the
//            evicted tokens' table cells (looked up with the ring classes
//            for the SN slots, which are all evicted)
//   outputs  slots, is_miss, visited bits; erase the evicted tokens
//            (Algorithm R deletions commute when each pre-step cluster is
//            done right to left by its rightmost marked cell)
//   insert   tentative parallel placement of the new tokens (the occupied
//            cells do not depend on order), entries naming the event; a key
//            alone in its final cluster takes its cell, and every other
//            cluster is redone in event order by one wave (a lane per cell).  Linear probing
//            with Algorithm R leaves the table equal to inserting the live
//            keys in insertion order, so the result is the sequential table
//            byte for byte.
//
// Shape preconditions, checked by the launcher: padded + 1 + topK <= 65535,
// topK < 16383, dbs <= 32 * 1024, htSize <= 32768.  State preconditions,
// checked in the kernel: the table indexes exactly the non-negative tokens of
// slots [0, dbs) (each found at its own slot), no hand wrap within the step;
// otherwise the row is restaged from HBM and the sequential recurrence runs.
#include "kvx_internal.h"
#include "sieve_common.h"

// the per-lane loops unroll in the fixed-count instantiations only
#pragma clang diagnostic ignored "-Wpass-failed"

namespace kvx {
namespace {

using namespace sieve;

// Global-memory pointers carry their address space, so the compiler emits
// global rather than flat instructions: flat ones also count against the LDS
// wait counter and stall the LDS work that follows them.
#define KVX_G __attribute__((address_space(1)))
// Uniform values this kernel does not write before reading them (lengths,
// the request index, the hand) load through the constant address space, as
// scalar loads that need no wave-wide copy into scalar registers.
#define KVX_C __attribute__((address_space(4)))
typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // 16-byte chunk
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));  // two 16-bit lanes of a register

constexpr int NT = kFastThreads;
constexpr int NWAVES = NT / 64;

constexpr uint32_t CLS_INV = 0u, CLS_EXT = 1u, CLS_HIT = 2u, CLS_CAND = 3u;
constexpr uint16_t VT_NONE = 0xFFFF, VT_EVICTED = 0x8000, VT_PASSED = 0x4000, VT_NOCONV = 0x3FFF;
constexpr uint16_t HV_EMPTY = 0xFFFF;  // compact form: slot without a token (hashes are masked below 2^15)
constexpr uint32_t NOCELL = 0xFFFFu;   // evicted slot without a table entry

// Phase timestamps for profiling builds (-DKVX_SIEVE_PHASE_STAMPS): thread 0
// of each workgroup records clock64() at phase boundaries into kvx_dbg_stamps,
// and into kvx_dbg_sub the constant-rate clock at entry [12] and exit [13],
// clock64() at entry [14] and the wave's HW_ID [10] and XCC_ID [11] (the
// shader clocks of different XCDs are not aligned; the constant-rate one is).
#ifdef KVX_SIEVE_PHASE_STAMPS
__device__ unsigned long long kvx_dbg_stamps[1024][16];
__device__ unsigned long long kvx_dbg_sub[1024][16];
// the arrays' addresses are taken once, at entry: a stamp is then a clock
// read and a store, with no address load queued ahead of the clock read.  The
// pointers carry the global address space: a flat store would also count
// against the LDS wait counter and hold up the phase after each stamp.
#define DBG_SETUP()                                                                         \
    KVX_G unsigned long long *dbgSt = (KVX_G unsigned long long *)&kvx_dbg_stamps[0][0];    \
    KVX_G unsigned long long *dbgSub = (KVX_G unsigned long long *)&kvx_dbg_sub[0][0];      \
    asm volatile("" : "+s"(dbgSt), "+s"(dbgSub))
#define STAMP(i)                                                        \
    do {                                                                \
        if (tid == 0 && bid < 1024) dbgSt[bid * 16 + (i)] = clock64();  \
    } while (0)
#define DBGVAL(i, v)                                                  \
    do {                                                              \
        if (tid == 0 && bid < 1024) dbgSub[bid * 16 + (i)] = (v);     \
    } while (0)
#else
#define DBG_SETUP()
#define STAMP(i) \
    do {         \
    } while (0)
#define DBGVAL(i, v) \
    do {             \
    } while (0)
#endif

struct Misc {
    unsigned long long evMask;  // in-order path: the events that placed a slot's final token
    int32_t nEv, handOut;
    int32_t bad, ovf, late, nSM, nUnd, uEnd, nTakes, nLead, nDone, snNext;
    int32_t diff;  // live tokens minus table entries
    uint32_t fp0, fpd;  // the staged tokens' fingerprint; its change by the step's new tokens
    uint32_t M;    // candidates (first occurrences of missing tokens)
    uint32_t uL[64];  // undecided SM slots in ring order: evictions settled before them with a larger k
    uint16_t ui[64];  // ... and their SM indices
};

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

// Inclusive prefix sum over the 64 lanes of a wave from DPP row shifts and
// row broadcasts (no LDS round trips).  Call with the whole wave active.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t x)
{
    int v = static_cast<int>(x);
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
    return static_cast<uint32_t>(v);
}

__device__ __forceinline__ uint32_t wave_sum(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(wave_incl_scan(v)), 63));
}

// Set bits of m below this lane.
__device__ __forceinline__ uint32_t lanes_below(uint64_t m)
{
    return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0u));
}

// Exclusive prefix counts over 64-bit ballot masks mk[e], e = block *
// NWAVES + wave (so entry e covers items 64e..64e+63 of a lane-strided
// index), computed by every wave for itself: lane L sums 2^lg consecutive
// entries.  Set up and query with the whole wave active.
struct MaskPrefix {
    const uint64_t *mk;
    const uint64_t *mk2;  // optional second array, OR'ed into mk (null: none)
    int32_t lg;
    uint32_t ex;     // prefix of this lane's first entry
    uint32_t total;  // set bits in all entries

    __device__ __forceinline__ uint64_t ent(int32_t x) const { return mk2 ? (mk[x] | mk2[x]) : mk[x]; }
    __device__ __forceinline__ void init(const uint64_t *m, int32_t nE, uint32_t lane, const uint64_t *m2 = nullptr)
    {
        mk = m;
        mk2 = m2;
        lg = 0;
        while ((64 << lg) < nE) ++lg;
        const int32_t e0 = static_cast<int32_t>(lane) << lg;
        uint32_t s = 0;
        for (int32_t x = e0; x < e0 + (1 << lg) && x < nE; ++x) s += static_cast<uint32_t>(__popcll(ent(x)));
        const uint32_t incl = wave_incl_scan(s);
        ex = incl - s;
        total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
    }
    // two prefixes from one scan (16-bit fields) when both fit one entry per lane
    static __device__ __forceinline__ void init_pair(MaskPrefix &a, const uint64_t *ma, int32_t na, MaskPrefix &b,
                                                     const uint64_t *mb, int32_t nb, uint32_t lane,
                                                     const uint64_t *mb2 = nullptr)
    {
        if (na > 64 || nb > 64) {
            a.init(ma, na, lane);
            b.init(mb, nb, lane, mb2);
            return;
        }
        a.mk = ma;
        b.mk = mb;
        a.mk2 = nullptr;
        b.mk2 = mb2;
        a.lg = b.lg = 0;
        const int32_t L = static_cast<int32_t>(lane);
        const uint32_t ca = L < na ? static_cast<uint32_t>(__popcll(a.ent(L))) : 0u;
        const uint32_t cb = L < nb ? static_cast<uint32_t>(__popcll(b.ent(L))) : 0u;
        const uint32_t packed = ca | (cb << 16);
        const uint32_t incl = wave_incl_scan(packed);
        const uint32_t ex = incl - packed;
        const uint32_t tot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), 63));
        a.ex = ex & 0xFFFFu;
        b.ex = ex >> 16;
        a.total = tot & 0xFFFFu;
        b.total = tot >> 16;
    }
    // set bits before entry e (e the same in the whole wave)
    __device__ __forceinline__ uint32_t base(int32_t e) const
    {
        const int32_t L = e >> lg;
        uint32_t c = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ex), L));
        for (int32_t x = L << lg; x < e; ++x) c += static_cast<uint32_t>(__popcll(ent(x)));
        return c;
    }
    // set bits before this lane's bit of entry e (e the same in the whole wave)
    __device__ __forceinline__ uint32_t own(int32_t e) const { return base(e) + lanes_below(ent(e)); }
    // set bits before bit `bit` of entry e (any entry per lane)
    __device__ __forceinline__ uint32_t before(int32_t e, uint32_t bit) const
    {
        const int32_t L = e >> lg;
        uint32_t c = static_cast<uint32_t>(__shfl(static_cast<int>(ex), L));
        for (int32_t x = L << lg; x < e; ++x) c += static_cast<uint32_t>(__popcll(ent(x)));
        return c + static_cast<uint32_t>(__popcll(ent(e) & ((1ull << bit) - 1ull)));
    }
};

// 16-bit LDS min via a CAS on the containing word.
__device__ __forceinline__ void lds_min16(uint32_t *w32, uint32_t i, uint16_t v)
{
    uint32_t *w = w32 + (i >> 1);
    const uint32_t sh = (i & 1u) * 16u;
    uint32_t old = *w;  // a stale value only costs a CAS retry
    for (;;) {
        const uint32_t cur = (old >> sh) & 0xFFFFu;
        if (cur <= v) return;
        const uint32_t nw = (old & ~(0xFFFFu << sh)) | (static_cast<uint32_t>(v) << sh);
        const uint32_t prev = atomicCAS(w, old, nw);
        if (prev == old) return;
        old = prev;
    }
}

// Claim the first free cell at or after `idx` in an occupancy bitmap (one
// bit per cell) with an atomic OR per try; a failed try moves to the next
// free cell the returned word shows.  Bits are only set while claims run, so
// every cell from idx to the one returned was occupied when passed.  Returns
// the cell, or -1 after a whole-table probe.
__device__ __forceinline__ int32_t lds_claim_bit(uint32_t *bm, int32_t idx, int32_t mask)
{
    for (int32_t n = 0; n <= mask; ++n) {
        const uint32_t b = static_cast<uint32_t>(idx) & 31u, bit = 1u << b;
        const uint32_t old = atomicOr(bm + (idx >> 5), bit);
        if (!(old & bit)) return idx;
        const uint32_t fr = ~old & (0xFFFFFFFEu << b);  // free cells above b in the word
        idx = fr ? ((idx & ~31) | __builtin_ctz(fr)) : (((idx | 31) + 1) & mask);
    }
    return -1;
}

// Algorithm R deletion of the entry at cell c (homes from the tokens row, or
// from the per-slot token hashes in the compact form); the cell left empty is
// cleared in the occupancy bitmap fin.
template <bool kC>
__device__ void rdel_at(uint16_t *ht, uint32_t *fin, const void *tokv, int32_t ntok, int32_t c, int32_t mask,
                        Guard &g)
{
    // the next cell is read with the current entry's token: a move writes
    // only cells left of the current one, never the next
    int32_t j = c, i = (c + 1) & mask;
    uint16_t e = ht[i];
    for (int32_t n = 0;; ++n) {
        if (n > mask) {
            g.code = kOverflowProbe;
            return;
        }
        if (e == 0) break;
        const int32_t inext = (i + 1) & mask;
        const uint16_t enext = ht[inext];
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
        i = inext;
        e = enext;
    }
    ht[j] = 0;
    atomicAnd(fin + (j >> 5), ~(1u << (j & 31)));
}

// Copy n bytes (multiple of 16) with the workgroup, four 16-byte chunks in
// flight per lane.  D and S are v4u in the LDS or global address space.
template <typename D, typename S>
__device__ __forceinline__ void wg_copy16(D *d, S *s, uint32_t n)
{
    const uint32_t n16 = n / 16u;
    uint32_t i = threadIdx.x;
    for (; i + 3u * NT < n16; i += 4u * NT) {
        const v4u a = s[i];
        const v4u b = s[i + NT];
        const v4u c = s[i + 2u * NT];
        const v4u e = s[i + 3u * NT];
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

// kC: compact LDS form.  PM, QM: positions and ring offsets per lane when
// fixed at compile time (the launcher picks an instantiation whose values
// equal ceil(topK / NT) and ceil(dbs / NT)); 0 = any shape.  With fixed
// counts the per-lane loops unroll and the lane's positions, their classes
// and its ring offsets' first-hit times stay in registers between phases.
template <bool kC, int PM, int QM>
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
    const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    DBG_SETUP();
    DBGVAL(12, __builtin_amdgcn_s_memrealtime());
    DBGVAL(14, clock64());
    DBGVAL(10, __builtin_amdgcn_s_getreg((31 << 11) | 4));   // HW_ID
    DBGVAL(11, __builtin_amdgcn_s_getreg((15 << 11) | 20));  // XCC_ID
    // (the grid is exactly maxNumReqs workgroups.)  The pointers are loaded
    // from the arguments in one batch, ahead of the first branch: fetched on
    // demand they would each cost a round trip.
    asm volatile("" : : "s"(a.topkIndices), "s"(a.reqPoolIndices), "s"(a.seqLens), "s"(a.prefillLens),
                 "s"(a.deviceBufferTokens), "s"(a.deviceBufferVisited), "s"(a.deviceBufferHt), "s"(a.sieveHand),
                 "s"(a.topKDeviceSlots), "s"(a.isMiss), "s"(a.numReal), "s"(a.topK), "s"(a.maxNumReqs),
                 "s"(a.htSize), "s"(a.poolSize), "s"(a.reserved));

    // num_real and the batch row's request and length in one round trip (the
    // row's entries exist for every bid < maxNumReqs, so they are read before
    // num_real is known; the asm use keeps them ahead of the branch)
    int32_t numReal = *(KVX_C const int32_t *)(a.numReal);
    const int64_t reqRaw = ((KVX_C const int64_t *)(a.reqPoolIndices))[bid];
    const int32_t seqLen = ((KVX_C const int32_t *)(a.seqLens))[bid];
    asm volatile("" : : "s"(reqRaw), "s"(seqLen));
    if (numReal > maxNumReqs) numReal = maxNumReqs;  // hisp_sieve_update.cpp:31-34
    KVX_G int32_t *rs = (KVX_G int32_t *)(a.topKDeviceSlots) + static_cast<int64_t>(bid) * K;
    KVX_G int8_t *rm = (KVX_G int8_t *)(a.isMiss) + static_cast<int64_t>(bid) * K;
    if (bid >= numReal) {
        write_dummy_row((int32_t *)rs, (int8_t *)rm, K);
        return;
    }
    // the topK row.  An invalid request index is acted on after staging (row
    // 0, which exists, is staged meanwhile): an early exit here would let the
    // compiler sink the loads below it, each then waited for on its own.
    KVX_G const int32_t *rt = (KVX_G const int32_t *)(a.topkIndices) + static_cast<int64_t>(bid) * K;
    // unconditional (clamped, K >= 1 here) loads: a load under a branch makes
    // the compiler wait for it at the branch's end
    const bool h0 = tid < K, h1 = tid + NT < K;
    const int32_t t0 = rt[min(tid, K - 1)], t1 = rt[min(tid + NT, K - 1)];
    const bool badReq = reqRaw < 0 || reqRaw >= poolSize;
    const int64_t reqIdx = badReq ? 0 : reqRaw;
    // direct token -> slot map over the tokens that can be looked up (below
    // both prefill and seqLen) when they fit the LDS left over after the
    // layout, 32-bit entries: all ones, slot+1 of the slot holding the token,
    // or padded+1+k for a missing token first seen at position k (the smallest
    // k, by an LDS min).  Cleared over min(seqLen, capacity) entries before the
    // state row lands.
    constexpr bool kFixed = PM > 0 && QM > 0;
    // fixed-count instantiations: compile-time offsets for the regions sized by topK and dbs
    const FastLayout lay = kFixed ? fast_layout_fixed<(kFixed ? PM : 1), (kFixed ? QM : 1)>(padded, H, visStrideB, kC)
                                  : fast_layout(padded, H, K, visStrideB, kC);
    // words of the visited bits set this step (bits of slots below dbs)
    const int32_t vsetWords = kFixed ? QM * NT / 32 : (visStrideB >> 2);
    const int32_t invCap = static_cast<int32_t>(a.reserved >> 8);
    uint32_t *inv = reinterpret_cast<uint32_t *>(smem + lay.total);
    if (!kC && invCap > 0 && seqLen > 0) {
        const int32_t n4 = (min(seqLen, invCap) + 3) >> 2;
        for (int32_t i = tid; i < n4; i += NT) reinterpret_cast<v4u *>(inv)[i] = v4u{~0u, ~0u, ~0u, ~0u};
    }
    if (tid == 0) {  // ordered before every update by the barrier in the staging pass
        ms.bad = ms.ovf = ms.late = 0;
        ms.nSM = ms.nUnd = ms.uEnd = ms.nTakes = ms.nLead = ms.nDone = ms.snNext = 0;
        ms.diff = 0;
        ms.fp0 = ms.fpd = 0u;
        ms.M = 0;
        ms.evMask = 0ull;
    }
    int32_t prefill = ((KVX_C const int32_t *)(a.prefillLens))[reqIdx];
    KVX_G int32_t *gTok = (KVX_G int32_t *)(a.deviceBufferTokens) + reqIdx * padded;
    KVX_G uint8_t *gVis = (KVX_G uint8_t *)(a.deviceBufferVisited) + reqIdx * visStrideB;
    KVX_G uint16_t *gHt = (KVX_G uint16_t *)(a.deviceBufferHt) + reqIdx * H;
    KVX_G int32_t *gHand = (KVX_G int32_t *)(a.sieveHand) + reqIdx * kHandStride;

    int32_t *tok = reinterpret_cast<int32_t *>(smem + lay.tok);    // full form: tokens
    uint16_t *hv = reinterpret_cast<uint16_t *>(smem + lay.tok);   // compact form: masked token hashes
    uint16_t *ht = reinterpret_cast<uint16_t *>(smem + lay.ht);
    uint32_t *ht32 = reinterpret_cast<uint32_t *>(smem + lay.ht);
    uint8_t *vis = smem + lay.vis;
    uint32_t *vis32 = reinterpret_cast<uint32_t *>(smem + lay.vis);
    int32_t *ptok = reinterpret_cast<int32_t *>(smem + lay.ptok);
    uint32_t *pinf = reinterpret_cast<uint32_t *>(smem + lay.pinf);
    // first-hit code per slot: 32 bits in the full form (an LDS min updates
    // it), 16 in the compact form (a CAS on the containing word)
    using VT = typename std::conditional<kC, uint16_t, uint32_t>::type;
    VT *vt = reinterpret_cast<VT *>(smem + lay.vt);
    uint16_t *evslot = reinterpret_cast<uint16_t *>(smem + lay.evslot);
    uint16_t *smKp = reinterpret_cast<uint16_t *>(smem + lay.smKp);  // k of SM slots that can be evicted, else 0
    uint16_t *eseq = reinterpret_cast<uint16_t *>(smem + lay.eseq);
    uint16_t *tb = reinterpret_cast<uint16_t *>(smem + lay.tb);
    uint32_t *smA = reinterpret_cast<uint32_t *>(smem + lay.smA);  // ring offset | k << 16
    uint32_t *smB = reinterpret_cast<uint32_t *>(smem + lay.smB);  // SN before | candidates before k << 16
    uint32_t *vset = reinterpret_cast<uint32_t *>(smem + lay.vset);
    uint32_t *ber = reinterpret_cast<uint32_t *>(smem + lay.ber);   // cells of evicted tokens
    uint32_t *occ = reinterpret_cast<uint32_t *>(smem + lay.occ);   // occupied cells of the pre-step table
    uint8_t *occ8 = smem + lay.occ;
    uint32_t *fin = reinterpret_cast<uint32_t *>(smem + lay.fin);   // occupied cells as erase and claims change them
    uint8_t *fin8 = smem + lay.fin;
    uint32_t *nkb = reinterpret_cast<uint32_t *>(smem + lay.nkb);   // cells claimed by new keys
    uint64_t *cmask = reinterpret_cast<uint64_t *>(smem + lay.cmask);  // first occurrences of candidates
    uint64_t *emask = reinterpret_cast<uint64_t *>(smem + lay.emask);  // conversion positions
    uint64_t *smask = reinterpret_cast<uint64_t *>(smem + lay.smask);  // evicted SM slots
    uint64_t *rsn = reinterpret_cast<uint64_t *>(smem + lay.rsn);      // SN slots by ring offset
    uint64_t *rsm = reinterpret_cast<uint64_t *>(smem + lay.rsm);      // SM slots by ring offset
    int32_t lim = 0;      // min(prefill, seqLen)
    bool direct = false;  // the direct map is in use (both set once the row's loads are in flight)
    // reuse of regions whose earlier contents are dead by then
    uint32_t *pcell = smA;                                   // classify: provisional cell per position
    uint16_t *undl = eseq;                                   // decide: undecided SM indices
    uint32_t *ecell = smA;                                   // per event: table cell | slot << 16
    uint16_t *lead = eseq;                                   // redo: start cell of each multi-key cluster
    int32_t *ntokv = reinterpret_cast<int32_t *>(smB);       // per event: the token inserted
    uint16_t *snList = evslot;                               // scan -> decide: the evicted SN slots in ring order
    uint16_t *smCell = smKp;                                 // events -> marks: table cell of each evicted SM slot
    // decide -> events: every SM slot's cell (fixed-count kernels, whose
    // topK tokens stay in registers: the row's region is dead after classify)
    uint16_t *smCellX = reinterpret_cast<uint16_t *>(ptok);

    // token of slot s equals t (th = its hash); the compact form checks the
    // hash in LDS and confirms with the HBM row
    auto tok_is = [&](uint32_t s, int32_t t, uint32_t th) -> bool {
        if constexpr (kC) return hv[s] == (th & static_cast<uint32_t>(mask)) && gTok[s] == t;
        else return tok[s] == t;
    };
    auto slot_live = [&](int32_t s) -> bool {
        if constexpr (kC) return hv[s] != HV_EMPTY;
        else return tok[s] >= 0;
    };
    auto slot_home = [&](int32_t s) -> int32_t {
        if constexpr (kC) return static_cast<int32_t>(hv[s]) & mask;
        else return static_cast<int32_t>(ht_hash(tok[s])) & mask;
    };
    // table cell of live slot s's entry, NOCELL when the probe does not find it
    auto cell_find = [&](int32_t s) -> uint32_t {
        int32_t idx = slot_home(s);
        for (int32_t n = 0; n <= mask; ++n) {
            const uint32_t ev = ht[idx];
            if (ev == static_cast<uint32_t>(s + 1)) return static_cast<uint32_t>(idx);
            if (ev == 0u) break;
            idx = (idx + 1) & mask;
        }
        return NOCELL;
    };
    // mark the cell of a live slot's entry in ber (a missing entry is a bound violation)
    auto cell_mark = [&](uint32_t cell) {
        if (cell == NOCELL) atomicOr(&ms.ovf, 1);
        else atomicOr(ber + (cell >> 5), 1u << (cell & 31u));
    };
    // table cell of slot s's entry (NOCELL for an empty slot), marked in ber
    auto cell_of = [&](int32_t s) -> uint32_t {
        uint32_t cell = NOCELL;
        if (slot_live(s)) {
            cell = cell_find(s);
            cell_mark(cell);
        }
        return cell;
    };

    const int32_t P = kFixed ? PM : (K + NT - 1) / NT;    // positions per lane: k = tid + q * NT
    const int32_t Q = kFixed ? QM : (dbs + NT - 1) / NT;  // ring offsets per lane: u = tid + j * NT
    constexpr int PR = kFixed ? PM : 1, QR = kFixed ? QM : 1;
    int32_t tR[PR];    // token of position tid + q * NT
    uint32_t iR[PR];   // its class word (pinf)
    uint32_t vR[QR];   // first-hit code (vt) of ring offset tid + j * NT

    // ---- stage the state row and the topK row; visited flags per slot (vt),
    // the direct map, the table's occupancy bitmap; count live tokens and
    // table entries
    STAMP(0);
    int32_t hand0 = ((KVX_C const int32_t *)gHand)[0];
    int32_t flagw = ((KVX_C const int32_t *)gHand)[1];
    // sieve_hand[row][2]: steps in a row this kernel could not take in parallel
    int32_t hintw = ((KVX_C const int32_t *)gHand)[2];
    // sieve_hand[row][3]: the fingerprint of the tokens a flagged row was left
    // with (a global-space load: this kernel writes the word later)
    const int32_t fpw = gHand[kFingerprintWord];

    // The in-order recurrence (hisp_sieve_update.cpp:115-163) on a staged copy
    // of the row, then its write back: registers for consistent rows of up to
    // 64 slots, else one lane for small tables, else 64 cells/slots per step.
    // canon: the row was consistent before the step.
    __shared__ int32_t s_dirty;
    auto run_inorder = [&](int32_t *tokF, uint16_t *htF, uint8_t *visF, bool canon) {
        STAMP(12);
        if (wave == 0) {
            int32_t hand = hand0;
            Guard g;
            bool dirty = false;
            if (canon && dbs <= 64 && 2 * invCap >= H + 64) {  // scratch: the direct map's region
                dirty = sieve_row_regs((const int32_t *)rt, (int32_t *)rs, (int8_t *)rm, K, seqLen, prefill, dbs, padded, mask, tokF, visF, htF,
                                       reinterpret_cast<uint16_t *>(inv), hand, g);
            } else if (H <= kSmallTable) {
                if (lane == 0) dirty = sieve_row_sequential((const int32_t *)rt, (int32_t *)rs, (int8_t *)rm, K, seqLen, prefill, dbs, padded, mask, tokF, visF, htF, hand, g);
            } else {
                dirty = sieve_row_wave((const int32_t *)rt, (int32_t *)rs, (int8_t *)rm, K, seqLen, prefill, dbs, padded, mask, tokF, visF, htF, hand, g);
            }
            if (lane == 0) {
                gHand[0] = hand;
                gHand[1] = (canon && g.code == 0) ? kCanonFlag : 0;
                // the staged (pre-step) tokens' fingerprint, changed by each
                // replaced token.  (The phase-stamp profiling build leaves it
                // out, its compiler run rejecting the store there: a stale
                // fingerprint only sends the row's next step to the full check.)
#ifndef KVX_SIEVE_PHASE_STAMPS
                gHand[kFingerprintWord] = static_cast<int32_t>(ms.fp0 + g.fpd);
#endif
                gHand[2] = min(hintw, (1 << 30)) + 1;
                s_dirty = dirty ? 1 : 0;
                report_overflow(L.overflowSlot, g.code);
            }
        }
        STAMP(13);
        __syncthreads();
        wg_copy16((KVX_G v4u *)gVis, reinterpret_cast<const v4u *>(visF), static_cast<uint32_t>(visStrideB));
        STAMP(14);
        if (s_dirty) {
            wg_copy16((KVX_G v4u *)gTok, reinterpret_cast<const v4u *>(tokF), static_cast<uint32_t>(padded) * 4u);
            wg_copy16((KVX_G v4u *)gHt, reinterpret_cast<const v4u *>(htF), static_cast<uint32_t>(H) * 2u);
        }
    };

    // Restage the pre-step row from HBM (nothing has been written back) and
    // run the in-order recurrence on it.
    auto restage_and_run = [&](bool canon) {
        __syncthreads();
        int32_t *tokF = reinterpret_cast<int32_t *>(smem);
        uint16_t *htF = reinterpret_cast<uint16_t *>(smem + static_cast<size_t>(padded) * 4u);
        uint8_t *visF = smem + static_cast<size_t>(padded) * 4u + static_cast<size_t>(H) * 2u;
        wg_copy16(reinterpret_cast<v4u *>(tokF), (KVX_G const v4u *)gTok, static_cast<uint32_t>(padded) * 4u);
        wg_copy16(reinterpret_cast<v4u *>(htF), (KVX_G const v4u *)gHt, static_cast<uint32_t>(H) * 2u);
        wg_copy16(reinterpret_cast<v4u *>(visF), (KVX_G const v4u *)gVis, static_cast<uint32_t>(visStrideB));
        __syncthreads();
        run_inorder(tokF, htF, visF, canon);
    };

    // ---- table update for Nev events (ecell[r]: the cell of the token the
    // event's slot loses, NOCELL for none, | slot << 16; ntokv[r]: the token
    // it gains, in event order): erase the lost tokens -- the rightmost
    // marked cell (ber) of each pre-step cluster (occ) leads it and deletes
    // right to left -- then place the gained ones (claims, clusters, redo).
    // setVset: also mark the events' slots visited in vset.  Sets ms.late on
    // a bound violation.  Every thread calls it.
    auto table_update = [&](int32_t Nev, bool setVset) {
        const int32_t Pn = (Nev + NT - 1) / NT;
        Guard g;
        uint32_t ecR = 0;  // ecell of the lane's first event, carried across the phases
        int32_t oldR = 0;  // compact form: the token that event's slot loses (read early, used at placement)
        for (int32_t q = 0; q < Pn; ++q) {
            const int32_t r = tid + q * NT;
            if (r >= Nev) break;
            const uint32_t ec = ecell[r];
            if (q == 0) {
                ecR = ec;
                if constexpr (kC) oldR = gTok[ec >> 16];
            }
            const uint32_t s = ec >> 16;
            if (setVset) atomicOr(vset + (s >> 5), 1u << (s & 31u));
            const uint32_t c = ec & 0xFFFFu;
            if (c == NOCELL) continue;
            bool ld = true;
            int32_t x = (static_cast<int32_t>(c) + 1) & mask;
            for (int32_t n = 0; n <= (H >> 5); ++n) {
                const uint32_t b = static_cast<uint32_t>(x) & 31u, span = 32u - b;
                const uint32_t o = occ[x >> 5] >> b, eb = ber[x >> 5] >> b;
                const uint32_t no = ~o;
                const uint32_t z = no ? static_cast<uint32_t>(__builtin_ctz(no)) : 32u;  // first empty cell
                const uint32_t below = (z >= 32u) ? 0xFFFFFFFFu : ((1u << z) - 1u);
                if (eb & below) {
                    ld = false;
                    break;
                }
                if (z < span) break;
                x = (x + static_cast<int32_t>(span)) & mask;
            }
            if (!ld) continue;
            // the cluster's marked cells right to left; cells left of a
            // deletion keep their pre-step contents, so the occupancy
            // snapshot finds the next marked cell and the cluster's start
            int32_t y = static_cast<int32_t>(c);
            for (int32_t n = 0; n <= H; ++n) {
                rdel_at<kC>(ht, fin, smem + lay.tok, padded, y, mask, g);
                int32_t nx = -1;
                int32_t x2 = (y - 1) & mask;  // scan words leftward from x2
                for (int32_t m = 0; m <= (H >> 5); ++m) {
                    const uint32_t b = static_cast<uint32_t>(x2) & 31u;
                    const uint32_t keep = (b == 31u) ? 0xFFFFFFFFu : ((2u << b) - 1u);  // bits 0..b
                    const uint32_t empt = ~occ[x2 >> 5] & keep, mk = ber[x2 >> 5] & keep;
                    const int32_t hiE = empt ? 31 - __builtin_clz(empt) : -1;  // cluster start boundary
                    const uint32_t live = (hiE >= 0) ? (mk & ~((2u << hiE) - 1u)) : mk;
                    if (live) {
                        nx = (x2 & ~31) + (31 - __builtin_clz(live));
                        break;
                    }
                    if (hiE >= 0) break;
                    x2 = ((x2 & ~31) - 1) & mask;
                }
                if (nx < 0) break;
                y = nx;
            }
        }
        __syncthreads();
        STAMP(7);
        // ---- new tokens; tentative placement (the final occupied cells do
        // not depend on order), entries padded+1+r name the event; the
        // fingerprint's change (each event's slot loses one token, gains one)
        uint32_t fpd = 0;
        for (int32_t q = 0; q < Pn; ++q) {
            const int32_t r = tid + q * NT;
            if (r >= Nev) break;
            const uint32_t s = ((q == 0) ? ecR : ecell[r]) >> 16;
            const int32_t t = ntokv[r];
            int32_t old;
            if constexpr (kC) {
                old = (q == 0) ? oldR : gTok[s];
                hv[s] = static_cast<uint16_t>(ht_hash(t) & static_cast<uint32_t>(mask));
                gTok[s] = t;
            } else {
                old = tok[s];
                tok[s] = t;
            }
            fpd += slot_token_mix(s, t) - slot_token_mix(s, old);
            const int32_t c = lds_claim_bit(fin, static_cast<int32_t>(ht_hash(t)) & mask, mask);
            if (c < 0) {
                g.code = kOverflowProbe;
                continue;
            }
            ht[c] = static_cast<uint16_t>(padded + 1 + r);
            atomicOr(nkb + (c >> 5), 1u << (c & 31));
            ecell[r] = static_cast<uint32_t>(c) | (s << 16);
            if (q == 0) ecR = static_cast<uint32_t>(c) | (s << 16);
        }
        {
            const uint32_t fw = wave_sum(fpd);
            if (lane == 0 && fw != 0u) atomicAdd(&ms.fpd, fw);
        }
        __syncthreads();
        STAMP(8);
        // ---- final cluster of each new key, from the bitmaps: the leftmost
        // new key of a cluster leads it; alone, the key takes its cell, with
        // others the leader queues the cluster's start for the redo
        const int32_t wmask = (H >> 5) - 1;
        for (int32_t q = 0; q < Pn; ++q) {
            const int32_t r = tid + q * NT;
            if (r >= Nev) break;
            const uint32_t ec = (q == 0) ? ecR : ecell[r];
            const int32_t c = static_cast<int32_t>(ec & 0xFFFFu) & mask;  // in range even after a failed claim
            // the bitmap words either side of c, read together
            const int32_t wl = ((c - 1) & mask) >> 5, wr = ((c + 1) & mask) >> 5;
            const uint32_t fL = fin[wl], nL = nkb[wl], fR = fin[wr], nR = nkb[wr];
            asm volatile("" : : "v"(fL), "v"(nL), "v"(fR), "v"(nR));
            // leftwards from c - 1 to the cluster's start: a new key on the
            // way leads instead
            int32_t st = -1;
            bool leads = true;
            {
                int32_t w = wl;
                uint32_t keep = (2u << ((c - 1) & 31)) - 1u, fw = fL, nw0 = nL;  // bits 0..(c-1)&31
                for (int32_t n = 0; n <= wmask; ++n) {
                    if (n > 0) {
                        fw = fin[w];
                        nw0 = nkb[w];
                    }
                    const uint32_t empt = ~fw & keep, nw = nw0 & keep;
                    const int32_t hiE = empt ? 31 - __builtin_clz(empt) : -1;
                    const uint32_t after = (hiE >= 0) ? (nw & ~((2u << hiE) - 1u)) : nw;
                    if (after) {
                        leads = false;
                        break;
                    }
                    if (hiE >= 0) {
                        st = ((w << 5) + hiE + 1) & mask;
                        break;
                    }
                    w = (w - 1) & wmask;
                    keep = 0xFFFFFFFFu;
                }
            }
            if (!leads) continue;
            if (st < 0) {
                g.code = kOverflowProbe;
                continue;
            }
            // rightwards from c + 1 to the cluster's end: another new key
            bool alone = true;
            {
                int32_t w = wr;
                uint32_t sel = 0xFFFFFFFFu << ((c + 1) & 31), fw = fR, nw = nR;
                for (int32_t n = 0; n <= wmask; ++n) {
                    if (n > 0) {
                        fw = fin[w];
                        nw = nkb[w];
                    }
                    const uint32_t empt = ~fw & sel;
                    const uint32_t before = empt ? ((1u << __builtin_ctz(empt)) - 1u) : 0xFFFFFFFFu;
                    if (nw & sel & before) {
                        alone = false;
                        break;
                    }
                    if (empt) break;
                    w = (w + 1) & wmask;
                    sel = 0xFFFFFFFFu;
                }
            }
            if (alone) ht[c] = static_cast<uint16_t>((ec >> 16) + 1u);
            else lead[atomicAdd(&ms.nLead, 1)] = static_cast<uint16_t>(st);
        }
        if (g.code) atomicOr(&ms.late, 1);
        __syncthreads();
        STAMP(9);
        // ---- redo: insert the cluster's new keys in event order.  The cells
        // still holding padded+1+r' are exactly the ones empty when the next
        // key is inserted, so key r probes from its home to the first of them
        // and swaps in; the key it displaces keeps its event number.  One
        // wave per cluster, a lane per cell (longer clusters: one lane).
        const int32_t nLead = ms.nLead;
        const int32_t st0 = lead[wave];  // read with nLead; used only when wave < nLead
        if (nLead == 0) return;
        for (int32_t li = wave; li < nLead; li += NWAVES) {
            const int32_t st = (li == wave) ? st0 : lead[li];
            const int32_t x = (st + static_cast<int32_t>(lane)) & mask;
            uint32_t e = ht[x];
            const uint64_t empt = __ballot(e == 0u);
            if (empt != 0ull) {
                const int32_t Lc = __builtin_ctzll(empt);  // cluster length
                bool un = static_cast<int32_t>(lane) < Lc && e > static_cast<uint32_t>(padded);
                // each unprocessed key's home (offset from st) and final
                // entry, read once; they move with the key when it is displaced
                int32_t hoff = 0;
                uint32_t fe = 0;
                if (un) {
                    const uint32_t rr = e - static_cast<uint32_t>(padded) - 1u;
                    hoff = ((static_cast<int32_t>(ht_hash(ntokv[rr])) & mask) - st) & mask;
                    fe = (ecell[rr] >> 16) + 1u;
                }
                const uint64_t um0 = __ballot(un);
                if (__popcll(um0) == 2) {
                    // two keys at a < b: the earlier event's key takes the
                    // first of them at or after its home, the other the rest
                    const int32_t a = __builtin_ctzll(um0), b = 63 - __builtin_clzll(um0);
                    const uint32_t ea = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e), a));
                    const uint32_t eb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e), b));
                    const uint32_t fa = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fe), a));
                    const uint32_t fb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fe), b));
                    const int32_t x0 = (ea < eb) ? a : b;
                    const int32_t hX = __builtin_amdgcn_readlane(hoff, x0);
                    const int32_t f = (hX <= a) ? a : (hX <= b) ? b : x0;
                    const uint32_t fX = (x0 == a) ? fa : fb, fY = (x0 == a) ? fb : fa;
                    if (static_cast<int32_t>(lane) == a) e = (f == a) ? fX : fY;
                    if (static_cast<int32_t>(lane) == b) e = (f == b) ? fX : fY;
                    un = false;
                }
                for (int32_t it = 0; it < 64; ++it) {
                    uint64_t um = __ballot(un);
                    if (um == 0ull) break;
                    uint32_t best = 0xFFFFFFFFu;
                    int32_t cm = 0;
                    for (; um != 0ull; um &= um - 1ull) {
                        const int32_t l = __builtin_ctzll(um);
                        const uint32_t v = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e), l));
                        if (v < best) {
                            best = v;
                            cm = l;
                        }
                    }
                    const int32_t hl = __builtin_amdgcn_readlane(hoff, cm);
                    const uint32_t fv = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fe), cm));
                    const uint64_t fm = __ballot(un && static_cast<int32_t>(lane) >= hl);
                    const int32_t f = fm ? __builtin_ctzll(fm) : cm;  // the home lies in the cluster
                    const uint32_t ef = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(e), f));
                    const int32_t hf = __builtin_amdgcn_readlane(hoff, f);
                    const uint32_t ff = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(fe), f));
                    if (static_cast<int32_t>(lane) == cm) {
                        e = ef;
                        hoff = hf;
                        fe = ff;
                    }
                    if (static_cast<int32_t>(lane) == f) {
                        e = fv;
                        un = false;
                    }
                }
                if (static_cast<int32_t>(lane) < Lc) ht[x] = static_cast<uint16_t>(e);
            } else if (lane == 0) {
                for (int32_t it = 0; it < H; ++it) {
                    uint32_t mn = 0xFFFFFFFFu;
                    int32_t cm = -1;
                    int32_t y = st;
                    for (int32_t n = 0; n < H && ht[y] != 0; ++n, y = (y + 1) & mask) {
                        const uint32_t ey = ht[y];
                        if (ey > static_cast<uint32_t>(padded) && ey < mn) {
                            mn = ey;
                            cm = y;
                        }
                    }
                    if (cm < 0) break;
                    const uint32_t rr = mn - static_cast<uint32_t>(padded) - 1u;
                    int32_t f = static_cast<int32_t>(ht_hash(ntokv[rr])) & mask;
                    for (int32_t n = 0; n < H && ht[f] <= static_cast<uint32_t>(padded); ++n) f = (f + 1) & mask;
                    ht[cm] = ht[f];
                    ht[f] = static_cast<uint16_t>((ecell[rr] >> 16) + 1u);
                }
            }
        }
        if (g.code) atomicOr(&ms.late, 1);
        __syncthreads();
    };
    {
        const int32_t nt = padded >> 2, nh = H >> 3, nv = visStrideB >> 4;  // 16-byte chunks
        KVX_G const v4u *sT = (KVX_G const v4u *)gTok;
        KVX_G const v4u *sH = (KVX_G const v4u *)gHt;
        KVX_G const v4u *sV = (KVX_G const v4u *)gVis;
        uint32_t nTok = 0, nEnt = 0, fpS = 0;
        // Each region loads into registers of its own, all before the first
        // use: loads that share a destination register across divergent
        // branches would each wait for the previous one to land.
        // pass p: token chunks [2 NT p, 2 NT (p+1)), table chunks [4 NT p, ...),
        // visited chunks [NT p, ...).  The first pass (all of it for rows up
        // to 8192 slots) is straight-line code: in a loop the compiler waits
        // for the previous iteration's loads before reusing their registers.
        auto stage_pass = [&](int32_t p) __attribute__((always_inline)) {
            v4u vT[2], vH[4], vV;
            uint32_t vB[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // unconditional (clamped) loads: a load under a branch makes
                // the compiler wait for it at the branch's end
                const int32_t c = min(2 * NT * p + tid + j * NT, nt - 1);
                vT[j] = sT[c];
                vB[j] = gVis[c >> 1];  // the visited bits of slots 8(c/2)..
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                vH[j] = sH[min(4 * NT * p + tid + j * NT, nh - 1)];
            }
            const int32_t cv = NT * p + tid;
            vV = sV[min(cv, nv - 1)];
            // the direct map's clearing is complete in every wave (the
            // barrier waits for LDS stores only, the loads stay in flight)
            // (the scalar values pass through the statement, so that nothing
            // computed from them is scheduled, and waited for, before the loads)
            if (p == 0) {
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" : "+s"(prefill), "+s"(hand0), "+s"(flagw), "+s"(hintw)
                             : : "memory");
                lim = min(prefill, seqLen);
                direct = !kC && lim > 0 && lim <= invCap;
            }
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int32_t c = 2 * NT * p + tid + j * NT;
                if (c < nt) {
                    const v4u x = vT[j];
                    const int32_t tt[4] = {static_cast<int32_t>(x.x), static_cast<int32_t>(x.y),
                                           static_cast<int32_t>(x.z), static_cast<int32_t>(x.w)};
                    if constexpr (kC) {
                        uint32_t hh[4];
#pragma unroll
                        for (int i = 0; i < 4; ++i) hh[i] = tt[i] < 0 ? HV_EMPTY : (ht_hash(tt[i]) & static_cast<uint32_t>(mask));
                        reinterpret_cast<uint2 *>(hv)[c] = make_uint2(hh[0] | (hh[1] << 16), hh[2] | (hh[3] << 16));
                    } else {
                        reinterpret_cast<v4u *>(tok)[c] = x;
                    }
                    if (4 * c < dbs) {  // first-hit codes of the ring's slots: 0 visited, 0xFFFF not
                        const uint32_t nv4 = ~(vB[j] >> ((c & 1) * 4));  // bit i: slot 4c+i not visited
                        if constexpr (kC) {
                            const uint2 code = make_uint2(((nv4 & 1u) | ((nv4 & 2u) << 15)) * 0xFFFFu,
                                                          (((nv4 >> 2) & 1u) | ((nv4 & 8u) << 13)) * 0xFFFFu);
                            reinterpret_cast<uint2 *>(vt)[c] = code;
                        } else {
                            reinterpret_cast<v4u *>(vt)[c] = v4u{(nv4 & 1u) * 0xFFFFu, ((nv4 >> 1) & 1u) * 0xFFFFu,
                                                                 ((nv4 >> 2) & 1u) * 0xFFFFu, ((nv4 >> 3) & 1u) * 0xFFFFu};
                        }
                    }
                    const int32_t s0 = c * 4, room = dbs - s0;  // slots of the chunk below dbs: i < room
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const bool live = i < room && tt[i] >= 0;
                        nTok += live ? 1u : 0u;
                        // masked, not branched on: the mix is a few full-rate instructions
                        fpS += slot_token_mix(static_cast<uint32_t>(s0 + i), tt[i]) & (i < room ? 0xFFFFFFFFu : 0u);
                        if (direct && i < room && static_cast<uint32_t>(tt[i]) < static_cast<uint32_t>(lim))
                            inv[tt[i]] = static_cast<uint32_t>(s0 + i + 1);
                    }
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int32_t c = 4 * NT * p + tid + j * NT;
                if (c < nh) {
                    const v4u x = vH[j];
                    reinterpret_cast<v4u *>(ht)[c] = x;
                    // occupied cells: min(cell, 1) per 16-bit half, the halves'
                    // bits gathered into bit 2q (low cell) and 2q+1 (high cell)
                    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
                    uint32_t m4[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) asm("v_pk_min_u16 %0, %1, %2" : "=v"(m4[q]) : "v"(w4[q]), "v"(0x00010001u));
                    const uint32_t xo = m4[0] | (m4[1] << 2) | (m4[2] << 4) | (m4[3] << 6);
                    const uint32_t ob = (xo | (xo >> 15)) & 0xFFu;
                    occ8[c] = static_cast<uint8_t>(ob);
                    fin8[c] = static_cast<uint8_t>(ob);
                    nEnt += static_cast<uint32_t>(__popc(ob));
                }
            }
            if (cv < nv) reinterpret_cast<v4u *>(vis)[cv] = vV;
        };
        stage_pass(0);
        if (hand0 < 0 || hand0 >= dbs) hand0 = 0;  // hisp_sieve_update.cpp:108-111
        for (int32_t p = 1; 2 * NT * p < nt || 4 * NT * p < nh || NT * p < nv; ++p) stage_pass(p);
        if (h0) ptok[tid] = t0;
        if (h1) ptok[tid + NT] = t1;
        for (int32_t k = tid + 2 * NT; k < K; k += NT) ptok[k] = rt[k];
        if constexpr (kFixed) {
#pragma unroll
            for (int q = 0; q < PR; ++q) {
                const int32_t k = tid + q * NT;
                tR[q] = (q == 0) ? t0 : (q == 1) ? t1 : (k < K ? ptok[k] : 0);
            }
        }
        for (int32_t i = tid; i < vsetWords; i += NT) vset[i] = 0u;
        for (int32_t i = tid; i < (H >> 5); i += NT) {
            ber[i] = 0u;
            nkb[i] = 0u;
        }
        for (int32_t i = tid; i < 2 * P * NWAVES; i += NT) emask[i] = 0ull;  // emask, smask (adjacent)
        const int32_t dw = static_cast<int32_t>(wave_sum(nTok)) - static_cast<int32_t>(wave_sum(nEnt));
        if (lane == 0 && dw != 0) atomicAdd(&ms.diff, dw);
        const uint32_t fw = wave_sum(fpS);
        if (lane == 0) atomicAdd(&ms.fp0, fw);
    }
    __syncthreads();
    STAMP(1);
    // the flag counts only while the tokens are the ones it was written with
    const bool flagged = flagw == kCanonFlag && ms.fp0 == static_cast<uint32_t>(fpw);
    if (badReq) {  // hisp_sieve_update.cpp:80-87: the row gets the dummy outputs, the state is untouched
        write_dummy_row((int32_t *)rs, (int8_t *)rm, K);
        return;
    }
    // ---- consistency: the table indexes exactly the non-negative tokens of
    // [0, dbs), each at its own slot.  A row this kernel wrote last carries
    // the flag (and the fingerprint of the tokens it left), and then only the
    // counts are checked.
    if (!flagged) {
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
        if (__ballot(bad) != 0ull && lane == 0) atomicOr(&ms.bad, 1);
        __syncthreads();
    }
    // A row whose recent steps all wrapped the hand (the parallel form's
    // bound) retries the parallel form after 8, 16, 32 and then every 64
    // such steps, a row of up to 64 slots (whose decisions in registers cost
    // about what the parallel form does, while a retry that fails restages
    // the row) after 8, 16 and then every 256; the other steps
    // run the in-order recurrence on the row as staged (known consistent when
    // it passed the check above and its entry count matches its live
    // tokens).  Consistent rows
    // of up to 64 slots take the recurrence's decisions in one wave's
    // registers and leave the table to the parallel update: the pre-step
    // token of every evicted slot leaves, the slots' final tokens arrive in
    // the order of the events that placed them.
    const bool retry = dbs <= 64 ? (hintw == 8 || hintw == 16 || (hintw & 255) == 0)
                                 : ((hintw >= 8 && __popc(static_cast<uint32_t>(hintw)) == 1) || (hintw & 63) == 0);
    if (!kC && hintw > 0 && !retry) {
        const bool canon = ms.bad == 0 && ms.diff == 0;
        if (!(canon && dbs <= 64)) {
            run_inorder(tok, ht, vis, canon);
            return;
        }
        if (wave == 0) {
            int32_t hand = hand0, tokFin = -1, lastEv = -1;
            uint64_t vmF = 0;
            const int32_t nev = sieve_row_regs_decide((const int32_t *)rt, (int32_t *)rs, (int8_t *)rm, K, seqLen,
                                                      prefill, dbs, padded, tok, vis, hand, tokFin, lastEv, vmF);
            const bool alive = lastEv >= 0;
            uint32_t rank = 0;  // among the slots' final placements, in event order
            if (nev <= 64) {
                if (alive) atomicOr(&ms.evMask, 1ull << lastEv);
                __threadfence_block();
                rank = static_cast<uint32_t>(__popcll(ms.evMask & ((1ull << (alive ? lastEv : 0)) - 1ull)));
            } else {
                for (int32_t l = 0; l < 64; ++l) {
                    const int32_t x = lane_value(lastEv, l);
                    rank += (x >= 0 && x < lastEv) ? 1u : 0u;
                }
            }
            if (alive) {
                ecell[rank] = cell_of(static_cast<int32_t>(lane)) | (lane << 16);  // the pre-step token's cell
                ntokv[rank] = tokFin;
            }
            if (static_cast<int32_t>(lane) < (dbs + 7) / 8) {  // visited bytes of slots [0, dbs)
                const int32_t b0 = static_cast<int32_t>(lane) * 8;
                const uint32_t keep = (dbs - b0 >= 8) ? 0u : (0xFFu << (dbs - b0)) & 0xFFu;
                vis[lane] = static_cast<uint8_t>((vis[lane] & keep) | (static_cast<uint32_t>(vmF >> b0) & 0xFFu & ~keep));
            }
            const uint64_t am = __ballot(alive);
            if (lane == 0) {
                ms.nEv = __popcll(am);
                ms.handOut = hand;
            }
        }
        __syncthreads();
        STAMP(15);
        const int32_t nAlive = ms.nEv;
        table_update(nAlive, false);
        if (!ms.late && !ms.ovf) {
            wg_copy16((KVX_G v4u *)gVis, reinterpret_cast<const v4u *>(vis), static_cast<uint32_t>(visStrideB));
            if (nAlive > 0) {
                wg_copy16((KVX_G v4u *)gTok, reinterpret_cast<const v4u *>(tok), static_cast<uint32_t>(padded) * 4u);
                wg_copy16((KVX_G v4u *)gHt, reinterpret_cast<const v4u *>(ht), static_cast<uint32_t>(H) * 2u);
            }
            if (tid == 0) {
                gHand[0] = ms.handOut;
                gHand[1] = kCanonFlag;
                gHand[2] = min(hintw, (1 << 30)) + 1;
                gHand[kFingerprintWord] = static_cast<int32_t>(ms.fp0 + ms.fpd);
            }
            return;
        }
        // a bound violation (only a corrupted table): nothing written back
        // but the outputs; the exact recurrence on the row restaged from HBM
        restage_and_run(false);
        return;
    }

    bool fast = ms.bad == 0 && ms.diff == 0;
    const bool canonical = fast;

    // ---- classify every position; dedup the candidates (smallest position
    // of each missing token).  With the direct map a hit is an entry naming a
    // slot and lowers the slot's first-hit code, and a missing token lowers
    // its entry to padded+1+k: both LDS mins, returning nothing, so a
    // position is one map read and one update.  Otherwise one probe of the
    // table does both: a hit stops at its entry (provisional entries only fill
    // empty cells, never the probe path of a resident token), a miss stops at
    // its token's provisional entry padded+1+k or claims the first empty cell
    if (fast && direct) {
        constexpr int PB = kFixed ? PM : 1;  // positions handled together
        for (int32_t q0 = 0; q0 < P; q0 += PB) {
            int32_t tq[PB];
            uint32_t wq[PB], inf[PB];
#pragma unroll
            for (int b = 0; b < PB; ++b) {
                const int32_t k = tid + (q0 + b) * NT;
                const int32_t t = k < K ? (kFixed ? tR[kFixed ? b : 0] : ptok[k]) : -1;
                tq[b] = t;
                inf[b] = (t < 0 || t >= seqLen) ? (CLS_INV << 30) : (t >= prefill) ? (CLS_EXT << 30) : 0xFFFFFFFFu;
                wq[b] = inf[b] == 0xFFFFFFFFu ? inv[t] : 0u;
            }
#pragma unroll
            for (int b = 0; b < PB; ++b) {
                const int32_t k = tid + (q0 + b) * NT;
                if (inf[b] == 0xFFFFFFFFu) {
                    const uint32_t cur0 = wq[b];
                    if (cur0 - 1u < static_cast<uint32_t>(dbs)) {  // first hit of the slot: the smallest k + 1
                        inf[b] = (CLS_HIT << 30) | (cur0 - 1u);
                        if constexpr (!kC) atomicMin(vt + (cur0 - 1u), static_cast<uint32_t>(k + 1));
                    } else {  // the entry stays all ones or provisional: resident entries are written in staging only
                        inf[b] = CLS_CAND << 30;
                        const uint32_t v = static_cast<uint32_t>(padded + 1 + k);
                        if (v < cur0) atomicMin(inv + tq[b], v);
                    }
                }
                if (k >= K) continue;
                if constexpr (kFixed) iR[b] = inf[b];
                else pinf[k] = inf[b];
            }
        }
        __syncthreads();
    } else if (fast) {
        Guard g;
#pragma unroll
        for (int32_t q = 0; q < P; ++q) {
            const int32_t k = tid + q * NT;
            if (k >= K) continue;
            const int32_t t = kFixed ? tR[kFixed ? q : 0] : ptok[k];
            uint32_t inf;
            if (t < 0 || t >= seqLen) {
                inf = CLS_INV << 30;
            } else if (t >= prefill) {
                inf = CLS_EXT << 30;
            } else {
                const uint32_t v = static_cast<uint32_t>(padded + 1 + k);
                const uint32_t th = ht_hash(t);
                int32_t idx = static_cast<int32_t>(th) & mask;
                inf = 0xFFFFFFFFu;
                for (int32_t n = 0; n <= mask; ++n) {
                    uint32_t *w = ht32 + (idx >> 1);
                    const uint32_t sh = (static_cast<uint32_t>(idx) & 1u) * 16u;
                    uint32_t old = *w;
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
                                if constexpr (kC) lds_min16(reinterpret_cast<uint32_t *>(vt), cur - 1u, static_cast<uint16_t>(k + 1));
                                else atomicMin(vt + (cur - 1u), static_cast<uint32_t>(k + 1));
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
            if constexpr (kFixed) iR[q] = inf;
            else pinf[k] = inf;
        }
        if (g.code) atomicOr(&ms.ovf, 1);
        __syncthreads();
        // probing form: every candidate reads its token's final provisional
        // entry before the first occurrences drop them
        if (!direct) {
#pragma unroll
            for (int32_t q = 0; q < P; ++q) {
                const int32_t k = tid + q * NT;
                if (k >= K) continue;
                const uint32_t inf = kFixed ? iR[kFixed ? q : 0] : pinf[k];
                if ((inf >> 30) != CLS_CAND) continue;
                const uint32_t e = ht[pcell[k]];
                const uint32_t ni = (CLS_CAND << 30) | (e - static_cast<uint32_t>(padded) - 1u);
                if constexpr (kFixed) iR[q] = ni;
                else pinf[k] = ni;
            }
            __syncthreads();
        }
        if (ms.ovf) fast = false;
    }
    STAMP(2);

    // ---- candidates' first occurrences (ballot masks in position order) and
    // the ring classes per offset from the hand, with one prefix scan; then
    // the SM list up to the M-th SN slot
    uint32_t snM = 0, smM = 0, M = 0;  // bit j: class of ring offset tid + j * NT
    MaskPrefix snP, smP;                // SN / SM slots before a ring offset
    if (fast) {
        uint32_t cw = 0;
        // the fixed-count kernels issue this half's LDS reads (map entries,
        // first-hit codes) together, unconditionally at clamped indices: a
        // read under a branch is waited for before the next one issues
        uint32_t mq[PR], vq[QR];
        if constexpr (kFixed) {
            if (direct) {
#pragma unroll
                for (int q = 0; q < PR; ++q) {
                    const bool cand = tid + q * NT < K && (iR[q] >> 30) == CLS_CAND;
                    mq[q] = inv[cand ? tR[q] : 0];  // a candidate's token lies below lim <= invCap
                }
            }
#pragma unroll
            for (int j = 0; j < QR; ++j) vq[j] = vt[ring_slot(hand0, min(tid + j * NT, dbs - 1), dbs)];
        }
#pragma unroll
        for (int32_t q = 0; q < P; ++q) {
            const int32_t k = tid + q * NT;
            bool f = false;
            if (k < K) {
                const uint32_t inf = kFixed ? iR[kFixed ? q : 0] : pinf[k];
                if ((inf >> 30) == CLS_CAND) {
                    uint32_t k1;
                    if (direct) {
                        const int32_t t = kFixed ? tR[kFixed ? q : 0] : ptok[k];
                        k1 = (kFixed ? mq[kFixed ? q : 0] : inv[t]) - static_cast<uint32_t>(padded) - 1u;
                        if constexpr (kFixed) iR[q] = (CLS_CAND << 30) | k1;
                        else pinf[k] = (CLS_CAND << 30) | k1;
                    } else {
                        k1 = inf & 0xFFFFu;
                    }
                    f = k1 == static_cast<uint32_t>(k);
                    if (f && !direct) ht[pcell[k]] = 0;
                }
            }
            const uint64_t m = __ballot(f);
            if (lane == 0) cmask[q * NWAVES + wave] = m;
            cw += static_cast<uint32_t>(__popcll(m));
        }
        // ring offsets are lane-strided so that the hand's walk (the first
        // offsets) spreads over all waves
#pragma unroll
        for (int32_t j = 0; j < Q; ++j) {
            const int32_t u = tid + j * NT;
            const uint32_t v = (u < dbs) ? (kFixed ? vq[kFixed ? j : 0] : vt[ring_slot(hand0, u, dbs)]) : 0u;
            if constexpr (kFixed) vR[j] = v;
            const bool sn = u < dbs && v == VT_NONE, sm = u < dbs && v != 0u && v != VT_NONE;
            snM |= (sn ? 1u : 0u) << j;
            smM |= (sm ? 1u : 0u) << j;
            const uint64_t bsn = __ballot(sn), bsm = __ballot(sm);
            if (lane == 0) {
                rsn[j * NWAVES + wave] = bsn;
                rsm[j * NWAVES + wave] = bsm;
            }
        }
        if (lane == 0 && cw != 0u) atomicAdd(&ms.M, cw);
        __syncthreads();
        M = ms.M;
        MaskPrefix::init_pair(snP, rsn, Q * NWAVES, smP, rsm, Q * NWAVES, lane);
        if (M > 0) {
            // only SM slots with fewer than M SN slots before them can be
            // reached (the SN slots before a slot are all evicted first, and
            // each conversion is paid by an SM eviction before it): the list
            // is a prefix of the SM slots in ring order
            MaskPrefix cp;
            cp.init(cmask, P * NWAVES, lane);
#pragma unroll
            for (int32_t j = 0; j < Q; ++j) {
                const int32_t e = j * NWAVES + wave;
                if (snP.base(e) >= M) continue;  // the whole block lies past the M-th SN slot
                const bool isSM = (smM >> j) & 1u, isSN = (snM >> j) & 1u;
                const int32_t u = tid + j * NT;
                // this wave's own ballots of block j, rebuilt from the lane's class
                // bits (no LDS read)
                const uint32_t nsn = snP.base(e) + lanes_below(__ballot(isSN)),
                               nsm = smP.base(e) + lanes_below(__ballot(isSM));
                uint32_t k = 0;
                if (isSM) k = (kFixed ? vR[kFixed ? j : 0] : static_cast<uint32_t>(vt[ring_slot(hand0, u, dbs)])) - 1u;
                uint32_t cc;
                if constexpr (kFixed) {
                    // one mask entry per lane (P * NWAVES <= 64): the prefix of entry
                    // k/64 and its bits below k, the two LDS reads issued together
                    const int32_t e2 = static_cast<int32_t>(k >> 6);
                    const uint32_t pre = static_cast<uint32_t>(__shfl(static_cast<int>(cp.ex), e2));
                    cc = pre + static_cast<uint32_t>(__popcll(cmask[e2] & ((1ull << (k & 63u)) - 1ull)));
                } else {
                    cc = cp.before(static_cast<int32_t>(k >> 6), k & 63u);
                }
                if (isSM && nsn < M) {
                    smA[nsm] = static_cast<uint32_t>(u) | (k << 16);
                    smB[nsm] = nsn | (cc << 16);
                    smKp[nsm] = (cc > nsn) ? static_cast<uint16_t>(k) : static_cast<uint16_t>(0);
                }
                // every SN slot before the M-th is evicted: listed for the
                // lookup of its token's table cell
                if (isSN && nsn < M) snList[nsn] = static_cast<uint16_t>(ring_slot(hand0, u, dbs));
                if (isSN && nsn + 1u == M) ms.nSM = static_cast<int32_t>(nsm);
            }
            if (tid == 0 && snP.total < M) ms.nSM = static_cast<int32_t>(smP.total);
        }
        __syncthreads();
    }
    STAMP(3);

    // ---- decide the SM slots.  In ring order, slot i (k_i, need0_i = SN
    // slots before it, cc_i = candidates before k_i) is evicted iff the
    // events before k_i outnumber the event being served on arrival:
    //   cc_i + #{evicted j < i: k_j < k_i} > need0_i + #{evicted j < i},
    // i.e. a_i = cc_i - need0_i - 1 >= D_i = #{evicted j < i: k_j > k_i}.
    // a_i < 0: passed.  a_i >= U_i = #{j < i: a_j >= 0, k_j > k_i} (a bound
    // on D_i): evicted.  The rest (rare) are settled in ring order.
    int32_t nSM = 0;
    if (fast) {
        nSM = ms.nSM;
        int32_t G = 1;  // lanes per SM slot for the U count
        while (G < 16 && 2 * G * nSM <= NT) G <<= 1;
        const int32_t part = tid & (G - 1);
        const uint4 *kp4 = reinterpret_cast<const uint4 *>(smKp);
        for (int32_t i = tid / G; i < nSM; i += NT / G) {
            const uint32_t eb = smB[i];
            const uint32_t ki = smA[i] >> 16;  // read with eb: a read under the branch would wait on its own
            const int32_t ai = static_cast<int32_t>(eb >> 16) - static_cast<int32_t>(eb & 0xFFFFu) - 1;
            uint16_t dec = 0;  // 0 passed, 1 evicted, 2 undecided
            if (ai >= 0) {
                uint32_t U = 0;
                const int32_t nb = i >> 3;  // blocks of 8 entirely before i
                // two entries per 32-bit word: saturating k_j - k_i, capped at
                // 1, summed in 16-bit halves
                const uint32_t kk = ki | (ki << 16), ones = 0x00010001u;
                u16x2 acc = {0, 0};
#pragma unroll 2
                for (int32_t b = part; b < nb; b += G) {
                    const uint4 x = kp4[b];
                    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        uint32_t gt;
                        asm("v_pk_sub_u16 %0, %1, %2 clamp\n\tv_pk_min_u16 %0, %0, %3"
                            : "=&v"(gt)
                            : "v"(w4[q]), "v"(kk), "v"(ones));
                        acc += __builtin_bit_cast(u16x2, gt);
                    }
                }
                U += static_cast<uint32_t>(acc.x) + static_cast<uint32_t>(acc.y);
                if ((i & 7) != 0 && (nb & (G - 1)) == part) {
                    const uint4 x = kp4[nb];
                    const uint32_t w4[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int32_t j = 8 * nb + 2 * q;
                        U += (j < i && (w4[q] & 0xFFFFu) > ki) ? 1u : 0u;
                        U += (j + 1 < i && (w4[q] >> 16) > ki) ? 1u : 0u;
                    }
                }
                // sum over the slot's G lanes (aligned within a row of 16) into its first lane
                int Ui = static_cast<int>(U);
                if (G >= 2) Ui += __builtin_amdgcn_update_dpp(0, Ui, 0x101, 0xF, 0xF, true);  // row_shl:1
                if (G >= 4) Ui += __builtin_amdgcn_update_dpp(0, Ui, 0x102, 0xF, 0xF, true);  // row_shl:2
                if (G >= 8) Ui += __builtin_amdgcn_update_dpp(0, Ui, 0x104, 0xF, 0xF, true);  // row_shl:4
                if (G >= 16) Ui += __builtin_amdgcn_update_dpp(0, Ui, 0x108, 0xF, 0xF, true); // row_shl:8
                U = static_cast<uint32_t>(Ui);
                dec = (ai >= static_cast<int32_t>(U)) ? 1 : 2;
                if (part == 0) {
                    if (dec == 2) {
                        // (the short list's settle finds them by their mark)
                        if (nSM > 4 * 64) undl[atomicAdd(&ms.nUnd, 1)] = static_cast<uint16_t>(i);
                    } else {  // evicted: its first hit converts
                        atomicOr(reinterpret_cast<unsigned long long *>(smask) + (i >> 6), 1ull << (i & 63));
                        atomicOr(reinterpret_cast<unsigned long long *>(emask) + (ki >> 6), 1ull << (ki & 63u));
                    }
                }
            }
            if (part == 0) tb[i] = dec;
        }
        const int32_t nSNev = static_cast<int32_t>(min(M, snP.total));
        if (nSM <= 4 * 64) {
            // short list: the last wave to finish the first pass settles the
            // undecided slots in ring order from registers (a lane per SM
            // slot of each 64-slot chunk); every wave then looks up the table
            // cells of the evicted SN slots, 64 at a time from a shared counter
            int32_t old = 0;
            if (lane == 0) {
                __threadfence_block();
                old = atomicAdd(&ms.nDone, 1);
            }
            if (lane_value(old, 0) == NWAVES - 1) {
                __threadfence_block();
                uint32_t kq[4], bq[4], tq[4];
                uint64_t evq[4], undq[4];
                // all twelve reads issued together (clamped, unconditional)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int32_t j = min(c * 64 + static_cast<int32_t>(lane), max(nSM - 1, 0));
                    tq[c] = tb[j];
                    kq[c] = smA[j];
                    bq[c] = smB[j];
                }
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const bool ok = c * 64 + static_cast<int32_t>(lane) < nSM;
                    kq[c] = ok ? (kq[c] >> 16) : 0u;
                    bq[c] = ok ? bq[c] : 0u;
                    evq[c] = __ballot(ok && tq[c] == 1u);
                    undq[c] = __ballot(ok && tq[c] == 2u);
                }
                if ((undq[0] | undq[1] | undq[2] | undq[3]) != 0ull) {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        for (uint64_t und = undq[c]; und != 0ull; und &= und - 1ull) {
                            const int f = __builtin_ctzll(und);
                            const uint32_t ki = static_cast<uint32_t>(lane_value(static_cast<int>(kq[c]), f));
                            const uint32_t eb = static_cast<uint32_t>(lane_value(static_cast<int>(bq[c]), f));
                            const int32_t ai = static_cast<int32_t>(eb >> 16) - static_cast<int32_t>(eb & 0xFFFFu) - 1;
                            uint32_t d = static_cast<uint32_t>(__popcll(__ballot(kq[c] > ki) & evq[c] & ((1ull << f) - 1ull)));
#pragma unroll
                            for (int c2 = 0; c2 < c; ++c2) d += static_cast<uint32_t>(__popcll(__ballot(kq[c2] > ki) & evq[c2]));
                            if (ai >= static_cast<int32_t>(d)) evq[c] |= 1ull << f;
                        }
                    }
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int32_t j = c * 64 + static_cast<int32_t>(lane);
                        if ((undq[c] >> lane) & 1ull) {
                            const bool evd = (evq[c] >> lane) & 1ull;
                            tb[j] = evd ? 1 : 0;
                            if (evd) {
                                atomicOr(reinterpret_cast<unsigned long long *>(smask) + (j >> 6), 1ull << (j & 63));
                                atomicOr(reinterpret_cast<unsigned long long *>(emask) + (kq[c] >> 6), 1ull << (kq[c] & 63u));
                            }
                        }
                    }
                }
            }
            // lookups 64 at a time from a shared counter: the evicted SN slots'
            // cells, then (fixed-count kernels) every SM slot's cell, kept
            // unmarked in smCellX for the events phase, which marks the ones
            // the settled decisions evict; the waves not settling do them
            const int32_t nLook = nSNev + (kFixed ? nSM : 0);
            for (;;) {
                int32_t x0 = 0;
                if (lane == 0) x0 = atomicAdd(&ms.snNext, 64);
                x0 = lane_value(x0, 0);
                if (x0 >= nLook) break;
                const int32_t x = x0 + static_cast<int32_t>(lane);
                if (x < nSNev) {
                    const int32_t sl = snList[x];
                    vt[sl] = static_cast<uint16_t>(cell_of(sl));
                } else if (x < nLook) {  // an SM slot holds the token its first hit found: live
                    const int32_t i = x - nSNev;
                    smCellX[i] = static_cast<uint16_t>(cell_find(ring_slot(hand0, static_cast<int32_t>(smA[i] & 0xFFFFu), dbs)));
                }
            }
            __syncthreads();
        } else {
        __syncthreads();
        // undecided slots, one wave each: count the evictions already settled
        // before them (L) and the undecided ones before them with a larger k
        // (X); with X == 0, D = L exactly.  A concurrent settle of j < i reads
        // either as undecided (counted in X) or settled (counted exactly):
        // both are safe.
        const int32_t nUnd = ms.nUnd;
        // the waves not settling undecided slots look up the table cells of
        // the evicted SN slots meanwhile (all waves, after, when none is free;
        // with no undecided slots the lookups overlap the events phase, which
        // does not touch what they write)
        const int32_t busy = nUnd == 0 ? 0 : nUnd <= 64 ? min(nUnd, NWAVES) : 1;
        auto sn_cells = [&](int32_t first, int32_t stride) {
            for (int32_t x = first; x < nSNev; x += stride) {
                const int32_t sl = snList[x];
                vt[sl] = static_cast<uint16_t>(cell_of(sl));
            }
        };
        if (wave >= busy) sn_cells(tid - busy * 64, NT - busy * 64);
        if (nUnd > 0 && nUnd <= 64) {
            // undecided slots (few): one wave each counts the evictions
            // settled in the first pass before it with a larger k (L) and
            // files it under its rank in ring order; the last wave to finish
            // then walks them in ring order, adding the evictions among the
            // undecided ones before each: D = L + #{undecided j < i evicted, k_j > k_i}
            if (wave < nUnd) {
                for (int32_t e = wave; e < nUnd; e += NWAVES) {
                    const int32_t i = static_cast<int32_t>(undl[e]);
                    const uint32_t ki = smA[i] >> 16;
                    uint32_t l = 0;
                    for (int32_t j = static_cast<int32_t>(lane); j < i; j += 64) {
                        l += (tb[j] == 1 && (smA[j] >> 16) > ki) ? 1u : 0u;
                    }
                    l = wave_sum(l);
                    const bool before = static_cast<int32_t>(lane) < nUnd && static_cast<int32_t>(undl[lane]) < i;
                    const int32_t rank = __popcll(__ballot(before));
                    if (lane == 0) {
                        ms.uL[rank] = l;
                        ms.ui[rank] = static_cast<uint16_t>(i);
                    }
                }
                int32_t old = 0;
                if (lane == 0) {
                    __threadfence_block();
                    old = atomicAdd(&ms.nDone, 1);
                }
                const int32_t waves = nUnd < NWAVES ? nUnd : NWAVES;
                if (lane_value(old, 0) == waves - 1) {  // every other wave has filed its slots
                    __threadfence_block();
                    const bool act = static_cast<int32_t>(lane) < nUnd;
                    const int32_t i = act ? static_cast<int32_t>(ms.ui[lane]) : 0;
                    const uint32_t ki = act ? (smA[i] >> 16) : 0u;
                    const uint32_t eb = act ? smB[i] : 0u;
                    const int32_t ai = static_cast<int32_t>(eb >> 16) - static_cast<int32_t>(eb & 0xFFFFu) - 1;
                    const uint32_t l = act ? ms.uL[lane] : 0u;
                    uint64_t ev = 0;  // undecided slots found evicted so far (by rank)
                    for (int32_t e = 0; e < nUnd; ++e) {
                        const uint32_t ke = static_cast<uint32_t>(lane_value(static_cast<int>(ki), e));
                        const int32_t ae = lane_value(ai, e);
                        const uint32_t le = static_cast<uint32_t>(lane_value(static_cast<int>(l), e));
                        const uint64_t larger = __ballot(static_cast<int32_t>(lane) < e && ki > ke);
                        const uint32_t d = le + static_cast<uint32_t>(__popcll(larger & ev));
                        if (ae >= static_cast<int32_t>(d)) ev |= 1ull << e;
                    }
                    if (act) {
                        const bool evd = (ev >> lane) & 1ull;
                        tb[i] = evd ? 1 : 0;
                        if (evd) {
                            atomicOr(reinterpret_cast<unsigned long long *>(smask) + (i >> 6), 1ull << (i & 63));
                            atomicOr(reinterpret_cast<unsigned long long *>(emask) + (ki >> 6), 1ull << (ki & 63u));
                        }
                    }
                }
            }
        } else if (nUnd > 64) {  // many undecided slots: one wave settles them in ring order
            if (wave == 0) {
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
                        if (lane == 0) {
                            const bool evd = ai >= static_cast<int32_t>(d);
                            tb[i] = evd ? 1 : 0;
                            if (evd) {
                                atomicOr(reinterpret_cast<unsigned long long *>(smask) + (i >> 6), 1ull << (i & 63));
                                atomicOr(reinterpret_cast<unsigned long long *>(emask) + (ki >> 6), 1ull << (ki & 63u));
                            }
                        }
                    }
                }
            }
        }
        if (busy == NWAVES) sn_cells(tid, NT);
        if (nUnd > 0) __syncthreads();
        }
    }
    STAMP(4);

    // ---- ballots of the evicted SM slots (in ring order) and of the event
    // positions (candidates' first occurrences and conversions -- first hits
    // of evicted SM slots); then the eviction prefix per SM slot and the
    // event sequence in position order
    int32_t N = 0;
    if (fast) {
        const int32_t Ps = (nSM + NT - 1) / NT;
        // the fixed-count kernels read this wave's own mask entries (evicted SM
        // slots; event positions) and, for the short list, its SM slots'
        // looked-up cells once, together with the prefix inputs
        constexpr int PS2 = kFixed ? 2 : 1;  // nSM <= topK <= 2 NT
        uint64_t entS[PS2], entE[PR];
        uint32_t cellX = 0;
        const bool smPre = kFixed && nSM <= 4 * 64;
        if constexpr (kFixed) {
#pragma unroll
            for (int q = 0; q < PS2; ++q) entS[q] = smask[q * NWAVES + wave];
#pragma unroll
            for (int q = 0; q < PR; ++q) entE[q] = cmask[q * NWAVES + wave] | emask[q * NWAVES + wave];
            if (smPre) cellX = smCellX[min(tid, 4 * 64 - 1)];
        }
        MaskPrefix sp, ep;
        // events: candidates' first occurrences (cmask) and conversions (emask)
        MaskPrefix::init_pair(sp, smask, Ps * NWAVES, ep, cmask, P * NWAVES, lane, emask);
        const uint32_t T = sp.total;
        for (int32_t q = 0; q < Ps; ++q) {
            const int32_t i = tid + q * NT;
            const uint64_t es = kFixed ? entS[kFixed ? q : 0] : sp.ent(q * NWAVES + wave);
            const uint32_t pre = sp.base(q * NWAVES + wave) + lanes_below(es);
            if (i < nSM) {
                const uint32_t tk = static_cast<uint32_t>((es >> lane) & 1ull);  // evicted
                tb[i] = static_cast<uint16_t>(pre | (tk << 15));
            }
        }
        if (tid == 0) tb[nSM] = static_cast<uint16_t>(T);
        N = static_cast<int32_t>(M + T);
#pragma unroll
        for (int32_t q = 0; q < P; ++q) {
            const int32_t k = tid + q * NT;
            const uint64_t ee = kFixed ? entE[kFixed ? q : 0] : ep.ent(q * NWAVES + wave);
            const uint32_t pre = ep.base(q * NWAVES + wave) + lanes_below(ee);
            if (k < K && ((ee >> lane) & 1ull)) {
                // the event inserts the position's own token: a candidate's,
                // or for a conversion the token of the slot its hit lost
                eseq[pre] = static_cast<uint16_t>(k);
                ntokv[pre] = kFixed ? tR[kFixed ? q : 0] : ptok[k];
            }
        }
        if (ep.total != static_cast<uint32_t>(N)) fast = false;  // same value in every wave
        // table cells of the evicted SM slots' tokens (looked up while
        // deciding when the short list's lookups ran there)
        for (int32_t q = 0; q < Ps; ++q) {
            const int32_t i = tid + q * NT;
            const uint64_t es = kFixed ? entS[kFixed ? q : 0] : smask[i >> 6];
            if (i < nSM && ((es >> (i & 63)) & 1ull)) {
                uint32_t cell;
                if (smPre) {
                    cell = cellX;  // smPre: nSM <= 256, so q == 0 and i == tid
                    cell_mark(cell);
                } else {
                    cell = cell_of(ring_slot(hand0, static_cast<int32_t>(smA[i] & 0xFFFFu), dbs));
                }
                smCell[i] = static_cast<uint16_t>(cell);
            }
        }
        __syncthreads();
    }
    STAMP(5);

    // ---- marks per ring offset: evicted by event r (at position p), or
    // passed while serving event p; each event's slot and the table cell of
    // the token it evicts (ber)
    if (fast) {
        Guard g;
        const uint32_t nSMu = static_cast<uint32_t>(nSM);  // tb[nSM] = T covers the unlisted SM slots
        uint32_t ntk = 0;
#pragma unroll
        for (int32_t j = 0; j < Q; ++j) {
            const int32_t u = tid + j * NT;
            const int32_t e = j * NWAVES + wave;
            // with N SN slots before the block, every offset in it has r >= N
            if (snP.base(e) >= static_cast<uint32_t>(N)) continue;
            const bool isSN = (snM >> j) & 1u, isSM = (smM >> j) & 1u;
            const uint32_t nsn2 = snP.base(e) + lanes_below(__ballot(isSN)),
                           nsm2 = min(smP.base(e) + lanes_below(__ballot(isSM)), nSMu);
            if (u >= dbs) continue;
            const int32_t s = ring_slot(hand0, u, dbs);
            // the evicted token's table cell, looked up (and marked in ber)
            // while deciding (SN: vt) or in the events phase (SM: smCell);
            // read with tb so the three reads wait together
            const uint32_t cellSN = vt[s], cellSM = smCell[nsm2];
            const uint32_t tbv = tb[nsm2];
            const int32_t r = static_cast<int32_t>(nsn2 + (tbv & 0x7FFFu));
            if (r < N) {
                const uint32_t p = eseq[r];
                if (isSN || (isSM && (tbv & 0x8000u))) {
                    evslot[p] = static_cast<uint16_t>(s);
                    ++ntk;
                    if (r == N - 1) ms.uEnd = u + 1;
                    if (isSM) {
                        const uint32_t v0 = kFixed ? vR[kFixed ? j : 0] : static_cast<uint32_t>(vt[s]);
                        vt[s] = static_cast<uint16_t>(VT_EVICTED | (v0 - 1u));
                    }
                    const uint32_t cell = isSN ? (cellSN & 0xFFFFu) : cellSM;
                    ecell[r] = cell | (static_cast<uint32_t>(s) << 16);
                } else {
                    vt[s] = static_cast<uint16_t>(VT_PASSED | p);
                }
            }
        }
        ntk = wave_sum(ntk);
        if (lane == 0 && ntk) atomicAdd(&ms.nTakes, static_cast<int32_t>(ntk));
        if (g.code) atomicOr(&ms.ovf, 1);
        __syncthreads();
        if (ms.nTakes != N || ms.ovf) fast = false;  // the hand would wrap within the step
    }
    STAMP(6);

    if (fast) {
        const int32_t uEnd = ms.uEnd;
        // ---- outputs and visited bits set this step (vset); erase the
        // evicted tokens: the rightmost marked cell of each pre-step cluster
        // (from the occupancy snapshot) leads it and deletes right to left.
        // The fixed-count kernels read every position's code (hit) and
        // event slot (candidate) together, at clamped indices.
        uint32_t vq[PR], eq[PR];
        if constexpr (kFixed) {
#pragma unroll
            for (int q = 0; q < PR; ++q) {
                const bool ok = tid + q * NT < K;
                const uint32_t cls = iR[q] >> 30, x = iR[q] & 0xFFFFu;
                vq[q] = vt[(ok && cls == CLS_HIT) ? x : 0u];
                eq[q] = evslot[(ok && cls == CLS_CAND) ? x : 0u];
            }
        }
#pragma unroll
        for (int32_t q = 0; q < P; ++q) {
            const int32_t k = tid + q * NT;
            if (k >= K) continue;
            const uint32_t inf = kFixed ? iR[kFixed ? q : 0] : pinf[k];
            const uint32_t cls = inf >> 30;
            int32_t slot = -1;
            int8_t miss = 0;
            if (cls == CLS_EXT) {
                slot = padded + ((kFixed ? tR[kFixed ? q : 0] : ptok[k]) - prefill);
            } else if (cls == CLS_HIT) {
                const uint32_t s0 = inf & 0xFFFFu;
                const uint16_t v = kFixed ? vq[kFixed ? q : 0] : vt[s0];
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
                slot = kFixed ? eq[kFixed ? q : 0] : evslot[k1];
                miss = (k1 == static_cast<uint32_t>(k)) ? 1 : 0;
            }
            rs[k] = slot;
            rm[k] = miss;
        }
        table_update(N, true);
        STAMP(10);
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
                ((KVX_G uint32_t *)gVis)[w] = (vis32[w] & ~clr) | (w < vsetWords ? vset[w] : 0u);
            }
            if (N > 0) {
                if constexpr (!kC) {  // compact: written in place
                    wg_copy16((KVX_G v4u *)gTok, reinterpret_cast<const v4u *>(tok), static_cast<uint32_t>(padded) * 4u);
                }
                wg_copy16((KVX_G v4u *)gHt, reinterpret_cast<const v4u *>(ht), static_cast<uint32_t>(H) * 2u);
            }
            if (tid == 0) {
                int32_t hd = hand0;
                if (N > 0) {
                    hd = hand0 + uEnd;
                    while (hd >= dbs) hd -= dbs;
                }
                gHand[0] = hd;
                gHand[1] = kCanonFlag;
                gHand[kFingerprintWord] = static_cast<int32_t>(ms.fp0 + ms.fpd);
                if (hintw != 0) gHand[2] = 0;
            }
            STAMP(11);
            DBGVAL(13, __builtin_amdgcn_s_memrealtime());
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
    restage_and_run(canonical);
}

}  // namespace

template <bool kC, int PM, int QM>
static hipError_t set_limit_one(size_t bytes)
{
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update_fast<kC, PM, QM>),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

constexpr int kP1 = kFixP, kQ1 = kFixQ1, kQ2 = kFixQ2;

hipError_t sieve_fast_set_lds_limit(size_t bytes)
{
    hipError_t e = hipSuccess;
    if ((e = set_limit_one<false, 0, 0>(bytes)) != hipSuccess) return e;
    if ((e = set_limit_one<false, kP1, kQ1>(bytes)) != hipSuccess) return e;
    if ((e = set_limit_one<false, kP1, kQ2>(bytes)) != hipSuccess) return e;
    if ((e = set_limit_one<true, 0, 0>(bytes)) != hipSuccess) return e;
    if ((e = set_limit_one<true, kP1, kQ1>(bytes)) != hipSuccess) return e;
    return set_limit_one<true, kP1, kQ2>(bytes);
}

template <bool kC>
static void launch_one(const KvxLaunch<HispSieveUpdateArgs> &L, size_t ldsBytes, hipStream_t stream)
{
    const HispSieveUpdateArgs &a = L.a;
    const uint32_t P = (a.topK + NT - 1) / NT, Q = (a.deviceBufferSize + NT - 1) / NT;
    if (P == kP1 && Q == kQ1) {
        hipLaunchKernelGGL((kvx_sieve_update_fast<kC, kP1, kQ1>), dim3(a.maxNumReqs), dim3(NT), ldsBytes, stream, L);
    } else if (P == kP1 && Q == kQ2) {
        hipLaunchKernelGGL((kvx_sieve_update_fast<kC, kP1, kQ2>), dim3(a.maxNumReqs), dim3(NT), ldsBytes, stream, L);
    } else {
        hipLaunchKernelGGL((kvx_sieve_update_fast<kC, 0, 0>), dim3(a.maxNumReqs), dim3(NT), ldsBytes, stream, L);
    }
}

hipError_t launch_sieve_update_fast(const HispSieveUpdateArgs &a, uint64_t overflowSlot, size_t ldsBytes, bool compact,
                                    hipStream_t stream)
{
    KvxLaunch<HispSieveUpdateArgs> L{a, overflowSlot};
    if (compact) launch_one<true>(L, ldsBytes, stream);
    else launch_one<false>(L, ldsBytes, stream);
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
