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
constexpr uint32_t INF_CONV = 1u << 29;  // a hit position that became a conversion
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
#else
#define STAMP(i) \
    do {         \
    } while (0)
#endif

struct Misc {
    int32_t nTok, nEnt, bad, ovf, late;
    int32_t M, nSM, T, nConv, N, smDone, uEnd, nTakes, nMulti;
    uint32_t wt0[NWAVES];
    uint32_t wt1[NWAVES];
};

__device__ __forceinline__ uint32_t lane_id() { return __lane_id(); }

__device__ __forceinline__ uint32_t readlane(uint32_t v, int l)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}

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
// the prefix and the total; ends with a barrier, after which `wt` is free.
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
    __syncthreads();
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

// Algorithm R deletion of the entry at cell c (homes from the tokens row).
__device__ void rdel_at(uint16_t *ht, const int32_t *tok, int32_t ntok, int32_t c, int32_t mask, Guard &g)
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
        const int32_t home = static_cast<int32_t>(ht_hash(tok_at(tok, e, ntok))) & mask;
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

    const FastLayout lay = fast_layout(padded, H, K, visStrideB);
    int32_t *tok = reinterpret_cast<int32_t *>(smem + lay.tok);
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
    uint16_t *cvlist = reinterpret_cast<uint16_t *>(smem + lay.cvlist);
    uint16_t *eseq = reinterpret_cast<uint16_t *>(smem + lay.eseq);
    uint16_t *tb = reinterpret_cast<uint16_t *>(smem + lay.tb);
    uint32_t *smA = reinterpret_cast<uint32_t *>(smem + lay.smA);  // ring offset | k << 16
    uint32_t *smB = reinterpret_cast<uint32_t *>(smem + lay.smB);  // SN before | candidates before k << 16
    uint32_t *ber = reinterpret_cast<uint32_t *>(smem + lay.ber);
    uint32_t *bg = reinterpret_cast<uint32_t *>(smem + lay.bg);
    uint32_t *bm = reinterpret_cast<uint32_t *>(smem + lay.bm);
    uint32_t *bnew = reinterpret_cast<uint32_t *>(smem + lay.bnew);
    // table-update phase reuse of dead regions
    uint32_t *kcell = smA;                                                   // erase cell / new token per event
    uint32_t *lead = smB;                                                    // erase leader flag per event
    uint64_t *mlist = reinterpret_cast<uint64_t *>(smem + lay.ptok);        // multi-cluster keys
    uint64_t *msort = reinterpret_cast<uint64_t *>(smem + lay.smA);         // the same, sorted

    // ---- stage the state row and the topK row
    STAMP(0);
    wg_copy16(tok, gTok, static_cast<uint32_t>(padded) * 4u);
    wg_copy16(ht, gHt, static_cast<uint32_t>(H) * 2u);
    wg_copy16(vis, gVis, static_cast<uint32_t>(visStrideB));
    for (int32_t k = tid; k < K; k += NT) ptok[k] = rt[k];
    for (int32_t i = tid; i < 4 * (H >> 5); i += NT) ber[i] = 0u;  // ber, bg, bm, bnew are contiguous
    if (tid == 0) {
        ms.nTok = ms.nEnt = ms.bad = ms.ovf = ms.late = 0;
        ms.M = ms.nSM = ms.T = ms.nConv = ms.N = ms.smDone = ms.uEnd = ms.nTakes = ms.nMulti = 0;
    }
    int32_t hand0 = gHand[0];
    if (hand0 < 0 || hand0 >= dbs) hand0 = 0;  // hisp_sieve_update.cpp:108-111
    const bool flagged = gHand[1] == kCanonFlag;
    __syncthreads();
    STAMP(1);

    // ---- consistency: the table indexes exactly the non-negative tokens of
    // [0, dbs), each at its own slot.  A row this kernel wrote last carries
    // the flag, and then only the counts are rechecked.
    {
        Guard g;
        uint32_t nTok = 0, nEnt = 0, bad = 0;
        for (int32_t s = tid; s < dbs; s += NT) {
            const int32_t t = tok[s];
            if (t < 0) continue;
            ++nTok;
            if (!flagged && ht_find(ht, tok, padded, t, mask, g) != s) bad = 1u;
        }
        for (int32_t c = tid; c < (H >> 1); c += NT) {
            const uint32_t w = ht32[c];
            nEnt += ((w & 0xFFFFu) != 0u) + ((w >> 16) != 0u);
        }
        nTok = wave_sum(nTok);
        nEnt = wave_sum(nEnt);
        const bool anyBad = __ballot(bad != 0u || g.code != 0) != 0ull;
        if (lane == 0) {
            atomicAdd(&ms.nTok, static_cast<int32_t>(nTok));
            atomicAdd(&ms.nEnt, static_cast<int32_t>(nEnt));
            if (anyBad) atomicOr(&ms.bad, 1);
        }
        for (int32_t s = tid; s < dbs; s += NT) vt[s] = vis_get(vis, s) ? 0 : VT_NONE;
    }
    __syncthreads();
    const bool canonical = ms.bad == 0 && ms.nTok == ms.nEnt;
    bool fast = canonical;
    STAMP(2);

    if (fast) {
        // ---- classify positions; first hit time per slot
        {
            Guard g;
            for (int32_t k = tid; k < K; k += NT) {
                const int32_t t = ptok[k];
                uint32_t inf;
                if (t < 0 || t >= seqLen) {
                    inf = CLS_INV << 30;
                } else if (t >= prefill) {
                    inf = CLS_EXT << 30;
                } else {
                    const int32_t s0 = ht_find(ht, tok, padded, t, mask, g);
                    if (s0 >= 0) {
                        inf = (CLS_HIT << 30) | static_cast<uint32_t>(s0);
                        lds_min16(vt32, static_cast<uint32_t>(s0), static_cast<uint16_t>(k + 1));
                    } else {
                        inf = CLS_CAND << 30;
                    }
                }
                pinf[k] = inf;
            }
            if (g.code) atomicOr(&ms.ovf, 1);
        }
        __syncthreads();
        STAMP(3);
        // ---- dedup: provisional entries padded+1+k; the smallest position of a token wins its cell
        for (int32_t k = tid; k < K; k += NT) {
            if ((pinf[k] >> 30) != CLS_CAND) continue;
            const int32_t t = ptok[k];
            const uint32_t v = static_cast<uint32_t>(padded + 1 + k);
            int32_t idx = static_cast<int32_t>(ht_hash(t)) & mask;
            bool done = false;
            for (int32_t n = 0; n <= mask && !done; ++n) {
                uint32_t *w = ht32 + (idx >> 1);
                const uint32_t sh = (static_cast<uint32_t>(idx) & 1u) * 16u;
                uint32_t old = *reinterpret_cast<volatile uint32_t *>(w);
                for (;;) {
                    const uint32_t cur = (old >> sh) & 0xFFFFu;
                    uint32_t nw;
                    if (cur == 0u) {
                        nw = old | (v << sh);
                    } else if (cur > static_cast<uint32_t>(padded) && ptok[cur - padded - 1] == t) {
                        if (v >= cur) {
                            done = true;
                            break;
                        }
                        nw = (old & ~(0xFFFFu << sh)) | (v << sh);
                    } else {
                        break;  // another key: next cell
                    }
                    const uint32_t prev = atomicCAS(w, old, nw);
                    if (prev == old) {
                        done = true;
                        break;
                    }
                    old = prev;
                }
                idx = (idx + 1) & mask;
            }
            if (!done) atomicOr(&ms.ovf, 1);
        }
        __syncthreads();
        // read back the first occurrence of each candidate token and its cell
        for (int32_t k = tid; k < K; k += NT) {
            if ((pinf[k] >> 30) != CLS_CAND) continue;
            const int32_t t = ptok[k];
            int32_t idx = static_cast<int32_t>(ht_hash(t)) & mask;
            for (int32_t n = 0; n <= mask; ++n) {
                const uint32_t e = ht[idx];
                if (e > static_cast<uint32_t>(padded) && ptok[e - padded - 1] == t) {
                    const uint32_t k1 = e - static_cast<uint32_t>(padded) - 1u;
                    pinf[k] = (CLS_CAND << 30) | k1;
                    if (k1 == static_cast<uint32_t>(k)) kcell[k] = static_cast<uint32_t>(idx);
                    break;
                }
                idx = (idx + 1) & mask;
            }
        }
        __syncthreads();
        // drop the provisional entries (one per first occurrence): the table is the pre-step table again
        for (int32_t k = tid; k < K; k += NT) {
            const uint32_t inf = pinf[k];
            if ((inf >> 30) == CLS_CAND && (inf & 0xFFFFu) == static_cast<uint32_t>(k)) ht[kcell[k]] = 0;
        }
        STAMP(4);
        // ---- candidate prefix counts per position (contiguous chunk per lane)
        {
            const int32_t P = (K + NT - 1) / NT;
            const int32_t k0 = tid * P;
            uint32_t cnt = 0, fl = 0;
            for (int32_t i = 0; i < P; ++i) {
                const int32_t k = k0 + i;
                if (k < K) {
                    const uint32_t inf = pinf[k];
                    const uint32_t f = ((inf >> 30) == CLS_CAND && (inf & 0xFFFFu) == static_cast<uint32_t>(k)) ? 1u : 0u;
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
        __syncthreads();
        STAMP(5);
        if (ms.ovf) fast = false;
    }

    // ---- ring classes per offset from the hand (contiguous chunk per lane)
    const int32_t Q = (dbs + NT - 1) / NT;
    const int32_t u0 = tid * Q;
    uint64_t snM = 0, smM = 0;
    uint32_t preSN = 0, preSM = 0;
    if (fast) {
        for (int32_t j = 0; j < Q; ++j) {
            const int32_t u = u0 + j;
            if (u >= dbs) break;
            const uint16_t v = vt[ring_slot(hand0, u, dbs)];
            if (v == VT_NONE) snM |= 1ull << j;
            else if (v != 0) smM |= 1ull << j;
        }
        const uint32_t cSN = static_cast<uint32_t>(__popcll(snM)), cSM = static_cast<uint32_t>(__popcll(smM));
        const uint32_t qb = bits_for(static_cast<uint32_t>(Q));
        uint32_t tot;
        const uint32_t pre = block_exscan(cSN | (cSM << 16), qb | (qb << 16), ms.wt0, tot);
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
                smA[nsm] = static_cast<uint32_t>(u) | (k << 16);
                smB[nsm] = nsn | (static_cast<uint32_t>(candPre[k]) << 16);
                ++nsm;
            }
        }
        if (tid == 0) ms.nSM = static_cast<int32_t>(tot >> 16);
        __syncthreads();
        STAMP(6);

        // ---- decide the SM slots, one wave, 64 at a time.  need = the event
        // index being served when the hand arrives; cnt = events before k.
        if (wave == 0) {
            const int32_t nSM = ms.nSM;
            int32_t T = 0, nConv = 0, Mtot = ms.M, done = 0;
            bool ended = false;
            for (int32_t b0 = 0; b0 < nSM && !ended; b0 += 64) {
                const int32_t i = b0 + static_cast<int32_t>(lane);
                const bool inb = i < nSM;
                const uint32_t ea = inb ? smA[i] : 0u;
                const uint32_t eb = inb ? smB[i] : 0u;
                const uint32_t k = ea >> 16;
                int32_t need = static_cast<int32_t>(eb & 0xFFFFu) + T;
                int32_t cnt = static_cast<int32_t>(eb >> 16);
                for (int32_t j = 0; j < nConv; ++j) cnt += (static_cast<uint32_t>(cvlist[j]) < k) ? 1 : 0;
                uint64_t active = __ballot(inb);
                uint64_t takenM = 0;
                const int32_t T0 = T;
                for (;;) {
                    const uint64_t tk = __ballot(cnt > need) & active;
                    const uint64_t ur = __ballot(need >= Mtot) & active;
                    const uint64_t any = tk | ur;
                    if (any == 0ull) break;
                    const int f = __builtin_ctzll(any);
                    if ((ur >> f) & 1ull) {  // the events run out before this slot: the walk ends
                        ended = true;
                        break;
                    }
                    takenM |= 1ull << f;
                    const uint32_t t = readlane(k, f);
                    const uint32_t uf = readlane(ea & 0xFFFFu, f);
                    if (lane == 0) {
                        evold[t] = static_cast<uint16_t>(ring_slot(hand0, static_cast<int32_t>(uf), dbs));
                        cvlist[nConv] = static_cast<uint16_t>(t);
                    }
                    ++T;
                    ++nConv;
                    ++Mtot;
                    active &= (f == 63) ? 0ull : (~0ull << (f + 1));
                    if (static_cast<int>(lane) > f) {
                        need += 1;
                        cnt += (k > t) ? 1 : 0;
                    }
                }
                if (inb) {
                    tb[i] = static_cast<uint16_t>((T0 + static_cast<int32_t>(lanes_below(takenM, lane))) |
                                                  (((takenM >> lane) & 1ull) ? 0x8000 : 0));
                }
                done = (b0 + 64 < nSM) ? b0 + 64 : nSM;
            }
            if (lane == 0) {
                ms.T = T;
                ms.nConv = nConv;
                ms.N = Mtot;
                ms.smDone = nSM < done ? nSM : done;
            }
        }
        __syncthreads();
        STAMP(7);
        {
            const int32_t nSM = ms.nSM, T = ms.T, nConv = ms.nConv;
            for (int32_t i = ms.smDone + tid; i <= nSM; i += NT) tb[i] = static_cast<uint16_t>(T);
            for (int32_t j = tid; j < nConv; j += NT) pinf[cvlist[j]] |= INF_CONV;
        }
        __syncthreads();
        // ---- the event sequence: candidates' first occurrences and conversions in position order
        {
            const int32_t P = (K + NT - 1) / NT;
            const int32_t k0 = tid * P;
            uint32_t cnt = 0, fl = 0;
            for (int32_t i = 0; i < P; ++i) {
                const int32_t k = k0 + i;
                if (k < K) {
                    const uint32_t inf = pinf[k];
                    const uint32_t c = inf >> 30;
                    const uint32_t f = ((c == CLS_CAND && (inf & 0xFFFFu) == static_cast<uint32_t>(k)) ||
                                        (c == CLS_HIT && (inf & INF_CONV)))
                                           ? 1u
                                           : 0u;
                    fl |= f << i;
                    cnt += f;
                }
            }
            uint32_t tot;
            uint32_t pre = block_exscan(cnt, bits_for(static_cast<uint32_t>(P)), ms.wt0, tot);
            for (int32_t i = 0; i < P; ++i) {
                if ((fl >> i) & 1u) eseq[pre++] = static_cast<uint16_t>(k0 + i);
            }
            if (tid == 0 && static_cast<int32_t>(tot) != ms.N) ms.ovf = 1;
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
        // ---- outputs and visited bits
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
                }
            } else if (cls == CLS_CAND) {
                const uint32_t k1 = inf & 0xFFFFu;
                slot = evslot[k1];
                miss = (k1 == static_cast<uint32_t>(k)) ? 1 : 0;
            }
            rs[k] = slot;
            rm[k] = miss;
        }
        for (int32_t u = tid; u < uEnd; u += NT) {
            const int32_t s = ring_slot(hand0, u, dbs);
            atomicAnd(vis32 + (s >> 5), ~(1u << (s & 31)));
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t s = evslot[eseq[i]];
            atomicOr(vis32 + (s >> 5), 1u << (s & 31u));
        }
        for (int32_t k = tid; k < K; k += NT) {
            const uint32_t inf = pinf[k];
            if ((inf >> 30) != CLS_HIT) continue;
            const uint32_t s0 = inf & 0xFFFFu;
            const uint16_t v = vt[s0];
            if (v & VT_EVICTED) continue;
            if ((v & VT_PASSED) && static_cast<uint32_t>(k) <= (v & VT_NOCONV)) continue;
            atomicOr(vis32 + (s0 >> 5), 1u << (s0 & 31u));
        }
        __syncthreads();
        STAMP(10);

        // ---- table: erase the evicted tokens (pre-step tokens give the homes)
        Guard g;
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t s = evslot[eseq[i]];
            const int32_t old = tok[s];
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
                else atomicOr(ber + (cell >> 5), 1u << (cell & 31u));
            }
            kcell[i] = cell;
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {  // leader: rightmost marked cell of its cluster
            const uint32_t c = kcell[i];
            uint32_t ld = 0;
            if (c != 0xFFFFFFFFu) {
                ld = 1;
                int32_t x = (static_cast<int32_t>(c) + 1) & mask;
                for (int32_t n = 0; n < H && ht[x] != 0; ++n, x = (x + 1) & mask) {
                    if (bit_get(ber, x)) {
                        ld = 0;
                        break;
                    }
                }
            }
            lead[i] = ld;
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {
            if (!lead[i]) continue;
            const int32_t c = static_cast<int32_t>(kcell[i]);
            rdel_at(ht, tok, padded, c, mask, g);
            int32_t x = (c - 1) & mask;
            for (int32_t n = 0; n < H && ht[x] != 0; ++n, x = (x - 1) & mask) {
                if (bit_get(ber, x)) rdel_at(ht, tok, padded, x, mask, g);
            }
        }
        __syncthreads();
        STAMP(11);
        // ---- token update: read every new token first (conversions re-insert a pre-step token)
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t p = eseq[i];
            kcell[i] = static_cast<uint32_t>((pinf[p] >> 30) == CLS_CAND ? ptok[p] : tok[evold[p]]);
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t s = evslot[eseq[i]];
            tok[s] = static_cast<int32_t>(kcell[i]);
        }
        __syncthreads();
        // ---- inserts: tentative placement (the final occupied cells do not depend on order)
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t s = evslot[eseq[i]];
            const int32_t c = lds_claim16(ht32, static_cast<int32_t>(ht_hash(tok[s])) & mask, mask,
                                          static_cast<uint16_t>(s + 1u));
            if (c < 0) g.code = kOverflowProbe;
            else atomicOr(bnew + (c >> 5), 1u << (c & 31));
        }
        __syncthreads();
        // final cluster of each new key (its start); clusters with two or more new keys are redone
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t s = evslot[eseq[i]];
            int32_t st = static_cast<int32_t>(ht_hash(tok[s])) & mask;
            for (int32_t n = 0; n < H && ht[(st - 1) & mask] != 0; ++n) st = (st - 1) & mask;
            const uint32_t bit = 1u << (st & 31);
            const uint32_t old = atomicOr(bg + (st >> 5), bit);
            if (old & bit) atomicOr(bm + (st >> 5), bit);
        }
        __syncthreads();
        for (int32_t i = tid; i < N; i += NT) {
            const uint32_t p = eseq[i];
            const uint32_t s = evslot[p];
            int32_t st = static_cast<int32_t>(ht_hash(tok[s])) & mask;
            for (int32_t n = 0; n < H && ht[(st - 1) & mask] != 0; ++n) st = (st - 1) & mask;
            if (bit_get(bm, static_cast<uint32_t>(st))) {
                const int32_t q = atomicAdd(&ms.nMulti, 1);
                mlist[q] = (static_cast<uint64_t>(st) << 32) | (static_cast<uint64_t>(p) << 16) | s;
            }
        }
        __syncthreads();
        STAMP(12);
        const int32_t nMulti = ms.nMulti;
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
                int32_t idx = static_cast<int32_t>(ht_hash(tok[s])) & mask;
                for (int32_t n = 0; n < H && ht[idx] != 0; ++n) idx = (idx + 1) & mask;
                ht[idx] = static_cast<uint16_t>(s + 1u);
            }
        }
        if (g.code) atomicOr(&ms.late, 1);
        __syncthreads();
        STAMP(13);
        if (!ms.late) {
            // ---- write back
            wg_copy16(gVis, vis, static_cast<uint32_t>(visStrideB));
            if (N > 0) {
                wg_copy16(gTok, tok, static_cast<uint32_t>(padded) * 4u);
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
        fast = false;
    }

    // ---- fallback: restage the pre-step row from HBM (nothing has been
    // written back) and run the sequential recurrence on it
    __syncthreads();
    wg_copy16(tok, gTok, static_cast<uint32_t>(padded) * 4u);
    wg_copy16(ht, gHt, static_cast<uint32_t>(H) * 2u);
    wg_copy16(vis, gVis, static_cast<uint32_t>(visStrideB));
    __syncthreads();
    __shared__ int32_t s_dirty;
    if (tid == 0) {
        int32_t hand = hand0;
        Guard g;
        const bool dirty = sieve_row_sequential(rt, rs, rm, K, seqLen, prefill, dbs, padded, mask, tok, vis, ht, hand, g);
        gHand[0] = hand;
        gHand[1] = (canonical && g.code == 0) ? kCanonFlag : 0;
        s_dirty = dirty ? 1 : 0;
        report_overflow(L.overflowSlot, g.code);
    }
    __syncthreads();
    wg_copy16(gVis, vis, static_cast<uint32_t>(visStrideB));
    if (s_dirty) {
        wg_copy16(gTok, tok, static_cast<uint32_t>(padded) * 4u);
        wg_copy16(gHt, ht, static_cast<uint32_t>(H) * 2u);
    }
}

}  // namespace

hipError_t sieve_fast_set_lds_limit(size_t bytes)
{
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update_fast),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_sieve_update_fast(const HispSieveUpdateArgs &a, uint64_t overflowSlot, size_t ldsBytes,
                                    hipStream_t stream)
{
    KvxLaunch<HispSieveUpdateArgs> L{a, overflowSlot};
    hipLaunchKernelGGL(kvx_sieve_update_fast, dim3(a.maxNumReqs), dim3(NT), ldsBytes, stream, L);
    return hipGetLastError();
}

}  // namespace kvx

#ifdef KVX_SIEVE_PHASE_STAMPS
extern "C" int kvx_dbg_read_stamps(unsigned long long *out, int rows)
{
    if (rows > 1024) rows = 1024;
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(kvx::kvx_dbg_stamps), sizeof(unsigned long long) * 16 * rows, 0,
                               hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif
