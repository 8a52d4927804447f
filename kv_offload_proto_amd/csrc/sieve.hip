// SIEVE (ring CLOCK) miss detector and hash-table build for gfx950.
//
// Semantics follow kvops/kernel/hisp_sieve_update.cpp:17-176 and
// hisp_sieve_ht_init.cpp:14-60 of the reference; the state format is that of
// hisp_kernel_common.h (uint16 entries = slot+1, Knuth hash, linear probing,
// backward-shift deletion, visited bitmap 8 slots per byte).
//
// Layout on the device: one workgroup per batch row.  The request's state row
// (tokens padded*4 B, hash table htSize*2 B, visited visStrideB B) is staged
// in LDS when it fits the per-workgroup LDS limit (160 KiB on gfx950) and
// written back at the end; otherwise the kernel works on the HBM-resident row
// in place.  Within the row, positions are processed in order -- the exact
// sequential recurrence of the reference -- by one wave whose probes, sweeps
// and shifts take 64 cells or slots per step (LDS-staged), or by one lane
// (HBM-resident).
#include "kvx_internal.h"
#include "sieve_common.h"

namespace kvx {
namespace {

using namespace sieve;

template <bool kLds>
__global__ __launch_bounds__(256) void kvx_sieve_update(KvxLaunch<HispSieveUpdateArgs> L)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int32_t s_dirty;
    const HispSieveUpdateArgs &a = L.a;
    const int32_t topK = static_cast<int32_t>(a.topK);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t visStrideB = static_cast<int32_t>(a.visitedStrideB);
    const int32_t maxNumReqs = static_cast<int32_t>(a.maxNumReqs);
    const int32_t htSize = static_cast<int32_t>(a.htSize);
    const int32_t poolSize = static_cast<int32_t>(a.poolSize);
    const int32_t bid = blockIdx.x;
    if (bid >= maxNumReqs) return;

    int32_t numReal = *reinterpret_cast<const int32_t *>(a.numReal);
    if (numReal > maxNumReqs) numReal = maxNumReqs;  // hisp_sieve_update.cpp:31-34

    int32_t *rs = reinterpret_cast<int32_t *>(a.topKDeviceSlots) + static_cast<int64_t>(bid) * topK;
    int8_t *rm = reinterpret_cast<int8_t *>(a.isMiss) + static_cast<int64_t>(bid) * topK;
    if (bid >= numReal) {  // padding rows (:72-78)
        write_dummy_row(rs, rm, topK);
        return;
    }
    const int64_t reqIdx = reinterpret_cast<const int64_t *>(a.reqPoolIndices)[bid];
    if (reqIdx < 0 || reqIdx >= poolSize) {  // (:80-88)
        write_dummy_row(rs, rm, topK);
        return;
    }
    const int32_t seqLen = reinterpret_cast<const int32_t *>(a.seqLens)[bid];
    const int32_t prefill = reinterpret_cast<const int32_t *>(a.prefillLens)[reqIdx];
    const int32_t *rt = reinterpret_cast<const int32_t *>(a.topkIndices) + static_cast<int64_t>(bid) * topK;
    int32_t *gTok = reinterpret_cast<int32_t *>(a.deviceBufferTokens) + reqIdx * padded;
    uint8_t *gVis = reinterpret_cast<uint8_t *>(a.deviceBufferVisited) + reqIdx * visStrideB;
    uint16_t *gHt = reinterpret_cast<uint16_t *>(a.deviceBufferHt) + reqIdx * htSize;
    int32_t *gHand = reinterpret_cast<int32_t *>(a.sieveHand) + reqIdx * kHandStride;

    int32_t *tok = gTok;
    uint8_t *vis = gVis;
    uint16_t *ht = gHt;
    if constexpr (kLds) {
        tok = reinterpret_cast<int32_t *>(smem);
        ht = reinterpret_cast<uint16_t *>(smem + static_cast<size_t>(padded) * 4);
        vis = smem + static_cast<size_t>(padded) * 4 + static_cast<size_t>(htSize) * 2;
        block_copy16(tok, gTok, static_cast<uint32_t>(padded) * 4u);
        block_copy16(ht, gHt, static_cast<uint32_t>(htSize) * 2u);
        block_copy16(vis, gVis, static_cast<uint32_t>(visStrideB));
        __syncthreads();
    }

    if (kLds && htSize > kSmallTable) {
        if (threadIdx.x < 64) {  // one wave: 64 cells/slots per probe, sweep and shift step
            int32_t hand = *gHand;
            if (hand < 0 || hand >= dbs) hand = 0;  // (:108-111)
            Guard g;
            const bool dirty =
                sieve_row_wave(rt, rs, rm, topK, seqLen, prefill, dbs, padded, htSize - 1, tok, vis, ht, hand, g);
            if (threadIdx.x == 0) {
                *gHand = hand;
                s_dirty = dirty ? 1 : 0;
                report_overflow(L.overflowSlot, g.code);
            }
        }
    } else if (threadIdx.x == 0) {
        int32_t hand = *gHand;
        if (hand < 0 || hand >= dbs) hand = 0;  // (:108-111)
        Guard g;
        const bool dirty =
            sieve_row_sequential(rt, rs, rm, topK, seqLen, prefill, dbs, padded, htSize - 1, tok, vis, ht, hand, g);
        *gHand = hand;
        s_dirty = dirty ? 1 : 0;
        report_overflow(L.overflowSlot, g.code);
    }
    if constexpr (kLds) {
        __syncthreads();
        block_copy16(gVis, vis, static_cast<uint32_t>(visStrideB));
        if (s_dirty) {  // (:165-172)
            block_copy16(gTok, tok, static_cast<uint32_t>(padded) * 4u);
            block_copy16(gHt, ht, static_cast<uint32_t>(htSize) * 2u);
        }
    }
}

// hisp_sieve_ht_init.cpp:14-60: block b -> (layer b/numReqs, pool row
// reqStart + b%numReqs); clear the row's table, insert tokens[s] >= 0 for
// s < dbs in increasing s, comparing through the HBM tokens row.
template <bool kLds>
__global__ __launch_bounds__(256) void kvx_sieve_ht_init(KvxLaunch<HispSieveHtInitArgs> L)
{
    extern __shared__ __align__(16) uint8_t smem[];
    const HispSieveHtInitArgs &a = L.a;
    const int32_t numReqs = static_cast<int32_t>(a.numReqs);
    const int32_t layerNum = static_cast<int32_t>(a.layerNum);
    const int32_t poolSize = static_cast<int32_t>(a.poolSize);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t htSize = static_cast<int32_t>(a.htSize);
    const int32_t b = blockIdx.x;
    if (b >= layerNum * numReqs) return;
    const int32_t layer = b / numReqs;
    const int64_t reqIdx = static_cast<int64_t>(a.reqStart) + b % numReqs;
    if (reqIdx < 0 || reqIdx >= poolSize) return;

    const int32_t *tok = reinterpret_cast<const int32_t *>(a.deviceBufferTokens) +
                         (static_cast<int64_t>(layer) * poolSize + reqIdx) * padded;
    uint16_t *gHt = reinterpret_cast<uint16_t *>(a.deviceBufferHt) +
                    (static_cast<int64_t>(layer) * poolSize + reqIdx) * htSize;
    uint16_t *ht = kLds ? reinterpret_cast<uint16_t *>(smem) : gHt;
    uint4 *ht16 = reinterpret_cast<uint4 *>(ht);
    for (int32_t i = threadIdx.x; i < htSize / 8; i += blockDim.x) ht16[i] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    if (threadIdx.x == 0) {
        Guard g;
        for (int32_t s = 0; s < dbs && g.code == 0; ++s) {
            const int32_t t = tok[s];
            if (t >= 0) ht_insert(ht, tok, padded, t, s, htSize - 1, g);
        }
        report_overflow(L.overflowSlot, g.code);
    }
    if constexpr (kLds) {
        __syncthreads();
        block_copy16(gHt, ht, static_cast<uint32_t>(htSize) * 2u);
    }
}

// Parallel form of the same build for tables that fit LDS, one 256-lane
// workgroup per (layer, pool row).  Linear probing fills the same set of
// cells whatever the insertion order: with n(c) keys homed at cell c, the
// backlog b(c) = max(0, b(c-1) + n(c) - 1) counts the keys homed at or before
// c still waiting for a cell, and c is in use iff b(c-1) + n(c) >= 1.  A key
// never leaves the cluster (maximal run of used cells) holding its home, so
// inserting each cluster's keys alone, in slot order, gives the sequential
// layout.  A later slot with a token already inserted meets the earlier entry
// on its probe path and is skipped (hisp_kernel_common.h:97-112); both share
// a home, so it is dropped from its home's list instead.
//
// LDS: table (2H B), per-home list ends (2H B, 16-bit, paired for atomics),
// the slots bucketed by home (2 B each), the used-cell bitmap (H/8 B), the
// scans' lane values (2 KiB); nothing static.
constexpr int32_t kInitThreads = 256;

__global__ __launch_bounds__(kInitThreads) void kvx_sieve_ht_init_par(KvxLaunch<HispSieveHtInitArgs> L)
{
    extern __shared__ __align__(16) uint8_t smem[];
    const HispSieveHtInitArgs &a = L.a;
    const int32_t numReqs = static_cast<int32_t>(a.numReqs);
    const int32_t layerNum = static_cast<int32_t>(a.layerNum);
    const int32_t poolSize = static_cast<int32_t>(a.poolSize);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t H = static_cast<int32_t>(a.htSize);
    const int32_t mask = H - 1;
    const int32_t b = blockIdx.x;
    if (b >= layerNum * numReqs) return;
    const int32_t layer = b / numReqs;
    const int64_t reqIdx = static_cast<int64_t>(a.reqStart) + b % numReqs;
    if (reqIdx < 0 || reqIdx >= poolSize) return;
    const int32_t *tok = reinterpret_cast<const int32_t *>(a.deviceBufferTokens) +
                         (static_cast<int64_t>(layer) * poolSize + reqIdx) * padded;
    uint16_t *gHt = reinterpret_cast<uint16_t *>(a.deviceBufferHt) +
                    (static_cast<int64_t>(layer) * poolSize + reqIdx) * H;

    const int32_t tid = threadIdx.x;
    const int32_t per = H / kInitThreads;  // cells (homes) per lane, >= 4 (H >= 1024)
    const int32_t c0 = tid * per;
    uint16_t *ht = reinterpret_cast<uint16_t *>(smem);
    uint16_t *ends = ht + H;  // per home: inclusive prefix of the counts, then (after the scatter) the list start
    uint32_t *ends32 = reinterpret_cast<uint32_t *>(ends);
    uint16_t *keys = ends + H;
    uint32_t *used = reinterpret_cast<uint32_t *>(keys + ((dbs + 7) & ~7));
    int32_t *sP = reinterpret_cast<int32_t *>(used + H / 32);  // the scans' lane values
    int32_t *sQ = sP + kInitThreads;
    int32_t &sTotal = sQ[kInitThreads];
    constexpr uint16_t kGone = 0xFFFF;  // a dropped duplicate or an inserted slot
    auto is_used = [&](int32_t c) { return (used[c >> 5] >> (c & 31)) & 1u; };

    // clear the table, the counts and the bitmap
    for (int32_t i = tid; i < H / 4; i += kInitThreads) reinterpret_cast<uint4 *>(smem)[i] = make_uint4(0, 0, 0, 0);  // 4H bytes
    for (int32_t i = tid; i < H / 32; i += kInitThreads) used[i] = 0u;
    __syncthreads();
    // keys per home (two 16-bit counts per word; a count stays below 2^16)
    for (int32_t s = tid; s < dbs; s += kInitThreads) {
        const int32_t t = tok[s];
        if (t >= 0) {
            const int32_t h = static_cast<int32_t>(ht_hash(t)) & mask;
            atomicAdd(ends32 + (h >> 1), 1u << ((h & 1) * 16));
        }
    }
    __syncthreads();
    // inclusive prefix over the homes: lane sums, a scan of the lane sums, then the lane's run
    int32_t sum = 0;
    for (int32_t i = 0; i < per; ++i) sum += ends[c0 + i];
    sP[tid] = sum;
    __syncthreads();
    for (int32_t o = 1; o < kInitThreads; o <<= 1) {
        const int32_t v = tid >= o ? sP[tid - o] : 0;
        __syncthreads();
        sP[tid] += v;
        __syncthreads();
    }
    int32_t run = sP[tid] - sum;
    for (int32_t i = 0; i < per; ++i) {
        run += ends[c0 + i];
        ends[c0 + i] = static_cast<uint16_t>(run);
    }
    if (tid == kInitThreads - 1) sTotal = sP[kInitThreads - 1];
    __syncthreads();
    // bucket the slots by home: each key takes the next position down from
    // its home's end, so the entry ends as the home's list start
    for (int32_t s = tid; s < dbs; s += kInitThreads) {
        const int32_t t = tok[s];
        if (t >= 0) {
            const int32_t h = static_cast<int32_t>(ht_hash(t)) & mask;
            const uint32_t sh = static_cast<uint32_t>(h & 1) * 16u;
            const uint32_t old = atomicSub(ends32 + (h >> 1), 1u << sh);
            keys[((old >> sh) & 0xFFFFu) - 1u] = static_cast<uint16_t>(s);
        }
    }
    __syncthreads();
    const int32_t total = sTotal;
    auto list_end = [&](int32_t h) { return h + 1 < H ? static_cast<int32_t>(ends[h + 1]) : total; };
    // per home: slot order, duplicates dropped, the count kept in the (still
    // empty) table cell; the lane's segment as a backlog map x -> max(P, x + Q)
    int32_t P = 0, Q = 0;
    for (int32_t i = 0; i < per; ++i) {
        const int32_t h = c0 + i;
        const int32_t st = ends[h], en = list_end(h);
        for (int32_t j = st + 1; j < en; ++j) {
            const uint16_t v = keys[j];
            int32_t k = j;
            for (; k > st && keys[k - 1] > v; --k) keys[k] = keys[k - 1];
            keys[k] = v;
        }
        int32_t n = 0;
        for (int32_t j = st; j < en; ++j) {
            bool dup = false;
            if (j > st) {
                const int32_t tj = tok[keys[j]];
                for (int32_t k = st; k < j && !dup; ++k) dup = keys[k] != kGone && tok[keys[k]] == tj;
            }
            if (dup) keys[j] = kGone;
            else ++n;
        }
        ht[h] = static_cast<uint16_t>(n);
        P = max(0, P + n - 1);
        Q += n - 1;
    }
    sP[tid] = P;
    sQ[tid] = Q;
    __syncthreads();
    // compose the segment maps in cell order (inclusive scan); the ring's map
    // has Q < 0 (fewer keys than cells), so its fixed point -- the backlog
    // entering cell 0 -- is its P
    for (int32_t o = 1; o < kInitThreads; o <<= 1) {
        const bool has = tid >= o;
        const int32_t pe = has ? sP[tid - o] : 0, qe = has ? sQ[tid - o] : 0;
        __syncthreads();
        if (has) {
            const int32_t pc = sP[tid], qc = sQ[tid];
            sP[tid] = max(pc, pe + qc);
            sQ[tid] = qe + qc;
        }
        __syncthreads();
    }
    const int32_t x0 = sP[kInitThreads - 1];
    int32_t x = tid == 0 ? x0 : max(sP[tid - 1], x0 + sQ[tid - 1]);
    for (int32_t i = 0; i < per; ++i) {
        const int32_t h = c0 + i;
        const int32_t n = ht[h];
        if (x + n >= 1) atomicOr(used + (h >> 5), 1u << (h & 31));
        x = max(0, x + n - 1);
        ht[h] = 0;
    }
    __syncthreads();
    // each cluster, by the lane holding its first cell: its keys in slot
    // order, each to the first free cell from its home (a cluster of L cells
    // costs O(L^2) LDS reads: short at these load factors, at most H/2 keys)
    for (int32_t i = 0; i < per; ++i) {
        const int32_t c = c0 + i;
        if (!is_used(c) || is_used((c - 1) & mask)) continue;
        int32_t len = 0;
        while (len < H && is_used((c + len) & mask)) ++len;
        for (;;) {
            int32_t best = 0x10000, bj = -1, bh = 0;
            for (int32_t u = 0; u < len; ++u) {
                const int32_t h = (c + u) & mask;
                const int32_t en = list_end(h);
                for (int32_t j = ends[h]; j < en; ++j) {
                    const int32_t v = keys[j];
                    if (v == kGone) continue;
                    if (v < best) {
                        best = v;
                        bj = j;
                        bh = h;
                    }
                    break;  // the home's list is in slot order
                }
            }
            if (bj < 0) break;
            keys[bj] = kGone;
            int32_t y = bh;
            for (int32_t n = 0; n < len && ht[y] != 0; ++n) y = (y + 1) & mask;
            ht[y] = static_cast<uint16_t>(best + 1);
        }
    }
    __syncthreads();
    block_copy16(gHt, ht, static_cast<uint32_t>(H) * 2u);
}

// Admission build for tables beyond the parallel form's LDS budget, one
// 256-lane workgroup per (layer, pool row); the table of the sequential
// inserts (hisp_sieve_ht_init.cpp:14-60).  Every lane first marks its slots'
// tokens in an LDS bitmap: a token met twice (a later slot would meet the
// earlier entry and insert nothing) or one beyond the bitmap sends the row to
// the one-lane inserts.  Otherwise one wave inserts 64 slots at a time over a
// three-level bitmap of used cells: each key's first free cell at or after its
// home in the table before the batch, then the free cells in increasing
// order, each taken by the earliest key of the batch whose first free cell is
// at or before it -- linear probing's cells in slot order.  A batch whose
// probe wraps past the table's end, or that has fewer free cells than keys at
// or after its last first-free cell (its sweep could wrap), inserts its keys
// one by one.
constexpr int32_t kWaveInitTokenBits = 1 << 20;
constexpr int32_t kFreeCap = 4;  // free cells counted between neighbouring first-free cells

__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__global__ __launch_bounds__(kInitThreads) void kvx_sieve_ht_init_wave(KvxLaunch<HispSieveHtInitArgs> L)
{
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ int32_t sInOrder;
    const HispSieveHtInitArgs &a = L.a;
    const int32_t numReqs = static_cast<int32_t>(a.numReqs);
    const int32_t layerNum = static_cast<int32_t>(a.layerNum);
    const int32_t poolSize = static_cast<int32_t>(a.poolSize);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t H = static_cast<int32_t>(a.htSize);  // a power of two in [65536, 2^20] (launcher)
    const int32_t mask = H - 1;
    const int32_t b = blockIdx.x;
    if (b >= layerNum * numReqs) return;
    const int32_t layer = b / numReqs;
    const int64_t reqIdx = static_cast<int64_t>(a.reqStart) + b % numReqs;
    if (reqIdx < 0 || reqIdx >= poolSize) return;
    // global-space pointers: flat accesses would also count against the LDS
    // wait counter, and every bitmap read would wait for the table's stores
    typedef __attribute__((address_space(1))) const int32_t GTok;
    typedef __attribute__((address_space(1))) uint16_t GCell;
    typedef uint32_t Chunk __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(1))) Chunk GChunk;
    GTok *tok = reinterpret_cast<GTok *>(a.deviceBufferTokens) + (static_cast<int64_t>(layer) * poolSize + reqIdx) * padded;
    GCell *gHt = reinterpret_cast<GCell *>(a.deviceBufferHt) + (static_cast<int64_t>(layer) * poolSize + reqIdx) * H;
    const int32_t tid = threadIdx.x;
    const int32_t lane = static_cast<int32_t>(__lane_id());

    // ---- clear the table; repeated and out-of-range tokens
    uint32_t *tbits = reinterpret_cast<uint32_t *>(smem);
    for (int32_t i = tid; i < H / 8; i += kInitThreads) reinterpret_cast<GChunk *>(gHt)[i] = Chunk{0u, 0u, 0u, 0u};
    for (int32_t i = tid; i < kWaveInitTokenBits / 128; i += kInitThreads) {
        reinterpret_cast<uint4 *>(smem)[i] = make_uint4(0, 0, 0, 0);
    }
    if (tid == 0) sInOrder = 0;
    __syncthreads();
    bool inOrder = false;
    for (int32_t s = tid; s < dbs; s += kInitThreads) {
        const int32_t t = tok[s];
        if (t < 0) continue;
        if (t >= kWaveInitTokenBits) {
            inOrder = true;
            continue;
        }
        const uint32_t bit = 1u << (t & 31);
        if (atomicOr(tbits + (t >> 5), bit) & bit) inOrder = true;
    }
    if (__ballot(inOrder) != 0ull && lane == 0) atomicOr(&sInOrder, 1);
    __syncthreads();
    if (sInOrder) {
        if (tid == 0) {
            Guard g;
            for (int32_t s = 0; s < dbs && g.code == 0; ++s) {
                const int32_t t = tok[s];
                if (t >= 0) ht_insert((uint16_t *)gHt, (const int32_t *)tok, padded, t, s, mask, g);
            }
            report_overflow(L.overflowSlot, g.code);
        }
        return;
    }
    if (tid >= 64) return;  // one wave from here on (no more workgroup barriers)

    // ---- used cells: word w bit i = cell 64w+i; full1 bit w = word w full;
    // full2 bit q = full1 word q full (bits past the last full1 word set)
    const int32_t nW = H >> 6, nS = nW >> 6, nT = (nS + 63) >> 6;
    uint64_t *used = reinterpret_cast<uint64_t *>(smem);
    uint64_t *full1 = used + nW;
    uint64_t *full2 = full1 + nS;
    for (int32_t i = lane; i < nW + nS; i += 64) used[i] = 0ull;
    for (int32_t i = lane; i < nT; i += 64) {
        const int32_t left = nS - i * 64;  // level-1 words covered by this word
        full2[i] = left >= 64 ? 0ull : ~((1ull << left) - 1ull);
    }
    wave_lds_sync();
    // first free cell in [x, H), -1 if none
    auto first_free = [&](int32_t x) -> int32_t {
        if (x >= H) return -1;
        int32_t w = x >> 6;
        const uint64_t u = used[w] | ((1ull << (x & 63)) - 1ull);
        if (u != ~0ull) return (w << 6) + __builtin_ctzll(~u);
        const int32_t w1 = w + 1;
        if (w1 >= nW) return -1;
        int32_t s1 = w1 >> 6;
        uint64_t f = full1[s1] | ((1ull << (w1 & 63)) - 1ull);
        if (f == ~0ull) {
            const int32_t s2 = s1 + 1;
            if (s2 >= nS) return -1;
            int32_t q = s2 >> 6;
            uint64_t g2 = full2[q] | ((1ull << (s2 & 63)) - 1ull);
            while (g2 == ~0ull) {
                if (++q >= nT) return -1;
                g2 = full2[q];
            }
            s1 = (q << 6) + __builtin_ctzll(~g2);
            f = full1[s1];
        }
        w = (s1 << 6) + __builtin_ctzll(~f);
        return (w << 6) + __builtin_ctzll(~used[w]);
    };
    // word w now holds bits u (written by lane 0); the levels above follow
    auto put_word = [&](int32_t w, uint64_t u) {
        if (lane == 0) {
            used[w] = u;
            if (u == ~0ull) {
                const int32_t s1 = w >> 6;
                const uint64_t f = full1[s1] | (1ull << (w & 63));
                full1[s1] = f;
                if (f == ~0ull) full2[s1 >> 6] |= 1ull << (s1 & 63);
            }
        }
        wave_lds_sync();
    };

    Guard g;
    const int32_t nb = (dbs + 63) >> 6;
    int32_t tNext = lane < dbs ? tok[lane] : -1;
    for (int32_t bi = 0; bi < nb && g.code == 0; ++bi) {
        const int32_t s = (bi << 6) + lane;
        const int32_t t = tNext;
        tNext = s + 64 < dbs ? tok[s + 64] : -1;  // the next batch's tokens, in flight meanwhile
        const bool valid = s < dbs && t >= 0;
        const uint64_t keys = __ballot(valid);
        if (keys == 0ull) continue;
        const int32_t h = valid ? static_cast<int32_t>(ht_hash(t)) & mask : 0;
        const int32_t tgt = valid ? first_free(h) : -1;
        const int32_t n = __popcll(keys);
        bool oneByOne = __ballot(valid && tgt < 0) != 0ull;
        // the keys in order of first-free cell (ties in slot order): rank by
        // comparing with every key, then each lane's cell and lane index move
        // to the lane of its rank (keys without a token rank last)
        int32_t rank = 0;
        if (!oneByOne) {
            for (uint64_t m = keys; m != 0ull; m &= m - 1ull) {
                const int32_t j = __builtin_ctzll(m);
                const int32_t tj = __builtin_amdgcn_readlane(tgt, j);
                rank += (tj < tgt || (tj == tgt && j < lane)) ? 1 : 0;
            }
            if (!valid) rank = n + __popcll(~keys & ((1ull << lane) - 1ull));
        }
        const int32_t sortedTgt = __builtin_amdgcn_ds_permute(rank << 2, tgt);
        const int32_t sortedLane = __builtin_amdgcn_ds_permute(rank << 2, lane);
        if (!oneByOne) {
            // free cells at or after the last first-free cell, counted up to the keys
            const int32_t tmax = __builtin_amdgcn_readlane(sortedTgt, n - 1);
            int32_t w = tmax >> 6;
            int32_t room = __popcll(~(used[w] | ((1ull << (tmax & 63)) - 1ull)));
            while (room < n) {
                const int32_t c = __builtin_amdgcn_readfirstlane(first_free((w + 1) << 6));
                if (c < 0) break;
                w = c >> 6;
                room += __popcll(~used[w]);
            }
            oneByOne = room < n;
        }
        if (oneByOne) {
            for (uint64_t m = keys; m != 0ull; m &= m - 1ull) {
                const int32_t j = __builtin_ctzll(m);
                const int32_t hj = __builtin_amdgcn_readlane(h, j);
                int32_t c = __builtin_amdgcn_readfirstlane(first_free(hj));
                if (c < 0) c = __builtin_amdgcn_readfirstlane(first_free(0));  // the probe wraps
                if (c < 0) {
                    g.code = kOverflowProbe;
                    break;
                }
                if (lane == j) gHt[c] = static_cast<uint16_t>(s + 1);
                put_word(c >> 6, used[c >> 6] | (1ull << (c & 63)));
            }
            continue;
        }
        // ---- keys that land on their own first-free cell, all at once.  In
        // rank order, key k's backlog b_k = max(0, b_{k-1} + 1 - D_k), D_k =
        // free cells in [t_{k-1}, t_k): the keys of earlier cells still
        // waiting when the sweep reaches t_k.  b_k = 0: key k takes t_k (the
        // earliest slot among keys of that cell).  D is counted up to
        // kFreeCap, which can only overstate b: such keys take the sweep.
        const bool rv = lane < n;
        const int32_t tk = sortedTgt;
        const int32_t tprev = __shfl_up(tk, 1);
        int32_t D = 0;
        if (rv && lane > 0 && tk > tprev) {
            D = 1;  // t_{k-1} itself
            for (int32_t x = tprev; D < kFreeCap;) {
                x = first_free(x + 1);
                if (x < 0 || x >= tk) break;
                ++D;
            }
        }
        // x -> max(P, x + Q) composed over ranks 0..k; rank 0 starts from b = 0
        int32_t P = 0, Q = lane == 0 ? -(1 << 24) : 1 - D;
        for (int32_t o = 1; o < 64; o <<= 1) {
            const int32_t Pp = __shfl_up(P, o), Qp = __shfl_up(Q, o);
            if (lane >= o) {
                P = max(P, Pp + Q);
                Q = Qp + Q;
            }
        }
        const bool direct = rv && P == 0;
        if (direct) {
            const int32_t slot = (bi << 6) + sortedLane;
            gHt[tk] = static_cast<uint16_t>(slot + 1);
            const int32_t w = tk >> 6;
            const uint64_t bit = 1ull << (tk & 63);
            if ((atomicOr(reinterpret_cast<unsigned long long *>(used) + w, bit) | bit) == ~0ull) {
                const int32_t s1 = w >> 6;
                const uint64_t bit1 = 1ull << (w & 63);
                if ((atomicOr(reinterpret_cast<unsigned long long *>(full1) + s1, bit1) | bit1) == ~0ull) {
                    atomicOr(reinterpret_cast<unsigned long long *>(full2) + (s1 >> 6), 1ull << (s1 & 63));
                }
            }
        }
        wave_lds_sync();
        const uint64_t congRank = __ballot(rv && !direct);
        if (congRank == 0ull) continue;
        // ---- the other keys: the sweep over the free cells, in rank order.
        // Their cells (ranked) move to lanes 0..m-1.
        const int32_t m = __popcll(congRank);
        const bool cg = (congRank >> lane) & 1ull;
        const int32_t below = __popcll(congRank & ((1ull << lane) - 1ull));
        const int32_t dest = cg ? below : m + (lane - below);
        const int32_t cTgt = __builtin_amdgcn_ds_permute(dest << 2, tk);
        const int32_t cLane = __builtin_amdgcn_ds_permute(dest << 2, sortedLane);
        uint64_t wait = 0ull;
        for (int32_t r = 0; r < m; ++r) wait |= 1ull << __builtin_amdgcn_readlane(cLane, r);
        // keys become ready in rank order as the cell passes their first-free
        // cell (which a key placed above may hold: the cell is the first free
        // one at or after it); the word holding the current cell stays in
        // registers
        uint64_t ready = 0ull;
        int32_t next = 0;  // keys of rank below it are ready or placed
        int32_t c = __builtin_amdgcn_readfirstlane(first_free(__builtin_amdgcn_readlane(cTgt, 0)));
        if (c < 0) {  // excluded by the room count; a corrupted launch only
            g.code = kOverflowProbe;
            break;
        }
        int32_t cw = c >> 6;
        uint64_t cbits = used[cw];
        while (wait != 0ull) {
            while (next < m && __builtin_amdgcn_readlane(cTgt, next) <= c) {
                ready |= 1ull << __builtin_amdgcn_readlane(cLane, next);
                ++next;
            }
            if (ready == 0ull) {  // no key waits at or before c: on to the next key's cell
                c = __builtin_amdgcn_readfirstlane(first_free(__builtin_amdgcn_readlane(cTgt, next)));
                if (c < 0) {
                    g.code = kOverflowProbe;
                    break;
                }
                if ((c >> 6) != cw) {
                    cw = c >> 6;
                    cbits = used[cw];
                }
                continue;
            }
            const int32_t j = __builtin_ctzll(ready);
            if (lane == j) gHt[c] = static_cast<uint16_t>(s + 1);
            cbits |= 1ull << (c & 63);
            put_word(cw, cbits);
            ready &= ~(1ull << j);
            wait &= ~(1ull << j);
            if (ready == 0ull) continue;  // the loop moves to the next key's cell
            // the next free cell: in the same word, else through the levels
            const uint64_t above = (c & 63) == 63 ? ~0ull : cbits | ((2ull << (c & 63)) - 1ull);
            if (above != ~0ull) {
                c = (cw << 6) + __builtin_ctzll(~above);
            } else {
                c = __builtin_amdgcn_readfirstlane(first_free((cw + 1) << 6));
                if (c < 0) {  // excluded by the room count; a corrupted launch only
                    g.code = kOverflowProbe;
                    break;
                }
                cw = c >> 6;
                cbits = used[cw];
            }
        }
    }
    if (lane == 0) report_overflow(L.overflowSlot, g.code);
}

}  // namespace

hipError_t sieve_set_lds_limit(size_t bytes)
{
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_ht_init<true>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_ht_init_par),
                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_ht_init_wave),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_sieve_update(const HispSieveUpdateArgs &a, uint64_t overflowSlot, int variant, size_t ldsBytes,
                               hipStream_t stream)
{
    KvxLaunch<HispSieveUpdateArgs> L{a, overflowSlot};
    const dim3 grid(a.maxNumReqs), block(256);
    if (variant == 0) {
        hipLaunchKernelGGL(kvx_sieve_update<true>, grid, block, ldsBytes, stream, L);
    } else {
        hipLaunchKernelGGL(kvx_sieve_update<false>, grid, block, 0, stream, L);
    }
    return hipGetLastError();
}

size_t sieve_ht_init_par_lds(uint32_t htSize, uint32_t dbs)
{
    if (htSize < 1024u || dbs >= htSize) return 0;  // 4+ cells per lane; fewer keys than cells
    return static_cast<size_t>(htSize) * 4u + static_cast<size_t>((dbs + 7u) & ~7u) * 2u + htSize / 8u +
           (2u * kInitThreads + 4u) * 4u;
}

size_t sieve_ht_init_wave_lds(uint32_t htSize, uint32_t dbs)
{
    if (htSize < 65536u || htSize > (1u << 20) || (htSize & (htSize - 1u)) != 0 || dbs >= htSize) return 0;
    const size_t cells = htSize / 8u + htSize / 512u + 8u * ((htSize + 262143u) / 262144u);
    const size_t tokens = kWaveInitTokenBits / 8u;
    return cells > tokens ? cells : tokens;
}

hipError_t launch_sieve_ht_init(const HispSieveHtInitArgs &a, uint64_t overflowSlot, size_t ldsBytes,
                                hipStream_t stream, InitForm form)
{
    KvxLaunch<HispSieveHtInitArgs> L{a, overflowSlot};
    const dim3 grid(a.layerNum * a.numReqs), block(256);
    if (form == InitForm::kParallel) {
        hipLaunchKernelGGL(kvx_sieve_ht_init_par, grid, dim3(kInitThreads), ldsBytes, stream, L);
    } else if (form == InitForm::kWave) {
        hipLaunchKernelGGL(kvx_sieve_ht_init_wave, grid, dim3(kInitThreads), ldsBytes, stream, L);
    } else if (ldsBytes != 0) {
        hipLaunchKernelGGL(kvx_sieve_ht_init<true>, grid, block, ldsBytes, stream, L);
    } else {
        hipLaunchKernelGGL(kvx_sieve_ht_init<false>, grid, block, 0, stream, L);
    }
    return hipGetLastError();
}

}  // namespace kvx
