// Row movers for gfx950: decode miss import (host segments -> HBM hot buffer)
// and prefill export (HBM -> host segments).
//
// Semantics follow kvops/kernel/kvc_gather_rows.cpp:12-96 and
// kvc_scatter_rows_alllayer.cpp:11-67 of the reference, with the row
// ownership of kv_layout.h.  The reference moves each row with one HCOMM
// ReadNbi/WriteNbi; here the host segments are pinned host memory mapped
// into the device address space.  The import runs in two launches: winners
// (the last miss position per destination row), then the listing and the
// copy, where 64 workgroups claim 256 positions at a time, list their rows in
// LDS with the reference's queued counts, and move them as 16-byte chunks, 8
// chunks in flight per lane.  A small batch (up to 4096 positions) takes one
// launch instead (below).
//
// Completion: the last workgroup to finish (atomicInc ticket) stores the
// status words with a system-scope release, after every workgroup fenced its
// own row stores.  The reference's per-block Commit/Drain + MTE3 flush has the
// same meaning: all rows of the launch have landed.
#include <cstddef>

#include "kvx_internal.h"

namespace kvx {
namespace {

constexpr int kWaves = 4;          // waves per workgroup
constexpr int kUnroll = 8;         // 16-byte chunks in flight per lane

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
// 16-byte chunk of device or host memory, addressed in the global address
// space (global_* instructions: flat ones also count against the LDS wait
// counter, and the copy loops read their row addresses from LDS)
typedef __attribute__((address_space(1))) u32x4 GVec;
// device and host memory read through global-space pointers, for the same reason
#define KVX_G __attribute__((address_space(1)))

// winner tags (the scratch table): relaxed device-scope max and load
__device__ __forceinline__ void win_max(unsigned long long *p, unsigned long long v)
{
    __hip_atomic_fetch_max((KVX_G unsigned long long *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned long long win_load(const unsigned long long *p)
{
    return __hip_atomic_load((const KVX_G unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct GatherExtra {
    uint64_t segBases[64];
    unsigned long long *win;
    uint64_t winEntries;
    uint32_t *chunkNext;   // next position chunk of the current import
    uint32_t *counters;
    uint32_t *errs;
    uint32_t *tickets;
    uint32_t *epoch;       // winner-tag epoch of the current call (device counter)
    uint32_t fused;
    uint32_t spanRows;
    uint32_t statusWords;
};

struct GatherParams {
    KvxLaunch<KvcGatherArgs> l;  // the reference launch block comes first
    GatherExtra x;
};

struct ExportExtra {
    uint32_t *tickets;
    uint64_t q0;          // first stripe owned by myNode
    uint64_t nStripes;    // stripes owned by myNode inside [rowLo, rowLo+rowCnt)
    uint64_t ownedRows;   // rows owned by myNode inside the range (reference queued / layer)
    uint32_t S;           // stripe rows used for item math (S == 0 mapped to 1)
    uint32_t N;           // node count used for item math (S == 0 mapped to 1)
};

struct ExportParams {
    KvxLaunch<KvcScatterAllArgs> l;
    ExportExtra x;
};

__device__ __forceinline__ int lane_id() { return __lane_id(); }

__device__ __forceinline__ void wave_sync_lds()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void store_status(uint64_t addr, uint64_t word)
{
    __hip_atomic_store(reinterpret_cast<uint64_t *>(addr), word, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Copy `n` rows whose byte addresses sit in src[0..n), dst[0..n) (LDS or
// global) with the whole wave: chunk c covers bytes [16*(c%cpr), +16) of row
// c/cpr.  kUnroll loads are issued before their stores.
__device__ __forceinline__ void wave_copy_rows(const uint64_t *src, const uint64_t *dst, uint32_t n, uint32_t cpr)
{
    const uint32_t total = n * cpr;
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    for (uint32_t base = 0; base < total; base += 64u * kUnroll) {
        u32x4 v[kUnroll];
        uint64_t d[kUnroll];
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) {
            const uint32_t c = base + static_cast<uint32_t>(j) * 64u + lane;
            d[j] = 0;
            if (c < total) {
                const uint32_t r = c / cpr;
                const uint32_t o = (c - r * cpr) * 16u;
                v[j] = __builtin_nontemporal_load(reinterpret_cast<const GVec *>(src[r] + o));
                d[j] = dst[r] + o;
            }
        }
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) {
            if (d[j] != 0) __builtin_nontemporal_store(v[j], reinterpret_cast<GVec *>(d[j]));
        }
    }
}

__device__ __forceinline__ int32_t clamp_num_real(uint64_t numRealAddr, uint32_t maxNumReqs)
{
    int32_t n = *reinterpret_cast<const int32_t *>(numRealAddr);
    if (n > static_cast<int32_t>(maxNumReqs)) n = static_cast<int32_t>(maxNumReqs);  // kvc_gather_rows.cpp:17-21
    return n < 0 ? 0 : n;
}

__device__ __forceinline__ uint64_t win_index(int64_t bid, int32_t slot, uint32_t spanRows)
{
    return static_cast<uint64_t>(bid) * spanRows + static_cast<uint64_t>(slot);
}

// Pass 1: per destination row, the last valid miss position (tagged with the
// call's epoch so the scratch never needs clearing; the epoch lives in device
// memory and the last copy workgroup advances it, so a captured graph replays
// correctly).  Block 0 also zeroes the chunk counter, the queued counters
// and the status words of the nodes this call reports.
__global__ __launch_bounds__(256) void kvx_gather_prep(GatherParams P)
{
    const KvcGatherArgs &a = P.l.a;
    const GatherExtra &x = P.x;
    const int32_t numReal = clamp_num_real(a.numReal, a.maxNumReqs);
    const int64_t total = static_cast<int64_t>(numReal) * a.topK;
    if (blockIdx.x == 0) {
        const uint32_t n0 = x.fused ? 0u : a.myNode;
        const uint32_t n1 = x.fused ? a.nodeNum : a.myNode + 1u;
        if (threadIdx.x == 0) *x.chunkNext = 0u;
        for (uint32_t i = threadIdx.x; i < (n1 - n0) * 8u; i += blockDim.x) {
            x.counters[n0 * 8u + i] = 0u;
            x.errs[n0 * 8u + i] = 0xFFFFFFFFu;  // lowest failing position, min-reduced
        }
        if (a.status != 0) {
            for (uint32_t i = threadIdx.x; i < (n1 - n0) * x.statusWords; i += blockDim.x) {
                const uint32_t node = n0 + i / x.statusWords, b = i % x.statusWords;
                store_status(a.status + node * 64ull + b * 8ull, 0ull);
            }
        }
    }
    const KVX_G int32_t *topk = reinterpret_cast<const KVX_G int32_t *>(a.topkIndices);
    const KVX_G int32_t *slots = reinterpret_cast<const KVX_G int32_t *>(a.topKDeviceSlots);
    const KVX_G int8_t *miss = reinterpret_cast<const KVX_G int8_t *>(a.isMiss);
    const KVX_G int64_t *pool = reinterpret_cast<const KVX_G int64_t *>(a.reqPoolIndices);
    const unsigned long long tagHi = static_cast<unsigned long long>(*x.epoch) << 32;
    for (int64_t p = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; p < total;
         p += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        if (miss[p] == 0) continue;
        const int32_t t = topk[p], s = slots[p];
        if (t < 0 || s < 0 || s >= 65536) continue;
        const int64_t bid = p / a.topK;
        if (pool[bid] < 0) continue;
        const uint64_t d = win_index(bid, s, x.spanRows);
        if (d < x.winEntries) win_max(x.win + d, tagHi | static_cast<unsigned long long>(p));
    }
}

// Pass 2: each workgroup claims kSpan consecutive positions at a time (a
// counter the first pass zeroes), lists the winners owned by the node(s) of
// this call in LDS while counting the queued rows per (node, status word),
// and moves them with its four waves; no row list passes through HBM.
// kSpanBlocks workgroups: fewer concurrent readers of host memory move more
// bytes per second over the link than one workgroup per chunk, and claiming
// chunks keeps them evenly loaded.  The last workgroup (ticket) advances the
// epoch and stores the status words.
constexpr uint32_t kSpan = 256;
constexpr uint32_t kSpanBlocks = 64;

__global__ __launch_bounds__(256) void kvx_gather_span(GatherParams P)
{
    __shared__ uint32_t sCnt[64 * 8];
    __shared__ uint64_t sSrc[kSpan], sDst[kSpan];
    __shared__ uint32_t sN, sEpoch, sChunk;
    __shared__ int sLast;
    const KvcGatherArgs &a = P.l.a;
    const GatherExtra &x = P.x;
    const uint32_t tid = threadIdx.x;
    const uint32_t wave = tid / 64u;
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    const uint32_t cpr = a.rowBytes / 16u;
    const int32_t numReal = clamp_num_real(a.numReal, a.maxNumReqs);
    const int64_t total = static_cast<int64_t>(numReal) * a.topK;
    const int64_t chunks = (total + kSpan - 1) / kSpan;
    const uint64_t ppc = a.positionsPerCore == 0 ? 1ull : a.positionsPerCore;
    const KVX_G int32_t *topk = reinterpret_cast<const KVX_G int32_t *>(a.topkIndices);
    const KVX_G int32_t *slots = reinterpret_cast<const KVX_G int32_t *>(a.topKDeviceSlots);
    const KVX_G int8_t *miss = reinterpret_cast<const KVX_G int8_t *>(a.isMiss);
    const KVX_G int64_t *pool = reinterpret_cast<const KVX_G int64_t *>(a.reqPoolIndices);
    const KVX_G int64_t *hostBase = reinterpret_cast<const KVX_G int64_t *>(a.reqHostBase);
    for (uint32_t i = tid; i < 64u * 8u; i += blockDim.x) sCnt[i] = 0u;
    if (tid == 0) sEpoch = *x.epoch;
    __syncthreads();
    const unsigned long long tagHi = static_cast<unsigned long long>(sEpoch) << 32;
    for (;;) {
        if (tid == 0) {
            sN = 0u;
            sChunk = atomicAdd(x.chunkNext, 1u);
        }
        __syncthreads();
        const int64_t chunk = sChunk;
        if (chunk >= chunks) break;
#pragma unroll
        for (uint32_t q = 0; q < kSpan / 256u; ++q) {
            const int64_t p = chunk * kSpan + q * 256u + tid;
            bool copy = false;
            uint64_t src = 0, dst = 0;
            if (p < total && miss[p] != 0) {
                const int32_t t = topk[p], s = slots[p];
                const int64_t bid = p / a.topK;
                if (t >= 0 && s >= 0 && pool[bid] >= 0) {
                    const uint32_t row = static_cast<uint32_t>(hostBase[bid] + t);  // kvc_gather_rows.cpp:69-73
                    const uint32_t node = kvx_node_of(row, a.stripeRows, a.nodeNum);
                    const bool owned = x.fused ? (node < a.nodeNum) : (node == a.myNode);
                    if (owned) {
                        const uint32_t key = node * 8u + static_cast<uint32_t>(static_cast<uint64_t>(p) / ppc);
                        atomicAdd(&sCnt[key], 1u);
                        bool winner = true;
                        if (s < 65536) {
                            const uint64_t d = win_index(bid, s, x.spanRows);
                            if (d < x.winEntries) winner = (win_load(x.win + d) == (tagHi | static_cast<unsigned long long>(p)));
                        }
                        const uint64_t segRow = kvx_seg_row_of(row, a.stripeRows, a.nodeNum);
                        if (segRow >= a.perLayerSegRows) {  // row outside the segment: report, do not read
                            atomicMin(&x.errs[key], static_cast<uint32_t>(p));
                            winner = false;
                        }
                        copy = winner;
                        const uint64_t segBase = x.fused ? x.segBases[node] : a.segBase;
                        src = segBase + (static_cast<uint64_t>(a.layerOffsetRows) + segRow) * a.rowBytes;
                        dst = a.hotRowBase +
                              (static_cast<uint64_t>(s) + static_cast<uint64_t>(bid) * a.hotReqStrideRows) * a.rowBytes;
                    }
                }
            }
            const uint64_t cm = __ballot(copy);
            uint32_t base = 0;
            if (lane == 0 && cm != 0ull) base = atomicAdd(&sN, static_cast<uint32_t>(__popcll(cm)));
            base = static_cast<uint32_t>(__shfl(static_cast<int>(base), 0));
            if (copy) {
                const uint32_t at = base + static_cast<uint32_t>(__popcll(cm & ((1ull << lane) - 1ull)));
                sSrc[at] = src;
                sDst[at] = dst;
            }
        }
        __syncthreads();
        const uint32_t n = sN, share = (n + kWaves - 1u) / kWaves, r0 = wave * share;
        if (r0 < n) wave_copy_rows(sSrc + r0, sDst + r0, (n - r0 < share) ? n - r0 : share, cpr);
        __syncthreads();  // the list and the chunk are rewritten by the next round
    }
    for (uint32_t i = tid; i < 64u * 8u; i += blockDim.x) {
        if (sCnt[i] != 0u) atomicAdd(&x.counters[i], sCnt[i]);
    }

    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned int ticket = atomicInc(&x.tickets[0], gridDim.x - 1u);
        sLast = (ticket == gridDim.x - 1u) ? 1 : 0;
    }
    __syncthreads();
    if (!sLast) return;
    // the next call's epoch; at the wrap to 0 the tags of 2^32 calls ago
    // could alias, so the table is cleared (once in 2^32 calls)
    if (sEpoch + 1u == 0u) {
        for (uint64_t i = tid; i < x.winEntries; i += blockDim.x) x.win[i] = 0ull;
    }
    if (tid == 0) *x.epoch = sEpoch + 1u;
    if (a.status == 0) return;
    __threadfence();
    const uint32_t n0 = x.fused ? 0u : a.myNode;
    const uint32_t n1 = x.fused ? a.nodeNum : a.myNode + 1u;
    for (uint32_t i = tid; i < (n1 - n0) * x.statusWords; i += blockDim.x) {
        const uint32_t node = n0 + i / x.statusWords, b = i % x.statusWords;
        uint64_t word = 1ull << 32;  // kvc_gather_rows.cpp:29-33, :93
        if (static_cast<int64_t>(b * ppc) < total) {
            const uint32_t q = __hip_atomic_load(&x.counters[node * 8u + b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t e = __hip_atomic_load(&x.errs[node * 8u + b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            word |= (static_cast<uint64_t>(q) << 40) | (e == 0xFFFFFFFFu ? 0u : row_error_code(e));
        }
        store_status(a.status + node * 64ull + b * 8ull, word);
    }
}

// Small batches (max_num_reqs * top_k <= kSmallMaxPositions): the three
// passes in one launch.  A winner is the last miss on its destination row;
// the rows of request b start at b * spanRows, so a row that a later request
// can also reach is one whose slot is at or past spanRows.  Each workgroup
// loads the slots of the requests its own kSmallSpan positions belong to
// into LDS; when none of its own positions has such a slot (the usual case),
// eight lanes per own position look for a later position of the same
// request with the same slot, and no global tags are needed.  Otherwise the
// workgroup tags every position of the call (relaxed device-scope max, as
// the two-launch path does) and reads its own positions' tags.  Each
// workgroup counts the queued rows and errors of all positions in its own
// LDS, then moves the winners among its own positions: the rows spread over
// ceil(positions / kSmallSpan) CUs (one CU reads only a few GB/s from host
// memory), with no counters shared between workgroups.  The last workgroup
// (ticket) advances the epoch and stores the status words.
constexpr uint32_t kSmallMaxPositions = 4096;
constexpr uint32_t kSmallSpan = 32;

__global__ __launch_bounds__(256) void kvx_gather_small(GatherParams P)
{
    __shared__ uint32_t sCnt[64 * 8], sErr[64 * 8];
    __shared__ uint64_t sSrc[kSmallSpan], sDst[kSmallSpan];
    __shared__ int32_t sKey[kSmallMaxPositions];  // slot of each position of the requests met, or -1
    __shared__ uint32_t sN, sEpoch, sLose;         // sLose bit i: own position lo + i is not a winner
    __shared__ int sLast;
    const KvcGatherArgs &a = P.l.a;
    const GatherExtra &x = P.x;
    const uint32_t tid = threadIdx.x;
    const int32_t numReal = clamp_num_real(a.numReal, a.maxNumReqs);
    const int64_t total = static_cast<int64_t>(numReal) * a.topK;  // <= kSmallMaxPositions (host)
    const uint32_t n0 = x.fused ? 0u : a.myNode;
    const uint32_t n1 = x.fused ? a.nodeNum : a.myNode + 1u;
    const uint64_t ppc = a.positionsPerCore == 0 ? 1ull : a.positionsPerCore;
    const KVX_G int32_t *topk = reinterpret_cast<const KVX_G int32_t *>(a.topkIndices);
    const KVX_G int32_t *slots = reinterpret_cast<const KVX_G int32_t *>(a.topKDeviceSlots);
    const KVX_G int8_t *miss = reinterpret_cast<const KVX_G int8_t *>(a.isMiss);
    const KVX_G int64_t *pool = reinterpret_cast<const KVX_G int64_t *>(a.reqPoolIndices);
    const KVX_G int64_t *hostBase = reinterpret_cast<const KVX_G int64_t *>(a.reqHostBase);
    if (blockIdx.x == 0 && a.status != 0) {  // the call's status words read 0 until its rows have landed
        for (uint32_t i = tid; i < (n1 - n0) * x.statusWords; i += blockDim.x) {
            const uint32_t node = n0 + i / x.statusWords, b = i % x.statusWords;
            store_status(a.status + node * 64ull + b * 8ull, 0ull);
        }
    }
    for (uint32_t i = tid; i < 64u * 8u; i += blockDim.x) {
        sCnt[i] = 0u;
        sErr[i] = 0xFFFFFFFFu;  // lowest failing position, min-reduced
    }
    if (tid == 0) {
        sN = 0u;
        sEpoch = *x.epoch;
    }
    __syncthreads();
    const unsigned long long tagHi = static_cast<unsigned long long>(sEpoch) << 32;
    const int64_t lo = static_cast<int64_t>(blockIdx.x) * kSmallSpan, hi = lo + kSmallSpan;
    // the slot of position p when p takes part in the winner rule, else -1
    // (the four reads issued together)
    auto tagged_slot = [&](int64_t p) -> int32_t {
        const int64_t bid = p / a.topK;
        const int8_t m = miss[p];
        const int32_t t = topk[p], s = slots[p];
        const int64_t pl = pool[bid];
        if (m == 0 || t < 0 || s < 0 || s >= 65536 || pl < 0) return -1;
        return win_index(bid, s, x.spanRows) < x.winEntries ? s : -1;
    };
    // the positions of the requests that [lo, hi) meets (at most the call's)
    const int64_t tagLo = lo < total ? (lo / a.topK) * a.topK : total;
    const int64_t tagHiPos = hi < total ? ((hi - 1) / a.topK + 1) * a.topK : total;
    int shared = 0;
    for (int64_t p = tagLo + tid; p < tagHiPos; p += blockDim.x) {
        const int32_t s = tagged_slot(p);
        sKey[p - tagLo] = s;
        shared |= (p >= lo && p < hi && s >= 0 && static_cast<uint32_t>(s) >= x.spanRows) ? 1 : 0;
    }
    if (tid == 0) sLose = 0u;
    const bool global = __syncthreads_or(shared) != 0;
    if (global) {
        for (int64_t p = tid; p < total; p += blockDim.x) {
            const int32_t s = tagged_slot(p);
            if (s >= 0) win_max(x.win + win_index(p / a.topK, s, x.spanRows), tagHi | static_cast<unsigned long long>(p));
        }
        __threadfence();
    } else {
        // lanes 8i .. 8i+7: own position lo + i against the later positions of its request
        const int64_t p = lo + static_cast<int64_t>(tid >> 3);
        int32_t s = -1;
        int64_t end = 0;
        if (p < hi && p < total) {
            s = sKey[p - tagLo];
            end = (p / a.topK + 1) * a.topK;
        }
        bool later = false;
        if (s >= 0) {
            for (int64_t q = p + 1 + static_cast<int64_t>(tid & 7u); q < end; q += 8) later |= sKey[q - tagLo] == s;
        }
        const uint64_t m = __ballot(later);
        const uint32_t lane = static_cast<uint32_t>(lane_id());
        if ((tid & 7u) == 0u && ((m >> lane) & 0xFFull) != 0ull) atomicOr(&sLose, 1u << (tid >> 3));
    }
    __syncthreads();
    for (int64_t p = tid; p < total; p += blockDim.x) {
        const int64_t bid = p / a.topK;
        const int8_t m = miss[p];  // the five reads issued together
        const int32_t t = topk[p], s = slots[p];
        const int64_t pl = pool[bid], hb = hostBase[bid];
        if (m == 0 || t < 0 || s < 0 || pl < 0) continue;
        const uint32_t row = static_cast<uint32_t>(hb + t);  // kvc_gather_rows.cpp:69-73
        const uint32_t node = kvx_node_of(row, a.stripeRows, a.nodeNum);
        const bool owned = x.fused ? (node < a.nodeNum) : (node == a.myNode);
        if (!owned) continue;
        const uint32_t key = node * 8u + static_cast<uint32_t>(static_cast<uint64_t>(p) / ppc);
        atomicAdd(&sCnt[key], 1u);
        const uint64_t segRow = kvx_seg_row_of(row, a.stripeRows, a.nodeNum);
        if (segRow >= a.perLayerSegRows) {  // row outside the segment: report, do not read
            atomicMin(&sErr[key], static_cast<uint32_t>(p));
            continue;
        }
        if (p < lo || p >= hi) continue;
        if (s < 65536) {
            const uint64_t d = win_index(bid, s, x.spanRows);
            if (d < x.winEntries && (global ? win_load(x.win + d) != (tagHi | static_cast<unsigned long long>(p))
                                            : ((sLose >> (p - lo)) & 1u) != 0u)) {
                continue;
            }
        }
        const uint64_t segBase = x.fused ? x.segBases[node] : a.segBase;
        const uint32_t at = atomicAdd(&sN, 1u);
        sSrc[at] = segBase + (static_cast<uint64_t>(a.layerOffsetRows) + segRow) * a.rowBytes;
        sDst[at] = a.hotRowBase + (static_cast<uint64_t>(s) + static_cast<uint64_t>(bid) * a.hotReqStrideRows) *
                                      a.rowBytes;
    }
    __syncthreads();
    {
        // the rows, shared among the waves
        const uint32_t n = sN, cpr = a.rowBytes / 16u, waves = blockDim.x / 64u, w = tid / 64u;
        const uint32_t share = (n + waves - 1u) / waves, r0 = w * share;
        if (r0 < n) wave_copy_rows(sSrc + r0, sDst + r0, (n - r0 < share) ? n - r0 : share, cpr);
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const unsigned int ticket = atomicInc(&x.tickets[3], gridDim.x - 1u);
        sLast = (ticket == gridDim.x - 1u) ? 1 : 0;
    }
    __syncthreads();
    if (!sLast) return;
    // the next call's epoch (at the wrap to 0, once in 2^32 calls, the table is cleared)
    if (sEpoch + 1u == 0u) {
        for (uint64_t i = tid; i < x.winEntries; i += blockDim.x) x.win[i] = 0ull;
    }
    if (tid == 0) *x.epoch = sEpoch + 1u;
    if (a.status == 0) return;
    __threadfence();
    for (uint32_t i = tid; i < (n1 - n0) * x.statusWords; i += blockDim.x) {
        const uint32_t node = n0 + i / x.statusWords, b = i % x.statusWords;
        uint64_t word = 1ull << 32;  // kvc_gather_rows.cpp:29-33, :93
        if (static_cast<int64_t>(b * ppc) < total) {
            const uint32_t e = sErr[node * 8u + b];
            word |= (static_cast<uint64_t>(sCnt[node * 8u + b]) << 40) | (e == 0xFFFFFFFFu ? 0u : row_error_code(e));
        }
        store_status(a.status + node * 64ull + b * 8ull, word);
    }
}

// Prefill export: item (layer l, owned stripe i) copies the stripe's winning
// row (its highest row inside the range) to segment row q/N of layer l.
__global__ __launch_bounds__(256) void kvx_export_alllayer(ExportParams P)
{
    __shared__ uint64_t sSrc[kWaves][64];
    __shared__ uint64_t sDst[kWaves][64];
    __shared__ int sLast;
    const KvcScatterAllArgs &a = P.l.a;
    const ExportExtra &x = P.x;
    const int wave = threadIdx.x / 64;
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    const uint64_t items = x.nStripes * a.layerNum;
    const uint64_t rowHi = static_cast<uint64_t>(a.rowLo) + a.rowCnt;
    const uint32_t cpr = a.rowBytes / 16u;

    for (uint64_t base = (static_cast<uint64_t>(blockIdx.x) * kWaves + wave) * 64ull; base < items;
         base += static_cast<uint64_t>(gridDim.x) * kWaves * 64ull) {
        const uint64_t it = base + lane;
        if (it < items) {
            const uint64_t l = it / x.nStripes, i = it - l * x.nStripes;
            const uint64_t q = x.q0 + i * x.N;
            uint64_t w = q * x.S + x.S - 1ull;
            if (w > rowHi - 1ull) w = rowHi - 1ull;
            const uint64_t segRow = q / x.N;
            sSrc[wave][lane] = a.srcLayer0Base + l * a.srcLayerStride + w * a.rowBytes;
            sDst[wave][lane] = a.segBase + (l * a.perLayerSegRows + segRow) * a.rowBytes;
        }
        wave_sync_lds();
        const uint64_t left = items - base;
        wave_copy_rows(sSrc[wave], sDst[wave], static_cast<uint32_t>(left < 64ull ? left : 64ull), cpr);
        wave_sync_lds();
    }

    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned int ticket = atomicInc(&x.tickets[1], gridDim.x - 1u);
        sLast = (ticket == gridDim.x - 1u) ? 1 : 0;
    }
    __syncthreads();
    if (!sLast || a.status == 0) return;
    __threadfence_system();
    const uint32_t words = a.blockDim == 0 ? 1u : a.blockDim;
    for (uint32_t b = threadIdx.x; b < words; b += blockDim.x) {
        uint64_t word = 1ull << 32;  // kvc_scatter_rows_alllayer.cpp:59-61
        if (b == 0) word |= (x.ownedRows * a.layerNum) << 40;
        store_status(a.status + a.myNode * 64ull + b * 8ull, word);
    }
}

// Decode-incremental export of one layer (the reference design's
// export_rows / kvc_scatter_rows, doc/kv_offload_design.md:322-327,394-396:
// the import's shape with the direction reversed).  Entry i < num_real names
// host row indices[i]; the row owned by myNode is copied from
// srcLayerBase + i*rowBytes to its segment row of layer layerId.  Entries
// naming one segment row resolve as a sequential walk would: the last wins.
struct ExportRowsParams {
    ExportRowsArgs a;
    uint64_t segBases[64];   // fused form: every node's segment base
    unsigned long long *win;
    uint64_t winEntries;
    uint32_t *counters;
    uint32_t *errs;
    uint32_t *tickets;
    uint32_t *epoch;
};

// Segment base of `node` from the kernel's argument block, read in place
// (the kernels' only argument starts at offset 0 of the argument segment):
// indexing the by-value argument at run time would copy the whole block to
// private memory.
__device__ __forceinline__ uint64_t export_seg_base(uint32_t node)
{
    typedef __attribute__((address_space(4))) const uint64_t KU64;
    typedef __attribute__((address_space(4))) const char KChar;
    const KChar *k = (KChar *)__builtin_amdgcn_kernarg_segment_ptr();
    return reinterpret_cast<KU64 *>(k + offsetof(ExportRowsParams, segBases))[node];
}

__device__ __forceinline__ bool export_row_target(const ExportRowsArgs &a, int64_t row, uint32_t &node,
                                                  uint32_t &segRow)
{
    if (row < 0) return false;
    const uint32_t r = static_cast<uint32_t>(row);  // the mapping is u32 math (kvc_common.h:81-89)
    node = kvx_node_of(r, a.stripeRows, a.nodeNum);
    if (a.fused ? node >= a.nodeNum : node != a.myNode) return false;
    segRow = kvx_seg_row_of(r, a.stripeRows, a.nodeNum);
    return true;
}

// Pass 1: the last entry per segment row (winner tags, as in the import);
// block 0 resets this node's counters and status words.
__global__ __launch_bounds__(256) void kvx_export_rows_prep(ExportRowsParams P)
{
    const ExportRowsArgs &a = P.a;
    const int32_t n = clamp_num_real(a.numReal, a.maxRows);
    const uint32_t n0 = a.fused ? 0u : a.myNode, n1 = a.fused ? a.nodeNum : a.myNode + 1u;
    if (blockIdx.x == 0) {
        for (uint32_t k = threadIdx.x; k < (n1 - n0) * a.statusWords; k += blockDim.x) {
            const uint32_t node = n0 + k / a.statusWords, b = k % a.statusWords;
            P.counters[node * 8u + b] = 0u;
            P.errs[node * 8u + b] = 0xFFFFFFFFu;  // lowest failing entry, min-reduced
            if (a.status != 0) store_status(a.status + node * 64ull + b * 8ull, 0ull);
        }
    }
    const KVX_G int64_t *idx = reinterpret_cast<const KVX_G int64_t *>(a.indicesHost);
    const unsigned long long tagHi = static_cast<unsigned long long>(*P.epoch) << 32;
    for (int32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        uint32_t node, segRow;
        if (!export_row_target(a, idx[i], node, segRow) || segRow >= a.perLayerSegRows) continue;
        const uint64_t w = (a.fused ? static_cast<uint64_t>(node) * a.perLayerSegRows : 0ull) + segRow;
        if (w < P.winEntries) win_max(P.win + w, tagHi | static_cast<unsigned long long>(i));
    }
}

// Pass 2: each wave takes kExportRowsPerWave entries (a decode step exports
// a few rows per layer: spread over many waves they move in one round trip),
// counts the owned ones per status word, records out-of-segment rows and
// copies its winners; the last workgroup advances the epoch and writes the
// status words.
constexpr int kExportRowsPerWave = 8;
__global__ __launch_bounds__(256) void kvx_export_rows_copy(ExportRowsParams P)
{
    __shared__ uint64_t sSrc[kWaves][64];
    __shared__ uint64_t sDst[kWaves][64];
    __shared__ int sLast;
    __shared__ uint32_t sEpoch;
    const ExportRowsArgs &a = P.a;
    const int wave = threadIdx.x / 64;
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    const int32_t n = clamp_num_real(a.numReal, a.maxRows);
    const KVX_G int64_t *idx = reinterpret_cast<const KVX_G int64_t *>(a.indicesHost);
    const unsigned long long tagHi = static_cast<unsigned long long>(*P.epoch) << 32;
    const uint32_t cpr = a.rowBytes / 16u;
    const uint32_t words = a.statusWords;
    const uint32_t ppc = (a.maxRows + words - 1u) / words;  // entries per status word
    constexpr int32_t R = kExportRowsPerWave;
    for (int32_t base = (blockIdx.x * kWaves + wave) * R; base < n; base += gridDim.x * kWaves * R) {
        const int32_t i = base + static_cast<int32_t>(lane);
        bool copy = false;
        uint64_t src = 0, dst = 0;
        uint32_t node, segRow;
        if (static_cast<int32_t>(lane) < R && i < n && export_row_target(a, idx[i], node, segRow)) {
            const uint32_t key = node * 8u + static_cast<uint32_t>(i) / ppc;
            atomicAdd(&P.counters[key], 1u);
            if (segRow >= a.perLayerSegRows) {  // outside the segment's layer region: report, do not write
                atomicMin(&P.errs[key], static_cast<uint32_t>(i));
            } else {
                const uint64_t w = (a.fused ? static_cast<uint64_t>(node) * a.perLayerSegRows : 0ull) + segRow;
                copy = w >= P.winEntries || win_load(P.win + w) == (tagHi | static_cast<unsigned long long>(i));
                src = a.srcLayerBase + static_cast<uint64_t>(i) * a.rowBytes;
                dst = (a.fused ? export_seg_base(node) : a.segBase) +
                      (static_cast<uint64_t>(a.layerId) * a.perLayerSegRows + segRow) * a.rowBytes;
            }
        }
        const uint64_t cm = __ballot(copy);
        if (copy) {
            const uint32_t at = static_cast<uint32_t>(__popcll(cm & ((1ull << lane) - 1ull)));
            sSrc[wave][at] = src;
            sDst[wave][at] = dst;
        }
        wave_sync_lds();
        wave_copy_rows(sSrc[wave], sDst[wave], static_cast<uint32_t>(__popcll(cm)), cpr);
        wave_sync_lds();
    }

    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned int ticket = atomicInc(&P.tickets[2], gridDim.x - 1u);
        sLast = (ticket == gridDim.x - 1u) ? 1 : 0;
    }
    __syncthreads();
    if (!sLast) return;
    if (threadIdx.x == 0) sEpoch = *P.epoch + 1u;
    __syncthreads();
    if (sEpoch == 0u) {
        for (uint64_t k = threadIdx.x; k < P.winEntries; k += blockDim.x) P.win[k] = 0ull;
    }
    if (threadIdx.x == 0) *P.epoch = sEpoch;
    if (a.status == 0) return;
    __threadfence_system();
    const uint32_t n0 = a.fused ? 0u : a.myNode, n1 = a.fused ? a.nodeNum : a.myNode + 1u;
    for (uint32_t k = threadIdx.x; k < (n1 - n0) * words; k += blockDim.x) {
        const uint32_t node = n0 + k / words, b = k % words;
        uint64_t word = 1ull << 32;
        if (static_cast<int64_t>(b) * ppc < n) {
            const uint32_t q = __hip_atomic_load(&P.counters[node * 8u + b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const uint32_t e = __hip_atomic_load(&P.errs[node * 8u + b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            word |= (static_cast<uint64_t>(q) << 40) | (e == 0xFFFFFFFFu ? 0u : row_error_code(e));
        }
        store_status(a.status + node * 64ull + b * 8ull, word);
    }
}

// Short exports (max_rows <= kExportSmallMax, the rows a decode step
// appends): both passes in one launch.  A winner is the last entry on its
// destination row.  Up to kExportSmallLds entries, every workgroup loads the
// destinations of all entries into LDS and eight lanes per own entry look for
// a later entry with the same destination (no device-scope atomics, no
// fence); above that, every workgroup tags the winners of all entries (the
// same atomicMax values, so the repeats are harmless) and reads its own
// entries' tags.  Each workgroup counts the owned entries and the lowest
// out-of-region entry per status word in its own LDS, then copies the
// winners among its own 32 entries (8 per wave); the last workgroup (ticket)
// advances the epoch and stores the status words from its counts.
constexpr uint32_t kExportSmallMax = 4096;
constexpr uint32_t kExportSmallLds = 1024;

__global__ __launch_bounds__(256) void kvx_export_rows_small(ExportRowsParams P)
{
    __shared__ uint64_t sSrc[kWaves][64];
    __shared__ uint64_t sDst[kWaves][64];
    __shared__ uint32_t sCnt[64 * 8], sErr[64 * 8];
    __shared__ uint64_t sDest[kExportSmallLds];  // destination of each entry (~0: none), for n <= kExportSmallLds
    __shared__ int sLast;
    __shared__ uint32_t sEpoch, sLose;  // sLose bit e: own entry e is not a winner
    const ExportRowsArgs &a = P.a;
    const int wave = threadIdx.x / 64;
    const uint32_t lane = static_cast<uint32_t>(lane_id());
    const int32_t n = clamp_num_real(a.numReal, a.maxRows);  // <= kExportSmallMax (host)
    const KVX_G int64_t *idx = reinterpret_cast<const KVX_G int64_t *>(a.indicesHost);
    const uint32_t cpr = a.rowBytes / 16u;
    const uint32_t words = a.statusWords;
    const uint32_t ppc = (a.maxRows + words - 1u) / words;  // entries per status word
    const uint32_t n0 = a.fused ? 0u : a.myNode, n1 = a.fused ? a.nodeNum : a.myNode + 1u;
    if (blockIdx.x == 0 && a.status != 0) {  // the call's status words read 0 until its rows have landed
        for (uint32_t k = threadIdx.x; k < (n1 - n0) * words; k += blockDim.x) {
            store_status(a.status + (n0 + k / words) * 64ull + (k % words) * 8ull, 0ull);
        }
    }
    for (uint32_t k = threadIdx.x; k < 64u * 8u; k += blockDim.x) {
        sCnt[k] = 0u;
        sErr[k] = 0xFFFFFFFFu;  // lowest failing entry, min-reduced
    }
    if (threadIdx.x == 0) sEpoch = *P.epoch;
    __syncthreads();
    const unsigned long long tagHi = static_cast<unsigned long long>(sEpoch) << 32;
    // the destination of entry i when the winner rule applies to it, else ~0
    auto entry_dest = [&](int32_t i) -> uint64_t {
        uint32_t node, segRow;
        if (!export_row_target(a, idx[i], node, segRow) || segRow >= a.perLayerSegRows) return ~0ull;
        const uint64_t w = (a.fused ? static_cast<uint64_t>(node) * a.perLayerSegRows : 0ull) + segRow;
        return w < P.winEntries ? w : ~0ull;
    };
    const int32_t first = static_cast<int32_t>(blockIdx.x) * kWaves * kExportRowsPerWave;  // own entries: 32 from here
    const bool inLds = n <= static_cast<int32_t>(kExportSmallLds);
    if (inLds) {
        for (int32_t i = threadIdx.x; i < n; i += blockDim.x) sDest[i] = entry_dest(i);
        if (threadIdx.x == 0) sLose = 0u;
        __syncthreads();
        // lanes 8e .. 8e+7: own entry first + e against the later entries
        const int32_t e = static_cast<int32_t>(threadIdx.x >> 3), i = first + e;
        bool later = false;
        if (i < n) {
            const uint64_t w = sDest[i];
            if (w != ~0ull) {
                for (int32_t j = i + 1 + static_cast<int32_t>(threadIdx.x & 7u); j < n; j += 8) later |= sDest[j] == w;
            }
        }
        const uint64_t m = __ballot(later);
        if ((threadIdx.x & 7u) == 0u && ((m >> lane) & 0xFFull) != 0ull) atomicOr(&sLose, 1u << e);
    } else {
        for (int32_t i = threadIdx.x; i < n; i += blockDim.x) {
            const uint64_t w = entry_dest(i);
            if (w != ~0ull) win_max(P.win + w, tagHi | static_cast<unsigned long long>(i));
        }
        __threadfence();
    }
    __syncthreads();
    for (int32_t i = threadIdx.x; i < n; i += blockDim.x) {
        uint32_t node, segRow;
        if (!export_row_target(a, idx[i], node, segRow)) continue;
        const uint32_t key = node * 8u + static_cast<uint32_t>(i) / ppc;
        atomicAdd(&sCnt[key], 1u);
        if (segRow >= a.perLayerSegRows) atomicMin(&sErr[key], static_cast<uint32_t>(i));
    }
    constexpr int32_t R = kExportRowsPerWave;
    {
        const int32_t i = (static_cast<int32_t>(blockIdx.x) * kWaves + wave) * R + static_cast<int32_t>(lane);
        bool copy = false;
        uint64_t src = 0, dst = 0;
        uint32_t node, segRow;
        if (static_cast<int32_t>(lane) < R && i < n && export_row_target(a, idx[i], node, segRow) &&
            segRow < a.perLayerSegRows) {
            const uint64_t w = (a.fused ? static_cast<uint64_t>(node) * a.perLayerSegRows : 0ull) + segRow;
            copy = w >= P.winEntries || (inLds ? ((sLose >> (i - first)) & 1u) == 0u
                                               : win_load(P.win + w) == (tagHi | static_cast<unsigned long long>(i)));
            src = a.srcLayerBase + static_cast<uint64_t>(i) * a.rowBytes;
            dst = (a.fused ? export_seg_base(node) : a.segBase) +
                  (static_cast<uint64_t>(a.layerId) * a.perLayerSegRows + segRow) * a.rowBytes;
        }
        const uint64_t cm = __ballot(copy);
        if (copy) {
            const uint32_t at = static_cast<uint32_t>(__popcll(cm & ((1ull << lane) - 1ull)));
            sSrc[wave][at] = src;
            sDst[wave][at] = dst;
        }
        wave_sync_lds();
        wave_copy_rows(sSrc[wave], sDst[wave], static_cast<uint32_t>(__popcll(cm)), cpr);
    }
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned int ticket = atomicInc(&P.tickets[4], gridDim.x - 1u);
        sLast = (ticket == gridDim.x - 1u) ? 1 : 0;
    }
    __syncthreads();
    if (!sLast) return;
    if (sEpoch + 1u == 0u) {  // at the wrap (once in 2^32 calls) the tag table is cleared
        for (uint64_t k = threadIdx.x; k < P.winEntries; k += blockDim.x) P.win[k] = 0ull;
    }
    if (threadIdx.x == 0) *P.epoch = sEpoch + 1u;
    if (a.status == 0) return;
    __threadfence_system();
    for (uint32_t k = threadIdx.x; k < (n1 - n0) * words; k += blockDim.x) {
        const uint32_t node = n0 + k / words, b = k % words;
        uint64_t word = 1ull << 32;
        if (static_cast<int64_t>(b) * ppc < n) {
            const uint32_t e = sErr[node * 8u + b];
            word |= (static_cast<uint64_t>(sCnt[node * 8u + b]) << 40) | (e == 0xFFFFFFFFu ? 0u : row_error_code(e));
        }
        store_status(a.status + node * 64ull + b * 8ull, word);
    }
}

// Plain streaming copy, 16 B per lane, kUnroll chunks in flight per lane.
__global__ __launch_bounds__(256) void kvx_stream_copy(u32x4 *dst, const u32x4 *src, uint64_t n16)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    for (; i + (kUnroll - 1) * stride < n16; i += kUnroll * stride) {
        u32x4 v[kUnroll];
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) v[j] = __builtin_nontemporal_load(src + i + j * stride);
#pragma unroll
        for (int j = 0; j < kUnroll; ++j) __builtin_nontemporal_store(v[j], dst + i + j * stride);
    }
    for (; i < n16; i += stride) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

}  // namespace

hipError_t launch_stream_copy(uint64_t dst, uint64_t src, uint64_t bytes, hipStream_t stream)
{
    const uint64_t n16 = bytes / 16;
    uint64_t blocks = (n16 + 255) / 256;
    if (blocks < 1) blocks = 1;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(kvx_stream_copy, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream,
                       reinterpret_cast<u32x4 *>(dst), reinterpret_cast<const u32x4 *>(src), n16);
    return hipGetLastError();
}

hipError_t launch_gather(const GatherPlan &plan, const RowScratch &scr, uint64_t overflowSlot, hipStream_t stream)
{
    GatherParams P{};
    P.l.a = plan.a;
    P.l.overflowSlot = overflowSlot;
    if (plan.fused) {
        for (uint32_t s = 0; s < plan.a.nodeNum && s < 64u; ++s) P.x.segBases[s] = plan.segBases[s];
    }
    P.x.win = scr.win;
    P.x.winEntries = scr.winEntries;
    P.x.chunkNext = scr.chunkNext;
    P.x.counters = scr.counters;
    P.x.errs = scr.errs;
    P.x.tickets = scr.tickets;
    P.x.fused = plan.fused;
    P.x.epoch = scr.epoch;
    P.x.spanRows = plan.spanRows;
    P.x.statusWords = plan.statusWords;
    const uint64_t positions = static_cast<uint64_t>(plan.a.maxNumReqs) * plan.a.topK;
    if (positions <= kSmallMaxPositions) {
        const uint32_t blocks = static_cast<uint32_t>((positions + kSmallSpan - 1u) / kSmallSpan);
        hipLaunchKernelGGL(kvx_gather_small, dim3(blocks), dim3(256), 0, stream, P);
        return hipGetLastError();
    }
    uint64_t prepBlocks = (positions + 255ull) / 256ull;
    if (prepBlocks < 1) prepBlocks = 1;
    if (prepBlocks > 2048) prepBlocks = 2048;
    hipLaunchKernelGGL(kvx_gather_prep, dim3(static_cast<uint32_t>(prepBlocks)), dim3(256), 0, stream, P);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t spanBlocks = (positions + kSpan - 1ull) / kSpan;
    if (spanBlocks > kSpanBlocks) spanBlocks = kSpanBlocks;
    hipLaunchKernelGGL(kvx_gather_span, dim3(static_cast<uint32_t>(spanBlocks)), dim3(256), 0, stream, P);
    return hipGetLastError();
}

hipError_t launch_export(const KvcScatterAllArgs &a, const RowScratch &scr, uint64_t overflowSlot,
                         hipStream_t stream)
{
    ExportParams P{};
    P.l.a = a;
    P.l.overflowSlot = overflowSlot;
    P.x.tickets = scr.tickets;
    const ExportGeometry geo = export_geometry(a);
    P.x.q0 = geo.q0;
    P.x.nStripes = geo.nStripes;
    P.x.ownedRows = geo.ownedRows;
    P.x.S = geo.S;
    P.x.N = geo.N;
    const uint64_t items = P.x.nStripes * a.layerNum;
    uint64_t blocks = (items + 64ull * kWaves - 1ull) / (64ull * kWaves);
    if (blocks < 1) blocks = 1;
    if (blocks > 2048) blocks = 2048;
    hipLaunchKernelGGL(kvx_export_alllayer, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, P);
    return hipGetLastError();
}

hipError_t launch_export_rows(const ExportRowsArgs &a, const uint64_t *segBases, const RowScratch &scr,
                              hipStream_t stream)
{
    ExportRowsParams P{};
    P.a = a;
    if (a.fused) {
        for (uint32_t s = 0; s < a.nodeNum && s < 64u; ++s) P.segBases[s] = segBases[s];
    }
    P.win = scr.win;
    P.winEntries = scr.winEntries;
    P.counters = scr.counters;
    P.errs = scr.errs;
    P.tickets = scr.tickets;
    P.epoch = scr.epoch;
    if (a.maxRows <= kExportSmallMax) {
        const uint32_t blocks = (a.maxRows + kExportRowsPerWave * kWaves - 1u) / (kExportRowsPerWave * kWaves);
        hipLaunchKernelGGL(kvx_export_rows_small, dim3(blocks), dim3(256), 0, stream, P);
        return hipGetLastError();
    }
    uint64_t prep = (static_cast<uint64_t>(a.maxRows) + 255ull) / 256ull;
    prep = prep < 1 ? 1 : (prep > 1024 ? 1024 : prep);
    hipLaunchKernelGGL(kvx_export_rows_prep, dim3(static_cast<uint32_t>(prep)), dim3(256), 0, stream, P);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    uint64_t copy = (static_cast<uint64_t>(a.maxRows) + kExportRowsPerWave * kWaves - 1ull) / (kExportRowsPerWave * kWaves);
    copy = copy < 1 ? 1 : (copy > 256 ? 256 : copy);
    hipLaunchKernelGGL(kvx_export_rows_copy, dim3(static_cast<uint32_t>(copy)), dim3(256), 0, stream, P);
    return hipGetLastError();
}

}  // namespace kvx
