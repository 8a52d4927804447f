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
// in place.  Within the row, positions are processed in order by one lane,
// which is the exact sequential recurrence of the reference.
#include "kvx_internal.h"

namespace kvx {
namespace {

struct Guard {
    uint64_t code = 0;
};

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
        dirty = true;
        rs[k] = h;
        rm[k] = 1;
        tok[h] = tp;
        vis_set(vis, h);
        hand = (h + 1 == dbs) ? 0 : h + 1;
    }
    return dirty;
}

// Copy n bytes (multiple of 16, both sides 16-byte aligned) with the block.
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

    if (threadIdx.x == 0) {
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

}  // namespace

hipError_t sieve_set_lds_limit(size_t bytes)
{
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_update<true>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
    if (e != hipSuccess) return e;
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_ht_init<true>),
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

hipError_t launch_sieve_ht_init(const HispSieveHtInitArgs &a, uint64_t overflowSlot, size_t ldsBytes,
                                hipStream_t stream)
{
    KvxLaunch<HispSieveHtInitArgs> L{a, overflowSlot};
    const dim3 grid(a.layerNum * a.numReqs), block(256);
    if (ldsBytes != 0) {
        hipLaunchKernelGGL(kvx_sieve_ht_init<true>, grid, block, ldsBytes, stream, L);
    } else {
        hipLaunchKernelGGL(kvx_sieve_ht_init<false>, grid, block, 0, stream, L);
    }
    return hipGetLastError();
}

}  // namespace kvx
