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
