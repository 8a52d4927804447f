// SIEVE update for rows whose state does not fit LDS (variant 3).
//
// One workgroup per batch row, state in HBM, updated in place.  The positions
// are processed in order -- the exact recurrence of hisp_sieve_update.cpp:
// 115-163 -- but every inner loop runs 64 cells or slots at a time on one
// wave: a probe reads 64 consecutive table cells and picks the first empty or
// matching one with a ballot, the hand sweep tests 64 visited bits at once,
// and Algorithm R's backward shift walks the cluster 64 cells per step,
// taking the moves in order with ballots.  Probes compare tokens through a
// per-launch shadow of the table (cell -> token of its entry, built by the
// whole workgroup first), so one probe step is two coalesced row reads
// instead of a chain of dependent slot lookups.  Long probe runs (adversarial
// keys that share home buckets) therefore cost runs/64 memory round trips.
#include "kvx_internal.h"
#include "sieve_hbm.h"

namespace kvx {
namespace {

using namespace sieve_hbm;

constexpr int WT = 256;  // all threads build the shadow; wave 0 runs the recurrence

__global__ __launch_bounds__(WT) void kvx_sieve_update_wave(KvxLaunch<HispSieveUpdateArgs> L, int32_t *shadow)
{
    const HispSieveUpdateArgs &a = L.a;
    const int32_t K = static_cast<int32_t>(a.topK);
    const int32_t dbs = static_cast<int32_t>(a.deviceBufferSize);
    const int32_t padded = static_cast<int32_t>(a.paddedBufferSize);
    const int32_t visStrideB = static_cast<int32_t>(a.visitedStrideB);
    const int32_t maxNumReqs = static_cast<int32_t>(a.maxNumReqs);
    const int32_t H = static_cast<int32_t>(a.htSize);
    const int32_t poolSize = static_cast<int32_t>(a.poolSize);
    const int32_t bid = blockIdx.x;
    if (bid >= maxNumReqs) return;

    int32_t numReal = *reinterpret_cast<const int32_t *>(a.numReal);
    if (numReal > maxNumReqs) numReal = maxNumReqs;  // hisp_sieve_update.cpp:31-34
    KVX_GM int32_t *rs = reinterpret_cast<KVX_GM int32_t *>(a.topKDeviceSlots) + static_cast<int64_t>(bid) * K;
    KVX_GM int8_t *rm = reinterpret_cast<KVX_GM int8_t *>(a.isMiss) + static_cast<int64_t>(bid) * K;
    if (bid >= numReal) {
        write_dummy_row((int32_t *)rs, (int8_t *)rm, K);
        return;
    }
    const int64_t reqIdx = reinterpret_cast<const int64_t *>(a.reqPoolIndices)[bid];
    if (reqIdx < 0 || reqIdx >= poolSize) {
        write_dummy_row((int32_t *)rs, (int8_t *)rm, K);
        return;
    }
    const int32_t seqLen = reinterpret_cast<const int32_t *>(a.seqLens)[bid];
    const int32_t prefill = reinterpret_cast<const int32_t *>(a.prefillLens)[reqIdx];
    const KVX_GM int32_t *rt = reinterpret_cast<const KVX_GM int32_t *>(a.topkIndices) + static_cast<int64_t>(bid) * K;
    Row r;
    r.tok = reinterpret_cast<KVX_GM int32_t *>(a.deviceBufferTokens) + reqIdx * padded;
    r.vis32 = reinterpret_cast<KVX_GM uint32_t *>(a.deviceBufferVisited + static_cast<uint64_t>(reqIdx) * visStrideB);
    r.ht = reinterpret_cast<KVX_GM uint16_t *>(a.deviceBufferHt) + reqIdx * H;
    r.ct = (KVX_GM int32_t *)shadow + static_cast<int64_t>(bid) * H;
    r.mask = H - 1;
    r.dbs = dbs;
    r.padded = padded;
    KVX_GM int32_t *gHand = reinterpret_cast<KVX_GM int32_t *>(a.sieveHand) + reqIdx * kHandStride;
    build_shadow(r);
    __threadfence_block();
    __syncthreads();
    if (threadIdx.x >= 64) return;
    recurrence(r, rt, rs, rm, K, seqLen, prefill, gHand, L.overflowSlot);
}

}  // namespace

hipError_t launch_sieve_update_wave(const HispSieveUpdateArgs &a, uint64_t overflowSlot, int32_t *shadow,
                                    hipStream_t stream)
{
    KvxLaunch<HispSieveUpdateArgs> L{a, overflowSlot};
    hipLaunchKernelGGL(kvx_sieve_update_wave, dim3(a.maxNumReqs), dim3(WT), 0, stream, L, shadow);
    return hipGetLastError();
}

}  // namespace kvx
