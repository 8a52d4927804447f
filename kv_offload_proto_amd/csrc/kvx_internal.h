// Internal declarations shared by the gfx950 kernels and the C-ABI layer.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "kvx/kv_layout.h"
#include "kvx/kvc_args.h"

namespace kvx {

// ---------------------------------------------------------------------------
// Hash and bitmap helpers (the state format of hisp_kernel_common.h:19-130).
// ---------------------------------------------------------------------------

// Knuth multiplicative hash, top 16 bits (hisp_kernel_common.h:23-26).
__host__ __device__ __forceinline__ uint32_t ht_hash(int32_t token)
{
    return (static_cast<uint32_t>(token) * 2654435761u) >> 16;
}

// Codes stored in the tail-slot word when a kernel stops a loop that the
// reference would spin on forever.
constexpr uint64_t kOverflowProbe = 0x50524F4245ull;   // probe run longer than the table
constexpr uint64_t kOverflowSweep = 0x5357454550ull;   // hand sweep longer than the buffer

// Status error code of a miss row whose segment row lies outside the
// segment's layer region: the reference's per-row band 0x2xx + (pos & 0xFF)
// with op return code 1 in bits 16.. (kvc_gather_rows.cpp:78-81).
__host__ __device__ __forceinline__ uint32_t row_error_code(uint64_t pos)
{
    return 0x200u + static_cast<uint32_t>(pos & 0xFFu) + (1u << 16);
}

// Stride of sieve_hand rows in int32 (64 bytes; hisp_kernel_common.h:20-21).
constexpr int32_t kHandStride = 16;
// sieve_hand[row][1]: set by the SIEVE kernels that left the row's table
// consistent with its tokens (every live token findable at its own slot, one
// entry per live slot); any other writer of the row clears it.
constexpr int32_t kCanonFlag = 0x4B565843;
// sieve_hand[row][3]: written with the flag, the sum over slots [0, dbs) of
// slot_token_mix(slot, token) (mod 2^32) of the tokens the kernel left.  A
// flagged row is trusted only while its tokens still sum to it, so a token
// edited in place without clearing the flag sends the row to the full check.
constexpr int32_t kFingerprintWord = 3;
// For a fixed slot the mix is a bijection of the token (every step is), so
// one edited token always changes the sum.  It uses only full-rate 24-bit
// multiplies (slot < 2^16): 32-bit ones issue at a quarter of the rate, and
// the parallel kernel mixes every slot of the row each step.  Step 3 is a
// bijection: its low 24 bits are x_lo * odd mod 2^24, which fixes x_lo, and
// then its top byte fixes x_hi.
__host__ __device__ __forceinline__ uint32_t slot_token_mix(uint32_t slot, int32_t token)
{
    uint32_t x = static_cast<uint32_t>(token) + (slot & 0xFFFFFFu) * 0x9E3779u;
    x ^= x >> 16;
    x = (x & 0xFFFFFFu) * 0x7FEB35u + (x & 0xFF000000u);
    x ^= x >> 15;
    return x;
}

// ---------------------------------------------------------------------------
// Scratch of the row movers.  The library keeps one set per stream (launches
// on one stream run in order and may share it; launches on different streams
// never do); the no-allocation entry point uses a fixed device array.
// ---------------------------------------------------------------------------
struct RowScratch {
    unsigned long long *win;   // winner tags, (epoch << 32) | position
    uint64_t winEntries;       // capacity of win[]
    uint32_t *counters;        // [64 nodes][8 status words] queued counts
    uint32_t *errs;            // [64 nodes][8 status words] first error code
    uint32_t *tickets;         // [8] last-block tickets (gather, export, export_rows, small gather, small export_rows)
    uint32_t *epoch;           // gather winner-tag epoch, advanced on the device by each call
    uint32_t *chunkNext;       // next position chunk of the current gather
};

// Control words of one scratch set: counters, error words, tickets, the
// import's chunk counter and the epoch, in this order (kControlWords uint32
// words).
constexpr uint32_t kControlWords = 64 * 8 * 2 + 8 + 8;

// Winner-table entries an import needs: request b's destinations are
// b*spanRows + slot with slot < 65536 (uint16 slot numbers).
__host__ __device__ __forceinline__ uint64_t gather_win_entries(uint32_t maxNumReqs, uint32_t hotReqStrideRows)
{
    const uint64_t span = hotReqStrideRows == 0 ? 0ull : (hotReqStrideRows < 65536u ? hotReqStrideRows : 65536u);
    return (maxNumReqs == 0 ? 0ull : static_cast<uint64_t>(maxNumReqs - 1u) * span) + 65536ull;
}

// Winner-table entries a decode-incremental export needs: one per segment row
// of the layer, for one segment or (fused) every segment.
__host__ __device__ __forceinline__ uint64_t export_rows_win_entries(uint32_t perLayerSegRows, uint32_t segments)
{
    const uint64_t n = static_cast<uint64_t>(perLayerSegRows) * segments;
    return n == 0 ? 1ull : n;
}

// ---------------------------------------------------------------------------
// LDS layout of the parallel SIEVE kernel (byte offsets, 16-byte aligned):
// the state row, then per-position, per-slot, per-event and per-cell scratch.
// ---------------------------------------------------------------------------
#ifndef KVX_FAST_THREADS
#define KVX_FAST_THREADS 1024
#endif
constexpr int kFastThreads = KVX_FAST_THREADS;

struct FastLayout {
    uint32_t tok, ht, vis, ptok, pinf, vt, evslot, smKp, eseq, tb, smA, smB, vset, ber, occ, fin, nkb, cmask, emask,
        smask, rsn, rsm, total;
};

__host__ __device__ __forceinline__ uint32_t align16(uint32_t x) { return (x + 15u) & ~15u; }

// LDS regions of the parallel SIEVE kernel for one batch row.  Regions with
// disjoint lifetimes share memory (the kernel names the aliases): the SM k
// list with the conversions' old slots, the event sequence with the list of
// undecided SM slots, and the SM list with the per-event cells and tokens.
// In the compact form (rows whose full layout does not fit) the tokens row is
// replaced by the Knuth hash of each slot's token (full tokens stay in HBM),
// and the per-slot first-hit codes (vt) take 16 bits instead of 32.
// cmask/emask/smask/rsn/rsm hold one 64-bit ballot per (wave, block of one
// entry per lane).  ber, occ, fin and nkb are one bit per table cell: cells
// of evicted tokens, the pre-step occupancy, the occupancy as the erase and
// insert phases change it, and the cells new keys claim.
__host__ __device__ __forceinline__ FastLayout fast_layout(uint32_t padded, uint32_t htSize, uint32_t topK,
                                                           uint32_t visStrideB, bool compact = false)
{
    FastLayout l{};
    uint32_t o = 0;
    const uint32_t bmBytes = htSize / 8u;
    const uint32_t blocks = (topK + kFastThreads - 1u) / kFastThreads;
    const uint32_t maskBytes = blocks * (kFastThreads / 64u) * 8u;
    l.tok = o;     o += align16(padded * (compact ? 2u : 4u));
    l.ht = o;      o += align16(htSize * 2u);
    l.vis = o;     o += align16(visStrideB);
    l.ptok = o;    o += align16(topK * 4u);
    l.pinf = o;    o += align16(topK * 4u);
    l.vt = o;      o += align16(padded * (compact ? 2u : 4u));
    l.evslot = o;  o += align16(topK * 2u);
    l.smKp = o;    o += align16(topK * 2u + 16u);
    l.eseq = o;    o += align16(topK * 2u);
    l.tb = o;      o += align16((topK + 1u) * 2u);
    l.smA = o;     o += align16(topK * 4u);
    l.smB = o;     o += align16(topK * 4u);
    l.vset = o;    o += align16(visStrideB);
    l.ber = o;     o += align16(bmBytes);
    l.occ = o;     o += align16(bmBytes);
    l.cmask = o;   o += maskBytes;
    l.emask = o;   o += maskBytes;
    l.smask = o;   o += maskBytes;
    const uint32_t ringMaskBytes = (padded + kFastThreads - 1u) / kFastThreads * (kFastThreads / 64u) * 8u;
    l.rsn = o;     o += ringMaskBytes;
    l.rsm = o;     o += ringMaskBytes;
    l.fin = o;     o += align16(bmBytes);
    l.nkb = o;     o += align16(bmBytes);
    l.total = o;
    return l;
}

// Fixed-count instantiations of the parallel kernel (positions and ring
// offsets per lane): topK up to 2048 with up to 4096 or 8192 slots.
constexpr int kFixP = 2048 / kFastThreads, kFixQ1 = 4096 / kFastThreads, kFixQ2 = 8192 / kFastThreads;

__host__ __device__ constexpr bool fast_fixed(uint32_t topK, uint32_t dbs, int &pm, int &qm)
{
    const uint32_t P = (topK + kFastThreads - 1u) / kFastThreads, Q = (dbs + kFastThreads - 1u) / kFastThreads;
    pm = static_cast<int>(P);
    qm = static_cast<int>(Q);
    return P == static_cast<uint32_t>(kFixP) && (Q == static_cast<uint32_t>(kFixQ1) || Q == static_cast<uint32_t>(kFixQ2));
}

// Layout of a fixed-count instantiation: the regions sized by topK or dbs
// take their bounds (PM or QM entries per lane), so their offsets are
// compile-time constants; the state row (tokens, table, visited bits) and the
// per-cell bitmaps follow at offsets that depend on padded and htSize.
template <int PM, int QM>
__host__ __device__ __forceinline__ FastLayout fast_layout_fixed(uint32_t padded, uint32_t htSize, uint32_t visStrideB,
                                                                 bool compact)
{
    constexpr uint32_t Kx = PM * kFastThreads, Dx = QM * kFastThreads, NW = kFastThreads / 64;
    FastLayout l{};
    uint32_t o = 0;
    l.ptok = o;    o += Kx * 4u;
    l.pinf = o;    o += Kx * 4u;
    l.vt = o;      o += Dx * (compact ? 2u : 4u);
    l.evslot = o;  o += Kx * 2u;
    l.smKp = o;    o += align16(Kx * 2u + 16u);
    l.eseq = o;    o += Kx * 2u;
    l.tb = o;      o += align16((Kx + 1u) * 2u);
    l.smA = o;     o += Kx * 4u;
    l.smB = o;     o += Kx * 4u;
    l.vset = o;    o += align16(Dx / 8u);
    l.cmask = o;   o += PM * NW * 8u;
    l.emask = o;   o += PM * NW * 8u;
    l.smask = o;   o += PM * NW * 8u;
    l.rsn = o;     o += QM * NW * 8u;
    l.rsm = o;     o += QM * NW * 8u;
    l.tok = o;     o += align16(padded * (compact ? 2u : 4u));
    l.ht = o;      o += align16(htSize * 2u);
    l.vis = o;     o += align16(visStrideB);
    l.ber = o;     o += align16(htSize / 8u);
    l.occ = o;     o += align16(htSize / 8u);
    // the two table bitmaps of the insert phases take the per-position
    // classes' region, which the fixed kernels keep in registers instead
    if (2u * align16(htSize / 8u) <= Kx * 4u) {
        l.fin = l.pinf;
        l.nkb = l.pinf + align16(htSize / 8u);
    } else {
        l.fin = o;  o += align16(htSize / 8u);
        l.nkb = o;  o += align16(htSize / 8u);
    }
    l.total = o;
    return l;
}

// The layout the launcher and the kernel use for a shape.
__host__ __device__ __forceinline__ FastLayout fast_layout_for(uint32_t padded, uint32_t htSize, uint32_t topK,
                                                               uint32_t dbs, uint32_t visStrideB, bool compact)
{
    int pm = 0, qm = 0;
    if (fast_fixed(topK, dbs, pm, qm)) {
        return qm == kFixQ1 ? fast_layout_fixed<kFixP, kFixQ1>(padded, htSize, visStrideB, compact)
                            : fast_layout_fixed<kFixP, kFixQ2>(padded, htSize, visStrideB, compact);
    }
    return fast_layout(padded, htSize, topK, visStrideB, compact);
}

// ---------------------------------------------------------------------------
// The batch HBM SIEVE kernel (sieve_batch.hip): one workgroup of
// kBatchThreads per batch row; LDS holds the row's visited and evicted
// bitmaps, a bitmap over the table cells, per-position codes and slots, and
// a stage of table cells; HBM scratch per row holds a token -> slot map,
// first-occurrence table and token bitmap of kBatchMapCap tokens and each
// position's resident slot.
// ---------------------------------------------------------------------------
constexpr int kBatchThreads = 1024;
constexpr int kBatchWaves = kBatchThreads / 64;
constexpr uint32_t kBatchStage = 4096;       // table cells staged per step of the deletion walk
constexpr uint32_t kBatchMapCap = 1u << 18;  // tokens the map holds (rows with larger tokens run in order)

struct BatchLayout {
    uint32_t vis, ev, del, slot, uni, uniL1, uniL2, stage, total;
};

__host__ __device__ __forceinline__ BatchLayout batch_layout(uint32_t dbs, uint32_t htSize, uint32_t topK)
{
    BatchLayout l{};
    const uint32_t nVisW = (dbs + 63u) / 64u, nCellW = htSize / 64u, nL1 = (nCellW + 63u) / 64u,
                   nL2 = (nL1 + 63u) / 64u;
    uint32_t o = 0;
    l.vis = o;    o += nVisW * 8u;
    l.ev = o;     o += nVisW * 8u;
    l.del = o;    o += nCellW * 8u;
    l.slot = o;   o += align16(topK * 4u);
    l.uni = o;
    l.uniL1 = o + nCellW * 8u;
    l.uniL2 = l.uniL1 + nL1 * 8u;
    const uint32_t bitBytes = (nCellW + nL1 + nL2) * 8u;
    const uint32_t uniBytes = topK * 4u > bitBytes ? topK * 4u : bitBytes;
    o += align16(uniBytes);
    l.stage = o;  o += kBatchStage * 4u;
    l.total = o;
    return l;
}

// The table rebuild of a step with misses (sieve_table.hip): per batch row,
// HBM scratch of its own (table_layout(H).words uint32 words a row; nothing in
// it needs to start zeroed, every launch writes what it reads):
//   meta [16]          0: rebuild pending, 1: new keys, 2: linearization cell
//   cellw [H]          per cell of the pre-step table: 0 empty, 0xFFFF0000 a
//                      deleted key, else (home << 16) | entry of a survivor
//   hist [min(H,2^16)] keys per home cell after the step (survivors + new keys)
//   newk [H/2]         new keys in event order: (home << 16) | (slot + 1)
//   evict [H/32]       the step's evicted slots (bitmap)
//   chunkA [H/kTblChunkCells]  per cell chunk: start of its cluster, or -1
constexpr uint32_t kTblChunkCells = 256;     // survivors' cells per chunk
constexpr uint32_t kTblChunkKeys = 256;      // new keys per chunk
constexpr uint32_t kTblWinBits = 3u << 16;   // free-cell window of a chunk (bits)
constexpr uint32_t kTblMaxHt = 1u << 18;     // largest table the rebuild takes

struct TableLayout {
    uint64_t meta, cellw, hist, newk, evict, chunkA, words;
};

__host__ __device__ __forceinline__ uint64_t align16w(uint64_t w) { return (w + 15u) & ~15ull; }

__host__ __device__ __forceinline__ TableLayout table_layout(uint32_t htSize)
{
    TableLayout t{};
    const uint64_t H = htSize, HH = htSize < 65536u ? htSize : 65536u;
    uint64_t o = 0;
    t.meta = o;    o += 16;
    t.cellw = o;   o += align16w(H);
    t.hist = o;    o += align16w(HH);
    t.newk = o;    o += align16w(H / 2);
    t.evict = o;   o += align16w(H / 32 + 2);
    t.chunkA = o;  o += align16w(H / kTblChunkCells + 1);
    t.words = o;
    return t;
}

// uint32 words of HBM scratch per row: map, first occurrences, a bitmap of
// the step's tokens, kBatchCounts counters (entries, last empty cell + 1,
// live tokens, a token past the map, the tokens' fingerprint) and each
// position's resident slot + 1 (htSize/2 >= topK words).  Every launch leaves
// them zeroed, whatever the shape of the next launch on the stream.
constexpr uint32_t kBatchCounts = 8;
__host__ __device__ __forceinline__ uint64_t batch_aux_words(uint32_t htSize)
{
    return 2ull * kBatchMapCap + kBatchMapCap / 32u + kBatchCounts + htSize / 2u;
}

// LDS bytes of the rebuild's chunk kernel: per-home counts (16 bits, 2^16
// homes and a 64-cell margin, read 8 at a time) and the free-cell window.
constexpr uint32_t kTblHistBytes = 65536u * 2u + 256u;
constexpr uint32_t kTblWinWords = kTblWinBits / 64u;
constexpr uint32_t kTblLdsBytes = kTblHistBytes + kTblWinWords * 8u;

// Launchers (implemented next to their kernels).
hipError_t launch_sieve_update(const HispSieveUpdateArgs &a, uint64_t overflowSlot, int variant,
                               size_t ldsBytes, hipStream_t stream);
// Forms of the admission build: kParallel (ldsBytes =
// sieve_ht_init_par_lds(htSize, dbs)), kWave (ldsBytes =
// sieve_ht_init_wave_lds(htSize, dbs)), kInOrder (one lane per table; the
// table in LDS when ldsBytes = 2 htSize, in HBM when 0).  The size functions
// return 0 where their form does not apply.
enum class InitForm { kParallel, kWave, kInOrder };
hipError_t launch_sieve_ht_init(const HispSieveHtInitArgs &a, uint64_t overflowSlot, size_t ldsBytes,
                                hipStream_t stream, InitForm form);
size_t sieve_ht_init_par_lds(uint32_t htSize, uint32_t dbs);
size_t sieve_ht_init_wave_lds(uint32_t htSize, uint32_t dbs);
hipError_t sieve_set_lds_limit(size_t bytes);
hipError_t sieve_fast_set_lds_limit(size_t bytes);
hipError_t launch_sieve_update_wave(const HispSieveUpdateArgs &a, uint64_t overflowSlot, int32_t *shadow,
                                    hipStream_t stream);
hipError_t launch_sieve_update_fast(const HispSieveUpdateArgs &a, uint64_t overflowSlot, size_t ldsBytes,
                                    bool compact, hipStream_t stream);
// tbl: the rebuild's scratch (rows of table_layout(htSize).words), or null
// for the table changes applied inside the batch kernel.
hipError_t launch_sieve_update_batch(const HispSieveUpdateArgs &a, uint64_t overflowSlot, int32_t *shadow,
                                     uint32_t *aux, uint32_t *tbl, hipStream_t stream);
hipError_t sieve_batch_set_lds_limit(size_t bytes);
// The table rebuild after the batch kernel (rows it left pending), on the
// same stream; table_rebuild_ok: the shape's windows fit (htSize <= kTblMaxHt).
hipError_t launch_sieve_table_rebuild(const HispSieveUpdateArgs &a, uint64_t overflowSlot, uint32_t *tbl,
                                      hipStream_t stream);
hipError_t sieve_table_set_lds_limit(size_t bytes);
__host__ __device__ __forceinline__ bool table_rebuild_ok(uint32_t htSize, uint32_t dbs, uint32_t topK)
{
    // windows: a survivor chunk spans its cluster (<= dbs cells) plus a chunk;
    // a new-key chunk spans the 2^16 homes plus every key it can pass
    return htSize >= 1024u && htSize <= kTblMaxHt && dbs <= 65535u && 65536ull + dbs + topK + 64u <= kTblWinBits &&
           dbs + kTblChunkCells + 64u <= kTblWinBits;
}

struct GatherPlan {
    KvcGatherArgs a;               // args of the first (or only) segment
    const uint64_t *segBases;      // device-visible bases of all segments (fused) or null
    uint32_t fused;                // 1: copy for every node; 0: only a.myNode
    uint32_t spanRows;             // bid stride used for the winner index
    uint32_t statusWords;          // words per node slot (block_dim)
};
hipError_t launch_gather(const GatherPlan &plan, const RowScratch &scr, uint64_t overflowSlot,
                         hipStream_t stream);
hipError_t launch_stream_copy(uint64_t dst, uint64_t src, uint64_t bytes, hipStream_t stream);
// Arguments of the decode-incremental single-layer export (the reference
// design's export_rows, doc/kv_offload_design.md:322-327; no args struct of
// the reference exists for it).
struct ExportRowsArgs {
    uint64_t segBase;         // host base of segment myNode
    uint64_t srcLayerBase;    // HBM rows: entry i at srcLayerBase + i*rowBytes
    uint64_t indicesHost;     // int64 host logical rows, one per entry
    uint64_t numReal;         // device int32: entries in use
    uint64_t status;          // status slot base (node myNode at +64*myNode)
    uint32_t layerId, perLayerSegRows, rowBytes, maxRows, stripeRows, nodeNum, myNode, statusWords;
    uint32_t fused;           // 1: every node's rows (segBases), status words of every node
};
hipError_t launch_export_rows(const ExportRowsArgs &a, const uint64_t *segBases, const RowScratch &scr,
                              hipStream_t stream);
hipError_t launch_export(const KvcScatterAllArgs &a, const RowScratch &scr, uint64_t overflowSlot,
                         hipStream_t stream);

// Export geometry of one segment: the stripes q of [rowLo, rowLo+rowCnt)
// owned by myNode are q0, q0+N, ... (nStripes of them); each contributes its
// highest in-range row.  ownedRows counts every in-range row of those stripes
// (the reference's queued count per layer).  S == 0 is the identity layout on
// node 0 (kv_layout.h:31-39), i.e. S = N = 1.
struct ExportGeometry {
    uint64_t q0 = 0, nStripes = 0, ownedRows = 0, maxSegRow = 0;
    uint32_t S = 1, N = 1;
};

inline ExportGeometry export_geometry(const KvcScatterAllArgs &a)
{
    ExportGeometry g;
    const uint64_t rowLo = a.rowLo, rowHi = static_cast<uint64_t>(a.rowLo) + a.rowCnt;
    uint64_t S = a.stripeRows, N = a.nodeNum;
    uint64_t my = a.myNode;
    bool none = (a.rowCnt == 0 || N == 0);
    if (S == 0) {
        S = 1;
        N = 1;
        if (a.myNode != 0) none = true;
        my = 0;
    }
    g.S = static_cast<uint32_t>(S);
    g.N = static_cast<uint32_t>(N);
    if (none) return g;
    const uint64_t qlo = rowLo / S, qhi = (rowHi - 1) / S;
    const uint64_t q0 = qlo + ((my + N - (qlo % N)) % N);
    if (q0 > qhi) return g;
    const uint64_t n = (qhi - q0) / N + 1;
    uint64_t owned = n * S;
    if (q0 == qlo) owned -= rowLo - qlo * S;
    const uint64_t qlast = q0 + (n - 1) * N;
    if (qlast == qhi) owned -= (qhi * S + S) - rowHi;
    g.q0 = q0;
    g.nStripes = n;
    g.ownedRows = owned;
    g.maxSegRow = qlast / N;
    return g;
}

}  // namespace kvx
