/*
 * CPU oracle for the decode-time KV data plane.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is a test oracle: it is built into
 * oracle/liboracle.so and loaded by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg.  Nothing in the product path links or calls it.
 *
 * It restates, in plain sequential C, the algorithms of the reference
 * (jsun8686/kv_offload_proto) for this path.  Each function cites the
 * reference file:line it follows.  Where the reference races or is
 * inconsistent, the rule chosen here is stated in the function comment.
 *
 * Parity pinning (what checks each function beyond this restatement):
 *   orc_ht_*            Knuth TAOCP 6.4 linear probing + Algorithm R; checked by
 *                       tests/test_oracle_hash.py against brute-force invariants
 *                       (every live key findable, no stray entries, table ==
 *                       live keys re-inserted in insertion order).
 *   orc_sieve_update    test_sieve_oracle.py literals (tests/golden/reference_kats.json),
 *                       an independent dict model (tests/sieve_model.py), ring
 *                       CLOCK invariants.
 *   orc_sieve_ht_init   invariants + equality with orc_ht_insert replay.
 *   orc_layout_*        test_layout.py literals + the reference's own
 *                       common/kv_layout.h compiled into oracle/_ref.
 *   orc_gather_rows     closed-form memcpy semantics checked by brute force
 *                       (tests/test_oracle_rows.py); parity with the reference
 *                       hardware path is unpinned (HCOMM ReadNbi is not vendored).
 *   orc_export_alllayer same as gather.
 *   orc_export_rows     the reference has only a design for it
 *                       (doc/kv_offload_design.md:322-327,394-396); checked in
 *                       tests/test_oracle_rows.py against orc_export_alllayer
 *                       (a contiguous index list must give the same segment
 *                       bytes) and brute-force last-entry-wins; parity with a
 *                       reference implementation is unpinned (none exists).
 */
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* Hash table: token -> slot, uint16 entries holding slot+1, 0 = empty.      */
/* ------------------------------------------------------------------------ */

/* kvops/kernel/hisp_kernel_common.h:23-26 — Knuth multiplicative hash, top 16 bits. */
uint32_t orc_ht_hash(int32_t token)
{
    return ((uint32_t)token * 2654435761u) >> 16;
}

/* Set when a probe loop ran over the whole table without terminating
 * (the reference would spin forever).  Cleared by orc_clear_error(). */
static int g_orc_error = 0;

int orc_get_error(void) { return g_orc_error; }
void orc_clear_error(void) { g_orc_error = 0; }

/* hisp_kernel_common.h:29-43 — find the slot holding `token`, or -1. */
int32_t orc_ht_find(const uint16_t *ht, const int32_t *tok, int32_t token, int32_t mask)
{
    int32_t idx = (int32_t)orc_ht_hash(token) & mask;
    for (int64_t n = 0; n <= mask; ++n) {
        uint16_t e = ht[idx];
        if (e == 0) return -1;
        if (tok[(int32_t)e - 1] == token) return (int32_t)e - 1;
        idx = (idx + 1) & mask;
    }
    g_orc_error = 1;
    return -1;
}

/* hisp_kernel_common.h:46-61 (and :97-112, the init variant, which probes the
 * same way) — insert token->slot; an entry whose slot already holds `token`
 * stops the insert (first inserted slot wins). */
void orc_ht_insert(uint16_t *ht, const int32_t *tok, int32_t token, int32_t slot, int32_t mask)
{
    int32_t idx = (int32_t)orc_ht_hash(token) & mask;
    for (int64_t n = 0; n <= mask; ++n) {
        uint16_t e = ht[idx];
        if (e == 0) {
            ht[idx] = (uint16_t)(slot + 1);
            return;
        }
        if (tok[(int32_t)e - 1] == token) return;
        idx = (idx + 1) & mask;
    }
    g_orc_error = 1;
}

/* hisp_kernel_common.h:64-94 — erase with backward shift (Knuth 6.4 Algorithm R).
 * The move test at :87: with hole j and scan position i, the entry at i moves
 * into j unless its home lies cyclically in (j, i]. */
void orc_ht_erase(uint16_t *ht, const int32_t *tok, int32_t token, int32_t mask)
{
    int32_t idx = (int32_t)orc_ht_hash(token) & mask;
    int64_t n = 0;
    for (;; ++n) {
        if (n > mask) { g_orc_error = 1; return; }
        uint16_t e = ht[idx];
        if (e == 0) return; /* not present */
        if (tok[(int32_t)e - 1] == token) break;
        idx = (idx + 1) & mask;
    }
    int32_t j = idx, i = idx;
    for (n = 0;; ++n) {
        if (n > mask) { g_orc_error = 1; return; }
        i = (i + 1) & mask;
        uint16_t e = ht[i];
        if (e == 0) break;
        int32_t home = (int32_t)orc_ht_hash(tok[(int32_t)e - 1]) & mask;
        int move = (j < i) ? (home <= j || home > i) : (home <= j && home > i);
        if (move) {
            ht[j] = e;
            j = i;
        }
    }
    ht[j] = 0;
}

/* ------------------------------------------------------------------------ */
/* Visited bitmap: bit (slot & 7) of byte (slot >> 3).                       */
/* hisp_kernel_common.h:115-130                                              */
/* ------------------------------------------------------------------------ */
static inline int vis_get(const uint8_t *v, int32_t s) { return (v[s >> 3] >> (s & 7)) & 1; }
static inline void vis_set(uint8_t *v, int32_t s) { v[s >> 3] = (uint8_t)(v[s >> 3] | (1u << (s & 7))); }
static inline void vis_clear(uint8_t *v, int32_t s) { v[s >> 3] = (uint8_t)(v[s >> 3] & ~(1u << (s & 7))); }

/* ------------------------------------------------------------------------ */
/* SIEVE (ring CLOCK) update for one layer slice.                           */
/* ------------------------------------------------------------------------ */

/* kvops/kernel/hisp_sieve_update.cpp:17-176.
 *
 * State arrays are the layer slice: tokens [pool, padded] int32,
 * vis [pool, visStrideB] u8, ht [pool, htSize] u16, hand [pool, 16] int32
 * (only element 0 of each 16-word row is used, hisp_kernel_common.h:20-21).
 * Outputs: slots/isMiss [maxNumReqs, topK], every row rewritten.
 *
 * Batch rows are processed in increasing bid order; each row is independent
 * of the block partition in the reference (:31-34), so the order only matters
 * when two batch rows name the same pool row, which callers must not do.
 * The reference stages state in UB and writes tokens/ht back only when a miss
 * occurred (:103-105, :165-172); in place, that is the same result.
 *
 * Returns the number of misses written.
 */
int64_t orc_sieve_update(const int32_t *topk, const int64_t *reqPool, const int32_t *seqLens,
                         const int32_t *prefillLens, int32_t *tokens, uint8_t *vis, uint16_t *ht,
                         int32_t *hand, int32_t *outSlots, int8_t *isMiss, int32_t numRealIn,
                         int32_t topK, int32_t dbs, int32_t padded, int32_t visStrideB,
                         int32_t maxNumReqs, int32_t htSize, int32_t poolSize)
{
    int32_t numReal = numRealIn;
    if (numReal > maxNumReqs) numReal = maxNumReqs; /* :31-34 */
    const int32_t mask = htSize - 1;
    int64_t misses = 0;
    for (int32_t bid = 0; bid < maxNumReqs; ++bid) {
        int32_t *rs = outSlots + (int64_t)bid * topK;
        int8_t *rm = isMiss + (int64_t)bid * topK;
        if (bid >= numReal) { /* :72-78 padding rows */
            for (int32_t k = 0; k < topK; ++k) { rs[k] = -1; rm[k] = 0; }
            continue;
        }
        const int64_t reqIdx = reqPool[bid];
        if (reqIdx < 0 || reqIdx >= poolSize) { /* :80-88 */
            for (int32_t k = 0; k < topK; ++k) { rs[k] = -1; rm[k] = 0; }
            continue;
        }
        const int32_t seqLen = seqLens[bid];
        const int32_t prefill = prefillLens[reqIdx];
        const int32_t *rt = topk + (int64_t)bid * topK;
        int32_t *tok = tokens + reqIdx * padded;
        uint8_t *v = vis + reqIdx * visStrideB;
        uint16_t *t = ht + reqIdx * htSize;
        int32_t hd = hand[reqIdx * 16];
        if (hd < 0 || hd >= dbs) hd = 0; /* :108-111 */

        for (int32_t k = 0; k < topK; ++k) { /* :115-163 */
            const int32_t tp = rt[k];
            if (tp < 0 || tp >= seqLen) { rs[k] = -1; rm[k] = 0; continue; }
            if (tp >= prefill) { rs[k] = padded + (tp - prefill); rm[k] = 0; continue; }
            const int32_t hit = orc_ht_find(t, tok, tp, mask);
            if (hit >= 0) { rs[k] = hit; rm[k] = 0; vis_set(v, hit); continue; }
            int32_t h = hd;
            int64_t guard = 0;
            while (vis_get(v, h)) { /* :139-146 */
                vis_clear(v, h);
                if (++h == dbs) h = 0;
                if (++guard > (int64_t)dbs + 1) { g_orc_error = 1; break; }
            }
            const int32_t old = tok[h];
            if (old >= 0) orc_ht_erase(t, tok, old, mask);
            orc_ht_insert(t, tok, tp, h, mask);
            rs[k] = h;
            rm[k] = 1;
            tok[h] = tp;
            vis_set(v, h);
            hd = h + 1;
            if (hd == dbs) hd = 0;
            ++misses;
        }
        hand[reqIdx * 16] = hd;
    }
    return misses;
}

/* kvops/kernel/hisp_sieve_ht_init.cpp:14-60: block b -> (layer b/numReqs,
 * pool row reqStart + b%numReqs); clear the row's table and insert tokens[s]
 * for s < dbs with tokens[s] >= 0, in increasing s.  Operates on the full 3D
 * tensors tokens [layerNum, pool, padded] and ht [layerNum, pool, htSize]. */
void orc_sieve_ht_init(const int32_t *tokens, uint16_t *ht, int64_t reqStart, int32_t numReqs,
                       int32_t layerNum, int32_t poolSize, int32_t dbs, int32_t padded, int32_t htSize)
{
    const int32_t mask = htSize - 1;
    for (int32_t b = 0; b < layerNum * numReqs; ++b) {
        const int32_t layer = b / numReqs;
        const int64_t reqIdx = reqStart + b % numReqs;
        if (reqIdx < 0 || reqIdx >= poolSize) continue;
        const int32_t *tok = tokens + ((int64_t)layer * poolSize + reqIdx) * padded;
        uint16_t *t = ht + ((int64_t)layer * poolSize + reqIdx) * htSize;
        memset(t, 0, (size_t)htSize * sizeof(uint16_t));
        for (int32_t s = 0; s < dbs; ++s) {
            if (tok[s] >= 0) orc_ht_insert(t, tok, tok[s], s, mask);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Host-side derivations (kvops/kvops_ext/kvops_ext.cpp:288-312).            */
/* ------------------------------------------------------------------------ */

/* :297-300 — power of two >= 2*(padded+topK), at least 1024. */
int64_t orc_ht_size(int64_t padded, int64_t topK)
{
    int64_t s = 1024;
    while (s < 2 * (padded + topK)) s <<= 1;
    return s;
}

/* :307-312 — requests per block, aligned so each block's output rows cover
 * whole 64-byte lines: align(ceil(maxNumReqs/blockDim), 64/gcd(topK,64)).
 * A block count below 1 reads as 1, as the launch layer maps block_dim 0
 * (the reference divides by it). */
int64_t orc_reqs_per_core(int64_t maxNumReqs, int64_t blockDim, int64_t topK)
{
    if (blockDim < 1) blockDim = 1;
    int64_t a = topK, b = 64;
    while (b != 0) { int64_t t = a % b; a = b; b = t; }
    const int64_t al = 64 / a;
    int64_t r = (maxNumReqs + blockDim - 1) / blockDim;
    r = (r + al - 1) / al * al;
    return r < 1 ? 1 : r;
}

/* ------------------------------------------------------------------------ */
/* Row ownership (common/kv_layout.h:26-57, kvc_common.h:81-89).            */
/* ------------------------------------------------------------------------ */
uint32_t orc_per_layer_seg_rows(uint32_t layerRows, uint32_t nodeNum)
{
    return (layerRows + nodeNum - 1) / nodeNum;
}
uint32_t orc_node_of(uint32_t row, uint32_t S, uint32_t N) { return S == 0 ? 0 : (row / S) % N; }
uint32_t orc_seg_row_of(uint32_t row, uint32_t S, uint32_t N) { return S == 0 ? row : (row / S) / N; }
uint64_t orc_seg_offset(uint32_t layer, uint32_t row, uint32_t S, uint32_t N, uint32_t plsr, uint32_t rowBytes)
{
    return ((uint64_t)layer * plsr + orc_seg_row_of(row, S, N)) * rowBytes;
}
/* kv_layout.h:49-57: 0 = valid, -1 = invalid. */
int orc_layout_validate(uint32_t nodeNum, uint32_t layerNum, uint32_t layerRows, uint32_t plsr,
                        uint32_t rowBytes, uint32_t S)
{
    if (nodeNum == 0 || nodeNum > 64 || layerNum == 0 || layerRows == 0 || rowBytes == 0 ||
        (rowBytes & 0x7F) != 0 || S == 0 || plsr != orc_per_layer_seg_rows(layerRows, nodeNum))
        return -1;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Row movers.                                                              */
/* ------------------------------------------------------------------------ */

/* kvops/kernel/kvc_gather_rows.cpp:12-96 for segment `myNode`.
 *
 * segs[s] is the host base of segment s (all N are passed so the winner rule
 * below can be applied across segments); hot is the hot-buffer base.
 * Positions p in [0, numReal*topK) with isMiss[p] != 0, topk[p] >= 0,
 * slots[p] >= 0 and reqPool[p/topK] >= 0 are "valid misses" (:54-68).
 * row = reqHostBase[bid] + token, truncated to 32 bits for the mapping (:69-73).
 * The destination row is slot + bid*hotReqStrideRows (stride 0 = the
 * reference's hotRowBase + slot, :76).
 *
 * Winner rule (the reference races here): the final content of a destination
 * row is the source row of the LAST valid miss position p that targets it,
 * over all segments.  This call copies exactly those winners owned by myNode,
 * so running it for every node leaves the hot buffer equal to the sequential
 * "for p in order: copy" result.
 *
 * statusWords[b] for b < blockDim receives the word block b of the reference
 * would write: (queued << 40) | (1 << 32), where queued counts the valid misses
 * owned by myNode in [b*ppc, min((b+1)*ppc, numReal*topK)), ppc =
 * ceil(maxNumReqs*topK / blockDim) (kvops_ext.cpp:250-251).  An empty range
 * gives 1 << 32 (:29-33).
 *
 * Rows outside the layer region (segRow >= perLayerSegRows): the reference
 * reads segBase + (layerOffsetRows + segRow)*rowBytes regardless (:74-77), i.e.
 * a row of the next layer's region, or past the segment's end for the last
 * layer, where HCOMM's ReadNbi fails with the 0x200 + (pos & 0xFF) +
 * (ret << 16) band (:78-81).  The rule here reads no such row: such a
 * position is still counted in queued and still takes part in the winner
 * rule (so a destination whose winner lies outside is left untouched), and
 * the word of its block carries 0x200 + (p & 0xFF) + (1 << 16) for the
 * lowest such position p owned by myNode.  perLayerSegRows = UINT32_MAX
 * disables the check (the reference's read, in-segment cases only).
 *
 * Returns the number of rows copied (winners owned by myNode).
 */
int64_t orc_gather_rows(uint8_t *const *segs, uint8_t *hot, uint32_t layerOffsetRows, uint32_t perLayerSegRows,
                        uint32_t rowBytes, const int32_t *topk, const int64_t *reqPool, const int64_t *reqHostBase,
                        const int32_t *slots, const int8_t *isMiss, int32_t numRealIn, uint32_t topK,
                        uint32_t maxNumReqs, uint32_t S, uint32_t N, uint32_t myNode,
                        uint32_t hotReqStrideRows, uint32_t blockDim, uint64_t *statusWords)
{
    int32_t numReal = numRealIn;
    if (numReal > (int32_t)maxNumReqs) numReal = (int32_t)maxNumReqs;
    if (numReal < 0) numReal = 0;
    const int64_t total = (int64_t)numReal * topK;
    if (blockDim == 0) blockDim = 1;
    const int64_t ppc = ((int64_t)maxNumReqs * topK + blockDim - 1) / blockDim;
    for (uint32_t b = 0; b < blockDim; ++b) statusWords[b] = 0;
    int64_t firstErr[8];
    for (uint32_t b = 0; b < 8; ++b) firstErr[b] = -1;

    int64_t copied = 0;
    /* Walk backwards: the first time a destination row is seen, that position
     * is its winner.  Destinations seen so far live in an open-addressing set
     * keyed by destination row + 1 (0 = empty). */
    uint64_t cap = 1024;
    while (cap < 2 * (uint64_t)(total + 1)) cap <<= 1;
    uint64_t *seen = (uint64_t *)calloc(cap, sizeof(uint64_t));
    if (seen == NULL) { g_orc_error = 2; return -1; }
    for (int64_t p = total - 1; p >= 0; --p) {
        if (isMiss[p] == 0) continue;
        const int64_t bid = p / topK;
        const int32_t tp = topk[p];
        const int32_t slot = slots[p];
        if (tp < 0 || slot < 0) continue;
        if (reqPool[bid] < 0) continue;
        const uint32_t row = (uint32_t)(reqHostBase[bid] + tp);
        const uint32_t node = orc_node_of(row, S, N);
        const int64_t blk = p / ppc;
        if (node == myNode && blk < (int64_t)blockDim) statusWords[blk] += 1;
        const uint64_t dst = (uint64_t)slot + (uint64_t)bid * hotReqStrideRows;
        uint64_t i = (dst * 0x9E3779B97F4A7C15ull) & (cap - 1);
        int winner = 1;
        while (seen[i] != 0) {
            if (seen[i] == dst + 1) { winner = 0; break; }
            i = (i + 1) & (cap - 1);
        }
        if (winner) seen[i] = dst + 1;
        if (node != myNode) continue;
        const uint64_t segRow = orc_seg_row_of(row, S, N);
        if (segRow >= perLayerSegRows) {
            if (blk < 8 && blk < (int64_t)blockDim) firstErr[blk] = p; /* walking backwards: the last write is the lowest */
            continue;
        }
        if (!winner) continue;
        memcpy(hot + dst * rowBytes, segs[node] + ((uint64_t)layerOffsetRows + segRow) * rowBytes, rowBytes);
        ++copied;
    }
    free(seen);
    for (uint32_t b = 0; b < blockDim; ++b) {
        const int64_t lo = (int64_t)b * ppc;
        if (lo >= total) { statusWords[b] = 1ull << 32; continue; }
        uint64_t err = 0;
        if (b < 8 && firstErr[b] >= 0) err = 0x200u + ((uint64_t)firstErr[b] & 0xFFu) + (1u << 16);
        statusWords[b] = (statusWords[b] << 40) | (1ull << 32) | err;
    }
    return copied;
}

/* Host staging step of the CPU serial pipeline (the baseline the reference
 * design replaces, doc/kv_offload_design.md:21: CPU miss list -> host copy
 * into a staging buffer -> one H2D -> device scatter).  Lists the winning
 * valid miss rows of every segment (the winner rule of orc_gather_rows), in
 * position order, and copies them into the dense `staging` buffer with
 * `threads` threads; dstRows[i] receives the hot row of staging row i.
 * Returns the number of staged rows (or -1 if memory runs out).  Timing
 * baseline only: the GPU path is checked against orc_gather_rows. */
struct orc_stage_job {
    uint8_t *staging;
    const uint8_t *const *src;
    int64_t lo, hi;
    uint32_t rowBytes;
};

static void *orc_stage_copy(void *arg)
{
    const struct orc_stage_job *j = (const struct orc_stage_job *)arg;
    for (int64_t i = j->lo; i < j->hi; ++i) memcpy(j->staging + (uint64_t)i * j->rowBytes, j->src[i], j->rowBytes);
    return NULL;
}

int64_t orc_stage_rows(uint8_t *const *segs, uint8_t *staging, int64_t *dstRows, uint32_t layerOffsetRows,
                       uint32_t rowBytes, const int32_t *topk, const int64_t *reqPool, const int64_t *reqHostBase,
                       const int32_t *slots, const int8_t *isMiss, int32_t numRealIn, uint32_t topK,
                       uint32_t maxNumReqs, uint32_t S, uint32_t N, uint32_t hotReqStrideRows, int32_t threads)
{
    int32_t numReal = numRealIn;
    if (numReal > (int32_t)maxNumReqs) numReal = (int32_t)maxNumReqs;
    if (numReal < 0) numReal = 0;
    const int64_t total = (int64_t)numReal * topK;
    uint64_t cap = 1024;
    while (cap < 2 * (uint64_t)(total + 1)) cap <<= 1;
    uint64_t *seen = (uint64_t *)calloc(cap, sizeof(uint64_t));
    const uint8_t **src = (const uint8_t **)malloc(sizeof(uint8_t *) * (size_t)(total + 1));
    if (seen == NULL || src == NULL) { free(seen); free(src); return -1; }
    int64_t n = 0;
    for (int64_t p = total - 1; p >= 0; --p) {  /* backwards: first seen = last position = winner */
        if (isMiss[p] == 0) continue;
        const int64_t bid = p / topK;
        const int32_t tp = topk[p], slot = slots[p];
        if (tp < 0 || slot < 0 || reqPool[bid] < 0) continue;
        const uint32_t row = (uint32_t)(reqHostBase[bid] + tp);
        const uint32_t node = orc_node_of(row, S, N);
        if (node >= N) continue;
        const uint64_t dst = (uint64_t)slot + (uint64_t)bid * hotReqStrideRows;
        uint64_t i = (dst * 0x9E3779B97F4A7C15ull) & (cap - 1);
        int winner = 1;
        while (seen[i] != 0) {
            if (seen[i] == dst + 1) { winner = 0; break; }
            i = (i + 1) & (cap - 1);
        }
        if (!winner) continue;
        seen[i] = dst + 1;
        src[n] = segs[node] + ((uint64_t)layerOffsetRows + orc_seg_row_of(row, S, N)) * rowBytes;
        dstRows[n] = (int64_t)dst;
        ++n;
    }
    free(seen);
    if (threads < 1) threads = 1;
    if (threads > 64) threads = 64;
    pthread_t tid[64];
    struct orc_stage_job job[64];
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        job[t].staging = staging;
        job[t].src = src;
        job[t].lo = n * t / threads;
        job[t].hi = n * (t + 1) / threads;
        job[t].rowBytes = rowBytes;
        if (t == threads - 1 || pthread_create(&tid[t], NULL, orc_stage_copy, &job[t]) != 0) {
            orc_stage_copy(&job[t]);
        } else {
            ++started;
        }
    }
    for (int t = 0; t < started; ++t) pthread_join(tid[t], NULL);
    free(src);
    return n;
}

/* kvops/kernel/kvc_scatter_rows_alllayer.cpp:11-67 for segment `myNode`:
 * for l < layerNum, row in [rowLo, rowLo+rowCnt) in increasing order, rows
 * owned by myNode are copied from src0 + l*srcLayerStride + row*rowBytes to
 * seg + (l*plsr + segRow(row))*rowBytes (:34-53).  With S > 1 several rows of
 * one stripe share a segment row; the sequential order makes the highest row
 * of the stripe the one left in the segment.
 * Returns the reference's queued count (rows owned x layers, :47). */
int64_t orc_export_alllayer(uint8_t *seg, const uint8_t *src0, uint64_t srcLayerStride, uint32_t plsr,
                            uint32_t rowBytes, uint32_t rowLo, uint32_t rowCnt, uint32_t layerNum,
                            uint32_t S, uint32_t N, uint32_t myNode)
{
    int64_t queued = 0;
    for (uint32_t l = 0; l < layerNum; ++l) {
        const uint8_t *srcL = src0 + (uint64_t)l * srcLayerStride;
        for (uint32_t row = rowLo; row < rowLo + rowCnt; ++row) {
            if (orc_node_of(row, S, N) != myNode) continue;
            const uint64_t segRow = orc_seg_row_of(row, S, N);
            memcpy(seg + ((uint64_t)l * plsr + segRow) * rowBytes, srcL + (uint64_t)row * rowBytes, rowBytes);
            ++queued;
        }
    }
    return queued;
}

/* Decode-incremental single-layer export (the reference design's export_rows /
 * kvc_scatter_rows, doc/kv_offload_design.md:322-327,353-354,394-396: the
 * import's arguments with the direction reversed).  For entries i in
 * [0, min(numReal, maxRows)) in increasing order: row = idx[i]; negative rows
 * are skipped; rows owned by myNode (kvc_common.h:81-89 mapping on the low 32
 * bits, as the import) are copied from src + i*rowBytes to
 * seg + (layerId*plsr + segRow)*rowBytes, so the last entry naming a segment
 * row wins.  A segment row >= plsr is not written; the status word of its
 * entry block records the lowest such entry (error code band of
 * kvc_gather_rows.cpp:78-81).  statusWords[b], b < blockDim:
 * (owned << 40) | (1 << 32) | err over entries [b*ppc, (b+1)*ppc),
 * ppc = ceil(maxRows/blockDim); an empty range gives 1 << 32.
 * Returns the number of entries written. */
int64_t orc_export_rows(uint8_t *seg, const uint8_t *src, const int64_t *idx, int32_t numRealIn, uint32_t maxRows,
                        uint32_t layerId, uint32_t plsr, uint32_t rowBytes, uint32_t S, uint32_t N, uint32_t myNode,
                        uint32_t blockDim, uint64_t *statusWords)
{
    int32_t n = numRealIn;
    if (n > (int32_t)maxRows) n = (int32_t)maxRows;
    if (n < 0) n = 0;
    if (blockDim == 0) blockDim = 1;
    const int64_t ppc = ((int64_t)maxRows + blockDim - 1) / blockDim;
    uint64_t owned[8] = {0};
    int64_t firstErr[8];
    for (uint32_t b = 0; b < 8; ++b) firstErr[b] = -1;
    int64_t written = 0;
    for (int32_t i = 0; i < n; ++i) {
        if (idx[i] < 0) continue;
        const uint32_t row = (uint32_t)idx[i];
        if (orc_node_of(row, S, N) != myNode) continue;
        const int64_t b = i / ppc;
        if (b < 8) owned[b] += 1;
        const uint64_t segRow = orc_seg_row_of(row, S, N);
        if (segRow >= plsr) {
            if (b < 8 && firstErr[b] < 0) firstErr[b] = i;
            continue;
        }
        memcpy(seg + ((uint64_t)layerId * plsr + segRow) * rowBytes, src + (uint64_t)i * rowBytes, rowBytes);
        ++written;
    }
    for (uint32_t b = 0; b < blockDim; ++b) {
        if ((int64_t)b * ppc >= n) { statusWords[b] = 1ull << 32; continue; }
        uint64_t err = 0;
        if (firstErr[b] >= 0) err = 0x200u + ((uint64_t)firstErr[b] & 0xFFu) + (1u << 16);
        statusWords[b] = (owned[b] << 40) | (1ull << 32) | err;
    }
    return written;
}
