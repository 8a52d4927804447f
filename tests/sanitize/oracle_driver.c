/* Runs every function of the CPU oracle (oracle/kvx_oracle.c) on random
 * shapes under AddressSanitizer and UndefinedBehaviorSanitizer: SIEVE steps
 * with padding rows, bad pool rows, num_real beyond the batch, invalid and
 * decode-extension positions, duplicates and wrapping rings; the table
 * build; the row movers with rows outside the segment region.  Buffers are
 * sized exactly for the accesses the oracle makes, so any read or write past
 * them is reported.  Exit status 0 = no finding. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

uint32_t orc_ht_hash(int32_t token);
int orc_get_error(void);
void orc_clear_error(void);
int32_t orc_ht_find(const uint16_t *ht, const int32_t *tok, int32_t token, int32_t mask);
void orc_ht_insert(uint16_t *ht, const int32_t *tok, int32_t token, int32_t slot, int32_t mask);
void orc_ht_erase(uint16_t *ht, const int32_t *tok, int32_t token, int32_t mask);
int64_t orc_sieve_update(const int32_t *topk, const int64_t *reqPool, const int32_t *seqLens,
                         const int32_t *prefillLens, int32_t *tokens, uint8_t *vis, uint16_t *ht, int32_t *hand,
                         int32_t *outSlots, int8_t *isMiss, int32_t numRealIn, int32_t topK, int32_t dbs,
                         int32_t padded, int32_t visStrideB, int32_t maxNumReqs, int32_t htSize, int32_t poolSize);
void orc_sieve_ht_init(const int32_t *tokens, uint16_t *ht, int64_t reqStart, int32_t numReqs, int32_t layerNum,
                       int32_t poolSize, int32_t dbs, int32_t padded, int32_t htSize);
int64_t orc_ht_size(int64_t padded, int64_t topK);
int64_t orc_reqs_per_core(int64_t maxNumReqs, int64_t blockDim, int64_t topK);
uint32_t orc_per_layer_seg_rows(uint32_t layerRows, uint32_t nodeNum);
uint32_t orc_node_of(uint32_t row, uint32_t S, uint32_t N);
uint32_t orc_seg_row_of(uint32_t row, uint32_t S, uint32_t N);
uint64_t orc_seg_offset(uint32_t layer, uint32_t row, uint32_t S, uint32_t N, uint32_t plsr, uint32_t rowBytes);
int orc_layout_validate(uint32_t nodeNum, uint32_t layerNum, uint32_t layerRows, uint32_t plsr, uint32_t rowBytes,
                        uint32_t S);
int64_t orc_gather_rows(uint8_t *const *segs, uint8_t *hot, uint32_t layerOffsetRows, uint32_t perLayerSegRows,
                        uint32_t rowBytes, const int32_t *topk, const int64_t *reqPool, const int64_t *reqHostBase, const int32_t *slots,
                        const int8_t *isMiss, int32_t numRealIn, uint32_t topK, uint32_t maxNumReqs, uint32_t S,
                        uint32_t N, uint32_t myNode, uint32_t hotReqStrideRows, uint32_t blockDim,
                        uint64_t *statusWords);
int64_t orc_stage_rows(uint8_t *const *segs, uint8_t *staging, int64_t *dstRows, uint32_t layerOffsetRows,
                       uint32_t rowBytes, const int32_t *topk, const int64_t *reqPool, const int64_t *reqHostBase,
                       const int32_t *slots, const int8_t *isMiss, int32_t numRealIn, uint32_t topK,
                       uint32_t maxNumReqs, uint32_t S, uint32_t N, uint32_t hotReqStrideRows, int32_t threads);
int64_t orc_export_alllayer(uint8_t *seg, const uint8_t *src0, uint64_t srcLayerStride, uint32_t plsr,
                            uint32_t rowBytes, uint32_t rowLo, uint32_t rowCnt, uint32_t layerNum, uint32_t S,
                            uint32_t N, uint32_t myNode);
int64_t orc_export_rows(uint8_t *seg, const uint8_t *src, const int64_t *idx, int32_t numRealIn, uint32_t maxRows,
                        uint32_t layerId, uint32_t plsr, uint32_t rowBytes, uint32_t S, uint32_t N, uint32_t myNode,
                        uint32_t blockDim, uint64_t *statusWords);

static uint64_t g_rng = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void)
{
    g_rng ^= g_rng << 13;
    g_rng ^= g_rng >> 7;
    g_rng ^= g_rng << 17;
    return (uint32_t)(g_rng >> 16);
}
static int32_t rint_in(int32_t lo, int32_t hi) { return lo + (int32_t)(rnd() % (uint32_t)(hi - lo + 1)); }
static void *xmalloc(size_t n) { void *p = malloc(n ? n : 1); if (!p) abort(); return p; }

#define ROWB 128u

static void sieve_and_rows(int trial)
{
    const int32_t dbs = rint_in(1, 300), padded = (dbs + 15) / 16 * 16, topK = rint_in(1, 200);
    const int32_t pool = rint_in(1, 6), maxReqs = rint_in(1, 7), visStride = ((padded + 7) / 8 + 63) / 64 * 64;
    const int32_t H = (int32_t)orc_ht_size(padded, topK);
    int32_t *prefill = xmalloc(sizeof(int32_t) * pool);
    int32_t *tokens = xmalloc(sizeof(int32_t) * (size_t)pool * padded);
    uint8_t *vis = xmalloc((size_t)pool * visStride);
    uint16_t *ht = xmalloc(sizeof(uint16_t) * (size_t)pool * H);
    int32_t *hand = xmalloc(sizeof(int32_t) * (size_t)pool * 16);
    memset(vis, 0, (size_t)pool * visStride);
    memset(hand, 0, sizeof(int32_t) * (size_t)pool * 16);
    for (int32_t r = 0; r < pool; ++r) {
        prefill[r] = rint_in(1, 4 * dbs + 8);
        for (int32_t s = 0; s < padded; ++s) tokens[(size_t)r * padded + s] = s < dbs && s < prefill[r] ? s : -1;
    }
    if (pool > 1) hand[16] = dbs + 3;  /* a dirty hand on pool row 1 */
    orc_sieve_ht_init(tokens, ht, 0, pool, 1, pool, dbs, padded, H);
    int32_t *topk = xmalloc(sizeof(int32_t) * (size_t)maxReqs * topK);
    int64_t *reqPool = xmalloc(sizeof(int64_t) * maxReqs);
    int32_t *seq = xmalloc(sizeof(int32_t) * maxReqs);
    int32_t *slots = xmalloc(sizeof(int32_t) * (size_t)maxReqs * topK);
    int8_t *miss = xmalloc((size_t)maxReqs * topK);
    int64_t *hostBase = xmalloc(sizeof(int64_t) * maxReqs);
    for (int step = 0; step < 6; ++step) {
        const int32_t numReal = rint_in(0, maxReqs + 2);
        int32_t maxSeq = 0;
        for (int32_t b = 0; b < maxReqs; ++b) {
            /* distinct pool rows for the real rows, -1 / out of range now and then */
            reqPool[b] = b < pool ? (b + step) % pool : -1;
            if (rnd() % 9 == 0) reqPool[b] = (rnd() & 1) ? -4 : pool + 3;
            const int32_t p = (reqPool[b] >= 0 && reqPool[b] < pool) ? prefill[reqPool[b]] : 5;
            seq[b] = p + rint_in(-3, 5);
            if (seq[b] > maxSeq) maxSeq = seq[b];
            hostBase[b] = rint_in(0, 50);
            for (int32_t k = 0; k < topK; ++k) topk[(size_t)b * topK + k] = rint_in(-3, seq[b] + 4);
            for (int32_t k = 0; k < topK; ++k)
                if (rnd() % 16 == 0) topk[(size_t)b * topK + k] = topk[(size_t)b * topK + rnd() % topK];
        }
        /* a batch may not name one pool row twice: keep the first */
        for (int32_t b = 0; b < maxReqs; ++b)
            for (int32_t c = 0; c < b; ++c)
                if (reqPool[b] >= 0 && reqPool[b] < pool && reqPool[c] == reqPool[b]) reqPool[b] = -1;
        orc_sieve_update(topk, reqPool, seq, prefill, tokens, vis, ht, hand, slots, miss, numReal, topK, dbs, padded,
                         visStride, maxReqs, H, pool);
        orc_clear_error();
        /* the import of every segment, and the staging pipeline */
        const uint32_t S = (uint32_t)rint_in(1, 4), N = (uint32_t)rint_in(1, 3), layerOff = (uint32_t)rint_in(0, 2);
        const uint32_t stride = (rnd() & 1) ? (uint32_t)padded : 0u;
        const uint32_t maxRow = 50u + (uint32_t)maxSeq + 8u;
        const uint32_t segRows = layerOff + maxRow / S / N + 2u;
        const size_t hotRows = (size_t)maxReqs * stride + (size_t)padded + (size_t)maxSeq + 16u;
        uint8_t *segs[3];
        for (uint32_t n = 0; n < N; ++n) {
            segs[n] = xmalloc((size_t)segRows * ROWB);
            memset(segs[n], (int)(n + 1), (size_t)segRows * ROWB);
        }
        uint8_t *hot = xmalloc(hotRows * ROWB);
        uint64_t status[8];
        for (uint32_t n = 0; n < N; ++n)
            orc_gather_rows(segs, hot, layerOff, (rnd() & 1) ? 0xFFFFFFFFu : maxRow / S / N / 2u, ROWB, topk, reqPool, hostBase, slots, miss, numReal, (uint32_t)topK,
                            (uint32_t)maxReqs, S, N, n, stride, (uint32_t)rint_in(1, 8), status);
        const size_t total = (size_t)maxReqs * topK;
        uint8_t *staging = xmalloc(total * ROWB);
        int64_t *dst = xmalloc(sizeof(int64_t) * total);
        orc_stage_rows(segs, staging, dst, layerOff, ROWB, topk, reqPool, hostBase, slots, miss, numReal,
                       (uint32_t)topK, (uint32_t)maxReqs, S, N, stride, rint_in(1, 3));
        free(staging);
        free(dst);
        free(hot);
        for (uint32_t n = 0; n < N; ++n) free(segs[n]);
    }
    /* direct table operations on one row */
    uint16_t *t = ht;
    for (int32_t i = 0; i < 50; ++i) {
        const int32_t s = rint_in(0, dbs - 1);
        orc_ht_find(t, tokens, rint_in(-2, 5 * dbs), H - 1);
        if (tokens[s] >= 0 && rnd() % 2) orc_ht_erase(t, tokens, tokens[s], H - 1);
        else if (tokens[s] >= 0) orc_ht_insert(t, tokens, tokens[s], s, H - 1);
    }
    orc_clear_error();
    (void)trial;
    free(prefill); free(tokens); free(vis); free(ht); free(hand); free(topk); free(reqPool); free(seq);
    free(slots); free(miss); free(hostBase);
}

static void exports(void)
{
    const uint32_t L = (uint32_t)rint_in(1, 3), N = (uint32_t)rint_in(1, 4), S = (uint32_t)rint_in(1, 5);
    const uint32_t layerRows = (uint32_t)rint_in(1, 200), plsr = orc_per_layer_seg_rows(layerRows, N);
    orc_layout_validate(N, L, layerRows, plsr, ROWB, S);
    uint8_t *src = xmalloc((size_t)L * layerRows * ROWB);
    memset(src, 7, (size_t)L * layerRows * ROWB);
    uint8_t *seg = xmalloc((size_t)L * plsr * ROWB);
    const uint32_t lo = (uint32_t)rint_in(0, (int32_t)layerRows - 1), cnt = (uint32_t)rint_in(0, (int32_t)(layerRows - lo));
    for (uint32_t n = 0; n < N; ++n) orc_export_alllayer(seg, src, (uint64_t)layerRows * ROWB, plsr, ROWB, lo, cnt, L, S, N, n);
    const uint32_t maxRows = (uint32_t)rint_in(1, 64);
    int64_t *idx = xmalloc(sizeof(int64_t) * maxRows);
    for (uint32_t i = 0; i < maxRows; ++i) idx[i] = rint_in(-2, (int32_t)layerRows + 5);
    uint8_t *rowsSrc = xmalloc((size_t)maxRows * ROWB);
    memset(rowsSrc, 9, (size_t)maxRows * ROWB);
    uint64_t status[8];
    for (uint32_t n = 0; n < N; ++n)
        orc_export_rows(seg, rowsSrc, idx, rint_in(0, (int32_t)maxRows + 2), maxRows, (uint32_t)rint_in(0, (int32_t)L - 1),
                        plsr, ROWB, S, N, n, (uint32_t)rint_in(1, 8), status);
    for (int i = 0; i < 20; ++i) {
        const uint32_t row = rnd(), s = (uint32_t)rint_in(0, 9), nn = (uint32_t)rint_in(1, 64);
        orc_seg_offset((uint32_t)rint_in(0, 60), row % 100000u, s, nn, plsr, ROWB);
        orc_node_of(row, s, nn);
        orc_reqs_per_core(rint_in(0, 300), rint_in(0, 9), rint_in(1, 9000));
    }
    free(src); free(seg); free(idx); free(rowsSrc);
}

int main(int argc, char **argv)
{
    const int trials = argc > 1 ? atoi(argv[1]) : 1000;
    for (int trial = 0; trial < trials; ++trial) {
        sieve_and_rows(trial);
        exports();
    }
    printf("oracle driver: %d trials, no sanitizer finding\n", trials);
    return 0;
}
