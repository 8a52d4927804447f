// The hash-table update of a SIEVE step with misses, rebuilt in parallel
// (after the batch HBM kernel, variant 5, for rows it leaves pending).
//
// The reference erases each evicted token with Algorithm R and inserts each
// new token by linear probing, one event at a time, in position order
// (hisp_sieve_update.cpp:147-155, hisp_kernel_common.h:46-94).  Algorithm R
// leaves a table exactly as if the deleted key had never been inserted
// (Knuth, TAOCP 6.4), so after the step the table is the first-come-first-
// served linear-probing table of the survivors in their insertion order
// followed by the new tokens in event order.  The pre-step table itself is
// that table for the survivors taken in cell order, starting after an empty
// cell: a key's probe path runs over cells that precede it in that order.
// So the step's table is built from scratch by inserting
//
//     the survivors in cell order, then the new keys in event order,
//
// each into the first free cell at or after its home.  Which cells a set of
// keys occupies does not depend on the order they go in: with n(x) keys homed
// at cell x, the backlog b(x) = max(0, b(x-1) + n(x) - 1) leaves cell x free
// iff b(x-1) + n(x) = 0.  That makes every chunk of the insertion sequence
// independent: its free cells are those of the keys before it, found by one
// histogram and one max-plus scan, and only the chunk's own keys go in one at
// a time.  Three kernels:
//
//  1. cells (many workgroups per row): each cell of the pre-step table is
//     tagged empty, deleted or a survivor with its home; the per-home counts
//     of every key after the step (survivors and new keys) are summed;
//  2. final (one workgroup per row): the cells the step's keys occupy (the
//     same scan, cyclic over the table), the cells that end empty (cleared
//     here), a cell empty before and after the step that starts the cell
//     order, and per chunk of cells the start of its cluster and whether a
//     deleted cell precedes it in the cluster (otherwise its survivors stay);
//  3. chunks (one workgroup per chunk of 256 cells or 256 new keys): the
//     chunk's free cells, then its keys in order; a survivor that lands on
//     another cell, and every new key, writes its entry there.
//
// Every cell is written by at most one workgroup (a cell is taken once, and a
// cell that ends empty is never taken), so the chunks run in any order.
#include "kvx_internal.h"
#include "sieve_common.h"

// device memory through global-space pointers (global_* instructions)
#define KVX_GM __attribute__((address_space(1)))

namespace kvx {
namespace {

using sieve::report_overflow;

constexpr int kTT = 1024;                  // threads of the final and chunk kernels
constexpr int kTW = kTT / 64;              // their waves
constexpr int kCellThreads = 256;          // threads of the cells kernel (8 cells each)
constexpr uint32_t kCellsPerBlock = kCellThreads * 8u;
constexpr uint32_t kDeleted = 0xFFFF0000u;  // cellw of a deleted key
constexpr int32_t kNegInf = -(1 << 29);

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct TblParams {
    KvxLaunch<HispSieveUpdateArgs> L;
    uint32_t *tbl;      // [maxNumReqs][t.words]
    TableLayout t;
};

__device__ __forceinline__ KVX_GM uint32_t *row_tbl(const TblParams &P, int32_t bid)
{
    return (KVX_GM uint32_t *)P.tbl + static_cast<uint64_t>(bid) * P.t.words;
}

// A map b -> max(p, b + q) of the backlog over a run of cells; a cell with n
// keys homed at it is {0, n - 1} (the backlog is never negative).
struct MP {
    int32_t p, q;
};
__device__ __forceinline__ MP mp_then(MP f, MP g)  // f, then g
{
    const int32_t fp = f.p + g.q;
    return MP{fp > g.p ? fp : g.p, f.q + g.q};
}
__device__ __forceinline__ int32_t mp_apply(MP m, int32_t b)
{
    const int32_t v = b + m.q;
    return v > m.p ? v : m.p;
}
__device__ __forceinline__ MP mp_cell(int32_t n)
{
    return MP{0, n - 1};
}

// Exclusive scan of one map per thread over the block (kTT threads) in thread
// order; `total` is every thread's maps composed.
__device__ __forceinline__ MP block_scan_mp(MP m, MP &total, MP *sPart)
{
    const int lane = __lane_id(), wave = threadIdx.x >> 6;
    MP inc = m;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        MP o;
        o.p = __shfl_up(inc.p, d);
        o.q = __shfl_up(inc.q, d);
        if (lane >= d) inc = mp_then(o, inc);
    }
    MP ex;
    ex.p = __shfl_up(inc.p, 1);
    ex.q = __shfl_up(inc.q, 1);
    if (lane == 0) ex = MP{kNegInf, 0};
    if (lane == 63) sPart[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        MP run{kNegInf, 0};
        for (int w = 0; w < kTW; ++w) {
            const MP v = sPart[w];
            sPart[w] = run;
            run = mp_then(run, v);
        }
        sPart[kTW] = run;
    }
    __syncthreads();
    total = sPart[kTW];
    const MP r = mp_then(sPart[wave], ex);
    __syncthreads();  // sPart is reused by the next scan
    return r;
}

// Three-level bitmap (a bit per cell of the window, per nonzero word, per
// nonzero summary word) in LDS; used by one wave, whose LDS operations
// complete in order.  First set bit at or after i, or -1.
struct Win {
    uint64_t *l0, *l1, *l2;
};
__device__ __forceinline__ uint64_t from_bit(uint32_t b) { return ~0ull << (b & 63u); }

__device__ __forceinline__ int32_t win_next(const Win &m, uint32_t i)
{
    if (i >= kTblWinBits) return -1;
    const uint32_t w = i >> 6;
    const uint64_t x0 = m.l0[w] & from_bit(i);
    if (x0) return static_cast<int32_t>((w << 6) + __builtin_ctzll(x0));
    const uint32_t s1 = w + 1u;
    if (s1 < kTblWinWords && (s1 & 63u)) {
        const uint64_t x1 = m.l1[s1 >> 6] & from_bit(s1);
        if (x1) {
            const uint32_t w0 = ((s1 >> 6) << 6) + static_cast<uint32_t>(__builtin_ctzll(x1));
            return static_cast<int32_t>((w0 << 6) + __builtin_ctzll(m.l0[w0]));
        }
    }
    const uint32_t s2 = (s1 + 63u) >> 6;  // summary words after the one searched
    if (s2 >= kTblWinL1) return -1;
    const uint64_t x2 = m.l2[0] & from_bit(s2);
    if (!x2) return -1;
    const uint32_t w1 = static_cast<uint32_t>(__builtin_ctzll(x2));
    const uint32_t w0 = (w1 << 6) + static_cast<uint32_t>(__builtin_ctzll(m.l1[w1]));
    return static_cast<int32_t>((w0 << 6) + __builtin_ctzll(m.l0[w0]));
}

__device__ __forceinline__ void win_clear(const Win &m, uint32_t i, bool writer)
{
    const uint32_t w = i >> 6, v = w >> 6;
    const uint64_t x0 = m.l0[w] & ~(1ull << (i & 63u));
    if (writer) m.l0[w] = x0;
    if (x0) return;
    const uint64_t x1 = m.l1[v] & ~(1ull << (w & 63u));
    if (writer) m.l1[v] = x1;
    if (x1) return;
    if (writer) m.l2[0] &= ~(1ull << v);
}

// The summary levels of the window, from its words (whole block).
__device__ __forceinline__ void win_summarize(const Win &m)
{
    for (uint32_t v = threadIdx.x; v < kTblWinL1; v += kTT) {
        uint64_t s = 0;
        for (uint32_t q = 0; q < 64u && (v << 6) + q < kTblWinWords; ++q) {
            if (m.l0[(v << 6) + q]) s |= 1ull << q;
        }
        m.l1[v] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t s = 0;
        for (uint32_t v = 0; v < kTblWinL1; ++v) {
            if (m.l1[v]) s |= 1ull << v;
        }
        m.l2[0] = s;
    }
    __syncthreads();
}

// ---- 1. cells ---------------------------------------------------------------
__global__ __launch_bounds__(kCellThreads) void kvx_sieve_table_cells(TblParams P)
{
    const HispSieveUpdateArgs &a = P.L.a;
    const int32_t bid = blockIdx.y;
    if (bid >= static_cast<int32_t>(a.maxNumReqs)) return;
    KVX_GM uint32_t *tb = row_tbl(P, bid);
    if (tb[P.t.meta] != 1u) return;  // no rebuild pending for this row
    const uint32_t H = a.htSize, mask = H - 1u, padded = a.paddedBufferSize;
    const int64_t reqIdx = reinterpret_cast<const KVX_GM int64_t *>(a.reqPoolIndices)[bid];
    const KVX_GM uint16_t *ht = reinterpret_cast<const KVX_GM uint16_t *>(a.deviceBufferHt) + reqIdx * H;
    const KVX_GM int32_t *tok = reinterpret_cast<const KVX_GM int32_t *>(a.deviceBufferTokens) + reqIdx * padded;
    KVX_GM uint32_t *cellw = tb + P.t.cellw;
    KVX_GM uint32_t *hist = tb + P.t.hist;
    const KVX_GM uint32_t *evict = tb + P.t.evict;
    const uint32_t c8 = blockIdx.x * kCellThreads + threadIdx.x;  // 8 cells
    if (c8 * 8u < H) {
        const u32x4 v = reinterpret_cast<const KVX_GM u32x4 *>(ht)[c8];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t out[8];
        int32_t tk[8];
#pragma unroll
        for (int h = 0; h < 8; ++h) {  // the survivors' tokens, loaded together
            const uint32_t e = (w[h >> 1] >> (16 * (h & 1))) & 0xFFFFu;
            const uint32_t s = e - 1u;
            const bool live = e != 0u && s < padded && !((evict[s >> 5] >> (s & 31u)) & 1u);
            tk[h] = live ? tok[s] : -1;
            out[h] = e == 0u ? 0u : (live ? e : kDeleted);
        }
#pragma unroll
        for (int h = 0; h < 8; ++h) {
            if (out[h] == 0u || out[h] == kDeleted) continue;
            const uint32_t home = ht_hash(tk[h]) & mask;
            out[h] |= home << 16;
            __hip_atomic_fetch_add(hist + home, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        KVX_GM u32x4 *cw4 = reinterpret_cast<KVX_GM u32x4 *>(cellw + c8 * 8u);
        cw4[0] = u32x4{out[0], out[1], out[2], out[3]};
        cw4[1] = u32x4{out[4], out[5], out[6], out[7]};
    }
    // the new keys' homes
    const uint32_t N = tb[P.t.meta + 1];
    const KVX_GM uint32_t *newk = tb + P.t.newk;
    for (uint32_t j = c8; j < N; j += gridDim.x * kCellThreads) {
        __hip_atomic_fetch_add(hist + (newk[j] >> 16), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---- 2. final ---------------------------------------------------------------
__global__ __launch_bounds__(kTT) void kvx_sieve_table_final(TblParams P)
{
    __shared__ MP sPart[kTW + 1];
    __shared__ int32_t sE;
    __shared__ int32_t sLastEmpty[kTblMaxHt / kTblChunkCells], sLastDel[kTblMaxHt / kTblChunkCells];
    __shared__ uint32_t sSurv[kTblMaxHt / kTblChunkCells];
    const HispSieveUpdateArgs &a = P.L.a;
    const int32_t bid = blockIdx.x;
    if (bid >= static_cast<int32_t>(a.maxNumReqs)) return;
    KVX_GM uint32_t *tb = row_tbl(P, bid);
    if (tb[P.t.meta] != 1u) return;
    const uint32_t H = a.htSize, mask = H - 1u, HH = H < 65536u ? H : 65536u;
    const int64_t reqIdx = reinterpret_cast<const KVX_GM int64_t *>(a.reqPoolIndices)[bid];
    KVX_GM uint16_t *ht = reinterpret_cast<KVX_GM uint16_t *>(a.deviceBufferHt) + reqIdx * H;
    const KVX_GM uint32_t *cellw = tb + P.t.cellw;
    const KVX_GM uint32_t *hist = tb + P.t.hist;
    const uint32_t tid = threadIdx.x;
    const uint32_t S = H / kTT;  // cells per thread (H >= 1024, a power of two)
    const uint32_t c0 = tid * S;

    // the cells occupied after the step, cyclic: the backlog entering cell 0
    // is the fixed point of the whole ring's map, max(p, b + q) with q < 0
    // (fewer keys than cells), i.e. p
    MP m{kNegInf, 0};
    for (uint32_t x = c0; x < c0 + S; ++x) m = mp_then(m, mp_cell(x < HH ? static_cast<int32_t>(hist[x]) : 0));
    MP total;
    const MP ex = block_scan_mp(m, total, sPart);
    if (tid == 0) sE = 0x7FFFFFFF;
    for (uint32_t i = tid; i < H / kTblChunkCells; i += kTT) {
        sLastEmpty[i] = -1;
        sLastDel[i] = -1;
        sSurv[i] = 0u;
    }
    __syncthreads();
    int32_t b = mp_apply(ex, total.p > 0 ? total.p : 0);
    int32_t eMin = 0x7FFFFFFF;
    for (uint32_t x = c0; x < c0 + S; ++x) {
        const int32_t n = x < HH ? static_cast<int32_t>(hist[x]) : 0;
        const bool occ = b + n >= 1;
        b = b + n - 1 > 0 ? b + n - 1 : 0;
        const uint32_t cw = cellw[x];
        if (cw != 0u && !occ) ht[x] = 0;  // occupied before the step, empty after
        if (cw == 0u && !occ && (H <= 65536u || x >= 65535u) && static_cast<int32_t>(x) < eMin) eMin = static_cast<int32_t>(x);
    }
    if (eMin != 0x7FFFFFFF) atomicMin(&sE, eMin);
    __syncthreads();
    const int32_t e = sE;
    if (e == 0x7FFFFFFF) {  // not reachable: fewer keys than cells leave one
        if (tid == 0) {
            report_overflow(P.L.overflowSlot, kOverflowProbe);
            tb[P.t.meta] = 0u;
        }
        return;
    }
    // chunks of the cell order (position x is cell (x + e + 1) mod H): the
    // last empty cell, the last deleted cell, whether any survivor is there
    for (uint32_t x = c0; x < c0 + S; ++x) {
        const uint32_t cw = cellw[(x + static_cast<uint32_t>(e) + 1u) & mask];
        const uint32_t g = x / kTblChunkCells;
        if (cw == 0u) atomicMax(&sLastEmpty[g], static_cast<int32_t>(x));
        else if (cw == kDeleted) atomicMax(&sLastDel[g], static_cast<int32_t>(x));
        else sSurv[g] = 1u;
    }
    __syncthreads();
    KVX_GM int32_t *chunkA = reinterpret_cast<KVX_GM int32_t *>(tb + P.t.chunkA);
    const uint32_t nChunks = H / kTblChunkCells;
    if (tid == 0) {
        // a chunk's cluster starts after the last empty cell before it (the
        // order starts after the empty cell e); its survivors can move only
        // if a deleted cell lies between that start and the chunk's end
        int32_t lastEmpty = -1, lastDel = -1;
        for (uint32_t g = 0; g < nChunks; ++g) {
            const int32_t start = lastEmpty + 1;
            if (sLastDel[g] > lastDel) lastDel = sLastDel[g];
            chunkA[g] = (sSurv[g] && lastDel >= start) ? start : -1;
            if (sLastEmpty[g] > lastEmpty) lastEmpty = sLastEmpty[g];
        }
        tb[P.t.meta + 2] = static_cast<uint32_t>(e);
    }
}

// ---- 3. chunks --------------------------------------------------------------
// The free cells of position window [wb, wb + kTblWinBits) after the keys
// counted in hist (per home, 16 bits each), scanning positions [x0, x1)
// (x0 and wb multiples of 64, backlog 0 at x0); homeOf(x) gives the count
// index of position x or -1.
template <typename CountAt>
__device__ __forceinline__ void chunk_free_cells(uint32_t x0, uint32_t x1, uint32_t wb, const Win &win,
                                                 CountAt countAt, MP *sPart)
{
    const uint32_t tid = threadIdx.x;
    for (uint32_t w = tid; w < kTblWinWords; w += kTT) win.l0[w] = 0ull;
    const uint32_t len = x1 - x0;
    const uint32_t seg = ((len + kTT - 1u) / kTT + 63u) & ~63u;  // whole 64-position words per thread
    const uint32_t s0 = x0 + tid * seg;
    const uint32_t s1 = s0 + seg < x1 ? s0 + seg : x1;
    MP m{kNegInf, 0};
    for (uint32_t x = s0; x < s1; ++x) m = mp_then(m, mp_cell(countAt(x)));
    MP total;
    const MP ex = block_scan_mp(m, total, sPart);  // (its barriers order the clearing above too)
    int32_t b = mp_apply(ex, 0);
    for (uint32_t xw = s0; xw < s1; xw += 64u) {
        uint64_t free = 0;
        const uint32_t xe = xw + 64u < s1 ? xw + 64u : s1;
        for (uint32_t x = xw; x < xe; ++x) {
            const int32_t n = countAt(x);
            if (b + n == 0) free |= 1ull << (x - xw);
            b = b + n - 1 > 0 ? b + n - 1 : 0;
        }
        if (xw >= wb && xw - wb < kTblWinBits) win.l0[(xw - wb) >> 6] = free;
    }
    __syncthreads();
    win_summarize(win);
}

__global__ __launch_bounds__(kTT) void kvx_sieve_table_chunks(TblParams P)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ MP sPart[kTW + 1];
    __shared__ uint32_t sCell[kTblChunkCells];
    __shared__ int32_t sLo;
    uint32_t *hist = reinterpret_cast<uint32_t *>(lds);  // two 16-bit counts a word
    const Win win{reinterpret_cast<uint64_t *>(lds + kTblHistBytes),
                  reinterpret_cast<uint64_t *>(lds + kTblHistBytes + kTblWinWords * 8u),
                  reinterpret_cast<uint64_t *>(lds + kTblHistBytes + (kTblWinWords + kTblWinL1) * 8u)};
    const HispSieveUpdateArgs &a = P.L.a;
    const int32_t bid = blockIdx.y;
    if (bid >= static_cast<int32_t>(a.maxNumReqs)) return;
    KVX_GM uint32_t *tb = row_tbl(P, bid);
    if (tb[P.t.meta] != 1u) return;
    const uint32_t H = a.htSize, mask = H - 1u, HH = H < 65536u ? H : 65536u;
    const uint32_t e = tb[P.t.meta + 2], N = tb[P.t.meta + 1];
    const int64_t reqIdx = reinterpret_cast<const KVX_GM int64_t *>(a.reqPoolIndices)[bid];
    KVX_GM uint16_t *ht = reinterpret_cast<KVX_GM uint16_t *>(a.deviceBufferHt) + reqIdx * H;
    const KVX_GM uint32_t *cellw = tb + P.t.cellw;
    const uint32_t tid = threadIdx.x, lane = __lane_id();
    const uint32_t nS = H / kTblChunkCells;
    auto tab = [&](uint32_t x) { return (x + e + 1u) & mask; };  // position -> cell
    auto pos = [&](uint32_t c) { return (c - e - 1u) & mask; };  // cell -> position
    auto count16 = [&](uint32_t i) { return static_cast<int32_t>((hist[i >> 1] >> (16u * (i & 1u))) & 0xFFFFu); };

    if (blockIdx.x < nS) {
        // survivors of positions [s0, s1), after those of [a0, s0) in the same cluster
        const int32_t a0 = reinterpret_cast<const KVX_GM int32_t *>(tb + P.t.chunkA)[blockIdx.x];
        if (a0 < 0) return;
        const uint32_t s0 = blockIdx.x * kTblChunkCells, s1 = s0 + kTblChunkCells;
        const uint32_t A = static_cast<uint32_t>(a0), wb = A & ~63u;
        const uint32_t nh = s0 - A;  // counted positions, and count slots (homes lie in [A, s0))
        if (tid < kTblChunkCells) sCell[tid] = cellw[tab(s0 + tid)];
        for (uint32_t i = tid; i < (nh + 1u) / 2u; i += kTT) hist[i] = 0u;
        __syncthreads();
        for (uint32_t x = A + tid; x < s0; x += kTT) {
            const uint32_t cw = cellw[tab(x)];
            if ((cw & 0xFFFFu) == 0u) continue;  // empty or deleted
            const uint32_t i = pos(cw >> 16) - A;
            if (i < nh) atomicAdd(&hist[i >> 1], 1u << (16u * (i & 1u)));
        }
        __syncthreads();
        chunk_free_cells(wb, s1, wb, win,
                         [&](uint32_t x) { return (x >= A && x < s0) ? count16(x - A) : 0; }, sPart);
        if (tid >= 64) return;
        const bool wr = lane == 0;
        for (uint32_t q = 0; q < kTblChunkCells; q += 64u) {
            const uint32_t cw = sCell[q + lane];
            const bool surv = (cw & 0xFFFFu) != 0u;
            const uint32_t hp = surv ? pos(cw >> 16) : 0u;
            uint64_t mm = __ballot(surv);
            while (mm) {
                const int j = __builtin_ctzll(mm);
                mm &= mm - 1ull;
                const uint32_t h = static_cast<uint32_t>(__shfl(static_cast<int>(hp), j));
                const uint32_t entry = static_cast<uint32_t>(__shfl(static_cast<int>(cw), j)) & 0xFFFFu;
                const uint32_t own = s0 + q + static_cast<uint32_t>(j);
                const int32_t y = h >= wb ? win_next(win, h - wb) : -1;
                if (y < 0 || static_cast<uint32_t>(y) + wb > own) {
                    // not reachable on a consistent table (the own cell is free)
                    if (wr) report_overflow(P.L.overflowSlot, kOverflowProbe);
                    continue;
                }
                win_clear(win, static_cast<uint32_t>(y), wr);
                if (wr && static_cast<uint32_t>(y) + wb != own) ht[tab(static_cast<uint32_t>(y) + wb)] = static_cast<uint16_t>(entry);
            }
        }
        return;
    }

    // new keys [j0, j1), after every survivor and the new keys before j0
    const uint32_t j0 = (blockIdx.x - nS) * kTblChunkKeys;
    if (j0 >= N) return;
    const uint32_t j1 = j0 + kTblChunkKeys < N ? j0 + kTblChunkKeys : N;
    const KVX_GM uint32_t *newk = tb + P.t.newk;
    const KVX_GM uint32_t *histAll = tb + P.t.hist;
    if (tid == 0) sLo = 0x7FFFFFFF;
    for (uint32_t i = tid; i < HH / 2u; i += kTT) hist[i] = (histAll[2u * i] & 0xFFFFu) | (histAll[2u * i + 1u] << 16);
    __syncthreads();
    for (uint32_t j = j0 + tid; j < N; j += kTT) {
        const uint32_t h = newk[j] >> 16;
        atomicSub(&hist[h >> 1], 1u << (16u * (h & 1u)));
        if (j < j1) atomicMin(&sLo, static_cast<int32_t>(pos(h)));
    }
    __syncthreads();
    const uint32_t wb = static_cast<uint32_t>(sLo) & ~63u;
    // homes lie in cells [0, HH): positions [pos(0), pos(0) + HH) (the order
    // starts past 65535 when the table is larger)
    const uint32_t x0 = H > 65536u ? (pos(0) & ~63u) : 0u;
    chunk_free_cells(x0, H, wb, win,
                     [&](uint32_t x) {
                         const uint32_t c = tab(x);
                         return c < HH ? count16(c) : 0;
                     },
                     sPart);
    if (tid >= 64) return;
    const bool wr = lane == 0;
    for (uint32_t q = j0; q < j1; q += 64u) {
        const uint32_t j = q + lane;
        const uint32_t nk = j < j1 ? newk[j] : 0u;
        const uint32_t hp = pos(nk >> 16);
        uint64_t mm = __ballot(j < j1);
        while (mm) {
            const int i = __builtin_ctzll(mm);
            mm &= mm - 1ull;
            const uint32_t h = static_cast<uint32_t>(__shfl(static_cast<int>(hp), i));
            const uint32_t ent = static_cast<uint32_t>(__shfl(static_cast<int>(nk), i)) & 0xFFFFu;
            const int32_t y = h >= wb ? win_next(win, h - wb) : -1;
            if (y < 0) {  // not reachable: the window holds every cell a key can reach
                if (wr) report_overflow(P.L.overflowSlot, kOverflowProbe);
                continue;
            }
            win_clear(win, static_cast<uint32_t>(y), wr);
            if (wr) ht[tab(static_cast<uint32_t>(y) + wb)] = static_cast<uint16_t>(ent);
        }
    }
}

}  // namespace

hipError_t sieve_table_set_lds_limit(size_t bytes)
{
    return hipFuncSetAttribute(reinterpret_cast<const void *>(&kvx_sieve_table_chunks),
                               hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes));
}

hipError_t launch_sieve_table_rebuild(const HispSieveUpdateArgs &a, uint64_t overflowSlot, uint32_t *tbl,
                                      hipStream_t stream)
{
    TblParams P{};
    P.L = KvxLaunch<HispSieveUpdateArgs>{a, overflowSlot};
    P.tbl = tbl;
    P.t = table_layout(a.htSize);
    const uint32_t cellBlocks = (a.htSize + kCellsPerBlock - 1u) / kCellsPerBlock;
    hipLaunchKernelGGL(kvx_sieve_table_cells, dim3(cellBlocks, a.maxNumReqs), dim3(kCellThreads), 0, stream, P);
    hipLaunchKernelGGL(kvx_sieve_table_final, dim3(a.maxNumReqs), dim3(kTT), 0, stream, P);
    const uint32_t chunks = a.htSize / kTblChunkCells + (a.topK + kTblChunkKeys - 1u) / kTblChunkKeys;
    hipLaunchKernelGGL(kvx_sieve_table_chunks, dim3(chunks, a.maxNumReqs), dim3(kTT), kTblLdsBytes, stream, P);
    return hipGetLastError();
}

}  // namespace kvx
