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
// Inclusive max over the block in thread order (kTT threads); -1 = none.
__device__ __forceinline__ int32_t block_scan_max(int32_t v, int32_t *sPart)
{
    const int lane = __lane_id(), wave = threadIdx.x >> 6;
    int32_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int32_t o = __shfl_up(inc, d);
        if (lane >= d && o > inc) inc = o;
    }
    if (lane == 63) sPart[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t run = -1;
        for (int w = 0; w < kTW; ++w) {
            const int32_t x = sPart[w];
            sPart[w] = run;
            if (x > run) run = x;
        }
    }
    __syncthreads();
    const int32_t before = sPart[wave];
    __syncthreads();
    return inc > before ? inc : before;
}

constexpr uint32_t kTblChunks = kTblMaxHt / kTblChunkCells;  // chunks of the largest table

__global__ __launch_bounds__(kTT) void kvx_sieve_table_final(TblParams P)
{
    __shared__ MP sPart[kTW + 1];
    __shared__ int32_t sMax[kTW];
    __shared__ int32_t sE, sEAligned;
    // per chunk of 256 cells (table order): the last empty cell, the last
    // deleted cell (offsets in the chunk, -1 = none), and whether a survivor is there
    __shared__ int32_t sLastEmpty[kTblChunks], sLastDel[kTblChunks];
    __shared__ uint32_t sSurv[kTblChunks];
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
    const uint32_t S = H / kTT;  // cells per thread (H >= 1024, a power of two: S a power of two)
    const uint32_t c0 = tid * S;
    const uint32_t nC = H / kTblChunkCells;
    // cells go four at a time (16-byte loads) when a thread has at least four
    const uint32_t step = S >= 4u ? 4u : S;
    auto load = [&](const KVX_GM uint32_t *a4, uint32_t x, uint32_t *out) {
        if (step == 4u) {
            const u32x4 v = reinterpret_cast<const KVX_GM u32x4 *>(a4)[x >> 2];
            out[0] = v.x;
            out[1] = v.y;
            out[2] = v.z;
            out[3] = v.w;
        } else {
            for (uint32_t h = 0; h < step; ++h) out[h] = a4[x + h];
        }
    };
    auto cnts = [&](uint32_t x, uint32_t *out) {  // counts of cells x .. x + step - 1
        if (x < HH) {
            load(hist, x, out);
        } else {
            for (uint32_t h = 0; h < 4u; ++h) out[h] = 0u;
        }
    };

    // the cells occupied after the step, cyclic: the backlog entering cell 0
    // is the fixed point of the whole ring's map, max(p, b + q) with q < 0
    // (fewer keys than cells), i.e. p
    MP m{kNegInf, 0};
    if (c0 >= HH) {
        m = MP{0, -static_cast<int32_t>(S)};  // no keys homed here
    } else {
        for (uint32_t x = c0; x < c0 + S; x += step) {
            uint32_t n[4];
            cnts(x, n);
            for (uint32_t h = 0; h < step; ++h) m = mp_then(m, mp_cell(static_cast<int32_t>(n[h])));
        }
    }
    MP total;
    const MP ex = block_scan_mp(m, total, sPart);
    if (tid == 0) {
        sE = 0x7FFFFFFF;
        sEAligned = 0x7FFFFFFF;
    }
    for (uint32_t i = tid; i < nC; i += kTT) {
        sLastEmpty[i] = -1;
        sLastDel[i] = -1;
        sSurv[i] = 0u;
    }
    __syncthreads();
    int32_t b = mp_apply(ex, total.p > 0 ? total.p : 0);
    int32_t eMin = 0x7FFFFFFF, eAl = 0x7FFFFFFF;
    // this thread's chunk statistics (one chunk at a time; S and 256 are powers of two)
    int32_t le = -1, ld = -1;
    uint32_t sv = 0u, g = c0 / kTblChunkCells;
    for (uint32_t x = c0; x < c0 + S; x += step) {
        uint32_t nn[4], ww[4];
        cnts(x, nn);
        load(cellw, x, ww);
        for (uint32_t h = 0; h < step; ++h) {
            const uint32_t c = x + h;
            const int32_t n = static_cast<int32_t>(nn[h]);
            const bool occ = b + n >= 1;
            b = b + n - 1 > 0 ? b + n - 1 : 0;
            const uint32_t cw = ww[h];
            if (cw != 0u && !occ) ht[c] = 0;  // occupied before the step, empty after
            if (cw == 0u && !occ && (H <= 65536u || c >= 65535u)) {
                if (static_cast<int32_t>(c) < eMin) eMin = static_cast<int32_t>(c);
                if ((c & (kTblChunkCells - 1u)) == kTblChunkCells - 1u && static_cast<int32_t>(c) < eAl)
                    eAl = static_cast<int32_t>(c);
            }
            const int32_t off = static_cast<int32_t>(c & (kTblChunkCells - 1u));
            if (cw == 0u) le = off;
            else if (cw == kDeleted) ld = off;
            else sv = 1u;
        }
        if (((x + step) & (kTblChunkCells - 1u)) == 0u || x + step == c0 + S) {
            // the chunk ends (or this thread's part of it): publish
            if (le >= 0) atomicMax(&sLastEmpty[g], le);
            if (ld >= 0) atomicMax(&sLastDel[g], ld);
            if (sv) sSurv[g] = 1u;
            le = -1;
            ld = -1;
            sv = 0u;
            g = (x + step) / kTblChunkCells;
        }
    }
    if (eMin != 0x7FFFFFFF) atomicMin(&sE, eMin);
    if (eAl != 0x7FFFFFFF) atomicMin(&sEAligned, eAl);
    __syncthreads();
    // the order starts after e; one that ends a chunk keeps the chunks whole
    const int32_t e = sEAligned != 0x7FFFFFFF ? sEAligned : sE;
    if (e == 0x7FFFFFFF) {  // not reachable: fewer keys than cells leave one
        if (tid == 0) {
            report_overflow(P.L.overflowSlot, kOverflowProbe);
            tb[P.t.meta] = 0u;
        }
        return;
    }
    if (sEAligned == 0x7FFFFFFF) {
        // chunks of the cell order straddle the table's: count them again in
        // positions (position x is cell (x + e + 1) mod H)
        __syncthreads();
        for (uint32_t i = tid; i < nC; i += kTT) {
            sLastEmpty[i] = -1;
            sLastDel[i] = -1;
            sSurv[i] = 0u;
        }
        __syncthreads();
        le = -1;
        ld = -1;
        sv = 0u;
        g = c0 / kTblChunkCells;
        for (uint32_t x = c0; x < c0 + S; ++x) {
            const uint32_t cw = cellw[(x + static_cast<uint32_t>(e) + 1u) & mask];
            const int32_t off = static_cast<int32_t>(x & (kTblChunkCells - 1u));
            if (cw == 0u) le = off;
            else if (cw == kDeleted) ld = off;
            else sv = 1u;
            if (((x + 1u) & (kTblChunkCells - 1u)) == 0u || x + 1u == c0 + S) {
                if (le >= 0) atomicMax(&sLastEmpty[g], le);
                if (ld >= 0) atomicMax(&sLastDel[g], ld);
                if (sv) sSurv[g] = 1u;
                le = -1;
                ld = -1;
                sv = 0u;
                g = (x + 1u) / kTblChunkCells;
            }
        }
        __syncthreads();
    }
    // position chunk q is table chunk (q + shift) mod nC (shift 0 when the
    // order does not start at a chunk boundary: the statistics were counted in positions)
    const uint32_t shift = sEAligned != 0x7FFFFFFF ? ((static_cast<uint32_t>(e) + 1u) / kTblChunkCells) % nC : 0u;
    // a chunk's cluster starts after the last empty cell before it; its
    // survivors can move only if a deleted cell lies between that start and
    // the chunk's end
    const uint32_t q = tid;
    int32_t myLe = -1, myLd = -1;
    uint32_t mySv = 0u;
    if (q < nC) {
        const uint32_t tc = (q + shift) % nC;
        const int32_t base = static_cast<int32_t>(q * kTblChunkCells);
        myLe = sLastEmpty[tc] >= 0 ? base + sLastEmpty[tc] : -1;
        myLd = sLastDel[tc] >= 0 ? base + sLastDel[tc] : -1;
        mySv = sSurv[tc];
    }
    const int32_t leInc = block_scan_max(myLe, sMax);
    const int32_t ldInc = block_scan_max(myLd, sMax);
    // the last empty cell strictly before chunk q: the inclusive max of chunk q - 1
    const int32_t lePrev = __shfl_up(leInc, 1);
    __shared__ int32_t sWaveLast[kTW];
    if ((tid & 63u) == 63u) sWaveLast[tid >> 6] = leInc;
    __syncthreads();
    const int32_t leBefore = (tid & 63u) ? lePrev : (tid >= 64u ? sWaveLast[(tid >> 6) - 1u] : -1);
    if (q < nC) {
        const int32_t start = leBefore + 1;
        KVX_GM int32_t *chunkA = reinterpret_cast<KVX_GM int32_t *>(tb + P.t.chunkA);
        chunkA[q] = (mySv && ldInc >= start) ? start : -1;
    }
    if (tid == 0) tb[P.t.meta + 2] = static_cast<uint32_t>(e);
}

// ---- 3. chunks --------------------------------------------------------------
// The free cells of position window [wb, wb + kTblWinBits) after the keys
// counted (per home, 16 bits each), scanning positions [x0, x1) (x0 and wb
// multiples of 64, backlog 0 at x0) into win[] (a bit per position).
// count8(x, c) gives the counts of positions x .. x+7 (x a multiple of 8).
template <typename Count8>
__device__ __forceinline__ void chunk_free_cells(uint32_t x0, uint32_t x1, uint32_t wb, uint64_t *win, Count8 count8,
                                                 MP *sPart)
{
    const uint32_t tid = threadIdx.x;
    for (uint32_t w = tid; w < kTblWinWords; w += kTT) win[w] = 0ull;
    const uint32_t len = x1 - x0;
    const uint32_t seg = ((len + kTT - 1u) / kTT + 63u) & ~63u;  // whole 64-position words per thread
    const uint32_t s0 = x0 + tid * seg;
    const uint32_t s1 = s0 + seg < x1 ? s0 + seg : x1;
    MP m{kNegInf, 0};
#pragma unroll 2
    for (uint32_t x = s0; x < s1; x += 8u) {
        int32_t c[8];
        count8(x, c);
#pragma unroll
        for (int h = 0; h < 8; ++h) m = mp_then(m, mp_cell(c[h]));
    }
    MP total;
    const MP ex = block_scan_mp(m, total, sPart);  // (its barriers order the clearing above too)
    int32_t b = mp_apply(ex, 0);
    for (uint32_t xw = s0; xw < s1; xw += 64u) {
        uint64_t free = 0;
#pragma unroll 2
        for (uint32_t x = xw; x < xw + 64u; x += 8u) {
            int32_t c[8];
            count8(x, c);
#pragma unroll
            for (int h = 0; h < 8; ++h) {
                if (b + c[h] == 0) free |= 1ull << (x - xw + static_cast<uint32_t>(h));
                b = b + c[h] - 1 > 0 ? b + c[h] - 1 : 0;
            }
        }
        if (xw >= wb && xw - wb < kTblWinBits) win[(xw - wb) >> 6] = free;
    }
    __syncthreads();
}

// The chunk's n <= 256 keys, in insertion order (home h, window-relative;
// entry; own cell, window-relative, or kNoOwn), each into the first free cell
// of win[] at or after its home, one after another.  The set of cells they
// take does not depend on that order: going in in home order, key j (sorted)
// takes the free cell of index r_j = max(p_j, r_{j-1} + 1), p_j the free cells
// before its home, i.e. r_j = j + max_{i<=j} (p_i - i); z_j its cell.  In
// insertion order each key then takes the first of those cells at or after
// its home not taken before it: an index search in a 256-bit mask.
constexpr uint32_t kNoOwn = 0xFFFFFFFFu;

struct PlaceLds {
    uint32_t *rank;   // [kTblWinWords + 1] free cells before each window word
    uint32_t *home, *ent, *own, *sortedH, *z, *res;  // [kTblChunkCells] each
};

__device__ __forceinline__ uint32_t select_bit64(uint64_t x, uint32_t r)  // offset of the r-th set bit
{
    uint32_t base = 0;
    for (uint32_t w = 32; w >= 1; w >>= 1) {
        const uint64_t lo = x & (w == 64u ? ~0ull : ((1ull << w) - 1ull));
        const uint32_t c = static_cast<uint32_t>(__builtin_popcountll(lo));
        if (r >= c) {
            r -= c;
            x >>= w;
            base += w;
        } else {
            x = lo;
        }
    }
    return base;
}

// All threads; the items are in L.home/ent/own [0, n).  Returns through L.res
// the window cell of each item.  False: a key found no cell (not reachable).
__device__ bool place_chunk(const PlaceLds &L, const uint64_t *win, uint32_t n, MP *sPart, int32_t *sMax)
{
    __shared__ uint32_t sBad;
    const uint32_t tid = threadIdx.x, lane = static_cast<uint32_t>(__lane_id());
    // free cells before each word
    uint32_t cnt = 0;
    for (uint32_t q = 0; q < kTblWinWords / kTT; ++q) cnt += static_cast<uint32_t>(__builtin_popcountll(win[tid * (kTblWinWords / kTT) + q]));
    // exclusive sum via the max-plus scan's partial array (a plain sum here)
    uint32_t inc = cnt;
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(inc), d));
        if (lane >= static_cast<uint32_t>(d)) inc += o;
    }
    uint32_t *sSum = reinterpret_cast<uint32_t *>(sMax);
    if (lane == 63u) sSum[tid >> 6] = inc;
    if (tid == 0) sBad = 0u;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (int w = 0; w < kTW; ++w) {
            const uint32_t x = sSum[w];
            sSum[w] = run;
            run += x;
        }
        L.rank[kTblWinWords] = run;
    }
    __syncthreads();
    {
        uint32_t r = sSum[tid >> 6] + inc - cnt;
        for (uint32_t q = 0; q < kTblWinWords / kTT; ++q) {
            const uint32_t w = tid * (kTblWinWords / kTT) + q;
            L.rank[w] = r;
            r += static_cast<uint32_t>(__builtin_popcountll(win[w]));
        }
    }
    __syncthreads();
    const uint32_t totalFree = L.rank[kTblWinWords];
    // homes in order (ties by insertion order)
    if (tid < n) {
        const uint32_t h = L.home[tid];
        uint32_t rk = 0;
        for (uint32_t j = 0; j < n; ++j) {
            const uint32_t hj = L.home[j];
            rk += (hj < h || (hj == h && j < tid)) ? 1u : 0u;
        }
        L.sortedH[rk] = h;
    }
    __syncthreads();
    // r_j = j + max_{i<=j} (p_i - i)
    int32_t v = -0x3FFFFFFF;
    if (tid < n) {
        const uint32_t h = L.sortedH[tid];
        const uint32_t w = h >> 6;
        const uint32_t p = L.rank[w] + static_cast<uint32_t>(__builtin_popcountll(win[w] & ((1ull << (h & 63u)) - 1ull)));
        v = static_cast<int32_t>(p) - static_cast<int32_t>(tid);
    }
    const int32_t pm = block_scan_max(v, sMax);
    if (tid < n) {
        const uint32_t r = static_cast<uint32_t>(pm + static_cast<int32_t>(tid));
        if (r >= totalFree) {
            sBad = 1u;
        } else {
            // the word holding free cell r: the last word whose rank is <= r
            uint32_t lo = 0, hi = kTblWinWords;
            while (hi - lo > 1u) {
                const uint32_t mid = (lo + hi) >> 1;
                if (L.rank[mid] <= r) lo = mid; else hi = mid;
            }
            L.z[tid] = (lo << 6) + select_bit64(win[lo], r - L.rank[lo]);
        }
    }
    __syncthreads();
    if (sBad) return false;
    // each key's first candidate cell: the cells before its home
    if (tid < n) {
        const uint32_t h = L.home[tid];
        uint32_t lo = 0, hi = n;  // first z >= h
        while (lo < hi) {
            const uint32_t mid = (lo + hi) >> 1;
            if (L.z[mid] < h) lo = mid + 1u; else hi = mid;
        }
        L.res[tid] = lo;
    }
    __syncthreads();
    // in insertion order, the first untaken candidate (one wave, 256-bit mask)
    if (tid < 64) {
        uint64_t tk0 = 0, tk1 = 0, tk2 = 0, tk3 = 0;
        uint32_t q4[4], r4[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t i = static_cast<uint32_t>(g) * 64u + lane;
            q4[g] = i < n ? L.res[i] : 0u;
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t lim = n > static_cast<uint32_t>(g) * 64u ? n - static_cast<uint32_t>(g) * 64u : 0u;
            for (uint32_t l = 0; l < (lim < 64u ? lim : 64u); ++l) {
                const uint32_t q = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(q4[g]), static_cast<int>(l)));
                const uint32_t wq = q >> 6;
                const uint64_t m0 = wq == 0u ? (~tk0 & (~0ull << (q & 63u))) : 0ull;
                const uint64_t m1 = wq <= 1u ? (~tk1 & (wq == 1u ? (~0ull << (q & 63u)) : ~0ull)) : 0ull;
                const uint64_t m2 = wq <= 2u ? (~tk2 & (wq == 2u ? (~0ull << (q & 63u)) : ~0ull)) : 0ull;
                const uint64_t m3 = ~tk3 & (wq == 3u ? (~0ull << (q & 63u)) : ~0ull);
                uint32_t idx;
                if (m0) { idx = static_cast<uint32_t>(__builtin_ctzll(m0)); tk0 |= 1ull << idx; }
                else if (m1) { idx = 64u + static_cast<uint32_t>(__builtin_ctzll(m1)); tk1 |= 1ull << (idx - 64u); }
                else if (m2) { idx = 128u + static_cast<uint32_t>(__builtin_ctzll(m2)); tk2 |= 1ull << (idx - 128u); }
                else { idx = 192u + static_cast<uint32_t>(__builtin_ctzll(m3)); tk3 |= 1ull << (idx - 192u); }
                if (lane == l) r4[g] = idx;
            }
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint32_t i = static_cast<uint32_t>(g) * 64u + lane;
            if (i < n) L.res[i] = L.z[r4[g]];
        }
    }
    __syncthreads();
    return true;
}

__global__ __launch_bounds__(kTT) void kvx_sieve_table_chunks(TblParams P)
{
    extern __shared__ __align__(16) unsigned char lds[];
    __shared__ MP sPart[kTW + 1];
    __shared__ int32_t sMax[kTW];
    __shared__ int32_t sLo;
    uint32_t *hist = reinterpret_cast<uint32_t *>(lds);  // two 16-bit counts a word
    uint64_t *win = reinterpret_cast<uint64_t *>(lds + kTblHistBytes);
    // after the scan the counts are dead: their LDS holds the placement's arrays
    PlaceLds pl;
    pl.rank = hist;
    pl.home = hist + kTblWinWords + 4u;
    pl.ent = pl.home + kTblChunkCells;
    pl.own = pl.ent + kTblChunkCells;
    pl.sortedH = pl.own + kTblChunkCells;
    pl.z = pl.sortedH + kTblChunkCells;
    pl.res = pl.z + kTblChunkCells;
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
    auto count8from = [&](uint32_t i, int32_t *c) {  // counts i .. i+7, i a multiple of 8
        const uint4 v = *reinterpret_cast<const uint4 *>(hist + (i >> 1));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            c[2 * h] = static_cast<int32_t>(w[h] & 0xFFFFu);
            c[2 * h + 1] = static_cast<int32_t>(w[h] >> 16);
        }
    };
#ifdef KVX_BATCH_STAMPS
    uint64_t t0 = __builtin_amdgcn_s_memtime(), t1 = 0, t2 = 0;
#endif
    uint32_t wb = 0, n = 0;
    bool survivors = blockIdx.x < nS;
    uint32_t s0 = 0;
    if (survivors) {
        // survivors of positions [s0, s0 + 256), after those of [A, s0) in the same cluster
        const int32_t a0 = reinterpret_cast<const KVX_GM int32_t *>(tb + P.t.chunkA)[blockIdx.x];
        if (a0 < 0) return;
        s0 = blockIdx.x * kTblChunkCells;
        const uint32_t s1 = s0 + kTblChunkCells;
        const uint32_t A = static_cast<uint32_t>(a0);
        wb = A & ~63u;
        const uint32_t nh = s0 - wb;  // counted positions [wb, s0), by position - wb
        uint32_t cw = 0u;
        if (tid < kTblChunkCells) cw = cellw[tab(s0 + tid)];
        for (uint32_t i = tid; i < (nh + 1u) / 2u + 4u; i += kTT) hist[i] = 0u;
        __syncthreads();
        for (uint32_t x = A + tid; x < s0; x += kTT) {
            const uint32_t c = cellw[tab(x)];
            if ((c & 0xFFFFu) == 0u) continue;  // empty or deleted
            const uint32_t i = pos(c >> 16) - wb;
            if (i < nh) atomicAdd(&hist[i >> 1], 1u << (16u * (i & 1u)));
        }
        __syncthreads();
#ifdef KVX_BATCH_STAMPS
        t1 = __builtin_amdgcn_s_memtime();
#endif
        chunk_free_cells(wb, s1, wb, win,
                         [&](uint32_t x, int32_t *c) {
                             if (x < s0) {
                                 count8from(x - wb, c);
                             } else {
#pragma unroll
                                 for (int h = 0; h < 8; ++h) c[h] = 0;
                             }
                         },
                         sPart);
#ifdef KVX_BATCH_STAMPS
        t2 = __builtin_amdgcn_s_memtime();
#endif
        // the chunk's survivors in cell order (its cells are threads 0..255: whole waves)
        __shared__ uint32_t sWaveCnt[kTblChunkCells / 64];
        const bool surv = tid < kTblChunkCells && (cw & 0xFFFFu) != 0u;
        const uint64_t bm = __ballot(surv);
        if (tid < kTblChunkCells && lane == 0u) sWaveCnt[tid >> 6] = static_cast<uint32_t>(__builtin_popcountll(bm));
        __syncthreads();
        if (surv) {
            uint32_t base = 0;
            for (uint32_t w = 0; w < (tid >> 6); ++w) base += sWaveCnt[w];
            const uint32_t at = base + static_cast<uint32_t>(__builtin_popcountll(bm & ((1ull << lane) - 1ull)));
            pl.home[at] = pos(cw >> 16) - wb;
            pl.ent[at] = cw & 0xFFFFu;
            pl.own[at] = s0 + tid - wb;
        }
        n = 0;
        for (uint32_t w = 0; w < kTblChunkCells / 64u; ++w) n += sWaveCnt[w];
        __syncthreads();
    } else {
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
        wb = static_cast<uint32_t>(sLo) & ~63u;
        // homes lie in cells [0, HH): positions [pos(0), pos(0) + HH) (the order
        // starts past 65535 when the table is larger)
        const uint32_t x0 = H > 65536u ? (pos(0) & ~63u) : 0u;
        const bool aligned = ((e + 1u) & 7u) == 0u;  // positions of 8 cells then read 8 counts at once
#ifdef KVX_BATCH_STAMPS
        t1 = __builtin_amdgcn_s_memtime();
#endif
        chunk_free_cells(x0, H, wb, win,
                         [&](uint32_t x, int32_t *c) {
                             const uint32_t c0 = tab(x);
                             if (aligned) {
                                 if (c0 < HH) {
                                     count8from(c0, c);
                                 } else {
#pragma unroll
                                     for (int h = 0; h < 8; ++h) c[h] = 0;
                                 }
                             } else {
#pragma unroll
                                 for (int h = 0; h < 8; ++h) {
                                     const uint32_t ch = tab(x + static_cast<uint32_t>(h));
                                     c[h] = ch < HH ? count16(ch) : 0;
                                 }
                             }
                         },
                         sPart);
#ifdef KVX_BATCH_STAMPS
        t2 = __builtin_amdgcn_s_memtime();
#endif
        n = j1 - j0;
        if (tid < n) {
            const uint32_t nk = newk[j0 + tid];
            pl.home[tid] = pos(nk >> 16) - wb;
            pl.ent[tid] = nk & 0xFFFFu;
            pl.own[tid] = kNoOwn;
        }
        __syncthreads();
    }
    if (n == 0u) return;
    if (!place_chunk(pl, win, n, sPart, sMax)) {
        if (tid == 0) report_overflow(P.L.overflowSlot, kOverflowProbe);  // not reachable: the window holds them
        return;
    }
    if (tid < n) {
        const uint32_t y = pl.res[tid], own = pl.own[tid];
        if (own != kNoOwn && y > own) {
            report_overflow(P.L.overflowSlot, kOverflowProbe);  // not reachable on a consistent table
        } else if (y != own) {
            ht[tab(y + wb)] = static_cast<uint16_t>(pl.ent[tid]);
        }
    }
#ifdef KVX_BATCH_STAMPS
    if (tid == 0 && bid == 0 && (blockIdx.x & 31u) == 0u)
        printf("chunk %u n %u: hist %llu scan %llu place %llu\n", blockIdx.x, n, (unsigned long long)(t1 - t0),
               (unsigned long long)(t2 - t1), (unsigned long long)(__builtin_amdgcn_s_memtime() - t2));
#endif
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
