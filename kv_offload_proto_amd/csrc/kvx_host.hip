// C-ABI of libkvx.so: validation, derived geometry, status slots, host
// segments and kernel launches.  Mirrors kvops/kvops_ext/kvops_ext.cpp of the
// reference (same entry points, argument meaning and error texts); the
// Ascend fatbin loading chain is replaced by kernels linked into this library.
#include <hip/hip_runtime.h>

#include <linux/mempolicy.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cerrno>
#include <cctype>
#include <chrono>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <map>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "kvx/kvx.h"
#include "kvx_internal.h"

namespace {

thread_local std::string t_lastError;

struct Alloc {
    uint64_t addr;
    uint64_t bytes;
};

// Scratch of the launches on one stream.  Launches on one stream run in
// order, so they share it; launches on different streams never do.  Buffers
// only grow, and a replaced buffer is kept until kvx_close: a captured graph
// or a launch still in flight may hold its address.
struct StreamScratch {
    uint64_t stream = 0;
    kvx::RowScratch rows{};
    int32_t *shadow = nullptr;      // HBM-resident SIEVE variants: per-cell token shadow
    uint64_t shadowCells = 0;
    uint32_t *aux = nullptr;        // batch HBM SIEVE variant: per-row map, first occurrences, homes
    uint64_t auxWords = 0;
    uint32_t *tbl = nullptr;        // its table rebuild: per-row cells, counts, new keys
    uint64_t tblWords = 0;
};

// Scratch of kvx_import_all_noalloc: a fixed array in the library's code
// object, so each GPU the library is loaded on holds its own copy from load
// to process exit, and the entry point allocates nothing.  Layout: the
// control words (counters, error words, tickets, chunk counter, epoch), then
// the winner table.  It starts zeroed; the kernels clear the counters, error
// words and chunk counter at the start of every call, and the winner table is
// tagged with the epoch that every call advances, so it is never cleared
// (except at the epoch's 2^32 wrap, by the last copy workgroup).
constexpr uint64_t kNoAllocMaxWinEntries = 34ull << 16;     // (max_num_reqs-1)*min(stride,65536) + 65536
constexpr uint64_t kNoAllocControlBytes = (kvx::kControlWords * 4 + 255) / 256 * 256;
constexpr uint64_t kNoAllocBytes = kNoAllocControlBytes + kNoAllocMaxWinEntries * 8;
static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

struct State {
    bool inited = false;
    int device = 0;
    uint64_t *overflow = nullptr;   // the 8-byte tail-slot word
    size_t ldsLimit = 0;            // dynamic LDS per workgroup usable by SIEVE
    size_t ldsBatch = 0;            // the same for the batch HBM kernel (more static LDS)
    std::vector<Alloc> status;      // kvx_alloc_status allocations
    std::vector<StreamScratch *> scratch;  // one per stream that launched or reserved
    std::vector<void *> retired;    // replaced scratch buffers, freed by kvx_close
    int lastSieveVariant = -1;
    int forcedSieveVariant = -1;
    bool tableRebuild = false;      // the device's LDS holds the rebuild's chunk kernel
    void *noAllocScratch[64] = {};  // device address of `scratch`, per device (set at init)
    // the last eager call of the no-allocation import per device: its stream
    // and an event recorded after its launches (created at init)
    hipEvent_t noAllocDone[64] = {};
    uint64_t noAllocStream[64] = {};
    bool noAllocPending[64] = {};
};

State g;
std::mutex g_hostMu;
std::map<uint64_t, uint64_t> g_hostAllocs;  // kvx_host_alloc: addr -> bytes
std::mutex g_statusMu;
std::mutex g_scratchMu;

struct Error : std::runtime_error {
    using std::runtime_error::runtime_error;
};

void hipCheck(hipError_t e, const char *what)
{
    if (e != hipSuccess) throw Error(std::string(what) + " failed: " + hipGetErrorString(e));
}

void EnsureInited()
{
    if (!g.inited) throw Error("kvops not inited");
}

template <typename F>
int Guarded(F &&f)
{
    try {
        f();
        t_lastError.clear();
        return 0;
    } catch (const std::exception &e) {
        t_lastError = e.what();
        return -1;
    }
}

hipStream_t AsStream(uint64_t s) { return reinterpret_cast<hipStream_t>(s); }

void CheckAligned16(uint64_t addr, const char *what)
{
    if ((addr & 15u) != 0) throw Error(std::string(what) + " must be 16-byte aligned");
}

// Host-visible pointer for a status word inside one of our allocations, or null.
volatile uint64_t *StatusWord(uint64_t addr)
{
    std::lock_guard<std::mutex> lk(g_statusMu);
    for (const Alloc &a : g.status) {
        if (addr >= a.addr && addr + 8 <= a.addr + a.bytes && (addr & 7u) == 0) {
            return reinterpret_cast<volatile uint64_t *>(addr);
        }
    }
    return nullptr;
}

// A status word outside the kvx_alloc_status blocks (device memory, or host
// memory HIP knows): read with an 8-byte copy per poll, as the reference polls
// any status address (kvops_ext.cpp:198-218).  An address HIP does not know,
// or a failed copy, gives -0x1000 (the reference's copy-failure code), a
// timeout -0x2000; done is the doneSeq byte, as for the direct reads.
int64_t PollCopiedWord(uint64_t addr, int64_t timeout_us)
{
    hipPointerAttribute_t attr{};
    if (addr == 0 || (addr & 7u) != 0 ||
        hipPointerGetAttributes(&attr, reinterpret_cast<const void *>(addr)) != hipSuccess ||
        attr.type == hipMemoryTypeUnregistered) {
        (void)hipGetLastError();
        t_lastError = "poll_status: not a status address known to the runtime";
        return -0x1000;
    }
    const auto t0 = std::chrono::steady_clock::now();
    while (true) {
        uint64_t v = 0;
        if (hipMemcpy(&v, reinterpret_cast<const void *>(addr), 8, hipMemcpyDefault) != hipSuccess) {
            (void)hipGetLastError();
            t_lastError = "poll_status: reading the status word failed";
            return -0x1000;
        }
        if (((v >> 32) & 0xFFu) == 1u) return static_cast<int64_t>(v & 0xFFFFFFFFull);
        if (timeout_us >= 0) {
            const auto us = std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0);
            if (us.count() >= timeout_us) return -0x2000;
        }
        std::this_thread::sleep_for(std::chrono::microseconds(20));
    }
}

// Clear `words` status words of node slot `node` from the host, before the
// launch is queued (kvops_ext.cpp:252,276 clear synchronously too).
void ClearStatusWords(uint64_t status, uint32_t node, uint32_t words)
{
    if (status == 0) return;
    for (uint32_t b = 0; b < words; ++b) {
        volatile uint64_t *w = StatusWord(status + node * 64ull + b * 8ull);
        if (w != nullptr) *w = 0;
    }
}

// A status block whose base lies inside a kvx_alloc_status allocation must
// end inside it: the kernels write node n's words at status + 64n + 8b.
void CheckStatusBlock(uint64_t status, uint32_t firstNode, uint32_t nodes, uint32_t words, const char *what)
{
    if (status == 0 || nodes == 0) return;
    const uint64_t lo = status;
    const uint64_t hi = status + (static_cast<uint64_t>(firstNode) + nodes - 1ull) * 64ull + words * 8ull;
    std::lock_guard<std::mutex> lk(g_statusMu);
    for (const Alloc &a : g.status) {
        if (lo >= a.addr && lo < a.addr + a.bytes) {
            if (hi > a.addr + a.bytes) {
                throw Error(std::string(what) + ": status slots of this call run past the end of their alloc_status block");
            }
            return;
        }
    }
}

// Scratch needs of one launch (entries of each buffer; 0 = not used).
struct ScratchNeed {
    uint64_t win = 0, shadow = 0, aux = 0, tbl = 0;
};

bool Capturing(hipStream_t s)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(s, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Device buffer of `bytes` zeroed in order on `stream` (no host sync).
void *ScratchAlloc(uint64_t bytes, hipStream_t stream, const char *what)
{
    void *p = nullptr;
    hipCheck(hipMalloc(&p, bytes), (std::string("hipMalloc(") + what + ")").c_str());
    const hipError_t e = hipMemsetAsync(p, 0, bytes, stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        hipCheck(e, "hipMemsetAsync(scratch)");
    }
    return p;
}

// The scratch of `stream`, created or grown to `need`.  Creation and growth
// allocate and queue a clear on the stream; both are refused while the stream
// is being captured (kvx_reserve_scratch sizes a stream beforehand).  The
// caller holds g_scratchMu.
StreamScratch &ScratchFor(uint64_t stream, const ScratchNeed &need, const char *what)
{
    StreamScratch *sc = nullptr;
    for (StreamScratch *s : g.scratch) {
        if (s->stream == stream) sc = s;
    }
    const bool create = sc == nullptr;
    const bool grow = create || sc->rows.winEntries < need.win || sc->shadowCells < need.shadow ||
                      sc->auxWords < need.aux || sc->tblWords < need.tbl;
    if (!grow) return *sc;
    hipStream_t st = AsStream(stream);
    if (Capturing(st)) {
        throw Error(std::string(what) + ": the scratch of this stream is too small for the call and cannot grow "
                    "during stream capture; call reserve_scratch for the stream before capturing");
    }
    if (create) {
        auto *s = new StreamScratch();
        s->stream = stream;
        uint32_t *c = static_cast<uint32_t *>(ScratchAlloc(kvx::kControlWords * sizeof(uint32_t), st, "scratch control"));
        s->rows.counters = c;
        s->rows.errs = c + 64 * 8;
        s->rows.tickets = c + 2 * 64 * 8;
        s->rows.chunkNext = s->rows.tickets + 8;
        s->rows.epoch = s->rows.tickets + 9;
        g.scratch.push_back(s);
        sc = s;
    }
    kvx::RowScratch &r = sc->rows;
    if (r.winEntries < need.win) {
        // a zeroed table is valid under any epoch
        const uint64_t cap = std::max<uint64_t>(need.win, std::max<uint64_t>(2 * r.winEntries, 65536));
        void *p = ScratchAlloc(cap * sizeof(unsigned long long), st, "winner table");
        if (r.win != nullptr) g.retired.push_back(r.win);
        r.win = static_cast<unsigned long long *>(p);
        r.winEntries = cap;
    }
    if (sc->shadowCells < need.shadow) {
        void *p = ScratchAlloc(need.shadow * sizeof(int32_t), st, "sieve shadow");
        if (sc->shadow != nullptr) g.retired.push_back(sc->shadow);
        sc->shadow = static_cast<int32_t *>(p);
        sc->shadowCells = need.shadow;
    }
    if (sc->auxWords < need.aux) {
        // zeroed: the batch kernel's maps must start empty (each launch leaves them empty)
        void *p = ScratchAlloc(need.aux * sizeof(uint32_t), st, "sieve batch scratch");
        if (sc->aux != nullptr) g.retired.push_back(sc->aux);
        sc->aux = static_cast<uint32_t *>(p);
        sc->auxWords = need.aux;
    }
    if (sc->tblWords < need.tbl) {
        void *p = ScratchAlloc(need.tbl * sizeof(uint32_t), st, "sieve table rebuild scratch");
        if (sc->tbl != nullptr) g.retired.push_back(sc->tbl);
        sc->tbl = static_cast<uint32_t *>(p);
        sc->tblWords = need.tbl;
    }
    return *sc;
}

// The SIEVE kernel a row shape launches: 2 = parallel LDS kernel, 4 = the same
// with the compact LDS layout (token hashes in LDS, tokens in HBM), 0 =
// sequential LDS kernel, 5 = batch HBM-resident kernel (state in HBM,
// decisions and bitmaps in LDS), 3 = sequential HBM-resident kernel with
// wave-wide probes (1 = the single-lane HBM kernel, only when forced).
struct SievePlan {
    int variant = 0;
    size_t ldsLaunch = 0;   // dynamic LDS of the launch
    uint32_t invCap = 0;    // entries of the parallel kernel's token -> slot map
    bool rebuild = false;   // variant 5: a step's table changes by the rebuild kernels
};

SievePlan PlanSieve(uint32_t top_k, uint32_t dbs, uint32_t padded, uint32_t visStrideB, uint32_t poolSize,
                    uint32_t htSize)
{
    SievePlan p;
    const size_t lds = static_cast<size_t>(padded) * 4 + static_cast<size_t>(htSize) * 2 + visStrideB;
    const bool fastShape = top_k >= 1 && poolSize >= 1 && top_k < 0x3FFF &&
                           static_cast<uint64_t>(padded) + 1 + top_k <= 65535 && dbs <= 32u * kvx::kFastThreads &&
                           htSize <= 32768;
    const size_t ldsFast = kvx::fast_layout_for(padded, htSize, top_k, dbs, visStrideB, false).total;
    const size_t ldsCompact = kvx::fast_layout_for(padded, htSize, top_k, dbs, visStrideB, true).total;
    const bool fastOk = fastShape && ldsFast <= g.ldsLimit;
    const bool compactOk = fastShape && ldsCompact <= g.ldsLimit && lds <= g.ldsLimit;
    const size_t ldsBatch = kvx::batch_layout(dbs, htSize, top_k).total;
    const bool batchOk = top_k >= 1 && top_k < (1u << 24) && dbs <= 65535 && htSize >= 1024 && ldsBatch <= g.ldsBatch;
    int v = fastOk ? 2 : (compactOk ? 4 : (lds <= g.ldsLimit ? 0 : (batchOk ? 5 : 3)));
    const int f = g.forcedSieveVariant;
    if (f == 0 && lds <= g.ldsLimit) v = 0;
    if (f == 1) v = 1;
    if (f == 2 && fastOk) v = 2;
    if (f == 3) v = 3;
    if (f == 4 && compactOk) v = 4;
    if ((f == 5 || f == 6) && batchOk) v = 5;
    p.variant = v;
    // the batch kernel hands a step's table changes to the rebuild kernels
    // where their windows fit (force 6: it applies them itself)
    p.rebuild = v == 5 && f != 6 && g.tableRebuild && kvx::table_rebuild_ok(htSize, dbs, top_k);
    p.ldsLaunch = v == 2 ? ldsFast
                         : (v == 4 ? std::max(ldsCompact, lds) : (v == 0 ? lds : (v == 5 ? ldsBatch : 0)));
    // the parallel kernel's direct token -> slot map (32-bit entries) takes the
    // LDS left over (rows whose prefill exceeds it probe the table instead)
    if (v == 2 && g.ldsLimit > ldsFast) {
        p.invCap = static_cast<uint32_t>(std::min<size_t>((g.ldsLimit - ldsFast) / 4, 65536)) & ~15u;
        p.ldsLaunch = ldsFast + static_cast<size_t>(p.invCap) * 4;
    }
    return p;
}

ScratchNeed SieveScratchNeed(const SievePlan &p, uint32_t maxNumReqs, uint32_t htSize)
{
    ScratchNeed n;
    if (p.variant == 3 || p.variant == 5) n.shadow = static_cast<uint64_t>(maxNumReqs) * htSize;
    if (p.variant == 5) n.aux = static_cast<uint64_t>(maxNumReqs) * kvx::batch_aux_words(htSize);
    if (p.variant == 5 && p.rebuild) n.tbl = static_cast<uint64_t>(maxNumReqs) * kvx::table_layout(htSize).words;
    return n;
}

struct GatherCall {
    uint64_t segBases[64];
    uint32_t nSeg;
    bool fused;
    uint64_t channel, segBase;
    uint32_t layerOffsetRows, perLayerSegRows, rowBytes;
    uint64_t topk, pool, hostBase, slots, isMiss, numReal, hotRowBase;
    uint32_t topK, maxNumReqs, stripeRows, nodeNum, myNode;
    uint64_t status, stream;
    uint32_t blockDim, stride;
};

void DoGather(const GatherCall &c, const kvx::RowScratch *fixed = nullptr)
{
    EnsureInited();
    if (c.blockDim > 8) throw Error("import blockDim must be <= 8 (status slot layout)");  // kvops_ext.cpp:228-230
    if (c.rowBytes == 0 || c.rowBytes % 16 != 0) throw Error("import_seg: row_bytes must be a positive multiple of 16");
    if (c.nodeNum == 0 || c.nodeNum > 64) throw Error("import_seg: node_num must be in [1, 64]");
    if (!c.fused && c.myNode >= c.nodeNum) throw Error("import_seg: my_node must be < node_num");
    CheckAligned16(c.hotRowBase, "import_seg: hot_row_base");
    if (c.fused) {
        for (uint32_t s = 0; s < c.nSeg; ++s) CheckAligned16(c.segBases[s], "import_all: seg_bases");
    } else {
        CheckAligned16(c.segBase, "import_seg: seg_base");
    }
    const uint32_t bd = c.blockDim == 0 ? 1u : c.blockDim;
    const uint64_t positions = static_cast<uint64_t>(c.maxNumReqs) * c.topK;
    if (positions == 0) return;

    kvx::GatherPlan plan{};
    KvcGatherArgs &a = plan.a;
    a.channel = c.channel;
    a.segBase = c.segBase;
    a.topkIndices = c.topk;
    a.reqPoolIndices = c.pool;
    a.reqHostBase = c.hostBase;
    a.topKDeviceSlots = c.slots;
    a.isMiss = c.isMiss;
    a.numReal = c.numReal;
    a.hotRowBase = c.hotRowBase;
    a.status = c.status;
    a.layerOffsetRows = c.layerOffsetRows;
    a.perLayerSegRows = c.perLayerSegRows;
    a.rowBytes = c.rowBytes;
    a.stripeRows = c.stripeRows;
    a.nodeNum = c.nodeNum;
    a.myNode = c.fused ? 0u : c.myNode;
    a.topK = c.topK;
    a.maxNumReqs = c.maxNumReqs;
    a.positionsPerCore = static_cast<uint32_t>((positions + bd - 1) / bd);  // kvops_ext.cpp:250-251
    a.hotReqStrideRows = c.stride;
    plan.segBases = c.segBases;
    plan.fused = c.fused ? 1u : 0u;
    plan.spanRows = c.stride == 0 ? 0u : std::min<uint32_t>(c.stride, 65536u);
    plan.statusWords = bd;

    ScratchNeed need;
    need.win = kvx::gather_win_entries(c.maxNumReqs, c.stride);
    hipStream_t st = AsStream(c.stream);
    if (c.fused) {
        CheckStatusBlock(c.status, 0, c.nodeNum, bd, "import_all");
    } else {
        CheckStatusBlock(c.status, c.myNode, 1, bd, "import_seg");
    }
    if (fixed != nullptr) {
        // the no-allocation form: the fixed scratch bounds the call
        if (need.win > fixed->winEntries) {
            throw Error("import_all_noalloc: winner rows (max_num_reqs-1)*min(stride,65536)+65536 = " +
                        std::to_string(need.win) + " (max " + std::to_string(fixed->winEntries) +
                        ") must fit the fixed scratch");
        }
        for (uint32_t s = 0; s < c.nodeNum; ++s) ClearStatusWords(c.status, s, bd);
        hipCheck(kvx::launch_gather(plan, *fixed, reinterpret_cast<uint64_t>(g.overflow), st), "kvc_gather_rows launch");
        return;
    }
    std::lock_guard<std::mutex> lk(g_scratchMu);
    const kvx::RowScratch scr = ScratchFor(c.stream, need, c.fused ? "import_all" : "import_seg").rows;
    if (c.fused) {
        for (uint32_t s = 0; s < c.nodeNum; ++s) ClearStatusWords(c.status, s, bd);
    } else {
        ClearStatusWords(c.status, c.myNode, bd);
    }
    hipCheck(kvx::launch_gather(plan, scr, reinterpret_cast<uint64_t>(g.overflow), st), "kvc_gather_rows launch");
}

void DoExportRows(const uint64_t *segBases, bool fused, uint32_t layer_id, uint32_t per_layer_seg_rows,
                  uint32_t row_bytes, uint64_t src_layer_base, uint64_t indices_host, uint64_t num_real,
                  uint32_t max_rows, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node, uint64_t status,
                  uint64_t stream, uint32_t block_dim)
{
    EnsureInited();
    if (block_dim > 8) throw Error("export blockDim must be <= 8 (status slot layout)");
    if (row_bytes == 0 || row_bytes % 16 != 0) throw Error("export_rows: row_bytes must be a positive multiple of 16");
    if (node_num == 0 || node_num > 64) throw Error("export_rows: node_num must be in [1, 64]");
    if (my_node >= node_num) throw Error("export_rows: my_node must be < node_num");
    const uint32_t nSeg = fused ? node_num : 1u;
    for (uint32_t s = 0; s < nSeg; ++s) CheckAligned16(segBases[s], "export_rows: seg_base");
    CheckAligned16(src_layer_base, "export_rows: src_layer_base");
    if (max_rows == 0) return;
    if (indices_host == 0 || num_real == 0) throw Error("export_rows: indices_host and num_real must be device addresses");
    kvx::ExportRowsArgs a{};
    a.segBase = segBases[0];
    a.srcLayerBase = src_layer_base;
    a.indicesHost = indices_host;
    a.numReal = num_real;
    a.status = status;
    a.layerId = layer_id;
    a.perLayerSegRows = per_layer_seg_rows;
    a.rowBytes = row_bytes;
    a.maxRows = max_rows;
    a.stripeRows = stripe_rows;
    a.nodeNum = node_num;
    a.myNode = fused ? 0u : my_node;
    a.statusWords = block_dim == 0 ? 1u : block_dim;
    a.fused = fused ? 1u : 0u;
    ScratchNeed need;
    need.win = kvx::export_rows_win_entries(per_layer_seg_rows, fused ? node_num : 1u);
    if (fused) {
        CheckStatusBlock(status, 0, node_num, a.statusWords, "export_rows_all");
    } else {
        CheckStatusBlock(status, my_node, 1, a.statusWords, "export_rows");
    }
    std::lock_guard<std::mutex> lk(g_scratchMu);
    const kvx::RowScratch scr = ScratchFor(stream, need, fused ? "export_rows_all" : "export_rows").rows;
    if (fused) {
        for (uint32_t s = 0; s < node_num; ++s) ClearStatusWords(status, s, a.statusWords);
    } else {
        ClearStatusWords(status, my_node, a.statusWords);
    }
    hipCheck(kvx::launch_export_rows(a, segBases, scr, AsStream(stream)), "export_rows launch");
}

// Node masks for the memory-policy system calls: up to 1024 nodes (the
// kernel's usual limit); maxnode counts one past the mask's bits, as the
// kernel expects.
constexpr unsigned long kMaskBits = 1024;
constexpr unsigned long kMaskWords = kMaskBits / (8 * sizeof(unsigned long));

long GetPolicy(int *mode, unsigned long *mask, void *addr, unsigned long flags)
{
    return syscall(SYS_get_mempolicy, mode, mask, mask == nullptr ? 0ul : kMaskBits + 1, addr, flags);
}

long SetPolicy(int mode, const unsigned long *mask)
{
    return syscall(SYS_set_mempolicy, mode, mask, mask == nullptr ? 0ul : kMaskBits + 1);
}

// Node holding the page at addr (-1 when the system cannot say).
int32_t PageNode(const void *addr)
{
    int node = -1;
    if (GetPolicy(&node, nullptr, const_cast<void *>(addr), MPOL_F_NODE | MPOL_F_ADDR) != 0) return -1;
    return node;
}


}  // namespace

extern "C" {

const char *kvx_last_error(void) { return t_lastError.c_str(); }

int kvx_init(int device_id, const char *code_object_path, const char *rt_lib)
{
    (void)code_object_path;
    (void)rt_lib;
    return Guarded([&] {
        if (g.inited) throw Error("kvops already inited");  // kvops_ext.cpp:141-143
        if (hipSetDevice(device_id) != hipSuccess) throw Error("hipSetDevice failed");
        g.device = device_id;
        void *p = nullptr;
        if (hipMalloc(&p, 8) != hipSuccess || p == nullptr) throw Error("alloc overflow buf failed");
        hipCheck(hipMemset(p, 0, 8), "hipMemset(overflow)");
        g.overflow = static_cast<uint64_t *>(p);
        int lds = 0;
        hipCheck(hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, device_id),
                 "hipDeviceGetAttribute(LDS)");
        g.ldsLimit = static_cast<size_t>(lds) - 1024;  // room for the kernels' static LDS (under 1 KiB)
        hipCheck(kvx::sieve_set_lds_limit(g.ldsLimit), "hipFuncSetAttribute(LDS)");
        hipCheck(kvx::sieve_fast_set_lds_limit(g.ldsLimit), "hipFuncSetAttribute(LDS fast)");
        g.ldsBatch = static_cast<size_t>(lds) - 6 * 1024;  // the batch kernel keeps ~4.7 KiB of static LDS
        hipCheck(kvx::sieve_batch_set_lds_limit(g.ldsBatch), "hipFuncSetAttribute(LDS batch)");
        // the rebuild's chunk kernel keeps ~1.3 KiB of static LDS beside its dynamic part
        g.tableRebuild = static_cast<size_t>(lds) >= kvx::kTblLdsBytes + 2 * 1024;
        if (g.tableRebuild) hipCheck(kvx::sieve_table_set_lds_limit(kvx::kTblLdsBytes), "hipFuncSetAttribute(LDS table)");
        {
            // the null stream's scratch at a default size, so that callers on
            // the null stream start without an allocation on the launch path
            std::lock_guard<std::mutex> lk(g_scratchMu);
            ScratchNeed need;
            need.win = 65536;
            (void)ScratchFor(0, need, "init");
        }
        // the no-allocation entry point's scratch on this device: the
        // symbol's device address (the host-side name is not one)
        if (device_id < 0 || device_id >= 64) throw Error("kvx_init: device_id must be in [0, 64)");
        if (g.noAllocScratch[device_id] == nullptr) {
            void *p = nullptr;
            hipCheck(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
            if (p == nullptr) throw Error("hipGetSymbolAddress(scratch) returned null");
            g.noAllocScratch[device_id] = p;
        }
        if (g.noAllocDone[device_id] == nullptr) {
            hipCheck(hipEventCreateWithFlags(&g.noAllocDone[device_id], hipEventDisableTiming),
                     "hipEventCreateWithFlags(no-allocation import)");
        }
        hipCheck(hipDeviceSynchronize(), "hipDeviceSynchronize");
        g.inited = true;
    });
}

int kvx_reserve_scratch(uint64_t stream, uint32_t max_num_reqs, uint32_t top_k, uint32_t hot_req_stride_rows,
                        uint32_t per_layer_seg_rows, uint32_t node_num, uint32_t device_buffer_size)
{
    return Guarded([&] {
        EnsureInited();
        if (node_num > 64) throw Error("reserve_scratch: node_num must be in [0, 64]");
        ScratchNeed need;
        need.win = std::max(kvx::gather_win_entries(max_num_reqs, hot_req_stride_rows),
                            kvx::export_rows_win_entries(per_layer_seg_rows, std::max<uint32_t>(node_num, 1u)));
        if (device_buffer_size > 0 && max_num_reqs > 0) {
            // the shape rules of the coordinator and kvops_ext.cpp:288-300
            const uint32_t padded = (device_buffer_size + 15u) & ~15u;
            const uint32_t vis = ((padded + 7u) / 8u + 63u) & ~63u;
            uint64_t ht = 1024;
            while (ht < 2ull * (static_cast<uint64_t>(padded) + top_k)) ht <<= 1;
            if (padded <= 65534 && ht <= (1ull << 31)) {
                const SievePlan p = PlanSieve(top_k, device_buffer_size, padded, vis, 1, static_cast<uint32_t>(ht));
                const ScratchNeed sn = SieveScratchNeed(p, max_num_reqs, static_cast<uint32_t>(ht));
                need.shadow = sn.shadow;
                need.aux = sn.aux;
                need.tbl = sn.tbl;
            }
        }
        std::lock_guard<std::mutex> lk(g_scratchMu);
        (void)ScratchFor(stream, need, "reserve_scratch");
    });
}

int kvx_scratch_bytes(uint64_t stream, uint64_t *out_bytes)
{
    return Guarded([&] {
        EnsureInited();
        std::lock_guard<std::mutex> lk(g_scratchMu);
        uint64_t b = 0;
        for (const StreamScratch *s : g.scratch) {
            if (s->stream != stream) continue;
            b = kvx::kControlWords * sizeof(uint32_t) + s->rows.winEntries * sizeof(unsigned long long) +
                s->shadowCells * sizeof(int32_t) + s->auxWords * sizeof(uint32_t) + s->tblWords * sizeof(uint32_t);
        }
        *out_bytes = b;
    });
}

int kvx_alloc_status(int count, uint64_t *out_addr)
{
    return Guarded([&] {
        EnsureInited();
        if (count <= 0) throw Error("alloc status failed");
        void *p = nullptr;
        const size_t bytes = static_cast<size_t>(count) * 64;
        if (hipHostMalloc(&p, bytes, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess || p == nullptr) {
            throw Error("alloc status failed");
        }
        void *d = nullptr;
        if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess || d != p) {
            (void)hipHostFree(p);
            throw Error("alloc status failed: device address differs from host address");
        }
        std::memset(p, 0, bytes);
        {
            std::lock_guard<std::mutex> lk(g_statusMu);
            g.status.push_back({reinterpret_cast<uint64_t>(p), bytes});
        }
        *out_addr = reinterpret_cast<uint64_t>(p);
    });
}

int64_t kvx_poll_status(uint64_t status_addr, int64_t timeout_us)
{
    if (!g.inited) {
        t_lastError = "kvops not inited";
        return -0x1000;
    }
    volatile uint64_t *w = StatusWord(status_addr);
    if (w == nullptr) return PollCopiedWord(status_addr, timeout_us);
    const auto t0 = std::chrono::steady_clock::now();
    uint32_t spins = 0;
    while (true) {
        const uint64_t v = __atomic_load_n(const_cast<uint64_t *>(w), __ATOMIC_ACQUIRE);
        if (((v >> 32) & 0xFFu) == 1u) return static_cast<int64_t>(v & 0xFFFFFFFFull);  // F2: doneSeq byte
        if (timeout_us >= 0) {
            const auto us = std::chrono::duration_cast<std::chrono::microseconds>(std::chrono::steady_clock::now() - t0);
            if (us.count() >= timeout_us) return -0x2000;
        }
        if (++spins < 4096) {
            __builtin_ia32_pause();
        } else {
            std::this_thread::sleep_for(std::chrono::microseconds(20));
        }
    }
}

int kvx_import_seg(uint64_t channel, uint64_t seg_base, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
                   uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices, uint64_t req_host_base,
                   uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base,
                   uint32_t top_k, uint32_t max_num_reqs, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node,
                   uint64_t status, uint64_t stream, uint32_t block_dim)
{
    return kvx_import_seg_strided(channel, seg_base, layer_offset_rows, per_layer_seg_rows, row_bytes, topk_indices,
                                  req_pool_indices, req_host_base, topk_device_slots, is_miss, num_real, hot_row_base,
                                  top_k, max_num_reqs, stripe_rows, node_num, my_node, status, stream, block_dim, 0);
}

int kvx_import_seg_strided(uint64_t channel, uint64_t seg_base, uint32_t layer_offset_rows,
                           uint32_t per_layer_seg_rows, uint32_t row_bytes, uint64_t topk_indices,
                           uint64_t req_pool_indices, uint64_t req_host_base, uint64_t topk_device_slots,
                           uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base, uint32_t top_k,
                           uint32_t max_num_reqs, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node,
                           uint64_t status, uint64_t stream, uint32_t block_dim, uint32_t hot_req_stride_rows)
{
    return Guarded([&] {
        GatherCall c{};
        c.fused = false;
        c.channel = channel;
        c.segBase = seg_base;
        c.layerOffsetRows = layer_offset_rows;
        c.perLayerSegRows = per_layer_seg_rows;
        c.rowBytes = row_bytes;
        c.topk = topk_indices;
        c.pool = req_pool_indices;
        c.hostBase = req_host_base;
        c.slots = topk_device_slots;
        c.isMiss = is_miss;
        c.numReal = num_real;
        c.hotRowBase = hot_row_base;
        c.topK = top_k;
        c.maxNumReqs = max_num_reqs;
        c.stripeRows = stripe_rows;
        c.nodeNum = node_num;
        c.myNode = my_node;
        c.status = status;
        c.stream = stream;
        c.blockDim = block_dim;
        c.stride = hot_req_stride_rows;
        DoGather(c);
    });
}

int kvx_import_all(const uint64_t *seg_bases, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
                   uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices, uint64_t req_host_base,
                   uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base,
                   uint32_t top_k, uint32_t max_num_reqs, uint32_t stripe_rows, uint32_t node_num, uint64_t status,
                   uint64_t stream, uint32_t block_dim, uint32_t hot_req_stride_rows)
{
    return Guarded([&] {
        if (seg_bases == nullptr) throw Error("import_all: seg_bases is null");
        if (node_num == 0 || node_num > 64) throw Error("import_seg: node_num must be in [1, 64]");
        GatherCall c{};
        c.fused = true;
        c.nSeg = node_num;
        for (uint32_t s = 0; s < node_num; ++s) c.segBases[s] = seg_bases[s];
        c.channel = 0;
        c.segBase = seg_bases[0];
        c.layerOffsetRows = layer_offset_rows;
        c.perLayerSegRows = per_layer_seg_rows;
        c.rowBytes = row_bytes;
        c.topk = topk_indices;
        c.pool = req_pool_indices;
        c.hostBase = req_host_base;
        c.slots = topk_device_slots;
        c.isMiss = is_miss;
        c.numReal = num_real;
        c.hotRowBase = hot_row_base;
        c.topK = top_k;
        c.maxNumReqs = max_num_reqs;
        c.stripeRows = stripe_rows;
        c.nodeNum = node_num;
        c.myNode = 0;
        c.status = status;
        c.stream = stream;
        c.blockDim = block_dim;
        c.stride = hot_req_stride_rows;
        DoGather(c);
    });
}

int kvx_import_all_noalloc(const uint64_t *seg_bases, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
                           uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices,
                           uint64_t req_host_base, uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real,
                           uint64_t hot_row_base, uint32_t top_k, uint32_t max_num_reqs, uint32_t stripe_rows,
                           uint32_t node_num, uint64_t status, uint64_t stream, uint32_t block_dim,
                           uint32_t hot_req_stride_rows)
{
    return Guarded([&] {
        EnsureInited();
        if (seg_bases == nullptr) throw Error("import_all_noalloc: seg_bases is null");
        if (node_num == 0 || node_num > 64) throw Error("import_seg: node_num must be in [1, 64]");
        void *base = g.noAllocScratch[g.device];
        if (base == nullptr) throw Error("import_all_noalloc: scratch address not set up on this device");
        unsigned char *b = static_cast<unsigned char *>(base);
        kvx::RowScratch fixed{};
        uint32_t *ctl = reinterpret_cast<uint32_t *>(b);
        fixed.counters = ctl;
        fixed.errs = ctl + 64 * 8;
        fixed.tickets = ctl + 2 * 64 * 8;
        fixed.chunkNext = fixed.tickets + 8;
        fixed.epoch = fixed.tickets + 9;
        fixed.win = reinterpret_cast<unsigned long long *>(b + kNoAllocControlBytes);
        fixed.winEntries = kNoAllocMaxWinEntries;
        // every call on this GPU shares the fixed scratch: a call on another
        // stream while the last one may still run is refused (the event query
        // and record allocate nothing; under capture neither is issued, and a
        // captured call must not overlap other calls of this entry point)
        const int dev = g.device;
        const bool capturing = Capturing(AsStream(stream));
        if (!capturing && g.noAllocPending[dev] && g.noAllocStream[dev] != stream) {
            const hipError_t q = hipEventQuery(g.noAllocDone[dev]);
            if (q == hipErrorNotReady) {
                throw Error("import_all_noalloc: a call on another stream may still be running on this GPU; its fixed "
                            "scratch is shared by every call, so order the calls (synchronize that stream first)");
            }
            if (q != hipSuccess) hipCheck(q, "hipEventQuery(no-allocation import)");
        }
        GatherCall c{};
        c.fused = true;
        c.nSeg = node_num;
        for (uint32_t s = 0; s < node_num; ++s) c.segBases[s] = seg_bases[s];
        c.segBase = seg_bases[0];
        c.layerOffsetRows = layer_offset_rows;
        c.perLayerSegRows = per_layer_seg_rows;
        c.rowBytes = row_bytes;
        c.topk = topk_indices;
        c.pool = req_pool_indices;
        c.hostBase = req_host_base;
        c.slots = topk_device_slots;
        c.isMiss = is_miss;
        c.numReal = num_real;
        c.hotRowBase = hot_row_base;
        c.topK = top_k;
        c.maxNumReqs = max_num_reqs;
        c.stripeRows = stripe_rows;
        c.nodeNum = node_num;
        c.status = status;
        c.stream = stream;
        c.blockDim = block_dim;
        c.stride = hot_req_stride_rows;
        DoGather(c, &fixed);
        if (!capturing) {
            hipCheck(hipEventRecord(g.noAllocDone[dev], AsStream(stream)), "hipEventRecord(no-allocation import)");
            g.noAllocStream[dev] = stream;
            g.noAllocPending[dev] = true;
        }
    });
}

int kvx_export_seg_alllayer(uint64_t channel, uint64_t seg_base, uint32_t per_layer_seg_rows, uint32_t row_bytes,
                            uint32_t row_lo, uint32_t row_cnt, uint32_t layer_num, uint64_t src_layer0_base,
                            uint64_t src_layer_stride, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node,
                            uint64_t status, uint64_t stream, uint32_t block_dim)
{
    return Guarded([&] {
        EnsureInited();
        if (block_dim > 8) throw Error("export blockDim must be <= 8 (status slot layout)");
        if (row_bytes == 0 || row_bytes % 16 != 0) throw Error("export_seg_alllayer: row_bytes must be a positive multiple of 16");
        if (node_num == 0 || node_num > 64) throw Error("export_seg_alllayer: node_num must be in [1, 64]");
        if (my_node >= node_num) throw Error("export_seg_alllayer: my_node must be < node_num");
        CheckAligned16(seg_base, "export_seg_alllayer: seg_base");
        CheckAligned16(src_layer0_base, "export_seg_alllayer: src_layer0_base");
        if (src_layer_stride % 16 != 0) throw Error("export_seg_alllayer: src_layer_stride must be a multiple of 16");
        if (static_cast<uint64_t>(row_lo) + row_cnt > 0xFFFFFFFFull) throw Error("export_seg_alllayer: row range exceeds 32 bits");
        KvcScatterAllArgs a{};
        a.channel = channel;
        a.segBase = seg_base;
        a.srcLayer0Base = src_layer0_base;
        a.srcLayerStride = src_layer_stride;
        a.status = status;
        a.perLayerSegRows = per_layer_seg_rows;
        a.rowBytes = row_bytes;
        a.rowLo = row_lo;
        a.rowCnt = row_cnt;
        a.layerNum = layer_num;
        a.stripeRows = stripe_rows;
        a.nodeNum = node_num;
        a.myNode = my_node;
        a.blockDim = block_dim == 0 ? 1u : block_dim;
        const kvx::ExportGeometry geo = kvx::export_geometry(a);
        if (geo.nStripes != 0 && geo.maxSegRow >= per_layer_seg_rows) {
            throw Error("export_seg_alllayer: rows [row_lo, row_lo+row_cnt) exceed per_layer_seg_rows of the segment");
        }
        CheckStatusBlock(status, my_node, 1, a.blockDim, "export_seg_alllayer");
        std::lock_guard<std::mutex> lk(g_scratchMu);
        const kvx::RowScratch scr = ScratchFor(stream, ScratchNeed{}, "export_seg_alllayer").rows;
        ClearStatusWords(status, my_node, a.blockDim);
        hipCheck(kvx::launch_export(a, scr, reinterpret_cast<uint64_t>(g.overflow), AsStream(stream)),
                 "kvc_scatter_rows_alllayer launch");
    });
}

int kvx_export_rows(uint64_t channel, uint64_t seg_base, uint32_t layer_id, uint32_t per_layer_seg_rows,
                    uint32_t row_bytes, uint64_t src_layer_base, uint64_t indices_host, uint64_t indices_dst_unused,
                    uint64_t num_real, uint32_t max_rows, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node,
                    uint64_t status, uint64_t stream, uint32_t block_dim)
{
    (void)channel;
    (void)indices_dst_unused;
    return Guarded([&] {
        DoExportRows(&seg_base, false, layer_id, per_layer_seg_rows, row_bytes, src_layer_base, indices_host, num_real,
                     max_rows, stripe_rows, node_num, my_node, status, stream, block_dim);
    });
}

int kvx_export_rows_all(const uint64_t *seg_bases, uint32_t layer_id, uint32_t per_layer_seg_rows, uint32_t row_bytes,
                        uint64_t src_layer_base, uint64_t indices_host, uint64_t indices_dst_unused, uint64_t num_real,
                        uint32_t max_rows, uint32_t stripe_rows, uint32_t node_num, uint64_t status, uint64_t stream,
                        uint32_t block_dim)
{
    (void)indices_dst_unused;
    return Guarded([&] {
        if (seg_bases == nullptr) throw Error("export_rows_all: seg_bases is null");
        DoExportRows(seg_bases, true, layer_id, per_layer_seg_rows, row_bytes, src_layer_base, indices_host, num_real,
                     max_rows, stripe_rows, node_num, 0, status, stream, block_dim);
    });
}

int kvx_sieve_update(uint64_t topk_indices, uint64_t req_pool_indices, uint64_t seq_lens, uint64_t prefill_lens,
                     uint64_t device_buffer_tokens, uint64_t device_buffer_visited, uint64_t device_buffer_ht,
                     uint64_t sieve_hand, uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real,
                     uint32_t top_k, uint32_t device_buffer_size, uint32_t padded_buffer_size,
                     uint32_t visited_stride_b, uint32_t max_num_reqs, uint32_t pool_size, uint64_t stream,
                     uint32_t block_dim)
{
    return Guarded([&] {
        EnsureInited();
        // kvops_ext.cpp:288-296, same messages
        if (padded_buffer_size % 16 != 0) {
            throw Error("sieve_update: padded_buffer_size must be a multiple of 16 (64-byte rows)");
        }
        if (padded_buffer_size > 65534) {
            throw Error("sieve_update: padded_buffer_size must be <= 65534 (uint16 hash slots)");
        }
        if (visited_stride_b % 64 != 0 || visited_stride_b < (padded_buffer_size + 7) / 8) {
            throw Error("sieve_update: visited bitmap stride must be 64B aligned and cover padded");
        }
        // The reference's sweep never terminates for an empty buffer; reject it.
        if (device_buffer_size < 1 || device_buffer_size > padded_buffer_size) {
            throw Error("sieve_update: device_buffer_size must be in [1, padded_buffer_size]");
        }
        CheckAligned16(device_buffer_tokens, "sieve_update: device_buffer_tokens");
        CheckAligned16(device_buffer_visited, "sieve_update: device_buffer_visited");
        CheckAligned16(device_buffer_ht, "sieve_update: device_buffer_ht");
        int64_t htSize = 1024;  // kvops_ext.cpp:297-300
        while (htSize < 2 * (static_cast<int64_t>(padded_buffer_size) + top_k)) htSize <<= 1;
        // kvops_ext.cpp:307-312 (kept for the args block; the grid is one workgroup per row)
        const uint32_t bd = block_dim == 0 ? 1u : block_dim;
        int64_t a0 = top_k, b0 = 64;
        while (b0 != 0) {
            const int64_t t = a0 % b0;
            a0 = b0;
            b0 = t;
        }
        const int64_t rpcAlign = 64 / (a0 == 0 ? 64 : a0);
        int64_t rpc = (static_cast<int64_t>(max_num_reqs) + bd - 1) / bd;
        rpc = (rpc + rpcAlign - 1) / rpcAlign * rpcAlign;
        if (rpc < 1) rpc = 1;

        HispSieveUpdateArgs a{};
        a.topkIndices = topk_indices;
        a.reqPoolIndices = req_pool_indices;
        a.seqLens = seq_lens;
        a.prefillLens = prefill_lens;
        a.deviceBufferTokens = device_buffer_tokens;
        a.deviceBufferVisited = device_buffer_visited;
        a.deviceBufferHt = device_buffer_ht;
        a.sieveHand = sieve_hand;
        a.topKDeviceSlots = topk_device_slots;
        a.isMiss = is_miss;
        a.numReal = num_real;
        a.status = 0;
        a.topK = top_k;
        a.deviceBufferSize = device_buffer_size;
        a.paddedBufferSize = padded_buffer_size;
        a.visitedStrideB = visited_stride_b;
        a.maxNumReqs = max_num_reqs;
        a.reqsPerCore = static_cast<uint32_t>(rpc);
        a.htSize = static_cast<uint32_t>(htSize);
        a.poolSize = pool_size;
        const SievePlan plan = PlanSieve(top_k, device_buffer_size, padded_buffer_size, visited_stride_b, pool_size,
                                         static_cast<uint32_t>(htSize));
        a.reserved = static_cast<uint32_t>(plan.variant) | (plan.invCap << 8);
        g.lastSieveVariant = plan.variant;
        if (max_num_reqs == 0) return;
        if (plan.variant == 2 || plan.variant == 4) {
            hipCheck(kvx::launch_sieve_update_fast(a, reinterpret_cast<uint64_t>(g.overflow), plan.ldsLaunch,
                                                   plan.variant == 4, AsStream(stream)),
                     "hisp_sieve_update launch");
        } else if (plan.variant == 3) {
            std::lock_guard<std::mutex> lk(g_scratchMu);
            int32_t *shadow = ScratchFor(stream, SieveScratchNeed(plan, max_num_reqs, static_cast<uint32_t>(htSize)),
                                         "sieve_update").shadow;
            hipCheck(kvx::launch_sieve_update_wave(a, reinterpret_cast<uint64_t>(g.overflow), shadow, AsStream(stream)),
                     "hisp_sieve_update launch");
        } else if (plan.variant == 5) {
            std::lock_guard<std::mutex> lk(g_scratchMu);
            const StreamScratch &sc =
                ScratchFor(stream, SieveScratchNeed(plan, max_num_reqs, static_cast<uint32_t>(htSize)), "sieve_update");
            hipCheck(kvx::launch_sieve_update_batch(a, reinterpret_cast<uint64_t>(g.overflow), sc.shadow, sc.aux,
                                                    plan.rebuild ? sc.tbl : nullptr, AsStream(stream)),
                     "hisp_sieve_update launch");
        } else {
            hipCheck(kvx::launch_sieve_update(a, reinterpret_cast<uint64_t>(g.overflow), plan.variant,
                                              plan.variant == 0 ? plan.ldsLaunch : 0, AsStream(stream)),
                     "hisp_sieve_update launch");
        }
    });
}

int kvx_sieve_ht_init(uint64_t device_buffer_tokens, uint64_t device_buffer_ht, uint64_t prefill_lens,
                      uint32_t req_start, uint32_t num_reqs, uint32_t layer_num, uint32_t pool_size,
                      uint32_t device_buffer_size, uint32_t padded_buffer_size, uint32_t ht_size, uint64_t stream,
                      uint32_t block_dim)
{
    (void)block_dim;
    return Guarded([&] {
        EnsureInited();
        if (ht_size < 8 || (ht_size & (ht_size - 1)) != 0) throw Error("sieve_ht_init: ht_size must be a power of two >= 8");
        if (device_buffer_size > padded_buffer_size) {
            throw Error("sieve_ht_init: device_buffer_size must be <= padded_buffer_size");
        }
        CheckAligned16(device_buffer_ht, "sieve_ht_init: device_buffer_ht");
        HispSieveHtInitArgs a{};
        a.deviceBufferTokens = device_buffer_tokens;
        a.deviceBufferHt = device_buffer_ht;
        a.prefillLens = prefill_lens;
        a.status = 0;
        a.reqStart = req_start;
        a.numReqs = num_reqs;
        a.layerNum = layer_num;
        a.poolSize = pool_size;
        a.deviceBufferSize = device_buffer_size;
        a.paddedBufferSize = padded_buffer_size;
        a.htSize = ht_size;
        if (static_cast<uint64_t>(num_reqs) * layer_num == 0) return;
        // the parallel build when its LDS form fits, else the batched wave
        // build (larger tables), else one lane per table on the table in LDS
        // or in HBM
        const size_t ldsPar = kvx::sieve_ht_init_par_lds(ht_size, device_buffer_size);
        const size_t ldsWave = kvx::sieve_ht_init_wave_lds(ht_size, device_buffer_size);
        kvx::InitForm form = kvx::InitForm::kInOrder;
        size_t lds = static_cast<size_t>(ht_size) * 2;
        if (ldsPar != 0 && ldsPar <= g.ldsLimit) {
            form = kvx::InitForm::kParallel;
            lds = ldsPar;
        } else if (ldsWave != 0 && ldsWave <= g.ldsLimit) {
            form = kvx::InitForm::kWave;
            lds = ldsWave;
        } else if (lds > g.ldsLimit) {
            lds = 0;
        }
        hipCheck(kvx::launch_sieve_ht_init(a, reinterpret_cast<uint64_t>(g.overflow), lds, AsStream(stream), form),
                 "hisp_sieve_ht_init launch");
    });
}

int kvx_close(void)
{
    return Guarded([&] {
        if (g.inited) (void)hipDeviceSynchronize();  // nothing in flight may still use the scratch
        if (g.overflow != nullptr) (void)hipFree(g.overflow);
        g.overflow = nullptr;
        {
            std::lock_guard<std::mutex> lk(g_scratchMu);
            for (StreamScratch *s : g.scratch) {
                if (s->rows.win != nullptr) (void)hipFree(s->rows.win);
                if (s->rows.counters != nullptr) (void)hipFree(s->rows.counters);
                if (s->shadow != nullptr) (void)hipFree(s->shadow);
                if (s->aux != nullptr) (void)hipFree(s->aux);
                if (s->tbl != nullptr) (void)hipFree(s->tbl);
                delete s;
            }
            g.scratch.clear();
            for (void *p : g.retired) (void)hipFree(p);
            g.retired.clear();
        }
        {
            std::lock_guard<std::mutex> lk(g_statusMu);
            for (const Alloc &a : g.status) (void)hipHostFree(reinterpret_cast<void *>(a.addr));
            g.status.clear();
        }
        for (int d = 0; d < 64; ++d) {
            if (g.noAllocDone[d] != nullptr) (void)hipEventDestroy(g.noAllocDone[d]);
            g.noAllocDone[d] = nullptr;
            g.noAllocPending[d] = false;
        }
        g.inited = false;
    });
}

int kvx_host_alloc(uint64_t bytes, uint32_t flags, uint64_t *out_addr)
{
    return Guarded([&] {
        if (bytes == 0) throw Error("host_alloc: bytes must be > 0");
        const unsigned f = hipHostMallocMapped | (flags == 1 ? hipHostMallocCoherent : hipHostMallocNonCoherent);
        void *p = nullptr;
        hipError_t e = hipHostMalloc(&p, bytes, f);
        if (e != hipSuccess || p == nullptr) {
            throw Error("host_alloc: hipHostMalloc of " + std::to_string(bytes) + " bytes failed: " + hipGetErrorString(e));
        }
        void *d = nullptr;
        if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess || d != p) {
            (void)hipHostFree(p);
            throw Error("host_alloc: device address differs from host address");
        }
        std::lock_guard<std::mutex> lk(g_hostMu);
        g_hostAllocs[reinterpret_cast<uint64_t>(p)] = bytes;
        *out_addr = reinterpret_cast<uint64_t>(p);
    });
}

int kvx_gpu_numa_node(int32_t device_id, int32_t *out_node)
{
    return Guarded([&] {
        if (out_node == nullptr) throw Error("gpu_numa_node: out_node is null");
        char bus[64] = {0};
        hipCheck(hipDeviceGetPCIBusId(bus, sizeof(bus), device_id), "hipDeviceGetPCIBusId");
        std::string id(bus);
        for (char &c : id) c = static_cast<char>(std::tolower(static_cast<unsigned char>(c)));
        std::ifstream f("/sys/bus/pci/devices/" + id + "/numa_node");
        int n = -1;
        if (!(f >> n)) n = -1;
        *out_node = n < 0 ? -1 : n;
    });
}

int kvx_host_alloc_node(uint64_t bytes, uint32_t flags, int32_t node, uint64_t *out_addr, int32_t *out_page_node)
{
    return Guarded([&] {
        if (node < 0) {
            const int rc = kvx_host_alloc(bytes, flags, out_addr);
            if (rc != 0) throw Error(kvx_last_error());
            if (out_page_node != nullptr) *out_page_node = PageNode(reinterpret_cast<void *>(*out_addr));
            return;
        }
        if (bytes == 0) throw Error("host_alloc: bytes must be > 0");
        if (static_cast<unsigned long>(node) >= kMaskBits) throw Error("host_alloc: node must be below 1024");
        // bind this thread's allocations to the node while the runtime
        // allocates and pins the pages, then restore its previous policy
        int prevMode = MPOL_DEFAULT;
        unsigned long prevMask[kMaskWords] = {0};
        if (GetPolicy(&prevMode, prevMask, nullptr, 0) != 0) {
            throw Error(std::string("host_alloc: get_mempolicy failed: ") + std::strerror(errno));
        }
        unsigned long mask[kMaskWords] = {0};
        mask[node / (8 * sizeof(unsigned long))] = 1ul << (node % (8 * sizeof(unsigned long)));
        if (SetPolicy(MPOL_BIND, mask) != 0) {
            throw Error("host_alloc: node " + std::to_string(node) + " is not available (set_mempolicy: " +
                        std::strerror(errno) + ")");
        }
        const unsigned f = hipHostMallocMapped | hipHostMallocNumaUser |
                           (flags == 1 ? hipHostMallocCoherent : hipHostMallocNonCoherent);
        void *p = nullptr;
        const hipError_t e = hipHostMalloc(&p, bytes, f);
        const bool restored = SetPolicy(prevMode, prevMode == MPOL_DEFAULT ? nullptr : prevMask) == 0;
        if (e != hipSuccess || p == nullptr) {
            throw Error("host_alloc: hipHostMalloc of " + std::to_string(bytes) + " bytes on node " +
                        std::to_string(node) + " failed: " + hipGetErrorString(e));
        }
        void *d = nullptr;
        if (!restored || hipHostGetDevicePointer(&d, p, 0) != hipSuccess || d != p) {
            (void)hipHostFree(p);
            throw Error(restored ? "host_alloc: device address differs from host address"
                                 : "host_alloc: could not restore the thread's memory policy");
        }
        {
            std::lock_guard<std::mutex> lk(g_hostMu);
            g_hostAllocs[reinterpret_cast<uint64_t>(p)] = bytes;
        }
        *out_addr = reinterpret_cast<uint64_t>(p);
        if (out_page_node != nullptr) *out_page_node = PageNode(p);
    });
}

int kvx_host_free(uint64_t addr)
{
    return Guarded([&] {
        std::lock_guard<std::mutex> lk(g_hostMu);
        auto it = g_hostAllocs.find(addr);
        if (it == g_hostAllocs.end()) throw Error("host_free: unknown address");
        hipCheck(hipHostFree(reinterpret_cast<void *>(addr)), "hipHostFree");
        g_hostAllocs.erase(it);
    });
}

int kvx_read_overflow(uint64_t *out_value)
{
    return Guarded([&] {
        EnsureInited();
        hipCheck(hipDeviceSynchronize(), "hipDeviceSynchronize");
        hipCheck(hipMemcpy(out_value, g.overflow, 8, hipMemcpyDeviceToHost), "hipMemcpy(overflow)");
    });
}

int kvx_clear_overflow(void)
{
    return Guarded([&] {
        EnsureInited();
        hipCheck(hipMemset(g.overflow, 0, 8), "hipMemset(overflow)");
    });
}

int kvx_last_sieve_variant(void) { return g.lastSieveVariant; }

int kvx_sieve_force_variant(int variant)
{
    return Guarded([&] {
        if (variant < -1 || variant > 6) throw Error("sieve_force_variant: variant must be -1 or 0..6");
        g.forcedSieveVariant = variant;
    });
}

int kvx_stream_copy(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream)
{
    return Guarded([&] {
        EnsureInited();
        if (bytes % 16 != 0) throw Error("stream_copy: bytes must be a multiple of 16");
        CheckAligned16(dst, "stream_copy: dst");
        CheckAligned16(src, "stream_copy: src");
        if (bytes == 0) return;
        hipCheck(kvx::launch_stream_copy(dst, src, bytes, AsStream(stream)), "stream_copy launch");
    });
}

}  // extern "C"
