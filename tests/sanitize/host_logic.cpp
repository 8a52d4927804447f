// Runs the host-side layout and sizing code shared by the launch layer and
// the kernels (csrc/kvx_internal.h, include/kvx/kv_layout.h) over ranges of
// shapes under AddressSanitizer and UndefinedBehaviorSanitizer, checking
// what the kernels rely on: every LDS region of the parallel SIEVE layout is
// 16-byte aligned and lies inside the layout, the regions a kernel uses at
// the same time do not overlap, the batch kernel's regions fit, the winner
// tables cover every destination, and the row mapping round-trips.
#include <cstdio>
#include <cstdlib>
#include <vector>

#include "kvx_internal.h"

static int g_fail = 0;
#define CHECK(c)                                                            \
    do {                                                                    \
        if (!(c)) {                                                         \
            std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #c); \
            if (++g_fail > 20) std::exit(1);                                \
        }                                                                   \
    } while (0)

struct Region {
    const char *name;
    uint32_t off, size;
};

static void check_fast(uint32_t padded, uint32_t H, uint32_t K, uint32_t dbs, uint32_t vis, bool compact)
{
    const kvx::FastLayout l = kvx::fast_layout_for(padded, H, K, dbs, vis, compact);
    int pm = 0, qm = 0;
    const bool fixed = kvx::fast_fixed(K, dbs, pm, qm);
    const uint32_t Kx = fixed ? pm * kvx::kFastThreads : K, Dx = fixed ? qm * kvx::kFastThreads : padded;
    const uint32_t bm = H / 8u;
    std::vector<Region> r = {
        {"tok", l.tok, padded * (compact ? 2u : 4u)}, {"ht", l.ht, H * 2u}, {"vis", l.vis, vis},
        {"ptok", l.ptok, Kx * 4u}, {"vt", l.vt, Dx * 2u}, {"evslot", l.evslot, Kx * 2u},
        {"smKp", l.smKp, Kx * 2u + 16u}, {"eseq", l.eseq, Kx * 2u}, {"tb", l.tb, (Kx + 1u) * 2u},
        {"smA", l.smA, Kx * 4u}, {"smB", l.smB, Kx * 4u}, {"vset", l.vset, fixed ? Dx / 8u : vis},
        {"ber", l.ber, bm}, {"occ", l.occ, bm}};
    const bool finShared = l.fin == l.pinf;  // the fixed kernels keep the classes in registers
    if (!finShared) {
        r.push_back({"pinf", l.pinf, Kx * 4u});
        r.push_back({"fin", l.fin, bm});
        r.push_back({"nkb", l.nkb, bm});
    } else {
        CHECK(l.nkb + bm <= l.pinf + Kx * 4u);
    }
    for (const Region &x : r) {
        CHECK(x.off % 16u == 0u);
        CHECK(static_cast<uint64_t>(x.off) + x.size <= l.total);
    }
    for (size_t i = 0; i < r.size(); ++i)
        for (size_t j = i + 1; j < r.size(); ++j) {
            const bool apart = r[i].off + r[i].size <= r[j].off || r[j].off + r[j].size <= r[i].off;
            if (!apart) std::fprintf(stderr, "overlap %s %s (padded %u H %u K %u)\n", r[i].name, r[j].name, padded, H, K);
            CHECK(apart);
        }
}

int main()
{
    // parallel SIEVE layouts: the shapes the host can select (topK < 16383,
    // padded + 1 + topK <= 65535, dbs <= 32 * threads)
    for (uint32_t padded = 16; padded <= 32768; padded *= 2)
        for (uint32_t K : {1u, 63u, 64u, 1000u, 1024u, 2047u, 2048u, 4096u, 16382u}) {
            if (padded + 1u + K > 65535u) continue;
            for (uint32_t dbs : {padded - 15u, padded}) {
                const uint32_t H = static_cast<uint32_t>(1024);
                uint32_t h = H;
                while (h < 2u * (padded + K)) h <<= 1;
                const uint32_t vis = ((padded + 7u) / 8u + 63u) / 64u * 64u;
                for (bool compact : {false, true}) check_fast(padded, h, K, dbs, vis, compact);
            }
        }
    // batch HBM kernel layout
    for (uint32_t dbs : {1u, 64u, 4096u, 65518u, 65535u})
        for (uint32_t K : {1u, 2048u, 8192u, 100000u}) {
            uint32_t h = 1024;
            while (h < 2u * (dbs + K)) h <<= 1;
            const kvx::BatchLayout b = kvx::batch_layout(dbs, h, K);
            CHECK(b.stage + kvx::kBatchStage * 4u == b.total);
            CHECK(b.slot + K * 4u <= b.uni);
            CHECK(b.uniL2 <= b.stage);
            CHECK(kvx::batch_aux_words(h) >= 2ull * kvx::kBatchMapCap);  // map, first occurrences
        }
    // winner tables: request b's destination b*min(stride, 65536) + slot, slot < 65536
    for (uint32_t reqs : {1u, 2u, 64u, 256u})
        for (uint32_t stride : {0u, 1u, 4096u, 65536u, 70000u}) {
            const uint64_t span = stride == 0 ? 0 : (stride < 65536u ? stride : 65536u);
            CHECK(kvx::gather_win_entries(reqs, stride) >= (reqs - 1u) * span + 65535u + 1u);
        }
    CHECK(kvx::export_rows_win_entries(0, 4) == 1u);
    // row mapping round trip (kv_layout.h): row -> (node, segment row) -> row
    for (uint32_t S : {1u, 2u, 64u})
        for (uint32_t N : {1u, 3u, 4u, 64u})
            for (uint32_t row = 0; row < 5000u; row += 7u) {
                const uint32_t n = kvx_node_of(row, S, N), q = kvx_seg_row_of(row, S, N);
                CHECK(n < N);
                CHECK((q * N + n) * S + row % S == row);
            }
    if (g_fail) return 1;
    std::printf("host logic: layouts, winner tables and row mapping checked, no sanitizer finding\n");
    return 0;
}
