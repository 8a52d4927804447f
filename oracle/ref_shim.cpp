// C entry points over two of the reference's own headers, compiled where the
// reference is mounted (see Makefile target `ref`).  TEST INFRASTRUCTURE ONLY:
// tests load oracle/_ref/libkvref.so to check the layout mapping and the
// launch-argument byte layout of kvx against the reference's code.
//
//   kv_layout.h  (common/kv_layout.h:26-57)   -> kvref_node/seg_row/offset/validate
//   kvc_args.h   (kvops/kernel/kvc_args.h)    -> kvref_args_layout (sizeof/offsetof)
#include <cstddef>
#include <cstdint>

#include "kv_layout.h"
#include "kvc_args.h"

extern "C" {

uint32_t kvref_per_layer_seg_rows(uint32_t layerRows, uint32_t nodeNum)
{
    return KvLayoutPerLayerSegRows(layerRows, nodeNum);
}

uint32_t kvref_node(uint32_t row, uint32_t stripeRows, uint32_t nodeNum)
{
    KvLayout l{nodeNum, 1, 1, 1, 128, stripeRows};
    return KvLayoutNode(row, &l);
}

uint32_t kvref_seg_row(uint32_t row, uint32_t stripeRows, uint32_t nodeNum)
{
    KvLayout l{nodeNum, 1, 1, 1, 128, stripeRows};
    return KvLayoutSegRow(row, &l);
}

uint64_t kvref_seg_offset(uint32_t layer, uint32_t row, uint32_t stripeRows, uint32_t nodeNum, uint32_t plsr,
                          uint32_t rowBytes)
{
    KvLayout l{nodeNum, 1, 1, plsr, rowBytes, stripeRows};
    return KvLayoutSegOffset(layer, row, &l);
}

int kvref_validate(uint32_t nodeNum, uint32_t layerNum, uint32_t layerRows, uint32_t plsr, uint32_t rowBytes,
                   uint32_t stripeRows)
{
    KvLayout l{nodeNum, layerNum, layerRows, plsr, rowBytes, stripeRows};
    return KvLayoutValidate(&l);
}

// out[] = sizeof and field offsets of the four launch structs, in the order
// documented in tests/test_boundary.py.
int kvref_args_layout(uint64_t *out, int cap)
{
    const uint64_t v[] = {
        sizeof(KvcGatherArgs),
        offsetof(KvcGatherArgs, segBase),
        offsetof(KvcGatherArgs, hotRowBase),
        offsetof(KvcGatherArgs, status),
        offsetof(KvcGatherArgs, layerOffsetRows),
        offsetof(KvcGatherArgs, myNode),
        offsetof(KvcGatherArgs, positionsPerCore),
        offsetof(KvcGatherArgs, reserved),
        sizeof(KvcScatterAllArgs),
        offsetof(KvcScatterAllArgs, srcLayerStride),
        offsetof(KvcScatterAllArgs, status),
        offsetof(KvcScatterAllArgs, rowLo),
        offsetof(KvcScatterAllArgs, myNode),
        sizeof(HispSieveUpdateArgs),
        offsetof(HispSieveUpdateArgs, sieveHand),
        offsetof(HispSieveUpdateArgs, numReal),
        offsetof(HispSieveUpdateArgs, topK),
        offsetof(HispSieveUpdateArgs, reqsPerCore),
        offsetof(HispSieveUpdateArgs, poolSize),
        sizeof(HispSieveHtInitArgs),
        offsetof(HispSieveHtInitArgs, reqStart),
        offsetof(HispSieveHtInitArgs, htSize),
    };
    const int n = static_cast<int>(sizeof(v) / sizeof(v[0]));
    for (int i = 0; i < n && i < cap; ++i) out[i] = v[i];
    return n;
}

}  // extern "C"
