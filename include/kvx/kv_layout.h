/*
 * Row ownership across the N host segments.
 *
 * The mapping is a format shared with every writer and reader of the
 * segments, so it is kept identical to the reference (common/kv_layout.h:26-57,
 * kvops/kernel/kvc_common.h:81-89):
 *
 *   node(row)    = (row / S) % N
 *   segRow(row)  = (row / S) / N
 *   offset(l,row)= (l * perLayerSegRows + segRow(row)) * rowBytes
 *   perLayerSegRows = ceil(layerRows / N)
 *
 * S == 0 maps every row to node 0 at segRow == row.  With S > 1 all S rows of
 * one stripe share a segment row (the reference's mapping is not injective
 * there); writers resolve that by letting the highest row of the stripe win.
 *
 * Usable from host C/C++ and from HIP device code.
 */
#ifndef KVX_KV_LAYOUT_H
#define KVX_KV_LAYOUT_H

#include <stdint.h>

#if defined(__HIPCC__)
#define KVX_HD __host__ __device__ __forceinline__
#else
#define KVX_HD static inline
#endif

KVX_HD uint32_t kvx_per_layer_seg_rows(uint32_t layerRows, uint32_t nodeNum)
{
    return (layerRows + nodeNum - 1u) / nodeNum;
}

KVX_HD uint32_t kvx_node_of(uint32_t row, uint32_t stripeRows, uint32_t nodeNum)
{
    return stripeRows == 0u ? 0u : (row / stripeRows) % nodeNum;
}

KVX_HD uint32_t kvx_seg_row_of(uint32_t row, uint32_t stripeRows, uint32_t nodeNum)
{
    return stripeRows == 0u ? row : (row / stripeRows) / nodeNum;
}

KVX_HD uint64_t kvx_seg_offset(uint32_t layer, uint32_t row, uint32_t stripeRows, uint32_t nodeNum,
                               uint32_t perLayerSegRows, uint32_t rowBytes)
{
    return ((uint64_t)layer * perLayerSegRows + kvx_seg_row_of(row, stripeRows, nodeNum)) * rowBytes;
}

/* 0 when the layout is usable, -1 otherwise (same rules as kv_layout.h:49-57). */
KVX_HD int kvx_layout_validate(uint32_t nodeNum, uint32_t layerNum, uint32_t layerRows,
                               uint32_t perLayerSegRows, uint32_t rowBytes, uint32_t stripeRows)
{
    if (nodeNum == 0u || nodeNum > 64u || layerNum == 0u || layerRows == 0u || rowBytes == 0u ||
        (rowBytes & 0x7Fu) != 0u || stripeRows == 0u ||
        perLayerSegRows != kvx_per_layer_seg_rows(layerRows, nodeNum)) {
        return -1;
    }
    return 0;
}

#endif /* KVX_KV_LAYOUT_H */
