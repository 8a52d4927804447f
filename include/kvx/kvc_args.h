/*
 * Launch-argument blocks for the four data-plane kernels.
 *
 * The field order, widths and therefore the byte layout are an ABI shared with
 * callers that build these blocks themselves: they match the reference's
 * kvops/kernel/kvc_args.h:17-97 byte for byte (sizes 120/80/136/64 B, checked
 * by the static_asserts below and by tests against the reference header).
 *
 * A launch passes the block followed by one 8-byte "tail slot" holding the
 * device address of an 8-byte device word (kvops_ext.cpp:106-129).  Here that
 * word is the device-side overflow/error word: a kernel that hits a bound the
 * reference would spin on (a probe run longer than the table) stores a
 * nonzero code there instead of hanging.
 */
#ifndef KVX_KVC_ARGS_H
#define KVX_KVC_ARGS_H

#include <stddef.h>
#include <stdint.h>

/* Decode miss import (kvc_args.h:17-38).  Scans positions [0, numReal*topK);
 * a position with isMiss != 0 whose row (reqHostBase[bid] + token) belongs to
 * myNode is copied from segment row (layerOffsetRows + segRow) into hot row
 * slot (+ bid * hotReqStrideRows). */
struct KvcGatherArgs {
    uint64_t channel;          /* segment index in kvx (HCOMM channel in the reference) */
    uint64_t segBase;          /* device-visible address of the segment's first byte */
    uint64_t topkIndices;      /* int32 [maxNumReqs, topK] */
    uint64_t reqPoolIndices;   /* int64 [maxNumReqs] */
    uint64_t reqHostBase;      /* int64 [maxNumReqs], first host row of each batch row */
    uint64_t topKDeviceSlots;  /* int32 [maxNumReqs, topK], SIEVE output */
    uint64_t isMiss;           /* int8  [maxNumReqs, topK], SIEVE output */
    uint64_t numReal;          /* int32 [1] */
    uint64_t hotRowBase;       /* byte address of hot row 0 */
    uint64_t status;           /* status ring base (64-byte slot per segment) */
    uint32_t layerOffsetRows;  /* layer * perLayerSegRows */
    uint32_t perLayerSegRows;
    uint32_t rowBytes;
    uint32_t stripeRows;       /* S */
    uint32_t nodeNum;          /* N */
    uint32_t myNode;
    uint32_t topK;
    uint32_t maxNumReqs;
    uint32_t positionsPerCore; /* ceil(maxNumReqs*topK / blockDim): status word partition */
    uint32_t hotReqStrideRows; /* "reserved" in the reference; 0 = reference semantics */
};

/* Prefill export of rows [rowLo, rowLo+rowCnt) of every layer (kvc_args.h:41-56). */
struct KvcScatterAllArgs {
    uint64_t channel;
    uint64_t segBase;
    uint64_t srcLayer0Base;    /* byte address of layer 0, row 0 in HBM */
    uint64_t srcLayerStride;   /* bytes between layers in HBM */
    uint64_t status;
    uint32_t perLayerSegRows;
    uint32_t rowBytes;
    uint32_t rowLo;
    uint32_t rowCnt;
    uint32_t layerNum;
    uint32_t stripeRows;
    uint32_t nodeNum;
    uint32_t myNode;
    uint32_t blockDim;         /* "reserved" in the reference: status words to write */
};

/* SIEVE update of one layer slice (kvc_args.h:59-81). */
struct HispSieveUpdateArgs {
    uint64_t topkIndices;          /* int32 [maxNumReqs, topK] */
    uint64_t reqPoolIndices;       /* int64 [maxNumReqs] */
    uint64_t seqLens;              /* int32 [maxNumReqs] */
    uint64_t prefillLens;          /* int32 [poolSize] */
    uint64_t deviceBufferTokens;   /* int32 [poolSize, padded] */
    uint64_t deviceBufferVisited;  /* uint8 [poolSize, visitedStrideB] bitmap */
    uint64_t deviceBufferHt;       /* uint16 [poolSize, htSize] */
    uint64_t sieveHand;            /* int32 [poolSize, 16], element 0 used */
    uint64_t topKDeviceSlots;      /* int32 [maxNumReqs, topK] out */
    uint64_t isMiss;               /* int8 [maxNumReqs, topK] out */
    uint64_t numReal;              /* int32 [1] */
    uint64_t status;               /* unused (0) */
    uint32_t topK;
    uint32_t deviceBufferSize;
    uint32_t paddedBufferSize;
    uint32_t visitedStrideB;
    uint32_t maxNumReqs;
    uint32_t reqsPerCore;          /* reference block partition; informational here */
    uint32_t htSize;
    uint32_t poolSize;
    uint32_t reserved;             /* kernel variant selected by the host (see kvx_host) */
};

/* Hash-table build for (layer, request) pairs (kvc_args.h:84-97). */
struct HispSieveHtInitArgs {
    uint64_t deviceBufferTokens;   /* int32 [layerNum, poolSize, padded] */
    uint64_t deviceBufferHt;       /* uint16 [layerNum, poolSize, htSize] */
    uint64_t prefillLens;          /* int32 [poolSize], unused by the kernel */
    uint64_t status;               /* unused (0) */
    uint32_t reqStart;
    uint32_t numReqs;
    uint32_t layerNum;
    uint32_t poolSize;
    uint32_t deviceBufferSize;
    uint32_t paddedBufferSize;
    uint32_t htSize;
    uint32_t reserved;
};

#ifdef __cplusplus
static_assert(sizeof(KvcGatherArgs) == 120, "KvcGatherArgs ABI");
static_assert(offsetof(KvcGatherArgs, status) == 72, "KvcGatherArgs.status");
static_assert(offsetof(KvcGatherArgs, layerOffsetRows) == 80, "KvcGatherArgs.layerOffsetRows");
static_assert(offsetof(KvcGatherArgs, hotReqStrideRows) == 116, "KvcGatherArgs.reserved");
static_assert(sizeof(KvcScatterAllArgs) == 80, "KvcScatterAllArgs ABI");
static_assert(sizeof(HispSieveUpdateArgs) == 136, "HispSieveUpdateArgs ABI");
static_assert(offsetof(HispSieveUpdateArgs, topK) == 96, "HispSieveUpdateArgs.topK");
static_assert(sizeof(HispSieveHtInitArgs) == 64, "HispSieveHtInitArgs ABI");

/* Args block plus the 8-byte tail slot, passed by value as the kernel's only
 * parameter, so the kernarg segment is exactly "struct + 8 B". */
template <typename A>
struct KvxLaunch {
    A a;
    uint64_t overflowSlot;
};
static_assert(sizeof(KvxLaunch<KvcGatherArgs>) == 128, "gather launch block");
static_assert(sizeof(KvxLaunch<KvcScatterAllArgs>) == 88, "scatter launch block");
static_assert(sizeof(KvxLaunch<HispSieveUpdateArgs>) == 144, "sieve launch block");
static_assert(sizeof(KvxLaunch<HispSieveHtInitArgs>) == 72, "ht init launch block");
#endif

#endif /* KVX_KVC_ARGS_H */
