/*
 * kvx — C ABI of the MI355X decode-time KV data plane (libkvx.so).
 *
 * Every entry point takes plain integers: device addresses of caller-owned
 * buffers (tensor.data_ptr()), sizes, and a hipStream_t passed as uint64_t
 * (0 = the null stream).  Launches are asynchronous and never synchronise the
 * host.  A nonzero return is an error; kvx_last_error() gives the message
 * (thread-local), with the same text the reference's pybind layer raises.
 *
 * Each declaration names the reference entry point it replaces
 * (jsun8686/kv_offload_proto, kvops/kvops_ext/kvops_ext.cpp).
 *
 * Status protocol (a fix of the reference's inconsistent layout): the status
 * ring is made of 64-byte slots; for a launch with status address `st`, the
 * word at st + myNode*64 + b*8 (b < block_dim <= 8) receives
 *     err (bits 0..31) | doneSeq=1 (bits 32..39) | queued (bits 40..63)
 * once every row of that launch has landed.  kvx_poll_status() masks the
 * doneSeq byte, so EmsPool-style waits that poll st + s*64 + b*8 work as-is.
 *
 * Streams and scratch: the row movers (import, export_rows, the prefill
 * export) and the HBM-resident SIEVE variant keep device scratch (winner
 * tags, counters, a table shadow).  The library holds one scratch
 * set per stream: launches on one stream run in order and share it, launches
 * on different streams (from any threads) never share it.  A stream's set is
 * created by its first launch (the null stream's by kvx_init) and grows when
 * a launch needs more; creation and growth allocate device memory and queue a
 * clear on that stream, and are refused during stream capture, so a stream
 * that will be captured is sized first with kvx_reserve_scratch.  Buffers are
 * never freed before kvx_close (a captured graph may hold their addresses).
 */
#ifndef KVX_KVX_H
#define KVX_KVX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* kvops_ext.cpp:139-185 kv_init.  Selects the device and allocates the 8-byte
 * tail-slot word.  The kernels are linked into libkvx.so, so code_object_path
 * and rt_lib are accepted for signature compatibility and not opened.
 * Errors: "kvops already inited", "hipSetDevice failed ...". */
int kvx_init(int device_id, const char *code_object_path, const char *rt_lib);

/* kvops_ext.cpp:187-196 kv_alloc_status.  count*64 zeroed bytes of coherent
 * pinned host memory whose host and device addresses are equal; *out_addr
 * receives that address. */
int kvx_alloc_status(int count, uint64_t *out_addr);

/* kvops_ext.cpp:198-218 kv_poll_status.  Reads the word at status_addr until
 * its doneSeq byte is 1 and returns the err field; returns -0x2000 after
 * timeout_us microseconds (timeout_us < 0 waits forever).  A word inside a
 * kvx_alloc_status block is read directly from the host; any other address
 * the runtime knows (device memory, pinned host memory) is read with an
 * 8-byte copy per poll; an unknown address or a failed copy gives -0x1000. */
int64_t kvx_poll_status(uint64_t status_addr, int64_t timeout_us);

/* kvops_ext.cpp:221-254 kv_import_seg: copy this segment's miss rows into the
 * hot buffer.  Error: "import blockDim must be <= 8 (status slot layout)". */
int kvx_import_seg(uint64_t channel, uint64_t seg_base, uint32_t layer_offset_rows,
                   uint32_t per_layer_seg_rows, uint32_t row_bytes, uint64_t topk_indices,
                   uint64_t req_pool_indices, uint64_t req_host_base, uint64_t topk_device_slots,
                   uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base, uint32_t top_k,
                   uint32_t max_num_reqs, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node,
                   uint64_t status, uint64_t stream, uint32_t block_dim);

/* kv_import_seg with the per-request hot-row stride the reference leaves in
 * KvcGatherArgs.reserved (kvc_args.h:37): hot row = slot + bid*stride. */
int kvx_import_seg_strided(uint64_t channel, uint64_t seg_base, uint32_t layer_offset_rows,
                           uint32_t per_layer_seg_rows, uint32_t row_bytes, uint64_t topk_indices,
                           uint64_t req_pool_indices, uint64_t req_host_base,
                           uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real,
                           uint64_t hot_row_base, uint32_t top_k, uint32_t max_num_reqs,
                           uint32_t stripe_rows, uint32_t node_num, uint32_t my_node, uint64_t status,
                           uint64_t stream, uint32_t block_dim, uint32_t hot_req_stride_rows);

/* All N segments in one launch sequence (xds_ems_pool.py:204-217 batch_read
 * issues N kv_import_seg calls; this is the fused form).  seg_bases points to
 * node_num host integers; status words are written for every node. */
int kvx_import_all(const uint64_t *seg_bases, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
                   uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices,
                   uint64_t req_host_base, uint64_t topk_device_slots, uint64_t is_miss,
                   uint64_t num_real, uint64_t hot_row_base, uint32_t top_k, uint32_t max_num_reqs,
                   uint32_t stripe_rows, uint32_t node_num, uint64_t status, uint64_t stream,
                   uint32_t block_dim, uint32_t hot_req_stride_rows);

/* No counterpart in the reference: kvx_import_all for callers that cannot
 * allocate device memory (launches under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation).  Same arguments, results and
 * status words as kvx_import_all; it allocates nothing and creates no
 * per-stream scratch: its scratch is one fixed array per GPU (17.8 MB, held
 * from library load to process exit) shared by every call of this entry
 * point on that GPU, so calls must not overlap on one GPU: a call on another
 * stream than the last one, while that one may still run, fails with an
 * error (calls captured in a graph are not checked; their replays must not
 * overlap other calls of this entry point).  Limit:
 * (max_num_reqs - 1) * min(hot_req_stride_rows, 65536) + 65536 <= 2228224;
 * a larger call fails with an error before anything is queued. */
int kvx_import_all_noalloc(const uint64_t *seg_bases, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
                           uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices,
                           uint64_t req_host_base, uint64_t topk_device_slots, uint64_t is_miss,
                           uint64_t num_real, uint64_t hot_row_base, uint32_t top_k, uint32_t max_num_reqs,
                           uint32_t stripe_rows, uint32_t node_num, uint64_t status, uint64_t stream,
                           uint32_t block_dim, uint32_t hot_req_stride_rows);

/* kvops_ext.cpp:256-278 kv_export_seg_alllayer: copy rows [row_lo,
 * row_lo+row_cnt) of every layer owned by my_node from HBM to the segment.
 * block_dim only sets how many status words are written (<= 8). */
int kvx_export_seg_alllayer(uint64_t channel, uint64_t seg_base, uint32_t per_layer_seg_rows,
                            uint32_t row_bytes, uint32_t row_lo, uint32_t row_cnt, uint32_t layer_num,
                            uint64_t src_layer0_base, uint64_t src_layer_stride, uint32_t stripe_rows,
                            uint32_t node_num, uint32_t my_node, uint64_t status, uint64_t stream,
                            uint32_t block_dim);

/* Decode-incremental single-layer export, the reference design's
 * kvops.export_rows / kvc_scatter_rows (doc/kv_offload_design.md:322-327,
 * 353-354, 394-396; design only, no implementation in the reference): entry
 * i < *num_real (int32 on the device, clamped to max_rows) names host row
 * indices_host[i] (int64 on the device); if that row maps to my_node, the
 * row_bytes at src_layer_base + i*row_bytes (HBM) are written to segment row
 * layer_id*per_layer_seg_rows + segRow(row).  Negative rows are skipped;
 * entries naming one segment row leave the last one's bytes (sequential
 * order).  Status word b (< block_dim <= 8) of node my_node covers entries
 * [b*ppc, (b+1)*ppc), ppc = ceil(max_rows/block_dim): (owned << 40) |
 * (1 << 32) | err, err = 0x200 + (i & 0xFF) + (1 << 16) for the lowest entry
 * i whose segment row lies outside the layer region (nothing written for
 * it), as the import reports (kvc_gather_rows.cpp:78-81).  channel and
 * indices_dst_unused are accepted and ignored, as in the design. */
int kvx_export_rows(uint64_t channel, uint64_t seg_base, uint32_t layer_id, uint32_t per_layer_seg_rows,
                    uint32_t row_bytes, uint64_t src_layer_base, uint64_t indices_host, uint64_t indices_dst_unused,
                    uint64_t num_real, uint32_t max_rows, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node,
                    uint64_t status, uint64_t stream, uint32_t block_dim);

/* All N segments of kvx_export_rows in one launch pair (the design issues one
 * export per segment, doc/kv_offload_design.md:353-354; this is the fused
 * form, like kvx_import_all): seg_bases points to node_num host integers;
 * status words are written for every node. */
int kvx_export_rows_all(const uint64_t *seg_bases, uint32_t layer_id, uint32_t per_layer_seg_rows, uint32_t row_bytes,
                        uint64_t src_layer_base, uint64_t indices_host, uint64_t indices_dst_unused, uint64_t num_real,
                        uint32_t max_rows, uint32_t stripe_rows, uint32_t node_num, uint64_t status, uint64_t stream,
                        uint32_t block_dim);

/* kvops_ext.cpp:281-336 kv_sieve_update.  Same validation messages; the hash
 * table size is derived identically; block_dim is accepted and only feeds the
 * informational reqsPerCore field (the grid is one workgroup per batch row).
 * Elements 1 and 2 of each 16-int sieve_hand record (unused by the reference)
 * carry a consistency flag and a count of steps that wrapped the hand;
 * zeroing them is always safe, and a caller that edits a row's tokens or
 * table outside these calls zeroes element 1. */
int kvx_sieve_update(uint64_t topk_indices, uint64_t req_pool_indices, uint64_t seq_lens,
                     uint64_t prefill_lens, uint64_t device_buffer_tokens,
                     uint64_t device_buffer_visited, uint64_t device_buffer_ht, uint64_t sieve_hand,
                     uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint32_t top_k,
                     uint32_t device_buffer_size, uint32_t padded_buffer_size,
                     uint32_t visited_stride_b, uint32_t max_num_reqs, uint32_t pool_size,
                     uint64_t stream, uint32_t block_dim);

/* kvops_ext.cpp:339-358 kv_sieve_ht_init.  The grid always covers
 * layer_num*num_reqs (layer, request) pairs; block_dim is accepted and unused. */
int kvx_sieve_ht_init(uint64_t device_buffer_tokens, uint64_t device_buffer_ht, uint64_t prefill_lens,
                      uint32_t req_start, uint32_t num_reqs, uint32_t layer_num, uint32_t pool_size,
                      uint32_t device_buffer_size, uint32_t padded_buffer_size, uint32_t ht_size,
                      uint64_t stream, uint32_t block_dim);

/* kvops_ext.cpp:360-371 kv_close.  Waits for the device, then frees the
 * tail-slot word, the status allocations and every stream's scratch;
 * idempotent. */
int kvx_close(void);

/* No counterpart in the reference (its launches keep no device scratch):
 * size the scratch of `stream` so that later launches on it allocate
 * nothing -- imports of up to max_num_reqs x top_k positions with
 * hot_req_stride_rows, decode-incremental exports into segments of
 * per_layer_seg_rows rows (node_num segments fused; 0 = none), and SIEVE
 * updates of max_num_reqs rows of device_buffer_size slots with top_k
 * positions (0 = none; only the HBM-resident variant keeps scratch).  Must be
 * called before capturing launches on `stream`. */
int kvx_reserve_scratch(uint64_t stream, uint32_t max_num_reqs, uint32_t top_k, uint32_t hot_req_stride_rows,
                        uint32_t per_layer_seg_rows, uint32_t node_num, uint32_t device_buffer_size);

/* Device bytes held by the scratch of `stream` (0 if it has none). */
int kvx_scratch_bytes(uint64_t stream, uint64_t *out_bytes);

/* Message of the last failing call on this thread ("" if none). */
const char *kvx_last_error(void);

/* Host segment memory (replaces the EMS daemon's mmap'd segments,
 * ems/emsd/pool_mgr.cc:23-41): pinned host memory mapped into the device
 * address space with equal host/device addresses.  flags: 0 = non-coherent
 * (coarse-grained), 1 = coherent (fine-grained). */
int kvx_host_alloc(uint64_t bytes, uint32_t flags, uint64_t *out_addr);
int kvx_host_free(uint64_t addr);

/* Placement of host segments (the reference's daemon maps anonymous memory
 * wherever the kernel puts it, ems/emsd/pool_mgr.cc:23-41).
 * kvx_gpu_numa_node: the NUMA node of the GPU's PCI function as the
 * platform reports it (sysfs), -1 when it reports none.
 * kvx_host_alloc_node: kvx_host_alloc with the pages bound to `node` (the
 * calling thread's memory policy is set to that node while the runtime
 * allocates and pins them, then restored); node < 0 = no binding.
 * *out_page_node (may be null) receives the node the first page landed on,
 * -1 if the system cannot say.  Free with kvx_host_free. */
int kvx_gpu_numa_node(int32_t device_id, int32_t *out_node);
int kvx_host_alloc_node(uint64_t bytes, uint32_t flags, int32_t node, uint64_t *out_addr, int32_t *out_page_node);

/* Value of the device tail-slot word (0 = no kernel hit a bound); reading it
 * synchronises the device.  kvx_clear_overflow() zeroes it. */
int kvx_read_overflow(uint64_t *out_value);
int kvx_clear_overflow(void);

/* Measurement utility, no counterpart in the reference: copy `bytes`
 * (multiple of 16, both addresses 16-byte aligned) from src to dst with a
 * grid-stride 16-byte streaming kernel on `stream`.  With src in a pinned
 * host segment it measures the zero-copy host-link read rate; with both in
 * HBM it is the known-size copy used to calibrate traffic counters. */
int kvx_stream_copy(uint64_t dst, uint64_t src, uint64_t bytes, uint64_t stream);

/* Which SIEVE kernel variant the last kvx_sieve_update launched:
 * 2 = parallel LDS-staged kernel, 4 = the same with the compact LDS layout
 * (16-bit token hashes in LDS, tokens in HBM) for rows whose full layout does
 * not fit, 0 = sequential LDS-staged kernel, 3 = sequential HBM-resident
 * kernel with wave-wide probes, 5 = batch HBM-resident kernel (rows too large
 * for LDS: decisions in one pass, the table's changes in batch, for a step
 * with misses rebuilt in parallel by kernels of their own), 1 = single-lane
 * HBM-resident kernel (only when forced).  For tests and benchmarks. */
int kvx_last_sieve_variant(void);

/* Testing and benchmarking knob, no counterpart in the reference: force the
 * SIEVE variant of later kvx_sieve_update calls (-1 = automatic, 0..5 as
 * above; 6 = variant 5 with a step's table deletions and inserts applied by
 * the batch kernel itself instead of the parallel rebuild; a variant whose
 * LDS needs do not fit falls back to automatic). */
int kvx_sieve_force_variant(int variant);

#ifdef __cplusplus
}
#endif

#endif /* KVX_KVX_H */
