// Python module `_kvops`: the reference's kvops_ext._kvops surface
// (kvops/kvops_ext/kvops_ext.cpp:373-401) over the libkvx.so C ABI.
// Same function names, argument names, defaults and exception texts; a
// nonzero C return becomes RuntimeError(kvx_last_error()).
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "kvx/kvx.h"

namespace py = pybind11;

namespace {

void Check(int rc)
{
    if (rc != 0) throw std::runtime_error(kvx_last_error());
}

}  // namespace

PYBIND11_MODULE(_kvops, m)
{
    m.doc() = "kvops launch extension for MI355X (gfx950): SIEVE miss detection and host-segment row movers";

    m.def(
        "init",
        [](int device_id, const std::string &fatbin_path, const std::string &rt_lib) {
            Check(kvx_init(device_id, fatbin_path.c_str(), rt_lib.c_str()));
        },
        py::arg("device_id"), py::arg("fatbin_path"), py::arg("rt_lib") = "libascendcl.so");

    m.def(
        "alloc_status",
        [](int count) {
            uint64_t addr = 0;
            Check(kvx_alloc_status(count, &addr));
            return addr;
        },
        py::arg("count"));

    m.def(
        "poll_status",
        [](uint64_t status_addr, int64_t timeout_us) {
            py::gil_scoped_release release;  // kvops_ext.cpp:201
            return kvx_poll_status(status_addr, timeout_us);
        },
        py::arg("status_addr"), py::arg("timeout_us") = -1);

    m.def(
        "import_seg",
        [](uint64_t channel, uint64_t seg_base, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
           uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices, uint64_t req_host_base,
           uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base, uint32_t top_k,
           uint32_t max_num_reqs, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node, uint64_t status,
           uint64_t stream, uint32_t block_dim, uint32_t hot_req_stride_rows) {
            Check(kvx_import_seg_strided(channel, seg_base, layer_offset_rows, per_layer_seg_rows, row_bytes,
                                         topk_indices, req_pool_indices, req_host_base, topk_device_slots, is_miss,
                                         num_real, hot_row_base, top_k, max_num_reqs, stripe_rows, node_num, my_node,
                                         status, stream, block_dim, hot_req_stride_rows));
        },
        py::arg("channel"), py::arg("seg_base"), py::arg("layer_offset_rows"), py::arg("per_layer_seg_rows"),
        py::arg("row_bytes"), py::arg("topk_indices"), py::arg("req_pool_indices"), py::arg("req_host_base"),
        py::arg("topk_device_slots"), py::arg("is_miss"), py::arg("num_real"), py::arg("hot_row_base"),
        py::arg("top_k"), py::arg("max_num_reqs"), py::arg("stripe_rows"), py::arg("node_num"), py::arg("my_node"),
        py::arg("status"), py::arg("stream") = 0, py::arg("block_dim") = 1, py::arg("hot_req_stride_rows") = 0);

    m.def(
        "import_all",
        [](const std::vector<uint64_t> &seg_bases, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
           uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices, uint64_t req_host_base,
           uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base, uint32_t top_k,
           uint32_t max_num_reqs, uint32_t stripe_rows, uint64_t status, uint64_t stream, uint32_t block_dim,
           uint32_t hot_req_stride_rows) {
            if (seg_bases.empty()) throw std::runtime_error("import_all: seg_bases is empty");
            Check(kvx_import_all(seg_bases.data(), layer_offset_rows, per_layer_seg_rows, row_bytes, topk_indices,
                                 req_pool_indices, req_host_base, topk_device_slots, is_miss, num_real, hot_row_base,
                                 top_k, max_num_reqs, stripe_rows, static_cast<uint32_t>(seg_bases.size()), status,
                                 stream, block_dim, hot_req_stride_rows));
        },
        py::arg("seg_bases"), py::arg("layer_offset_rows"), py::arg("per_layer_seg_rows"), py::arg("row_bytes"),
        py::arg("topk_indices"), py::arg("req_pool_indices"), py::arg("req_host_base"), py::arg("topk_device_slots"),
        py::arg("is_miss"), py::arg("num_real"), py::arg("hot_row_base"), py::arg("top_k"), py::arg("max_num_reqs"),
        py::arg("stripe_rows"), py::arg("status"), py::arg("stream") = 0, py::arg("block_dim") = 1,
        py::arg("hot_req_stride_rows") = 0);

    m.def(
        "import_all_noalloc",
        [](const std::vector<uint64_t> &seg_bases, uint32_t layer_offset_rows, uint32_t per_layer_seg_rows,
           uint32_t row_bytes, uint64_t topk_indices, uint64_t req_pool_indices, uint64_t req_host_base,
           uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint64_t hot_row_base, uint32_t top_k,
           uint32_t max_num_reqs, uint32_t stripe_rows, uint64_t status, uint64_t stream, uint32_t block_dim,
           uint32_t hot_req_stride_rows) {
            if (seg_bases.empty()) throw std::runtime_error("import_all_noalloc: seg_bases is empty");
            Check(kvx_import_all_noalloc(seg_bases.data(), layer_offset_rows, per_layer_seg_rows, row_bytes,
                                         topk_indices, req_pool_indices, req_host_base, topk_device_slots, is_miss,
                                         num_real, hot_row_base, top_k, max_num_reqs, stripe_rows,
                                         static_cast<uint32_t>(seg_bases.size()), status, stream, block_dim,
                                         hot_req_stride_rows));
        },
        py::arg("seg_bases"), py::arg("layer_offset_rows"), py::arg("per_layer_seg_rows"), py::arg("row_bytes"),
        py::arg("topk_indices"), py::arg("req_pool_indices"), py::arg("req_host_base"), py::arg("topk_device_slots"),
        py::arg("is_miss"), py::arg("num_real"), py::arg("hot_row_base"), py::arg("top_k"), py::arg("max_num_reqs"),
        py::arg("stripe_rows"), py::arg("status"), py::arg("stream") = 0, py::arg("block_dim") = 1,
        py::arg("hot_req_stride_rows") = 0);

    m.def(
        "export_seg_alllayer",
        [](uint64_t channel, uint64_t seg_base, uint32_t per_layer_seg_rows, uint32_t row_bytes, uint32_t row_lo,
           uint32_t row_cnt, uint32_t layer_num, uint64_t src_layer0_base, uint64_t src_layer_stride,
           uint32_t stripe_rows, uint32_t node_num, uint32_t my_node, uint64_t status, uint64_t stream,
           uint32_t block_dim) {
            Check(kvx_export_seg_alllayer(channel, seg_base, per_layer_seg_rows, row_bytes, row_lo, row_cnt,
                                          layer_num, src_layer0_base, src_layer_stride, stripe_rows, node_num, my_node,
                                          status, stream, block_dim));
        },
        py::arg("channel"), py::arg("seg_base"), py::arg("per_layer_seg_rows"), py::arg("row_bytes"),
        py::arg("row_lo"), py::arg("row_cnt"), py::arg("layer_num"), py::arg("src_layer0_base"),
        py::arg("src_layer_stride"), py::arg("stripe_rows"), py::arg("node_num"), py::arg("my_node"),
        py::arg("status"), py::arg("stream") = 0, py::arg("block_dim") = 1);

    m.def(
        "export_rows",
        [](uint64_t channel, uint64_t seg_base, uint32_t layer_id, uint32_t per_layer_seg_rows, uint32_t row_bytes,
           uint64_t src_layer_base, uint64_t indices_host, uint64_t indices_dst_unused, uint64_t num_real,
           uint32_t max_rows, uint32_t stripe_rows, uint32_t node_num, uint32_t my_node, uint64_t status,
           uint64_t stream, uint32_t block_dim) {
            Check(kvx_export_rows(channel, seg_base, layer_id, per_layer_seg_rows, row_bytes, src_layer_base,
                                  indices_host, indices_dst_unused, num_real, max_rows, stripe_rows, node_num, my_node,
                                  status, stream, block_dim));
        },
        py::arg("channel"), py::arg("seg_base"), py::arg("layer_id"), py::arg("per_layer_seg_rows"),
        py::arg("row_bytes"), py::arg("src_layer_base"), py::arg("indices_host"), py::arg("indices_dst_unused"),
        py::arg("num_real"), py::arg("max_rows"), py::arg("stripe_rows"), py::arg("node_num"), py::arg("my_node"),
        py::arg("status"), py::arg("stream") = 0, py::arg("block_dim") = 1);

    m.def(
        "export_rows_all",
        [](const std::vector<uint64_t> &seg_bases, uint32_t layer_id, uint32_t per_layer_seg_rows, uint32_t row_bytes,
           uint64_t src_layer_base, uint64_t indices_host, uint64_t indices_dst_unused, uint64_t num_real,
           uint32_t max_rows, uint32_t stripe_rows, uint64_t status, uint64_t stream, uint32_t block_dim) {
            if (seg_bases.empty()) throw std::runtime_error("export_rows_all: seg_bases is empty");
            Check(kvx_export_rows_all(seg_bases.data(), layer_id, per_layer_seg_rows, row_bytes, src_layer_base,
                                      indices_host, indices_dst_unused, num_real, max_rows, stripe_rows,
                                      static_cast<uint32_t>(seg_bases.size()), status, stream, block_dim));
        },
        py::arg("seg_bases"), py::arg("layer_id"), py::arg("per_layer_seg_rows"), py::arg("row_bytes"),
        py::arg("src_layer_base"), py::arg("indices_host"), py::arg("indices_dst_unused"), py::arg("num_real"),
        py::arg("max_rows"), py::arg("stripe_rows"), py::arg("status"), py::arg("stream") = 0,
        py::arg("block_dim") = 1);

    m.def(
        "sieve_update",
        [](uint64_t topk_indices, uint64_t req_pool_indices, uint64_t seq_lens, uint64_t prefill_lens,
           uint64_t device_buffer_tokens, uint64_t device_buffer_visited, uint64_t device_buffer_ht,
           uint64_t sieve_hand, uint64_t topk_device_slots, uint64_t is_miss, uint64_t num_real, uint32_t top_k,
           uint32_t device_buffer_size, uint32_t padded_buffer_size, uint32_t visited_stride_b,
           uint32_t max_num_reqs, uint32_t pool_size, uint64_t stream, uint32_t block_dim) {
            Check(kvx_sieve_update(topk_indices, req_pool_indices, seq_lens, prefill_lens, device_buffer_tokens,
                                   device_buffer_visited, device_buffer_ht, sieve_hand, topk_device_slots, is_miss,
                                   num_real, top_k, device_buffer_size, padded_buffer_size, visited_stride_b,
                                   max_num_reqs, pool_size, stream, block_dim));
        },
        py::arg("topk_indices"), py::arg("req_pool_indices"), py::arg("seq_lens"), py::arg("prefill_lens"),
        py::arg("device_buffer_tokens"), py::arg("device_buffer_visited"), py::arg("device_buffer_ht"),
        py::arg("sieve_hand"), py::arg("topk_device_slots"), py::arg("is_miss"), py::arg("num_real"),
        py::arg("top_k"), py::arg("device_buffer_size"), py::arg("padded_buffer_size"),
        py::arg("visited_stride_b"), py::arg("max_num_reqs"), py::arg("pool_size"), py::arg("stream") = 0,
        py::arg("block_dim") = 8);

    m.def(
        "sieve_ht_init",
        [](uint64_t device_buffer_tokens, uint64_t device_buffer_ht, uint64_t prefill_lens, uint32_t req_start,
           uint32_t num_reqs, uint32_t layer_num, uint32_t pool_size, uint32_t device_buffer_size,
           uint32_t padded_buffer_size, uint32_t ht_size, uint64_t stream, uint32_t block_dim) {
            Check(kvx_sieve_ht_init(device_buffer_tokens, device_buffer_ht, prefill_lens, req_start, num_reqs,
                                    layer_num, pool_size, device_buffer_size, padded_buffer_size, ht_size, stream,
                                    block_dim));
        },
        py::arg("device_buffer_tokens"), py::arg("device_buffer_ht"), py::arg("prefill_lens"), py::arg("req_start"),
        py::arg("num_reqs"), py::arg("layer_num"), py::arg("pool_size"), py::arg("device_buffer_size"),
        py::arg("padded_buffer_size"), py::arg("ht_size"), py::arg("stream") = 0, py::arg("block_dim") = 0);

    m.def("close", []() { Check(kvx_close()); });

    // ---- additions of kvx (no counterpart in the reference) ----
    m.def(
        "host_alloc",
        [](uint64_t nbytes, bool coherent) {
            uint64_t addr = 0;
            Check(kvx_host_alloc(nbytes, coherent ? 1u : 0u, &addr));
            return addr;
        },
        py::arg("nbytes"), py::arg("coherent") = false);
    m.def("host_free", [](uint64_t addr) { Check(kvx_host_free(addr)); }, py::arg("addr"));
    m.def(
        "host_alloc_node",
        [](uint64_t nbytes, bool coherent, int32_t node) {
            uint64_t addr = 0;
            int32_t pageNode = -1;
            Check(kvx_host_alloc_node(nbytes, coherent ? 1u : 0u, node, &addr, &pageNode));
            return py::make_tuple(addr, pageNode);
        },
        py::arg("nbytes"), py::arg("coherent") = false, py::arg("node") = -1);
    m.def(
        "gpu_numa_node",
        [](int32_t device_id) {
            int32_t node = -1;
            Check(kvx_gpu_numa_node(device_id, &node));
            return node;
        },
        py::arg("device_id") = 0);
    m.def("read_overflow", []() {
        uint64_t v = 0;
        Check(kvx_read_overflow(&v));
        return v;
    });
    m.def("clear_overflow", []() { Check(kvx_clear_overflow()); });
    m.def(
        "reserve_scratch",
        [](uint64_t stream, uint32_t max_num_reqs, uint32_t top_k, uint32_t hot_req_stride_rows,
           uint32_t per_layer_seg_rows, uint32_t node_num, uint32_t device_buffer_size) {
            Check(kvx_reserve_scratch(stream, max_num_reqs, top_k, hot_req_stride_rows, per_layer_seg_rows, node_num,
                                      device_buffer_size));
        },
        py::arg("stream"), py::arg("max_num_reqs"), py::arg("top_k"), py::arg("hot_req_stride_rows") = 0,
        py::arg("per_layer_seg_rows") = 0, py::arg("node_num") = 0, py::arg("device_buffer_size") = 0);
    m.def(
        "scratch_bytes",
        [](uint64_t stream) {
            uint64_t b = 0;
            Check(kvx_scratch_bytes(stream, &b));
            return b;
        },
        py::arg("stream") = 0);
    m.def("last_sieve_variant", []() { return kvx_last_sieve_variant(); });
    m.def("sieve_force_variant", [](int variant) { Check(kvx_sieve_force_variant(variant)); }, py::arg("variant"));
    m.def(
        "stream_copy",
        [](uint64_t dst, uint64_t src, uint64_t nbytes, uint64_t stream) {
            Check(kvx_stream_copy(dst, src, nbytes, stream));
        },
        py::arg("dst"), py::arg("src"), py::arg("nbytes"), py::arg("stream") = 0);
}
