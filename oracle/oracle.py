"""numpy/ctypes front end of the C oracle (oracle/kvx_oracle.c).

TEST INFRASTRUCTURE ONLY: loaded by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg.

Functions mirror the reference's algorithms on numpy arrays:
  sieve_update       kvops/kernel/hisp_sieve_update.cpp:17-176
  sieve_ht_init      kvops/kernel/hisp_sieve_ht_init.cpp:14-60
  gather_rows        kvops/kernel/kvc_gather_rows.cpp:12-96 (+ last-position-wins rule)
  stage_rows         the host staging step of the CPU serial pipeline (bench baseline)
  export_alllayer    kvops/kernel/kvc_scatter_rows_alllayer.cpp:11-67
  layout helpers     common/kv_layout.h:26-57
  ht_size, reqs_per_core  kvops/kvops_ext/kvops_ext.cpp:297-312
"""
import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i8p = ctypes.POINTER(ctypes.c_int8)
_u64p = ctypes.POINTER(ctypes.c_uint64)


def lib_path():
    return os.path.join(_HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(lib_path()):
            build()
        L = ctypes.CDLL(lib_path())
        L.orc_ht_hash.restype = ctypes.c_uint32
        L.orc_ht_hash.argtypes = [ctypes.c_int32]
        L.orc_ht_find.restype = ctypes.c_int32
        L.orc_ht_find.argtypes = [_u16p, _i32p, ctypes.c_int32, ctypes.c_int32]
        L.orc_ht_insert.restype = None
        L.orc_ht_insert.argtypes = [_u16p, _i32p, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.orc_ht_erase.restype = None
        L.orc_ht_erase.argtypes = [_u16p, _i32p, ctypes.c_int32, ctypes.c_int32]
        L.orc_get_error.restype = ctypes.c_int
        L.orc_clear_error.restype = None
        L.orc_sieve_update.restype = ctypes.c_int64
        L.orc_sieve_update.argtypes = [_i32p, _i64p, _i32p, _i32p, _i32p, _u8p, _u16p, _i32p, _i32p, _i8p,
                                       ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                       ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.orc_sieve_ht_init.restype = None
        L.orc_sieve_ht_init.argtypes = [_i32p, _u16p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                        ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32]
        L.orc_ht_size.restype = ctypes.c_int64
        L.orc_ht_size.argtypes = [ctypes.c_int64, ctypes.c_int64]
        L.orc_reqs_per_core.restype = ctypes.c_int64
        L.orc_reqs_per_core.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
        for name in ("orc_per_layer_seg_rows", "orc_node_of", "orc_seg_row_of"):
            getattr(L, name).restype = ctypes.c_uint32
        L.orc_per_layer_seg_rows.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        L.orc_node_of.argtypes = [ctypes.c_uint32] * 3
        L.orc_seg_row_of.argtypes = [ctypes.c_uint32] * 3
        L.orc_seg_offset.restype = ctypes.c_uint64
        L.orc_seg_offset.argtypes = [ctypes.c_uint32] * 6
        L.orc_layout_validate.restype = ctypes.c_int
        L.orc_layout_validate.argtypes = [ctypes.c_uint32] * 6
        L.orc_gather_rows.restype = ctypes.c_int64
        L.orc_gather_rows.argtypes = [ctypes.POINTER(_u8p), _u8p, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      _i32p, _i64p,
                                      _i64p, _i32p, _i8p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                      ctypes.c_uint32, _u64p]
        L.orc_export_alllayer.restype = ctypes.c_int64
        L.orc_export_alllayer.argtypes = [_u8p, _u8p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                          ctypes.c_uint32, ctypes.c_uint32]
        L.orc_stage_rows.restype = ctypes.c_int64
        L.orc_stage_rows.argtypes = [ctypes.POINTER(_u8p), _u8p, _i64p, ctypes.c_uint32, ctypes.c_uint32, _i32p,
                                     _i64p, _i64p, _i32p, _i8p, ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32,
                                     ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int32]
        L.orc_export_rows.restype = ctypes.c_int64
        L.orc_export_rows.argtypes = [_u8p, _u8p, _i64p, ctypes.c_int32] + [ctypes.c_uint32] * 8 + [_u64p]
        _LIB = L
    return _LIB


def _p(a, typ):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(typ)


def clear_error():
    lib().orc_clear_error()


def get_error():
    return lib().orc_get_error()


# ---------------------------------------------------------------- hash table
def ht_hash(token):
    return int(lib().orc_ht_hash(int(token)))


def ht_find(ht, tok, token):
    return int(lib().orc_ht_find(_p(ht, _u16p), _p(tok, _i32p), int(token), ht.size - 1))


def ht_insert(ht, tok, token, slot):
    lib().orc_ht_insert(_p(ht, _u16p), _p(tok, _i32p), int(token), int(slot), ht.size - 1)


def ht_erase(ht, tok, token):
    lib().orc_ht_erase(_p(ht, _u16p), _p(tok, _i32p), int(token), ht.size - 1)


# ---------------------------------------------------------------- derivations
def ht_size(padded, top_k):
    return int(lib().orc_ht_size(padded, top_k))


def reqs_per_core(max_num_reqs, block_dim, top_k):
    return int(lib().orc_reqs_per_core(max_num_reqs, block_dim, top_k))


def padded_of(dbs):
    return -(-dbs // 16) * 16


def vis_stride_of(padded):
    return -(-((padded + 7) // 8) // 64) * 64


# ---------------------------------------------------------------- layout
def per_layer_seg_rows(layer_rows, node_num):
    return int(lib().orc_per_layer_seg_rows(layer_rows, node_num))


def node_of(row, stripe_rows, node_num):
    return int(lib().orc_node_of(row, stripe_rows, node_num))


def seg_row_of(row, stripe_rows, node_num):
    return int(lib().orc_seg_row_of(row, stripe_rows, node_num))


def seg_offset(layer, row, stripe_rows, node_num, plsr, row_bytes):
    return int(lib().orc_seg_offset(layer, row, stripe_rows, node_num, plsr, row_bytes))


def layout_validate(node_num, layer_num, layer_rows, plsr, row_bytes, stripe_rows):
    return int(lib().orc_layout_validate(node_num, layer_num, layer_rows, plsr, row_bytes, stripe_rows))


# ---------------------------------------------------------------- SIEVE
class SieveState:
    """Host copy of the SIEVE state tensors of all layers (same shapes/dtypes
    as the coordinator's device tensors, ht as uint16)."""

    def __init__(self, layer_num, pool_size, dbs, top_k):
        self.layer_num, self.pool_size, self.dbs, self.top_k = layer_num, pool_size, dbs, top_k
        self.padded = padded_of(dbs)
        self.vis_stride = vis_stride_of(self.padded)
        self.ht_size = ht_size(self.padded, top_k)
        self.tokens = np.full((layer_num, pool_size, self.padded), -1, dtype=np.int32)
        self.vis = np.zeros((layer_num, pool_size, self.vis_stride), dtype=np.uint8)
        self.ht = np.zeros((layer_num, pool_size, self.ht_size), dtype=np.uint16)
        self.hand = np.zeros((layer_num, pool_size, 16), dtype=np.int32)
        self.prefill_lens = np.zeros(pool_size, dtype=np.int32)

    def admit(self, pool_idx, prefill_len):
        """Identity admission (xds_offload.py:56-77 with the row reset to -1 first)."""
        init_n = min(prefill_len, self.dbs)
        self.tokens[:, pool_idx, :] = -1
        self.tokens[:, pool_idx, :init_n] = np.arange(init_n, dtype=np.int32)
        self.vis[:, pool_idx, :] = 0
        self.hand[:, pool_idx, :] = 0
        self.prefill_lens[pool_idx] = prefill_len
        sieve_ht_init(self.tokens, self.ht, pool_idx, 1, self.layer_num, self.pool_size, self.dbs, self.padded,
                      self.ht_size)

    def copy(self):
        c = SieveState.__new__(SieveState)
        c.__dict__.update({k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in self.__dict__.items()})
        return c

    def update(self, layer, topk, req_pool, seq_lens, num_real, max_num_reqs=None, threads=1):
        """One sieve_update of `layer`; returns (slots, is_miss) of shape [maxNumReqs, topK].

        threads > 1 runs the batch rows on a thread pool, one oracle call per
        row (the C call releases the GIL), when no two rows name the same pool
        row; each row then sees exactly the state the in-order call gives it."""
        topk = np.ascontiguousarray(topk, dtype=np.int32)
        mnr = topk.shape[0] if max_num_reqs is None else max_num_reqs
        top_k = topk.shape[1]
        if ht_size(self.padded, top_k) != self.ht_size:
            raise ValueError("topK {} derives a different table size than the state's".format(top_k))
        slots = np.empty((mnr, top_k), dtype=np.int32)
        miss = np.empty((mnr, top_k), dtype=np.int8)
        tl, vl, hl, hdl = self.tokens[layer], self.vis[layer], self.ht[layer], self.hand[layer]
        req_pool = np.ascontiguousarray(req_pool, dtype=np.int64)
        seq_lens = np.ascontiguousarray(seq_lens, dtype=np.int32)
        nr = max(0, min(int(num_real), mnr))
        live = [int(r) for r in req_pool[:nr] if 0 <= int(r) < self.pool_size]
        if threads > 1 and nr > 1 and len(set(live)) == len(live):
            from concurrent.futures import ThreadPoolExecutor

            def one(b):
                sieve_update(topk[b:b + 1], req_pool[b:b + 1], seq_lens[b:b + 1], self.prefill_lens, tl, vl, hl,
                             hdl, slots[b:b + 1], miss[b:b + 1], 1 if b < nr else 0, top_k, self.dbs, self.padded,
                             self.vis_stride, 1, self.ht_size, self.pool_size)

            with ThreadPoolExecutor(max_workers=threads) as ex:
                list(ex.map(one, range(mnr)))
            return slots, miss
        sieve_update(topk, req_pool, seq_lens, self.prefill_lens, tl, vl, hl, hdl, slots, miss,
                     num_real, top_k, self.dbs, self.padded, self.vis_stride, mnr, self.ht_size, self.pool_size)
        return slots, miss


def sieve_update(topk, req_pool, seq_lens, prefill_lens, tokens, vis, ht, hand, out_slots, out_miss, num_real,
                 top_k, dbs, padded, vis_stride, max_num_reqs, ht_size_, pool_size):
    """In-place oracle update of one layer slice; returns the miss count."""
    return int(lib().orc_sieve_update(_p(topk, _i32p), _p(req_pool, _i64p), _p(seq_lens, _i32p),
                                      _p(prefill_lens, _i32p), _p(tokens, _i32p), _p(vis, _u8p), _p(ht, _u16p),
                                      _p(hand, _i32p), _p(out_slots, _i32p), _p(out_miss, _i8p), int(num_real),
                                      top_k, dbs, padded, vis_stride, max_num_reqs, ht_size_, pool_size))


def sieve_ht_init(tokens, ht, req_start, num_reqs, layer_num, pool_size, dbs, padded, ht_size_):
    lib().orc_sieve_ht_init(_p(tokens, _i32p), _p(ht, _u16p), req_start, num_reqs, layer_num, pool_size, dbs,
                            padded, ht_size_)


# ---------------------------------------------------------------- row movers
def gather_rows(segs, hot, layer_offset_rows, row_bytes, topk, req_pool, req_host_base, slots, is_miss, num_real,
                top_k, max_num_reqs, stripe_rows, node_num, my_node, hot_req_stride_rows=0, block_dim=1,
                per_layer_seg_rows=None):
    """Oracle import for segment my_node.  segs: list of N uint8 arrays (whole
    segments); hot: uint8 hot buffer.  per_layer_seg_rows: rows of one layer's
    region in a segment; a host row whose segment row lies past it is not read
    and its status word carries the 0x200 error band (None: every segment row
    is read, as the reference does).  Returns (rows copied, status words)."""
    arr = (_u8p * len(segs))(*[_p(s, _u8p) for s in segs])
    words = np.zeros(max(block_dim, 1), dtype=np.uint64)
    plsr = 0xFFFFFFFF if per_layer_seg_rows is None else int(per_layer_seg_rows)
    n = lib().orc_gather_rows(arr, _p(hot, _u8p), layer_offset_rows, plsr, row_bytes,
                              _p(np.ascontiguousarray(topk, dtype=np.int32), _i32p),
                              _p(np.ascontiguousarray(req_pool, dtype=np.int64), _i64p),
                              _p(np.ascontiguousarray(req_host_base, dtype=np.int64), _i64p),
                              _p(np.ascontiguousarray(slots, dtype=np.int32), _i32p),
                              _p(np.ascontiguousarray(is_miss, dtype=np.int8), _i8p), int(num_real), top_k,
                              max_num_reqs, stripe_rows, node_num, my_node, hot_req_stride_rows, max(block_dim, 1),
                              _p(words, _u64p))
    return int(n), words


def stage_rows(segs, staging, dst_rows, layer_offset_rows, row_bytes, topk, req_pool, req_host_base, slots, is_miss,
               num_real, top_k, max_num_reqs, stripe_rows, node_num, hot_req_stride_rows, threads):
    """Host staging step of the CPU serial pipeline: the winning miss rows of
    every segment copied into `staging` (uint8, rows x row_bytes) with
    `threads` threads; dst_rows (int64) receives each staged row's hot row.
    Returns the number of rows staged."""
    arr = (_u8p * len(segs))(*[_p(s, _u8p) for s in segs])
    return int(lib().orc_stage_rows(arr, _p(staging, _u8p), _p(dst_rows, _i64p), layer_offset_rows, row_bytes,
                                    _p(np.ascontiguousarray(topk, dtype=np.int32), _i32p),
                                    _p(np.ascontiguousarray(req_pool, dtype=np.int64), _i64p),
                                    _p(np.ascontiguousarray(req_host_base, dtype=np.int64), _i64p),
                                    _p(np.ascontiguousarray(slots, dtype=np.int32), _i32p),
                                    _p(np.ascontiguousarray(is_miss, dtype=np.int8), _i8p), int(num_real), top_k,
                                    max_num_reqs, stripe_rows, node_num, hot_req_stride_rows, int(threads)))


def export_rows(seg, src, indices, num_real, max_rows, layer_id, plsr, row_bytes, stripe_rows, node_num, my_node,
                block_dim=1):
    """Oracle decode-incremental export into one segment (uint8 array) from src
    (uint8 array of max_rows rows).  Returns (entries written, status words)."""
    words = np.zeros(max(block_dim, 1), dtype=np.uint64)
    n = lib().orc_export_rows(_p(seg, _u8p), _p(src, _u8p), _p(np.ascontiguousarray(indices, dtype=np.int64), _i64p),
                              int(num_real), max_rows, layer_id, plsr, row_bytes, stripe_rows, node_num, my_node,
                              max(block_dim, 1), _p(words, _u64p))
    return int(n), words


def export_alllayer(seg, src, src_layer_stride, plsr, row_bytes, row_lo, row_cnt, layer_num, stripe_rows, node_num,
                    my_node):
    """Oracle export into one segment (uint8 array) from src (uint8 array of
    layer_num * src_layer_stride bytes).  Returns the reference's queued count."""
    return int(lib().orc_export_alllayer(_p(seg, _u8p), _p(src, _u8p), src_layer_stride, plsr, row_bytes, row_lo,
                                         row_cnt, layer_num, stripe_rows, node_num, my_node))
