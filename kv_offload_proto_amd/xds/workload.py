"""End-to-end decode workload on one GPU: prefill export, admission, streams,
and per-layer decode steps (SIEVE update + miss import).

This is the flow of the reference driver (xds/xds_decode.py:121-289) on the
MI355X data plane: the HBM layer pool is filled, exported to the N host
segments, every request is admitted with the identity layout, and each decode
step runs ``sieve_update`` then the miss import for one layer.  The hot buffer
of layer l is ``hot[l]``, rows ``slot + bid*padded`` (one slice per request).
"""
import time
from collections import namedtuple

import numpy as np
import torch

from ..kvops_ext import _kvops
from . import streams
from .xds_offload import XdsOffloadCoordinator
from .xds_seg_pool import HostSegPool


# One layer-step of a generated stream: the topK batch (device and host
# copies), the miss count (sum of is_miss), the rows the import moves
# (distinct destination rows after the last-position-wins rule) and the
# distinct host segment rows it reads (fewer when S > 1 aliases a stripe's
# rows to one segment row, or when requests share host rows).
LayerStep = namedtuple("LayerStep", "step layer topk batch misses moved unique_src")


def allocate_host_rows(pool, cfg):
    """Host rows of the workload's requests from the pool's row allocator: one
    run of `prefill` rows per exported request, which must be contiguous (the
    import reads host row = host base + token; xds_decode.py:172-176).
    Decode requests beyond the exported set reuse an exported request's run.
    Returns the host base of every decode request."""
    allocator = pool.make_allocator()
    bases = []
    for _ in range(cfg.host_reqs):
        rows = allocator.alloc(cfg.prefill)
        if rows != list(range(rows[0], rows[0] + cfg.prefill)):
            raise RuntimeError("host rows of a request are not contiguous: the import reads host base + token")
        bases.append(rows[0])
    return [bases[r % cfg.host_reqs] for r in range(cfg.req_num)]


class DecodeRunner:
    def __init__(self, cfg, device=0, fill="fp16", coherent=False, log=print, block_dim=8):
        self.cfg = cfg
        self.log = log
        self.block_dim = block_dim
        self.dev = torch.device("cuda", device)
        torch.cuda.set_device(self.dev)
        L, rows, rb = cfg.layers, cfg.layer_rows, cfg.row_bytes
        # HBM layer pool [L, layer_rows, row_bytes]: fp16 rows uniform in [-1, 1)
        t0 = time.perf_counter()
        self.src = torch.empty((L, rows, rb), dtype=torch.uint8, device=self.dev)
        gen = torch.Generator(device=self.dev)
        gen.manual_seed(cfg.seed)
        if fill == "fp16":
            h = self.src.view(torch.float16)
            for l in range(L):
                h[l].uniform_(-1.0, 1.0, generator=gen)
        else:
            self.src.random_(0, 256, generator=gen)
        self.pool = HostSegPool(device, L, rows, rb, stripe_rows=cfg.stripe_rows, node_num=cfg.node_num,
                                coherent=coherent)
        self.pool.create_pool()
        torch.cuda.synchronize()
        self.setup_s = time.perf_counter() - t0
        self.export_us = None

        self.coord = XdsOffloadCoordinator(self.dev, L, cfg.req_num, cfg.dbs, cfg.top_k, cfg.req_num, cfg.prefill)
        self.padded = self.coord.padded_buffer_size
        self.hot = torch.zeros((L, cfg.req_num * self.padded, rb), dtype=torch.uint8, device=self.dev)
        self.req_pool = torch.arange(cfg.req_num, dtype=torch.int64, device=self.dev)
        self.seq_lens = torch.full((cfg.req_num,), cfg.prefill, dtype=torch.int32, device=self.dev)
        self.seg_bases = [sg.seg_base for sg in self.pool.pool.segments]
        self.status = self.pool.next_status()
        self.host_bases = allocate_host_rows(self.pool, cfg)

    # ---- prefill export (xds_decode.py:167-189) ----
    def export_prefill(self):
        cfg = self.cfg
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        st = self.pool.batch_write_alllayers(0, cfg.host_reqs * cfg.prefill, self.src, cfg.layer_rows * cfg.row_bytes,
                                             stream=stream.cuda_stream)
        e1.record(stream)
        self.pool.wait(st)
        torch.cuda.synchronize()
        self.export_us = e0.elapsed_time(e1) * 1e3
        rows = cfg.host_reqs * cfg.prefill
        self.export_bytes = cfg.layers * rows * cfg.row_bytes
        # with S > 1 a stripe's rows share one segment row and only the
        # stripe's last row lands there (kvc_scatter_rows_alllayer.cpp:34-52,
        # kvc_common.h:86-89)
        S = max(1, cfg.stripe_rows)
        self.export_moved_bytes = cfg.layers * ((rows + S - 1) // S) * cfg.row_bytes
        return self.export_us

    def admit_all(self):
        cfg = self.cfg
        for r in range(cfg.req_num):
            self.coord.admit_request(r, r, cfg.prefill, self.host_bases[r])
        self.coord.set_batch(self.req_pool, self.seq_lens)
        torch.cuda.synchronize()

    # ---- state snapshot for replays ----
    def snapshot(self):
        c = self.coord
        return [t.clone() for t in (c.device_buffer_tokens, c.device_buffer_visited, c.device_buffer_ht,
                                    c.sieve_hand)]

    def restore(self, snap):
        c = self.coord
        for dst, src in zip((c.device_buffer_tokens, c.device_buffer_visited, c.device_buffer_ht, c.sieve_hand),
                            snap):
            dst.copy_(src)
        torch.cuda.synchronize()

    # ---- streams ----
    def schedule(self, n_steps):
        """(step, layer) pairs in execution order: every layer every step for
        state-driven streams, one layer per step for the reference stream."""
        cfg = self.cfg
        if cfg.stream == "ref":
            return [(s, s % cfg.layers) for s in range(n_steps)]
        return [(s, l) for s in range(n_steps) for l in range(cfg.layers)]

    def generate(self, n_steps, seed=None):
        """Draw the topK batches of n_steps decode steps by running SIEVE on the
        GPU state (no imports), recording each layer-step's batch and miss
        count; the state is restored afterwards so a replay reproduces it."""
        cfg = self.cfg
        rng = np.random.default_rng(cfg.seed if seed is None else seed)
        pool = streams.adversarial_pool(cfg.prefill, cfg.adversarial_hash_below) if cfg.adversarial else None
        snap = self.snapshot()
        plan = []
        for step, layer in self.schedule(n_steps):
            if cfg.stream == "ref":
                batch = streams.ref_batch(rng, cfg.req_num, cfg.top_k, cfg.prefill, cfg.dbs, cfg.miss_ratio)
            else:
                toks = self.coord.device_buffer_tokens[layer, :, :cfg.dbs].cpu().numpy()
                batch = streams.state_batch(rng, toks, cfg.prefill, cfg.top_k, cfg.miss_ratio, zipf_s=cfg.zipf_s,
                                            miss_pool=pool)
            topk_d = torch.from_numpy(batch).to(self.dev)
            self.coord.sieve_update(layer, topk_d, block_dim=self.block_dim)
            misses, moved, unique_src = self.import_counts(topk_d)
            plan.append(LayerStep(step, layer, topk_d, batch, misses, moved, unique_src))
        self.restore(snap)
        return plan, snap

    def import_counts(self, topk_d):
        """(misses, rows moved, distinct host segment rows) of the import of
        the last SIEVE update's outputs."""
        cfg, c = self.cfg, self.coord
        miss = c.is_miss.bool()
        misses = int(miss.sum().item())
        valid = miss & (topk_d >= 0) & (c.top_k_device_slots >= 0)
        pos = torch.nonzero(valid.reshape(-1)).reshape(-1)
        if pos.numel() == 0:
            return misses, 0, 0
        bid = pos // cfg.top_k
        dest = c.top_k_device_slots.reshape(-1)[pos].to(torch.int64) + bid * self.padded
        moved = int(torch.unique(dest).numel())
        row = (c.req_host_base[bid] + topk_d.reshape(-1)[pos].to(torch.int64)) & 0xFFFFFFFF
        S, N = max(cfg.stripe_rows, 1), cfg.node_num
        q = row // S
        key = (q % N) * self.pool.per_layer_seg_rows + q // N
        return misses, moved, int(torch.unique(key).numel())

    # ---- one decode layer-step ----
    def sieve(self, layer, topk_d):
        self.coord.sieve_update(layer, topk_d, block_dim=self.block_dim)

    def gather(self, layer, topk_d, fused=True, block_dim=1):
        cfg, c = self.cfg, self.coord
        stream = torch.cuda.current_stream().cuda_stream
        if fused:
            _kvops.import_all(self.seg_bases, layer * self.pool.per_layer_seg_rows, self.pool.per_layer_seg_rows,
                              cfg.row_bytes, topk_d.data_ptr(), self.req_pool.data_ptr(), c.req_host_base.data_ptr(),
                              c.top_k_device_slots.data_ptr(), c.is_miss.data_ptr(), c.num_real.data_ptr(),
                              self.hot[layer].data_ptr(), cfg.top_k, cfg.req_num, cfg.stripe_rows, self.status,
                              stream, block_dim, self.padded)
        else:
            self.status = self.pool.batch_read(layer, topk_d, self.req_pool, c.req_host_base, c.top_k_device_slots,
                                               c.is_miss, c.num_real, self.hot[layer], cfg.req_num, cfg.top_k,
                                               stream=stream, block_dim=block_dim,
                                               hot_req_stride_rows=self.padded)

    def verify_last_gather(self, layer, topk_d):
        """Every miss row of the last step is byte-equal to its source row
        (the stripe's exported row when S > 1), checked on the GPU."""
        cfg, c = self.cfg, self.coord
        miss = c.is_miss.bool()
        pos = torch.arange(miss.numel(), device=self.dev).view_as(miss)[miss]
        bid = pos // cfg.top_k
        tok = topk_d[miss].long()
        slot = c.top_k_device_slots[miss].long()
        dest = slot + bid * self.padded
        # several misses of one step can land on one slot (a sweep that wraps);
        # the last one in position order is what the hot row holds
        last = torch.full((int(dest.max().item()) + 1 if dest.numel() else 1,), -1, dtype=torch.long,
                          device=self.dev)
        last.scatter_reduce_(0, dest, pos, reduce="amax")
        keep = last[dest] == pos
        bid, tok, slot = bid[keep], tok[keep], slot[keep]
        row = c.req_host_base[bid] + tok
        S, N = cfg.stripe_rows, cfg.node_num
        q = row // S
        win = torch.minimum(q * S + S - 1, torch.full_like(q, cfg.host_reqs * cfg.prefill - 1))
        src_rows = self.src[layer].index_select(0, win)
        dst_rows = self.hot[layer].index_select(0, slot + bid * self.padded)
        return bool(torch.equal(src_rows, dst_rows)), int(miss.sum().item())

    def close(self):
        self.pool.destroy(close_ext=False)
