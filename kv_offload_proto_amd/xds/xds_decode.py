"""Decode pipeline driver on one MI355X: prefill export, admission, then decode
steps of SIEVE update + miss import, each checked byte for byte.

The counterpart of the reference's driver (xds/xds_decode.py:21-289): the same
flags, the same row fingerprint, the same acceptance log lines
(README.md:82-89) and the same ``--oracle`` per-step check of slots and
is_miss against a CPU SIEVE model.  The EMS pool is replaced by N pinned host
segments (``--node-num``); ``--ems-master``, ``--rootinfo`` and ``--fatbin``
are accepted and have no effect.

Run: ``python -m kv_offload_proto_amd.xds.xds_decode [options]``.

Differences from the reference driver, each on purpose:

* host bases come from the pool's row allocator (first fit), with the
  contiguity assert of the reference (xds_decode.py:172-176); at the end every
  request's rows go back to the allocator and the driver asserts that none is
  left in use;
* the hot buffer is a tensor of its own, ``[layers, req_num * hot_stride,
  row_bytes]``, and request b's slot s of a layer is row ``b * hot_stride +
  s`` (``--hot-stride``, default the padded buffer size, so that requests do
  not overwrite each other; ``--hot-stride 0`` is the reference's fixed
  offset ``hotRowBase + slot`` shared by every request);
* the check after each step covers every byte of the layer's hot buffer: each
  row holds the fingerprint of the host row that the last miss position
  naming it in this or an earlier step imported (with S > 1, the stripe's
  exported row), and rows never imported are zero;
* the ``--oracle`` model keeps one state per (layer, request), as the kernel
  does (the reference's model keeps one per request, xds_decode.py:66-84, so
  it only agrees with the kernel while every step uses the same layer);
* ``--layer-rows`` defaults to ``req_num * prefill`` (the reference's default
  of 1024 rows cannot hold its own default batch of 8 x 256 rows);
* ``--stream state`` draws each step's topK from the current SIEVE state
  (resident tokens with a Zipf recency bias for hits, non-resident ones for
  misses) instead of the reference's stream (``ref``, the default, which
  reproduces the reference's numpy call order from the same seed).
"""
import argparse
import os
import sys
import time

import numpy as np

# row fingerprint constants (xds_decode.py:18)
P1, P2, M1, M2 = 0x9E3779B1, 0x85EBCA77, 0x27220A95, 0x165667B1


def parse_args(argv=None):
    p = argparse.ArgumentParser(description="decode pipeline driver (MI355X KV data plane)")
    p.add_argument("--ems-master", default="local", help="accepted for compatibility; segments are local")
    p.add_argument("--device", type=int, default=0)
    p.add_argument("--rootinfo", default="/etc/hccl_rootinfo.json", help="accepted for compatibility")
    p.add_argument("--fatbin", default="", help="accepted for compatibility (kernels are linked in)")
    p.add_argument("--layers", type=int, default=2)
    p.add_argument("--layer-rows", type=int, default=0, help="rows per layer (default req_num * prefill)")
    p.add_argument("--kv-lora-rank", type=int, default=512)
    p.add_argument("--qk-rope", type=int, default=64)
    p.add_argument("--stripe-rows", type=int, default=1)
    p.add_argument("--node-num", type=int, default=2, help="host segments (the reference's resource nodes)")
    p.add_argument("--req-num", type=int, default=8)
    p.add_argument("--prefill", type=int, default=256)
    p.add_argument("--topk", type=int, default=64)
    p.add_argument("--device-buffer-size", type=int, default=64)
    p.add_argument("--miss-ratio", type=float, default=0.5)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--seed", type=int, default=42)
    p.add_argument("--block-dim", type=int, default=8)
    p.add_argument("--oracle", action="store_true", help="check slots and is_miss against the CPU model every step")
    p.add_argument("--run-dir", default="./log", help="log directory (xds_decode.log is rewritten each run)")
    p.add_argument("--hot-stride", type=int, default=-1,
                   help="hot rows per request (-1 = padded buffer size, 0 = one shared slice)")
    p.add_argument("--stream", choices=("ref", "state"), default="ref")
    p.add_argument("--zipf", type=float, default=1.1, help="recency bias of hits for --stream state")
    p.add_argument("--fill", choices=("fingerprint", "fp16"), default="fingerprint")
    p.add_argument("--fused", action="store_true", help="one import launch for all segments per step")
    p.add_argument("--no-check", action="store_true", help="skip the hot-buffer check")
    return p.parse_args(argv)


class Log:
    def __init__(self, run_dir):
        os.makedirs(run_dir, exist_ok=True)
        self.path = os.path.join(run_dir, "xds_decode.log")
        self._f = open(self.path, "w", encoding="utf-8")

    def __call__(self, msg):
        print(msg, flush=True)
        self._f.write(msg + "\n")
        self._f.flush()

    def close(self):
        self._f.close()


def fingerprint_rows(torch, rows, layer, words):
    """int32 [len(rows), words]: 32-bit word k of row r in layer l is
    ((r*P1 + l*P2)*M1 ^ M2) + k*M1 mod 2^32 (xds_decode.py:60-63); a row of
    row_bytes holds row_bytes/4 such words."""
    mask = 0xFFFFFFFF
    a = (rows.to(torch.int64) * P1 + layer * P2) & mask
    v = ((a * M1) & mask) ^ M2
    k = torch.arange(words, dtype=torch.int64, device=rows.device) * M1
    w = (v[:, None] + k[None, :]) & mask
    w = torch.where(w >= (1 << 31), w - (1 << 32), w)
    return w.to(torch.int32)


class CpuSieve:
    """CPU model of one request's SIEVE state for the --oracle check: slot ->
    token array, visited flags, the hand and a token -> slot map; ``update``
    maps a topK row to (slots, is_miss) by the rules of
    kvops/kernel/hisp_sieve_update.cpp:115-160 (invalid positions -1/0,
    decode-extension positions padded + offset, hits set visited, misses
    take the first unvisited slot from the hand, clearing visited flags on
    the way, and evict its token)."""

    def __init__(self, prefill, dbs, padded):
        n = min(prefill, dbs)
        self.prefill, self.dbs, self.padded = prefill, dbs, padded
        self.tok = np.full(dbs, -1, dtype=np.int64)
        self.tok[:n] = np.arange(n)
        self.vis = np.zeros(dbs, dtype=bool)
        self.hand = 0
        self.where = {t: s for s, t in enumerate(range(n))}

    def update(self, row, seq_len):
        slots = np.empty(len(row), dtype=np.int32)
        miss = np.zeros(len(row), dtype=np.int8)
        for k, t in enumerate(int(x) for x in row):
            if t < 0 or t >= seq_len:
                slots[k] = -1
            elif t >= self.prefill:
                slots[k] = self.padded + (t - self.prefill)
            elif t in self.where:
                s = self.where[t]
                self.vis[s] = True
                slots[k] = s
            else:
                h = self.hand
                while self.vis[h]:
                    self.vis[h] = False
                    h = h + 1 if h + 1 < self.dbs else 0
                old = int(self.tok[h])
                if old >= 0:
                    del self.where[old]
                self.tok[h] = t
                self.where[t] = h
                self.vis[h] = True
                self.hand = h + 1 if h + 1 < self.dbs else 0
                slots[k] = h
                miss[k] = 1
        return slots, miss


def main(argv=None):
    args = parse_args(argv)
    log = Log(args.run_dir)
    try:
        return _run(args, log)
    finally:
        log.close()


def _run(args, log):
    import torch

    if not torch.cuda.is_available():
        log("[xds][ERROR] no GPU visible")
        return 1
    from ..kvops_ext import _kvops
    from . import streams
    from .xds_offload import XdsOffloadCoordinator
    from .xds_seg_pool import HostSegPool

    rng = np.random.default_rng(args.seed)
    row_words = args.kv_lora_rank + args.qk_rope
    row_bytes = -(-(row_words * 2) // 128) * 128
    R, prefill, dbs, top_k, L = args.req_num, args.prefill, args.device_buffer_size, args.topk, args.layers
    layer_rows = args.layer_rows if args.layer_rows > 0 else R * prefill
    if dbs >= prefill:
        log("[xds][WARN] device-buffer-size >= prefill: no misses, --miss-ratio has no effect")
    dev = torch.device("cuda", args.device)
    torch.cuda.set_device(dev)
    log("[xds] config: layers={} layerRows={} rowWords={} rowBytes={} stripe={} reqs={} prefill={} topK={} dbs={} "
        "missRatio={}".format(L, layer_rows, row_words, row_bytes, args.stripe_rows, R, prefill, top_k, dbs,
                              args.miss_ratio))

    pool = HostSegPool(args.device, L, layer_rows, row_bytes, stripe_rows=args.stripe_rows, node_num=args.node_num)
    pool.create_pool(fatbin_path=args.fatbin)
    try:
        log("[xds] pool ready: nodes={} perLayerSegRows={} channels={} fatbin={}".format(
            pool.node_num, pool.per_layer_seg_rows, len(pool.channels), args.fatbin or "(linked)"))
        coord = XdsOffloadCoordinator(dev, L, R, dbs, top_k, R, prefill)
        padded = coord.padded_buffer_size
        log("[xds] coordinator: padded={} visitedStrideB={} htSize={}".format(
            padded, coord.visited_stride_b, coord.ht_size))
        stride = padded if args.hot_stride < 0 else args.hot_stride
        hot_rows = (R - 1) * stride + padded if stride > 0 else padded

        # prefill: rows from the allocator (contiguity contract), fill, export
        allocator = pool.make_allocator()
        host_bases, held = [], []
        for r in range(R):
            rows = allocator.alloc(prefill)
            if rows != list(range(rows[0], rows[0] + prefill)):
                log("[xds][ERROR] row allocation broke the contiguity contract for request {}".format(r))
                return 1
            host_bases.append(rows[0])
            held.append(rows)
        lo, hi = min(host_bases), max(host_bases) + prefill
        src = torch.zeros((L, layer_rows, row_bytes), dtype=torch.uint8, device=dev)
        if args.fill == "fingerprint":
            ids = torch.arange(lo, hi, dtype=torch.int64, device=dev)
            for l in range(L):
                src[l, lo:hi].view(torch.int32)[:] = fingerprint_rows(torch, ids, l, row_bytes // 4)
        else:
            g = torch.Generator(device=dev)
            g.manual_seed(args.seed)
            for l in range(L):
                src[l, lo:hi, :row_words * 2].view(torch.float16).uniform_(-1.0, 1.0, generator=g)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        st = pool.batch_write_alllayers(lo, hi - lo, src, layer_rows * row_bytes)
        pool.wait(st)
        t_export = time.perf_counter() - t0
        log("[xds] prefill export: {} rows x {} layers = {} B in {:.1f} us".format(
            hi - lo, L, L * (hi - lo) * row_bytes, t_export * 1e6))

        # admission (identity layout + table build of every layer)
        # one model per (layer, request): every layer keeps its own SIEVE state
        model = [[CpuSieve(prefill, dbs, padded) for _ in range(R)] for _ in range(L)] if args.oracle else None
        for r in range(R):
            coord.admit_request(r, r, prefill, host_bases[r])
        req_pool = torch.arange(R, dtype=torch.int64, device=dev)
        seq_lens = torch.full((R,), prefill, dtype=torch.int32, device=dev)
        coord.set_batch(req_pool, seq_lens)
        hot = torch.zeros((L, hot_rows, row_bytes), dtype=torch.uint8, device=dev)
        # host row each hot row must hold (-1: never imported, so zero)
        expect = torch.full((L, hot_rows), -1, dtype=torch.int64, device=dev)
        bases = torch.tensor(host_bases, dtype=torch.int64, device=dev)
        S = max(args.stripe_rows, 1)
        if args.fill == "fp16":
            ref_rows = src  # kept for the check
        else:
            del src
            ref_rows = None
        torch.cuda.synchronize()

        total_miss, t_total = 0, 0.0
        for step in range(args.steps):
            layer = step % L
            if args.stream == "ref":
                batch = streams.ref_batch(rng, R, top_k, prefill, dbs, args.miss_ratio)
            else:
                toks = coord.device_buffer_tokens[layer, :, :dbs].cpu().numpy()
                batch = streams.state_batch(rng, toks, prefill, top_k, args.miss_ratio, zipf_s=args.zipf)
            topk_d = torch.from_numpy(batch).to(dev)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            coord.sieve_update(layer, topk_d, block_dim=args.block_dim)
            read = pool.batch_read_fused if args.fused else pool.batch_read
            bd = min(args.block_dim, 8)
            st = read(layer, topk_d, req_pool, coord.req_host_base, coord.top_k_device_slots, coord.is_miss,
                      coord.num_real, hot[layer], R, top_k, block_dim=bd, hot_req_stride_rows=stride)
            pool.wait(st, block_dim=bd)
            dt = time.perf_counter() - t0
            t_total += dt
            miss_cnt = int(coord.miss_count().item())
            total_miss += miss_cnt

            if model is not None:
                g_slots = coord.top_k_device_slots.cpu().numpy()
                g_miss = coord.is_miss.cpu().numpy()
                for r in range(R):
                    e_slots, e_miss = model[layer][r].update(batch[r], prefill)
                    if not np.array_equal(g_miss[r], e_miss):
                        log("[xds][ERROR] oracle is_miss mismatch step={} req={}\n gpu={}\n exp={}".format(
                            step, r, g_miss[r].tolist(), e_miss.tolist()))
                        return 1
                    if not np.array_equal(g_slots[r], e_slots):
                        log("[xds][ERROR] oracle slots mismatch step={} req={}\n gpu={}\n exp={}".format(
                            step, r, g_slots[r].tolist(), e_slots.tolist()))
                        return 1

            checked = 0
            if not args.no_check:
                checked = _check_hot(torch, coord, topk_d, hot[layer], expect[layer], bases, stride, S,
                                     hi, layer, ref_rows)
                if checked < 0:
                    bad = -checked - 1
                    log("[xds][ERROR] verify failed step={} layer={} hot row {}: bytes differ from host row {}".format(
                        step, layer, bad, int(expect[layer, bad].item())))
                    return 1
            log("[xds] step {}: layer={} miss={} rows in {:.1f} us (checked={})".format(
                step, layer, miss_cnt, dt * 1e6, checked))

        if total_miss > 0:
            bw = total_miss * row_bytes / t_total / 1e9 if t_total > 0 else 0.0
            log("[xds] summary: imported {} miss rows, avg {:.1f} us/row, aggregate {:.2f} GB/s".format(
                total_miss, t_total * 1e6 / total_miss, bw))
        else:
            log("[xds] summary: no miss rows imported")
        for rows in held:
            allocator.free(rows)
        if allocator.used_rows() != 0:
            log("[xds][ERROR] row allocator leaked {} rows".format(allocator.used_rows()))
            return 1
        if _kvops.read_overflow() != 0:
            log("[xds][ERROR] a kernel stopped a runaway probe or sweep (tail slot {:#x})".format(
                _kvops.read_overflow()))
            return 1
    finally:
        pool.destroy()
    log("[xds] all done, log: {}".format(log.path))
    return 0


def _check_hot(torch, coord, topk_d, hot_l, expect_l, bases, stride, S, row_hi, layer, ref_rows):
    """Update the expected host row of each hot row of the layer from this
    step's outputs (the last valid miss position naming a hot row wins) and
    compare every byte.  Returns the number of rows imported this step, or
    -(row + 1) for the first hot row that differs."""
    top_k = topk_d.shape[1]
    miss = coord.is_miss.bool()
    slots = coord.top_k_device_slots
    valid = miss & (topk_d >= 0) & (slots >= 0)
    pos = torch.nonzero(valid.reshape(-1)).reshape(-1)
    n = 0
    if pos.numel():
        bid = pos // top_k
        tok = topk_d.reshape(-1)[pos].to(torch.int64)
        dest = slots.reshape(-1)[pos].to(torch.int64) + bid * stride
        last = torch.full((expect_l.shape[0],), -1, dtype=torch.int64, device=hot_l.device)
        last.scatter_reduce_(0, dest, pos, reduce="amax")
        keep = last[dest] == pos
        row = (bases[bid[keep]] + tok[keep]) & 0xFFFFFFFF
        # with S > 1 a stripe's rows share one segment row, which holds the
        # stripe's last exported row
        q = row // S
        row = torch.minimum(q * S + S - 1, torch.full_like(q, row_hi - 1)) if S > 1 else row
        expect_l[dest[keep]] = row
        n = int(keep.sum().item())
    have = expect_l >= 0
    want = torch.zeros_like(hot_l)
    if bool(have.any()):
        idx = torch.nonzero(have).reshape(-1)
        if ref_rows is None:
            words = fingerprint_rows(torch, expect_l[idx], layer, hot_l.shape[1] // 4)
            want[idx] = words.view(torch.uint8).reshape(idx.numel(), hot_l.shape[1])
        else:
            want[idx] = ref_rows[layer].index_select(0, expect_l[idx])
    diff = (hot_l != want).any(dim=1)
    if bool(diff.any()):
        return -(int(torch.nonzero(diff)[0].item()) + 1)
    return n


if __name__ == "__main__":
    sys.exit(main())
