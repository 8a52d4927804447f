#!/usr/bin/env python3
"""Benchmark of the decode-time KV data plane on one MI355X.

A step is one decode step of the workload: for every layer, the SIEVE update
of that layer's hot-buffer state followed by the import of its miss rows from
the N host-pinned segments into the layer's hot buffer (for the reference
stream, one layer per step).  Inputs (topK batches) are generated beforehand
by running SIEVE over the same state and are resident in HBM; the state is
restored before the timed replay, which therefore repeats the same work.

Prints one JSON line.  ``value`` is miss rows imported per second through the
whole path (SIEVE + import) over the timed steps.  SIEVE us/layer, import
GB/s against the measured host-link peak, the prefill export rate, the
roofline of the dominant kernel and the CPU oracle's rate are reported beside.
"""
import argparse
import json
import os
import sys
import time

METRIC = "SIEVE µs/layer; miss-row gather GB/s (% of host-link peak); rows/sec"
HBM_PEAK_GBPS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=5)
    p.add_argument("--warmup", type=int, default=2)
    p.add_argument("--config", type=int, default=2, help="workload id (0-4), default 2 = DSA-decode scale")
    p.add_argument("--per-segment", action="store_true", help="N per-segment imports instead of the fused import")
    p.add_argument("--coherent", action="store_true", help="fine-grained (coherent) pinned segments")
    p.add_argument("--cpu-sample-s", type=float, default=12.0, help="seconds of CPU oracle work for the baseline")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--verify", action="store_true", help="check the last step's imported rows on the GPU")
    p.add_argument("--link-mib", type=int, default=256)
    p.add_argument("--no-graph", action="store_true",
                   help="skip the replay of the timed steps as captured HIP graphs")
    p.add_argument("--sieve-variant", type=int, default=-1,
                   help="force a SIEVE kernel variant (0-4, see include/kvx/kvx.h); -1 = chosen per shape")
    return p.parse_args()


def pct(xs, q):
    import numpy as np

    return float(np.percentile(np.asarray(xs), q)) if len(xs) else None


def measure_link_peak(runner, mib, log):
    """Best of hipMemcpyAsync H2D from pinned memory and a zero-copy streaming
    read from a host segment (16 B loads), both of `mib` MiB."""
    import torch
    from kv_offload_proto_amd.kvops_ext import _kvops

    n = mib << 20
    dst = torch.empty(n, dtype=torch.uint8, device=runner.dev)
    pinned = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    pinned.fill_(1)
    stream = torch.cuda.current_stream()
    res = {}
    best = 0.0
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        dst.copy_(pinned, non_blocking=True)
        e1.record(stream)
        torch.cuda.synchronize()
        best = max(best, n / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    res["memcpy_h2d_GBps"] = best
    seg = runner.seg_bases[0]
    seg_bytes = runner.pool.pool.segments[0].size_bytes
    m = min(n, seg_bytes // 16 * 16)
    best = 0.0
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        _kvops.stream_copy(dst.data_ptr(), seg, m, stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        best = max(best, m / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    res["zero_copy_read_GBps"] = best
    res["peak_GBps"] = max(res["memcpy_h2d_GBps"], res["zero_copy_read_GBps"])
    # HBM -> HBM copy of the same size with the same streaming kernel: the
    # known-size copy that calibrates FETCH_SIZE / WRITE_SIZE readings
    src = torch.empty(n, dtype=torch.uint8, device=runner.dev)
    src.fill_(3)
    best = 0.0
    for _ in range(5):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        _kvops.stream_copy(dst.data_ptr(), src.data_ptr(), n, stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        best = max(best, 2 * n / (e0.elapsed_time(e1) * 1e-3) / 1e9)
    res["hbm_copy_GBps"] = best
    del src
    log("[bench] host link: memcpy H2D {:.1f} GB/s, zero-copy read {:.1f} GB/s; HBM copy {:.0f} GB/s (read+write)".format(
        res["memcpy_h2d_GBps"], res["zero_copy_read_GBps"], res["hbm_copy_GBps"]))
    del dst, pinned
    return res


def sieve_bytes(cfg, padded, vis_stride, ht_size, dirty_reqs):
    """Algorithmic HBM bytes of one SIEVE launch: per request topk/slots/miss
    (9 B per position), 24 B of per-request scalars, the visited row in and
    out, and the tokens + table rows in, and out again when the request had a
    miss (the staging traffic of hisp_sieve_update.cpp:103-105,165-172)."""
    per_req = 9 * cfg.top_k + 24 + 2 * vis_stride + (padded * 4 + ht_size * 2)
    return cfg.req_num * per_req + dirty_reqs * (padded * 4 + ht_size * 2)


# Counter profiles committed for a workload: HBM bytes per dispatch, from
# FETCH_SIZE and WRITE_SIZE runs scaled by a known-size copy.
TRAFFIC_PROFILES = {"c2-dsa-decode": "profiles/pmc_traffic_dsa_decode.md"}


def load_traffic(workload):
    """{kernel: bytes per dispatch} from the workload's counter profile, or {}."""
    rel = TRAFFIC_PROFILES.get(workload)
    if rel is None:
        return {}, None
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), rel)
    if not os.path.exists(path):
        return {}, None
    out = {}
    for line in open(path):
        f = line.split()
        if len(f) == 3 and f[0] == "traffic_bytes":
            out[f[1]] = float(f[2])
    return out, rel


def graph_pass(runner, snap, warm, timed, fused, eager_ms, log):
    """Replay the timed layer-steps again from the same starting state, each
    decode step as one captured HIP graph (SIEVE update + fused import of all
    its layers), and check that the final state and hot rows equal the eager
    run's."""
    import torch
    from kv_offload_proto_amd.xds import DecodeStepGraph

    if not fused:
        return {"skipped": "per-segment imports are not captured"}
    c = runner.coord
    names = ("device_buffer_tokens", "device_buffer_visited", "device_buffer_ht", "sieve_hand")
    ref_state = [getattr(c, n).clone() for n in names]
    ref_outs = [c.top_k_device_slots.clone(), c.is_miss.clone()]
    hot_bytes = runner.hot.numel()
    ref_hot = runner.hot.clone() if torch.cuda.mem_get_info()[0] > 2 * hot_bytes + (8 << 30) else None
    runner.restore(snap)
    runner.hot.zero_()  # the eager run started from a zeroed hot buffer too
    for _, layer, topk_d, _, _ in warm:
        runner.sieve(layer, topk_d)
        runner.gather(layer, topk_d, fused=True)
    steps = {}
    for step, layer, topk_d, _, _ in timed:
        steps.setdefault(step, []).append((layer, topk_d))
    t0 = time.perf_counter()
    graphs = []
    for step in sorted(steps):
        layers = [l for l, _ in steps[step]]
        g = DecodeStepGraph(c, runner.pool, layers, [t for _, t in steps[step]], [runner.hot[l] for l in layers],
                            hot_req_stride_rows=runner.padded, block_dim=1, sieve_block_dim=runner.block_dim)
        g.capture()
        graphs.append(g)
    capture_s = time.perf_counter() - t0
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for g in graphs:
        g.replay(clear_status=False)
    e1.record(stream)
    torch.cuda.synchronize()
    graph_ms = e0.elapsed_time(e1)
    graphs[-1].wait()
    state_ok = all(torch.equal(a, getattr(c, n)) for a, n in zip(ref_state, names))
    outs_ok = torch.equal(ref_outs[0], c.top_k_device_slots) and torch.equal(ref_outs[1], c.is_miss)
    hot_ok = None if ref_hot is None else torch.equal(ref_hot, runner.hot)
    del ref_hot, ref_state
    # launch overhead alone: the same layer-steps with num_real = 0 (every
    # kernel launched, no row does work), eager calls against graph replays
    saved = c.num_real.clone()
    c.num_real.zero_()
    torch.cuda.synchronize()
    e0.record(stream)
    for _, layer, topk_d, _, _ in timed:
        runner.sieve(layer, topk_d)
        runner.gather(layer, topk_d, fused=True)
    e1.record(stream)
    torch.cuda.synchronize()
    idle_eager_ms = e0.elapsed_time(e1)
    e0.record(stream)
    for g in graphs:
        g.replay(clear_status=False)
    e1.record(stream)
    torch.cuda.synchronize()
    idle_graph_ms = e0.elapsed_time(e1)
    c.num_real.copy_(saved)
    torch.cuda.synchronize()
    n = len(timed)
    res = {"steps": len(graphs), "layer_steps": n, "capture_s": capture_s,
           "us_per_layer": graph_ms * 1e3 / n, "eager_us_per_layer": eager_ms * 1e3 / n,
           "speedup": eager_ms / graph_ms, "state_match": state_ok, "outputs_match": outs_ok, "hot_match": hot_ok,
           "launch_only_us_per_layer": {"eager": idle_eager_ms * 1e3 / n, "graph": idle_graph_ms * 1e3 / n,
                                        "graph_over_eager": idle_graph_ms / idle_eager_ms}}
    log("[bench] graph replay: {:.2f} us/layer vs eager {:.2f} us/layer ({} step graphs, capture {:.1f} s); "
        "state {} outputs {} hot rows {}; launches alone (num_real 0): graph {:.2f} vs eager {:.2f} us/layer".format(
            res["us_per_layer"], res["eager_us_per_layer"], len(graphs), capture_s, state_ok, outs_ok, hot_ok,
            idle_graph_ms * 1e3 / n, idle_eager_ms * 1e3 / n))
    return res


def sieve_pipelined(runner, snap, warm, timed, log):
    """SIEVE alone over the timed layer-steps, launched back to back from the
    same starting state with HIP events only around the whole sequence: the
    per-layer cost in a stream of launches, without an event pair per launch.
    The final state must equal the eager run's."""
    import torch

    c = runner.coord
    names = ("device_buffer_tokens", "device_buffer_visited", "device_buffer_ht", "sieve_hand")
    ref = [getattr(c, n).clone() for n in names]
    runner.restore(snap)
    for _, layer, topk_d, _, _ in warm:
        runner.sieve(layer, topk_d)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _, layer, topk_d, _, _ in timed:
        runner.sieve(layer, topk_d)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / len(timed)
    ok = all(torch.equal(a, getattr(c, n)) for a, n in zip(ref, names))
    log("[bench] SIEVE back to back: {:.2f} us/layer over {} launches; state equal to the eager run: {}".format(
        us, len(timed), ok))
    return {"us_per_layer": us, "launches": len(timed), "state_match": ok}


def export_rows_pass(runner, log, reps=3):
    """Decode-incremental export: one row per request per layer (the row a
    decode step would append; here the last prefill row, rewritten with the
    bytes it already holds), timed per layer with HIP events, then checked in
    the host segments."""
    import numpy as np
    import torch

    cfg, pool = runner.cfg, runner.pool
    R = cfg.req_num
    rows = [cfg.host_base(r) + cfg.prefill - 1 for r in range(R)]
    rows_d = torch.tensor(rows, dtype=torch.int64, device=runner.dev)
    nr = torch.tensor([R], dtype=torch.int32, device=runner.dev)
    srcs = [runner.src[l].index_select(0, rows_d).contiguous() for l in range(cfg.layers)]
    stream = torch.cuda.current_stream()
    timing = {}
    for name, export in (("per_segment", pool.batch_export_rows), ("fused", pool.batch_export_rows_fused)):
        us = []
        st = None
        for _ in range(reps):
            for l in range(cfg.layers):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                st = export(l, srcs[l], rows_d, nr, R, stream=stream.cuda_stream)
                e1.record(stream)
                us.append((e0, e1))
            pool.wait(st)
        torch.cuda.synchronize()
        timing[name] = [a.elapsed_time(b) * 1e3 for a, b in us]
    views = pool.segment_views()
    S, N = max(cfg.stripe_rows, 1), cfg.node_num
    ok = True
    for l in (0, cfg.layers // 2, cfg.layers - 1):
        want = srcs[l].cpu().numpy()
        for r, row in enumerate(rows):
            node, seg_row = (row // S) % N, (row // S) // N
            ok = ok and bool(np.array_equal(views[node][l, seg_row], want[r]))
    med, med_seg = pct(timing["fused"], 50), pct(timing["per_segment"], 50)
    log("[bench] export_rows: {} rows per layer over {} segments, {:.1f} us/layer median fused ({:.1f} per segment); "
        "segments hold the rows: {}".format(R, N, med, med_seg, ok))
    return {"rows_per_layer": R, "segments": N, "us_per_layer_median": med, "us_per_layer_p99": pct(timing["fused"], 99),
            "per_segment_us_per_layer_median": med_seg, "GBps": R * cfg.row_bytes / (med * 1e-6) / 1e9, "match": ok}


def cpu_baseline(runner, plan, n_warm, budget_s, log):
    """The C oracle (oracle/liboracle.so) replaying the same batches from the
    same initial state on one host core: the warmup layer-steps untimed
    (SIEVE only, to reach the state the timed steps start from), then SIEVE +
    import over the timed layer-steps for about budget_s."""
    import numpy as np
    import torch
    from oracle import oracle as orc

    cfg = runner.cfg
    st = orc.SieveState(cfg.layers, cfg.req_num, cfg.dbs, cfg.top_k)
    c = runner.coord
    st.tokens[:] = c.device_buffer_tokens.cpu().numpy()
    st.vis[:] = c.device_buffer_visited.cpu().numpy()
    st.ht[:] = c.device_buffer_ht.cpu().numpy().view(np.uint16)
    st.hand[:] = c.sieve_hand.cpu().numpy()
    st.prefill_lens[:] = c.prefill_lens.cpu().numpy()
    segs = [sg.view() for sg in runner.pool.pool.segments]
    hot = np.zeros(cfg.req_num * runner.padded * cfg.row_bytes, dtype=np.uint8)
    req_pool = np.arange(cfg.req_num, dtype=np.int64)
    seq = np.full(cfg.req_num, cfg.prefill, dtype=np.int32)
    host_base = np.array([cfg.host_base(r) for r in range(cfg.req_num)], dtype=np.int64)
    plsr = runner.pool.per_layer_seg_rows
    t_sieve = t_gather = 0.0
    rows = done = 0
    sieve_mismatch = 0
    for step, layer, _, batch, gpu_misses in plan[:n_warm]:
        st.update(layer, batch, req_pool, seq, cfg.req_num)
    # a short stream is replayed from the same state until the budget is
    # spent (at most 1000 passes), so small workloads are timed over more
    # than a few microseconds of work
    start = [a.copy() for a in (st.tokens, st.vis, st.ht, st.hand)]
    timed_plan = plan[n_warm:]
    passes = 0
    while passes < 1000 and (passes == 0 or t_sieve + t_gather < budget_s):
        if passes > 0:
            for dst, src in zip((st.tokens, st.vis, st.ht, st.hand), start):
                np.copyto(dst, src)
        passes += 1
        for step, layer, _, batch, gpu_misses in timed_plan:
            t0 = time.perf_counter()
            slots, miss = st.update(layer, batch, req_pool, seq, cfg.req_num)
            t1 = time.perf_counter()
            for s in range(cfg.node_num):
                orc.gather_rows(segs, hot, layer * plsr, cfg.row_bytes, batch, req_pool, host_base, slots, miss,
                                cfg.req_num, cfg.top_k, cfg.req_num, cfg.stripe_rows, cfg.node_num, s,
                                hot_req_stride_rows=runner.padded)
            t2 = time.perf_counter()
            t_sieve += t1 - t0
            t_gather += t2 - t1
            n = int(miss.sum())
            sieve_mismatch += int(n != gpu_misses)
            rows += n
            done += 1
            if t_sieve + t_gather >= budget_s:
                break
    total = t_sieve + t_gather
    log("[bench] cpu oracle: {} layer-steps ({} passes) in {:.1f} s, {:.0f} rows/s, sieve {:.0f} us/layer".format(
        done, passes, total, rows / total, t_sieve / done * 1e6))
    return {
        "value": rows / total,
        "unit": "rows/s",
        "cores": 1,
        "kind": "port",
        "sample": "{} timed layer-steps of the benchmark stream ({} passes over its first {}; {} miss rows), oracle "
                  "SIEVE + import, 1 thread".format(done, passes, min(done, len(timed_plan)), rows),
        "sieve_us_per_layer": t_sieve / done * 1e6,
        "gather_GBps": rows * cfg.row_bytes / t_gather / 1e9 if t_gather > 0 else None,
        "miss_count_mismatches": sieve_mismatch,
        "cpu": _cpu_model(),
    }


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def main():
    args = parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this data plane runs on a single MI355X here "
              "(--gpus {} is not supported; run with --gpus 1)".format(args.gpus), file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    import numpy as np
    import torch

    import kv_offload_proto_amd  # noqa: F401  (loads the native module)
    from kv_offload_proto_amd.xds.configs import CONFIGS
    from kv_offload_proto_amd.xds.workload import DecodeRunner

    def log(msg):
        print(msg, file=sys.stderr, flush=True)

    if not torch.cuda.is_available():
        log("[bench] no GPU visible")
        return 1
    cfg = CONFIGS[args.config]
    t_start = time.perf_counter()
    runner = DecodeRunner(cfg, coherent=args.coherent, log=log)
    if args.sieve_variant >= 0:
        from kv_offload_proto_amd.kvops_ext import _kvops
        _kvops.sieve_force_variant(args.sieve_variant)
    log("[bench] {}: setup {:.1f} s (HBM pool + {} pinned segments of {:.2f} GiB)".format(
        cfg.name, runner.setup_s, cfg.node_num, runner.pool.pool.segments[0].size_bytes / 2**30))
    export_us = runner.export_prefill()
    export_gbps = runner.export_moved_bytes / (export_us * 1e-6) / 1e9
    log("[bench] prefill export: {} rows x {} layers ({} B of rows, {} B moved) in {:.1f} us ({:.1f} GB/s moved)".format(
        cfg.host_reqs * cfg.prefill, cfg.layers, runner.export_bytes, runner.export_moved_bytes, export_us,
        export_gbps))
    runner.admit_all()
    link = measure_link_peak(runner, args.link_mib, log)

    n_steps = args.warmup + args.steps
    t0 = time.perf_counter()
    plan, snap = runner.generate(n_steps)
    log("[bench] generated {} layer-steps in {:.1f} s".format(len(plan), time.perf_counter() - t0))
    per_step = len(plan) // n_steps if cfg.stream != "ref" else 1
    warm, timed = plan[: args.warmup * per_step], plan[args.warmup * per_step:]

    fused = not args.per_segment
    stream = torch.cuda.current_stream()
    for _, layer, topk_d, _, _ in warm:
        runner.sieve(layer, topk_d)
        runner.gather(layer, topk_d, fused=fused)
    torch.cuda.synchronize()

    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in timed]
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for (a, b, c), (_, layer, topk_d, _, _) in zip(ev, timed):
        a.record(stream)
        runner.sieve(layer, topk_d)
        b.record(stream)
        runner.gather(layer, topk_d, fused=fused)
        c.record(stream)
    end.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    sieve_us = [a.elapsed_time(b) * 1e3 for a, b, _ in ev]
    gather_us = [b.elapsed_time(c) * 1e3 for _, b, c in ev]
    rows = sum(m for *_, m in timed)
    ok, checked = (None, 0)
    if args.verify and timed:
        ok, checked = runner.verify_last_gather(timed[-1][1], timed[-1][2])
        log("[bench] verify last step: {} ({} rows)".format(ok, checked))

    # roofline of the dominant kernel
    c = runner.coord
    positions = cfg.req_num * cfg.top_k
    gather_bytes = [m * cfg.row_bytes * 2 + positions * 9 for *_, m in timed]
    gather_gbps_alg = sum(gather_bytes) / (sum(gather_us) * 1e-6) / 1e9
    link_gbps = rows * cfg.row_bytes / (sum(gather_us) * 1e-6) / 1e9
    sb = sieve_bytes(cfg, c.padded_buffer_size, c.visited_stride_b, c.ht_size, cfg.req_num)
    sieve_gbps_alg = sb * len(timed) / (sum(sieve_us) * 1e-6) / 1e9
    traffic, traffic_src = load_traffic(cfg.name)

    def traffic_of(*prefixes):
        """Summed bytes per dispatch of the profiled kernels named by each
        prefix (a template kernel is listed with its arguments), or None."""
        total = 0.0
        for pre in prefixes:
            hits = [v for k, v in traffic.items() if k == pre or k.startswith(pre + "<")]
            if not hits:
                return None
            total += sum(hits)
        return total

    gather_kernels = ("kvx_gather_prep", "kvx_gather_list", "kvx_gather_copy")
    gather_roof = {"kernel": "+".join(gather_kernels), "bound": "hbm", "achieved": gather_gbps_alg,
                   "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": gather_gbps_alg / HBM_PEAK_GBPS,
                   "traffic": traffic_of(*gather_kernels), "traffic_source": traffic_src,
                   "bytes_per_launch": sum(gather_bytes) / len(timed),
                   "avg_launch_us": sum(gather_us) / len(timed),
                   "link": {"achieved": link_gbps, "peak": link["peak_GBps"], "unit": "GB/s",
                            "frac": link_gbps / link["peak_GBps"]}}
    sieve_roof = {"kernel": "kvx_sieve_update", "bound": "hbm", "achieved": sieve_gbps_alg, "peak": HBM_PEAK_GBPS,
                  "unit": "GB/s", "frac": sieve_gbps_alg / HBM_PEAK_GBPS,
                  "traffic": traffic_of("kvx_sieve_update_fast"), "traffic_source": traffic_src, "bytes_per_launch": sb,
                  "avg_launch_us": sum(sieve_us) / len(timed)}
    dominant, other = (gather_roof, sieve_roof) if sum(gather_us) >= sum(sieve_us) else (sieve_roof, gather_roof)

    n_timed_steps = args.steps
    value = rows / (total_ms * 1e-3)
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": n_timed_steps,
        "warmup": args.warmup,
        "ms_per_step": total_ms / n_timed_steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic (seeded topK streams, fp16 rows uniform in [-1,1))",
        "config": {"workload": cfg.name, "req_num": cfg.req_num, "prefill": cfg.prefill, "top_k": cfg.top_k,
                   "device_buffer_size": cfg.dbs, "miss_ratio": cfg.miss_ratio, "layers": cfg.layers,
                   "node_num": cfg.node_num, "stripe_rows": cfg.stripe_rows, "row_bytes": cfg.row_bytes,
                   "stream": cfg.stream, "zipf_s": cfg.zipf_s, "import": "fused" if fused else "per-segment",
                   "segments": "coherent" if args.coherent else "non-coherent"},
        "sieve_us_per_layer": {"median": pct(sieve_us, 50), "p99": pct(sieve_us, 99),
                               "mean": sum(sieve_us) / len(sieve_us)},
        "gather": {"us_per_layer_median": pct(gather_us, 50), "GBps": link_gbps,
                   "frac_of_link_peak": link_gbps / link["peak_GBps"], "frac_of_hbm_peak": link_gbps / HBM_PEAK_GBPS,
                   "rows_per_s": rows / (sum(gather_us) * 1e-6), "rows": rows},
        "host_link": link,
        "export": {"row_bytes_total": runner.export_bytes, "bytes_moved": runner.export_moved_bytes,
                   "us": export_us, "GBps_moved": export_gbps},
        "roofline": dominant,
        "roofline_other": other,
        "verify": ok,
    }
    out["sieve_back_to_back"] = sieve_pipelined(runner, snap, warm, timed, log)
    out["graph"] = None if args.no_graph else graph_pass(runner, snap, warm, timed, fused, total_ms, log)
    out["export_rows"] = export_rows_pass(runner, log)
    if not args.no_cpu:
        runner.restore(snap)
        out["cpu_baseline"] = cpu_baseline(runner, plan, len(warm), args.cpu_sample_s, log)
    else:
        out["cpu_baseline"] = None
    out["wall_s"] = time.perf_counter() - t_start
    runner.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
