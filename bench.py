#!/usr/bin/env python3
"""Benchmark of the decode-time KV data plane on one MI355X.

A step is one decode step of the workload: for every layer, the SIEVE update
of that layer's hot-buffer state followed by the import of its miss rows from
the N host-pinned segments into the layer's hot buffer (for the reference
stream, one layer per step).  Inputs (topK batches) are generated beforehand
by running SIEVE over the same state and are resident in HBM; the state is
restored before the timed replay, which therefore repeats the same work.

Prints one JSON line.  ``value`` is miss rows imported per second through the
whole path (SIEVE + import) over the timed steps.  Beside it: SIEVE us/layer,
the import's rate against the measured host-link peak (its bound) and against
HBM, the prefill export rate, the decode-step graph replay and its launch
overhead, the CPU baseline (the oracle on 1 thread and on all cores, and the
CPU serial pipeline for the import), and ``verify``: every layer's final
SIEVE state and hot buffer compared with an independent oracle replay of all
the layer-steps.
"""
import argparse
import json
import os
import sys
import time
from concurrent.futures import ThreadPoolExecutor

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
    p.add_argument("--cpu-sample-s", type=float, default=12.0, help="seconds of CPU work for the baseline")
    p.add_argument("--cpu-threads", type=int, default=16, help="threads of the all-cores CPU baseline")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-verify", action="store_true", help="skip the oracle replay of the timed run")
    p.add_argument("--link-mib", type=int, default=256)
    p.add_argument("--no-graph", action="store_true",
                   help="skip the replay of the timed steps as captured HIP graphs")
    p.add_argument("--sieve-variant", type=int, default=-1,
                   help="force a SIEVE kernel variant (0-6, see include/kvx/kvx.h); -1 = chosen per shape")
    p.add_argument("--loop-only", action="store_true",
                   help="only the decode loop (no extra passes, no CPU baseline): for counter profiles")
    return p.parse_args()


class FenceFreeEvents:
    """HIP timing events created with hipEventDisableSystemFence (0x20000000).

    Recording a torch.cuda.Event releases to system scope, which writes the
    GPU caches back to memory; around a 20 us kernel that adds about 1.8 us
    to the bracketed time (device-scope release events cost the same here:
    the XCDs' L2 caches are written back either way).  These events record
    without a release, so the bracket holds the launch gap and the kernel.
    They bind the HIP runtime torch loaded (RTLD_NOLOAD), never a second one.
    """

    FLAGS = 0x20000000

    def __init__(self):
        import ctypes

        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD)
        self.made = []

    def event(self):
        e = self.ct.c_void_p()
        rc = self.hip.hipEventCreateWithFlags(self.ct.byref(e), self.ct.c_uint(self.FLAGS))
        if rc != 0:
            raise RuntimeError("hipEventCreateWithFlags failed: {}".format(rc))
        self.made.append(e)
        return e

    def record(self, e, stream):
        rc = self.hip.hipEventRecord(e, self.ct.c_void_p(stream.cuda_stream))
        if rc != 0:
            raise RuntimeError("hipEventRecord failed: {}".format(rc))

    def elapsed_ms(self, a, b):
        ms = self.ct.c_float()
        rc = self.hip.hipEventElapsedTime(self.ct.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError("hipEventElapsedTime failed: {}".format(rc))
        return ms.value

    def close(self):
        for e in self.made:
            self.hip.hipEventDestroy(e)
        self.made = []


def head_start():
    """Queue a GPU spin of about a millisecond before a timed region. After a
    synchronize the queue is empty, so without it the first timed launch also
    carries the host's submission latency (about 100 us measured); with it the
    host has queued the first launches before the GPU reaches them, as it has
    throughout a running decode loop. The spin precedes the region's first
    event and is not timed."""
    import torch

    torch.cuda._sleep(2_000_000)


def pct(xs, q):
    import numpy as np

    return float(np.percentile(np.asarray(xs), q)) if len(xs) else None


def cpu_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        usable = os.cpu_count()
    return {"model": model, "cpus_visible": os.cpu_count(), "cpus_usable": usable}


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

    def best_of(fn, nbytes):
        best = 0.0
        for _ in range(5):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            fn()
            e1.record(stream)
            torch.cuda.synchronize()
            best = max(best, nbytes / (e0.elapsed_time(e1) * 1e-3) / 1e9)
        return best

    res["memcpy_h2d_GBps"] = best_of(lambda: dst.copy_(pinned, non_blocking=True), n)
    seg = runner.seg_bases[0]
    m = min(n, runner.pool.pool.segments[0].size_bytes // 16 * 16)
    res["zero_copy_read_GBps"] = best_of(lambda: _kvops.stream_copy(dst.data_ptr(), seg, m, stream.cuda_stream), m)
    res["peak_GBps"] = max(res["memcpy_h2d_GBps"], res["zero_copy_read_GBps"])
    # HBM -> HBM copy with the same streaming kernel: the known-size copy that
    # calibrates FETCH_SIZE / WRITE_SIZE readings
    src = torch.empty(n, dtype=torch.uint8, device=runner.dev)
    src.fill_(3)
    res["hbm_copy_GBps"] = best_of(lambda: _kvops.stream_copy(dst.data_ptr(), src.data_ptr(), n, stream.cuda_stream),
                                   2 * n)
    del src, dst, pinned
    log("[bench] host link: memcpy H2D {:.1f} GB/s, zero-copy read {:.1f} GB/s; HBM copy {:.0f} GB/s (read+write)".format(
        res["memcpy_h2d_GBps"], res["zero_copy_read_GBps"], res["hbm_copy_GBps"]))
    return res


def sieve_bytes(cfg, padded, vis_stride, ht_size, dirty_reqs):
    """Algorithmic HBM bytes of one SIEVE launch: per request topk/slots/miss
    (9 B per position), 24 B of per-request scalars, the visited row in and
    out, and the tokens + table rows in, and out again when the request had a
    miss (the staging traffic of hisp_sieve_update.cpp:103-105,165-172)."""
    per_req = 9 * cfg.top_k + 24 + 2 * vis_stride + (padded * 4 + ht_size * 2)
    return cfg.req_num * per_req + dirty_reqs * (padded * 4 + ht_size * 2)


# Counter profiles committed per workload: HBM bytes per dispatch, from
# FETCH_SIZE and WRITE_SIZE runs scaled by a known-size copy.
TRAFFIC_PROFILES = {"c2-dsa-decode": "profiles/pmc_traffic_dsa_decode.md",
                    "c3-large-batch-export": "profiles/pmc_traffic_large_batch_export.md",
                    "c4-slot-limit-stress": "profiles/pmc_traffic_slot_limit_stress.md"}
# SIEVE kernel of each variant (kvx_last_sieve_variant), as named in the profiles
SIEVE_KERNELS = {0: ("kvx_sieve_update",), 1: ("kvx_sieve_update",), 2: ("kvx_sieve_update_fast",),
                 3: ("kvx_sieve_update_wave",), 4: ("kvx_sieve_update_fast",),
                 5: ("kvx_sieve_batch_pre", "kvx_sieve_batch_slots", "kvx_sieve_update_batch")}
# variant 5's table rebuild, when the step's launches include it
SIEVE_TABLE_KERNELS = ("kvx_sieve_table_cells", "kvx_sieve_table_final", "kvx_sieve_table_chunks")


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


# ---------------------------------------------------------------- oracle replays
def _layer_state(runner, snap, layer):
    """Oracle SieveState of one layer (a one-layer state) from the snapshot."""
    import numpy as np
    from oracle import oracle as orc

    cfg = runner.cfg
    st = orc.SieveState(1, cfg.req_num, cfg.dbs, cfg.top_k)
    st.tokens[0] = snap[0][layer].cpu().numpy()
    st.vis[0] = snap[1][layer].cpu().numpy()
    st.ht[0] = snap[2][layer].cpu().numpy().view(np.uint16)
    st.hand[0] = snap[3][layer].cpu().numpy()
    st.prefill_lens[:] = runner.coord.prefill_lens.cpu().numpy()
    return st


class _Batch:
    """Host-side batch context of the workload for oracle calls."""

    def __init__(self, runner):
        import numpy as np

        cfg = runner.cfg
        self.R = cfg.req_num
        self.req_pool = np.arange(cfg.req_num, dtype=np.int64)
        self.seq = np.full(cfg.req_num, cfg.prefill, dtype=np.int32)
        self.host_base = np.array(runner.host_bases, dtype=np.int64)
        self.segs = [sg.view() for sg in runner.pool.pool.segments]
        self.plsr = runner.pool.per_layer_seg_rows


def verify_against_oracle(runner, snap, plan, threads, log):
    """Replay every layer-step of `plan` (warmup and timed) on the oracle,
    layer by layer from the snapshot, SIEVE then the import of every segment
    into a zeroed hot buffer, and compare each layer's final SIEVE state
    (tokens, visited, table, hand) and every byte of its hot buffer with the
    GPU's after the timed run."""
    import numpy as np
    from oracle import oracle as orc

    cfg, c = runner.cfg, runner.coord
    b = _Batch(runner)
    final = [t.cpu().numpy() for t in (c.device_buffer_tokens, c.device_buffer_visited, c.device_buffer_ht,
                                       c.sieve_hand)]
    final[2] = final[2].view(np.uint16)
    by_layer = {}
    for ls in plan:
        by_layer.setdefault(ls.layer, []).append(ls)
    hot_bytes = runner.hot[0].numel()
    workers = max(1, min(threads, int((24 << 30) // (2 * hot_bytes))))
    # threads left over when there are fewer layers than threads go to the
    # requests of each layer-step (the slot-limit stress: 4 layers x 4 requests)
    inner = max(1, min(cfg.req_num, threads // max(1, min(workers, len(by_layer)))))

    def one(layer):
        st = _layer_state(runner, snap, layer)
        hot = np.zeros(hot_bytes, dtype=np.uint8)
        for ls in by_layer[layer]:
            slots, miss = st.update(0, ls.batch, b.req_pool, b.seq, b.R, threads=inner)
            for s in range(cfg.node_num):
                orc.gather_rows(b.segs, hot, layer * b.plsr, cfg.row_bytes, ls.batch, b.req_pool, b.host_base,
                                slots, miss, b.R, cfg.top_k, b.R, cfg.stripe_rows, cfg.node_num, s,
                                hot_req_stride_rows=runner.padded)
        state_ok = (np.array_equal(st.tokens[0], final[0][layer]) and np.array_equal(st.vis[0], final[1][layer])
                    and np.array_equal(st.ht[0], final[2][layer])
                    and np.array_equal(st.hand[0][:, 0], final[3][layer][:, 0]))
        hot_ok = bool(np.array_equal(hot, runner.hot[layer].cpu().numpy().reshape(-1)))
        return layer, state_ok, hot_ok

    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=workers) as ex:
        res = list(ex.map(one, sorted(by_layer)))
    bad_state = [l for l, s, _ in res if not s]
    bad_hot = [l for l, _, h in res if not h]
    ok = not bad_state and not bad_hot and orc.get_error() == 0
    log("[bench] verify: {} layers x {} layer-steps replayed on the oracle ({} threads, {:.1f} s): state {} hot rows "
        "{}".format(len(res), len(plan), workers, time.perf_counter() - t0, "equal" if not bad_state else bad_state,
                    "equal" if not bad_hot else bad_hot))
    return {"ok": ok, "layers": len(res), "layer_steps": len(plan), "state_mismatch_layers": bad_state,
            "hot_mismatch_layers": bad_hot,
            "what": "final SIEVE state and every hot-buffer byte of each layer vs the oracle's replay of all "
                    "layer-steps (SIEVE + import of every segment)"}


def cpu_baseline(runner, snap, plan, n_warm, budget_s, threads, log):
    """The oracle on the box's host cores over the same stream.

    * SIEVE: the layer-steps replayed in order on 1 thread, and layers spread
      over `threads` threads (the layers' states are independent), from the
      state the timed steps start from.
    * Import, as the CPU serial pipeline the reference design replaces
      (doc/kv_offload_design.md:21): the winning miss rows are copied on the
      host into a pinned staging buffer (1 thread, then `threads` threads),
      then one host-to-device copy and a device scatter into the hot buffer.
    ``value`` is the pipeline's rows/s on `threads` threads:
    misses / (SIEVE + staging + copy + scatter) per layer-step."""
    import numpy as np
    import torch
    from oracle import oracle as orc

    cfg = runner.cfg
    b = _Batch(runner)
    layers = sorted({ls.layer for ls in plan})
    states = {l: _layer_state(runner, snap, l) for l in layers}
    for ls in plan[:n_warm]:  # the state the timed steps start from (untimed)
        states[ls.layer].update(0, ls.batch, b.req_pool, b.seq, b.R)
    timed = plan[n_warm:]
    start = {l: st.copy() for l, st in states.items()}

    # SIEVE on one thread, in order, for about a third of the budget
    outs = []
    t_one = 0.0
    for ls in timed:
        t0 = time.perf_counter()
        slots, miss = states[ls.layer].update(0, ls.batch, b.req_pool, b.seq, b.R)
        t_one += time.perf_counter() - t0
        outs.append((ls, slots, miss))
        if t_one >= budget_s / 3:
            break
    n_one = len(outs)
    sieve_us_1 = t_one / n_one * 1e6

    # SIEVE on `threads` threads: layers spread over the threads, each layer's
    # timed steps in order; as many layers as keep it near a third of the budget
    per_layer = max(1, len(timed) // max(1, len(layers)))
    fit = int(threads * (budget_s / 3) / (per_layer * sieve_us_1 * 1e-6)) if sieve_us_1 > 0 else len(layers)
    use = layers[:max(1, min(len(layers), max(fit, threads)))]
    steps_of = {l: [ls for ls in timed if ls.layer == l] for l in use}
    work = {l: start[l].copy() for l in use}

    def run_layer(l):
        st = work[l]
        for ls in steps_of[l]:
            st.update(0, ls.batch, b.req_pool, b.seq, b.R)
        return len(steps_of[l])

    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        n_t = sum(ex.map(run_layer, use))
    sieve_us_t = (time.perf_counter() - t0) / n_t * 1e6

    # the serial pipeline over the layer-steps SIEVE'd on one thread
    R, padded, rb = cfg.req_num, runner.padded, cfg.row_bytes
    cap = R * cfg.top_k
    staging = torch.empty((cap, rb), dtype=torch.uint8, pin_memory=True)
    dst_rows = torch.empty(cap, dtype=torch.int64, pin_memory=True)
    staging_np, dst_np = staging.numpy(), dst_rows.numpy()
    staging_d = torch.empty((cap, rb), dtype=torch.uint8, device=runner.dev)
    dst_d = torch.empty(cap, dtype=torch.int64, device=runner.dev)
    hot = torch.zeros((R * padded, rb), dtype=torch.uint8, device=runner.dev)

    def pipeline(nthreads, budget):
        rows = 0
        t = 0.0
        done = 0
        for ls, slots, miss in outs:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            n = orc.stage_rows(b.segs, staging_np, dst_np, ls.layer * b.plsr, rb, ls.batch, b.req_pool, b.host_base,
                               slots, miss, R, cfg.top_k, R, cfg.stripe_rows, cfg.node_num, padded, nthreads)
            if n > 0:
                staging_d[:n].copy_(staging[:n], non_blocking=True)
                dst_d[:n].copy_(dst_rows[:n], non_blocking=True)
                hot.index_copy_(0, dst_d[:n], staging_d[:n])
            torch.cuda.synchronize()
            t += time.perf_counter() - t0
            rows += n
            done += 1
            if t >= budget:
                break
        return t / done * 1e6, rows / t / 1e9 * rb if t > 0 else None, done

    pipe_us_1, pipe_gbps_1, n_p1 = pipeline(1, budget_s / 6)
    pipe_us_t, pipe_gbps_t, n_pt = pipeline(threads, budget_s / 6)
    misses = float(np.mean([ls.misses for ls, _, _ in outs]))
    rows_1 = misses / ((sieve_us_1 + pipe_us_1) * 1e-6)
    rows_t = misses / ((sieve_us_t + pipe_us_t) * 1e-6)
    info = cpu_info()
    log("[bench] cpu baseline ({}): SIEVE {:.0f} us/layer on 1 thread, {:.0f} on {} threads; serial pipeline "
        "{:.1f} GB/s on 1 thread, {:.1f} on {}; {:.0f} / {:.0f} rows/s".format(
            info["model"], sieve_us_1, sieve_us_t, threads, pipe_gbps_1 or 0, pipe_gbps_t or 0, threads, rows_1,
            rows_t))
    return {
        "value": rows_t,
        "unit": "rows/s",
        "cores": threads,
        "kind": "port",
        "sample": "timed layer-steps of the benchmark stream from the state they start from: SIEVE on 1 thread "
                  "over {} of them, on {} threads over {} ({} layers); the serial pipeline (host staging, one H2D, "
                  "device scatter) over {} / {}".format(n_one, threads, n_t, len(use), n_p1, n_pt),
        "single_thread": {"sieve_us_per_layer": sieve_us_1, "pipeline_us_per_layer": pipe_us_1,
                          "gather_GBps": pipe_gbps_1, "rows_per_s": rows_1},
        "all_cores": {"threads": threads, "sieve_us_per_layer": sieve_us_t, "pipeline_us_per_layer": pipe_us_t,
                      "gather_GBps": pipe_gbps_t, "rows_per_s": rows_t},
        "cpu": info,
    }


# ---------------------------------------------------------------- GPU passes
def graph_pass(runner, snap, warm, timed, fused, eager_ms, log):
    """Replay the timed layer-steps again from the same starting state, each
    decode step as one captured HIP graph (SIEVE update + fused import of all
    its layers), and check that the final state and hot rows equal the eager
    run's.  Launch overhead, the reference design's graph-mode target
    (doc/kv_offload_design.md:94: under 50% of per-call launches): the host
    time to issue a step's launches, eager calls against one graph replay, and
    the GPU time of the launches alone (num_real = 0)."""
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
    for ls in warm:
        runner.sieve(ls.layer, ls.topk)
        runner.gather(ls.layer, ls.topk, fused=True)
    steps = {}
    for ls in timed:
        steps.setdefault(ls.step, []).append((ls.layer, ls.topk))
    t0 = time.perf_counter()
    graphs = []
    cap_stream = torch.cuda.Stream(device=runner.dev)
    for step in sorted(steps):
        layers = [l for l, _ in steps[step]]
        g = DecodeStepGraph(c, runner.pool, layers, [t for _, t in steps[step]], [runner.hot[l] for l in layers],
                            hot_req_stride_rows=runner.padded, block_dim=1, sieve_block_dim=runner.block_dim,
                            capture_stream=cap_stream)
        g.capture()
        graphs.append(g)
    capture_s = time.perf_counter() - t0
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    head_start()
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
    # launch overhead: the same layer-steps with num_real = 0 (every kernel
    # launched, no row does work)
    saved = c.num_real.clone()
    c.num_real.zero_()
    torch.cuda.synchronize()
    n = len(timed)
    h0 = time.perf_counter()
    e0.record(stream)
    for ls in timed:
        runner.sieve(ls.layer, ls.topk)
        runner.gather(ls.layer, ls.topk, fused=True)
    e1.record(stream)
    host_eager = time.perf_counter() - h0
    torch.cuda.synchronize()
    idle_eager_ms = e0.elapsed_time(e1)
    h0 = time.perf_counter()
    e0.record(stream)
    for g in graphs:
        g.replay(clear_status=False)
    e1.record(stream)
    host_graph = time.perf_counter() - h0
    torch.cuda.synchronize()
    idle_graph_ms = e0.elapsed_time(e1)
    c.num_real.copy_(saved)
    torch.cuda.synchronize()
    res = {"steps": len(graphs), "layer_steps": n, "capture_s": capture_s,
           "us_per_layer": graph_ms * 1e3 / n, "eager_us_per_layer": eager_ms * 1e3 / n,
           "speedup": eager_ms / graph_ms, "state_match": state_ok, "outputs_match": outs_ok, "hot_match": hot_ok,
           "launch_overhead": {
               "host_issue_us_per_layer": {"eager": host_eager * 1e6 / n, "graph": host_graph * 1e6 / n,
                                           "graph_over_eager": host_graph / host_eager},
               "gpu_launch_only_us_per_layer": {"eager": idle_eager_ms * 1e3 / n, "graph": idle_graph_ms * 1e3 / n,
                                                "graph_over_eager": idle_graph_ms / idle_eager_ms},
               "target_graph_over_eager": 0.5}}
    log("[bench] graph replay: {:.2f} us/layer vs eager {:.2f} us/layer ({} step graphs, capture {:.1f} s); "
        "state {} outputs {} hot rows {}; launch overhead per layer: host {:.2f} vs {:.2f} us ({:.2f}x), "
        "GPU (num_real 0) {:.2f} vs {:.2f} us".format(
            res["us_per_layer"], res["eager_us_per_layer"], len(graphs), capture_s, state_ok, outs_ok, hot_ok,
            host_graph * 1e6 / n, host_eager * 1e6 / n, host_graph / host_eager, idle_graph_ms * 1e3 / n,
            idle_eager_ms * 1e3 / n))
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
    for ls in warm:
        runner.sieve(ls.layer, ls.topk)
    stream = torch.cuda.current_stream()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    head_start()
    e0.record(stream)
    for ls in timed:
        runner.sieve(ls.layer, ls.topk)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / len(timed)
    ok = all(torch.equal(a, getattr(c, n)) for a, n in zip(ref, names))
    # the same launches one by one, each bracketed by a torch event pair and
    # then by a fence-free pair: the cost of the event kind itself
    per = {}
    for kind in ("torch_events", "fence_free_events"):
        runner.restore(snap)
        for ls in warm:
            runner.sieve(ls.layer, ls.topk)
        torch.cuda.synchronize()
        head_start()
        if kind == "torch_events":
            pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in timed]
            for (a, b), ls in zip(pairs, timed):
                a.record(stream)
                runner.sieve(ls.layer, ls.topk)
                b.record(stream)
            torch.cuda.synchronize()
            per[kind] = pct([a.elapsed_time(b) * 1e3 for a, b in pairs], 50)
        else:
            fev = FenceFreeEvents()
            pairs = [(fev.event(), fev.event()) for _ in timed]
            for (a, b), ls in zip(pairs, timed):
                fev.record(a, stream)
                runner.sieve(ls.layer, ls.topk)
                fev.record(b, stream)
            torch.cuda.synchronize()
            per[kind] = pct([fev.elapsed_ms(a, b) * 1e3 for a, b in pairs], 50)
            fev.close()
    log("[bench] SIEVE back to back: {:.2f} us/layer over {} launches; state equal to the eager run: {}; "
        "one by one: median {:.2f} us with torch events, {:.2f} us with fence-free events".format(
            us, len(timed), ok, per["torch_events"], per["fence_free_events"]))
    return {"us_per_layer": us, "launches": len(timed), "state_match": ok,
            "per_launch_median_us": per}


def sieve_standard_events(runner, snap, warm, timed, fused, log):
    """The decode loop again from the same starting state, each SIEVE launch
    bracketed by torch events, whose record releases to system scope (a
    write-back of the GPU caches): per-launch times that include that
    write-back, beside the fence-free figures of the main loop."""
    import torch

    runner.restore(snap)
    for ls in warm:
        runner.sieve(ls.layer, ls.topk)
        runner.gather(ls.layer, ls.topk, fused=fused)
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in timed]
    head_start()
    for (a, b), ls in zip(evs, timed):
        a.record()
        runner.sieve(ls.layer, ls.topk)
        b.record()
        runner.gather(ls.layer, ls.topk, fused=fused)
    torch.cuda.synchronize()
    us = [a.elapsed_time(b) * 1e3 for a, b in evs]
    log("[bench] SIEVE per launch with standard (system-release) events: median {:.2f} us, p99 {:.2f}".format(
        pct(us, 50), pct(us, 99)))
    return {"median": pct(us, 50), "p99": pct(us, 99), "mean": sum(us) / len(us),
            "timing": "per launch inside the decode loop, torch events (system-scope release: includes the cache "
                      "write-back each event record costs)"}


def import_curve(runner, log, reps=20, warm=3):
    """Import latency against batch size (the reference design's import
    batch-size curve): one request of n positions, every one a miss with its
    own token and slot, fused over the workload's segments, n = 16 .. 4096 rows
    (the one-launch form) and 8192, 16384 (two launches)."""
    import numpy as np
    import torch
    from kv_offload_proto_amd.kvops_ext import _kvops

    cfg = runner.cfg
    dev = runner.dev
    rb, plsr = cfg.row_bytes, runner.pool.per_layer_seg_rows
    fev = FenceFreeEvents()
    stream = torch.cuda.current_stream()
    status = runner.pool.next_status()
    out = []
    n_max = min(16384, cfg.layer_rows, runner.hot[0].shape[0])
    n = 16
    while n <= n_max:
        rng = np.random.default_rng(n)
        topk = torch.from_numpy(rng.permutation(min(cfg.layer_rows, 1 << 22))[:n].astype(np.int32)).to(dev).view(1, n)
        slots = torch.arange(n, dtype=torch.int32, device=dev).view(1, n)
        miss = torch.ones((1, n), dtype=torch.int8, device=dev)
        pool_idx = torch.zeros(1, dtype=torch.int64, device=dev)
        base = torch.zeros(1, dtype=torch.int64, device=dev)
        nr = torch.ones(1, dtype=torch.int32, device=dev)
        hot = runner.hot[0]

        def once():
            _kvops.import_all(runner.seg_bases, 0, plsr, rb, topk.data_ptr(), pool_idx.data_ptr(), base.data_ptr(),
                              slots.data_ptr(), miss.data_ptr(), nr.data_ptr(), hot.data_ptr(), n, 1,
                              cfg.stripe_rows, status, stream.cuda_stream, 1, 0)

        for _ in range(warm):
            once()
        torch.cuda.synchronize()
        evs = [(fev.event(), fev.event()) for _ in range(reps)]
        for a, b in evs:
            fev.record(a, stream)
            once()
            fev.record(b, stream)
        torch.cuda.synchronize()
        us = [fev.elapsed_ms(a, b) * 1e3 for a, b in evs]
        med = pct(us, 50)
        out.append({"rows": n, "us_median": med, "GBps": n * rb / (med * 1e-6) / 1e9})
        n *= 2
    fev.close()
    log("[bench] import latency by rows per layer: " + ", ".join(
        "{}: {:.1f} us".format(e["rows"], e["us_median"]) for e in out))
    return {"points": out, "what": "one request of n miss positions (own tokens and slots), fused import over the "
                                   "segments, median of {} launches between fence-free events".format(reps)}


def export_rows_pass(runner, log, reps=3):
    """Decode-incremental export: one row per request per layer (the row a
    decode step would append; here the last prefill row, rewritten with the
    bytes it already holds), timed per layer with HIP events, then checked in
    the host segments."""
    import numpy as np
    import torch

    cfg, pool = runner.cfg, runner.pool
    R = cfg.req_num
    rows = [runner.host_bases[r] + cfg.prefill - 1 for r in range(R)]
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


def main():
    args = parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this data plane runs on a single MI355X here "
              "(--gpus {} is not supported; run with --gpus 1)".format(args.gpus), file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
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
    threads = max(1, min(args.cpu_threads, cpu_info()["cpus_usable"] or 1))
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
    for ls in warm:
        runner.sieve(ls.layer, ls.topk)
        runner.gather(ls.layer, ls.topk, fused=fused)
    torch.cuda.synchronize()

    fev = FenceFreeEvents()
    ev = [(fev.event(), fev.event(), fev.event()) for _ in timed]
    start, end = fev.event(), fev.event()
    torch.cuda.synchronize()
    head_start()
    fev.record(start, stream)
    for (a, b, c), ls in zip(ev, timed):
        fev.record(a, stream)
        runner.sieve(ls.layer, ls.topk)
        fev.record(b, stream)
        runner.gather(ls.layer, ls.topk, fused=fused)
        fev.record(c, stream)
    fev.record(end, stream)
    torch.cuda.synchronize()
    total_ms = fev.elapsed_ms(start, end)
    sieve_us = [fev.elapsed_ms(a, b) * 1e3 for a, b, _ in ev]
    gather_us = [fev.elapsed_ms(b, c) * 1e3 for _, b, c in ev]
    fev.close()
    rows = sum(ls.misses for ls in timed)
    moved = sum(ls.moved for ls in timed)
    unique_src = sum(ls.unique_src for ls in timed)

    verify = None if args.no_verify else verify_against_oracle(runner, snap, plan, threads, log)

    # rooflines: the import is bound by the host link, SIEVE by HBM
    c = runner.coord
    positions = cfg.req_num * cfg.top_k
    t_gather = sum(gather_us) * 1e-6
    link_gbps = moved * cfg.row_bytes / t_gather / 1e9
    unique_gbps = unique_src * cfg.row_bytes / t_gather / 1e9
    hbm_bytes = [ls.moved * cfg.row_bytes * 2 + positions * 9 for ls in timed]
    hbm_gbps = sum(hbm_bytes) / t_gather / 1e9
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

    # the library imports up to 4096 positions in one launch, larger batches in two
    gather_kernels = ("kvx_gather_small",) if positions <= 4096 else ("kvx_gather_prep", "kvx_gather_span")
    gather_roof = {"kernel": "+".join(gather_kernels), "bound": "host-link", "achieved": link_gbps,
                   "peak": link["peak_GBps"], "unit": "GB/s", "frac": link_gbps / link["peak_GBps"],
                   "traffic": traffic_of(*gather_kernels), "traffic_source": traffic_src,
                   "bytes_per_launch": moved * cfg.row_bytes / len(timed),
                   "bytes_rule": "rows moved (distinct destinations after the winner rule) x row_bytes, read over "
                                 "the host link",
                   "traffic_basis": "FETCH_SIZE + WRITE_SIZE of the listed kernels per layer-step: the host rows "
                                    "read, the hot rows written and the index scan",
                   "algorithmic_traffic": sum(hbm_bytes) / len(timed),
                   "avg_launch_us": sum(gather_us) / len(timed),
                   "hbm": {"achieved": hbm_gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": hbm_gbps / HBM_PEAK_GBPS,
                           "bytes_rule": "rows moved x row_bytes read + written, + 9 B per position of index scan"}}
    from kv_offload_proto_amd.kvops_ext import _kvops

    sieve_kernels = SIEVE_KERNELS.get(_kvops.last_sieve_variant(), ("kvx_sieve_update",))
    if sieve_kernels[-1] == "kvx_sieve_update_batch" and traffic_of(*SIEVE_TABLE_KERNELS) is not None:
        sieve_kernels = sieve_kernels + SIEVE_TABLE_KERNELS
    sieve_roof = {"kernel": "+".join(sieve_kernels), "bound": "hbm", "achieved": sieve_gbps_alg,
                  "peak": HBM_PEAK_GBPS, "unit": "GB/s", "frac": sieve_gbps_alg / HBM_PEAK_GBPS,
                  "traffic": traffic_of(*sieve_kernels), "traffic_source": traffic_src, "bytes_per_launch": sb,
                  "traffic_basis": "FETCH_SIZE + WRITE_SIZE of the kernel per launch, against bytes_per_launch (the "
                                   "row state read and written back, the batch row read, the outputs written)",
                  "algorithmic_traffic": sb,
                  "avg_launch_us": sum(sieve_us) / len(timed)}
    for roof in (gather_roof, sieve_roof):
        t_, a_ = roof.get("traffic"), roof.get("algorithmic_traffic")
        roof["traffic_over_algorithmic"] = (t_ / a_) if (t_ and a_) else None
    dominant, other = (gather_roof, sieve_roof) if sum(gather_us) >= sum(sieve_us) else (sieve_roof, gather_roof)

    value = rows / (total_ms * 1e-3)
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": total_ms / args.steps,
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
                               "mean": sum(sieve_us) / len(sieve_us),
                               "timing": "per launch inside the decode loop, hipEventDisableSystemFence events"},
        "gather": {"us_per_layer_median": pct(gather_us, 50), "GBps": link_gbps,
                   "frac_of_link_peak": link_gbps / link["peak_GBps"], "frac_of_hbm_peak": link_gbps / HBM_PEAK_GBPS,
                   "unique_host_GBps": unique_gbps, "unique_host_frac_of_link_peak": unique_gbps / link["peak_GBps"],
                   "rows_moved_per_s": moved / t_gather, "miss_rows_per_s": rows / t_gather, "rows_moved": moved,
                   "miss_rows": rows, "unique_host_rows": unique_src},
        "host_link": link,
        "export": {"row_bytes_total": runner.export_bytes, "bytes_moved": runner.export_moved_bytes,
                   "us": export_us, "GBps_moved": export_gbps},
        "roofline": dominant,
        "roofline_other": other,
        "verify": None if verify is None else verify["ok"],
        "verify_detail": verify,
    }
    if args.loop_only:  # counter profiles: only the decode loop's dispatches
        out["sieve_us_per_layer"]["standard_events"] = None
        out["sieve_back_to_back"] = out["graph"] = out["export_rows"] = out["import_curve"] = None
    else:
        out["sieve_us_per_layer"]["standard_events"] = sieve_standard_events(runner, snap, warm, timed, fused, log)
        out["sieve_back_to_back"] = sieve_pipelined(runner, snap, warm, timed, log)
        out["graph"] = None if args.no_graph else graph_pass(runner, snap, warm, timed, fused, total_ms, log)
        out["export_rows"] = export_rows_pass(runner, log)
        out["import_curve"] = import_curve(runner, log)
    if not args.no_cpu and not args.loop_only:
        out["cpu_baseline"] = cpu_baseline(runner, snap, plan, len(warm), args.cpu_sample_s, threads, log)
    else:
        out["cpu_baseline"] = None
    out["wall_s"] = time.perf_counter() - t_start
    runner.close()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
