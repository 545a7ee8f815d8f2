#!/usr/bin/env python3
"""VecMarket benchmark on one MI355X: quote-matches/s, market-steps/s, p50 step latency.

A *step* is one ``add_two_sided_quotes`` over all markets (plus ``get_bbos`` when
the config asks for it every step), i.e. one lock-step batch of two-sided quotes
through the hot path. Inputs come from the deterministic counter-based generator
(astra_cuda.workloads), run on the device; the steps from the warm-up on are
generated up front and resident in HBM before timing starts.

The default run (config 3, the headline) also measures configs 2, 4 and 5 of
BASELINE.json, each over the end of its own run with the same window rule, and
reports them under "configs". ``--sweep 1000,10000,...`` instead prints
quote-matches/s at config 3's shape for each market count.

The timed window is the END of the config's run: a config defines a run of
``steps`` steps (config 3: 1,000, whose order ring wraps at step 512 and evicts
from then on), and ``--warmup W --steps K`` time steps [S + W, S + W + K) with
S = max(0, run steps - W - K). Steps [0, S) are a pre-roll through the same API,
untimed, so a short run measures the book in the state the config defines (for
config 3 the eviction regime) rather than an empty one. ``--start`` overrides S.
The window is reported in ``config.timed_steps``.

Phases (only A is the headline; B-D replay the same steps from clones of the
pre-timed state, so they see exactly the same work):
  A  throughput: exactly K steps, no host sync inside, bracketed by
     torch.cuda.synchronize() on both sides;
  B  latency: per-step host time with the stream synced (p50 / p99 / max);
  C  device time: HIP events on the launch stream around the K matching-kernel
     launches issued back to back (then around K get_bbos launches), so the
     mean per launch is the kernel's average duration;
  D  work counts: the diagnostic kernel variant counts inserts, fill rows and
     emptied levels, for the algorithmic-byte roofline;
  R  the timed steps again with a FillBatch in the row layout
     (new_fill_batch(layout="rows"), not the reference's), reported beside the
     headline as value_rows_layout;
  S  the timed steps as ONE launch of the multi-step kernel
     (add_two_sided_quotes_steps, not in the reference; every step's BBOs kept),
     reported beside the headline under "multistep";
  G  the timed steps captured in one HIP graph through the drop-in API and
     replayed once (the TID counter is in device memory), under "graph_replay".
Then the CPU baseline: the oracle (a C port of the reference algorithm) on a
bounded subset of the same markets, replaying the same pre-roll and warm-up
untimed and timing the same window, on all host threads and on 1 thread.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "astra-cuda_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published


def log(msg: str) -> None:
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


class HostInputs:
    """The host generator's steps (QuoteStream, numpy), uploaded one by one: the
    same int32 inputs as DeviceQuoteStream, with no generator kernels on the GPU."""

    def __init__(self, cfg, markets, dev):
        from astra_cuda.workloads import QuoteStream
        self.qs, self.dev = QuoteStream(cfg, markets), dev

    def step(self, t):
        import numpy as np
        import torch
        return tuple(torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(self.dev)
                     for x in self.qs.step(t))

    def steps(self, t0, t1):
        import torch
        rows = [self.step(t) for t in range(t0, t1)]
        return tuple(torch.stack([r[i] for r in rows]) for i in range(5))


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=900, help="timed steps K")
    ap.add_argument("--warmup", type=int, default=100, help="untimed warm-up steps W")
    ap.add_argument("--start", type=int, default=None,
                    help="untimed pre-roll steps S before the warm-up (default: the config's run "
                         "length - W - K, so the timed steps are the last K of the run)")
    ap.add_argument("--config", type=int, default=3,
                    help="BASELINE.json config index (2, 3 or 4; 5 = the high-low game step; "
                         "6 = the reference's own game benchmark workload, "
                         "src/tests/benchmarks/high_low_benchmark.py)")
    ap.add_argument("--episodes", type=int, default=30, help="config 6: episodes timed")
    ap.add_argument("--markets", type=int, default=0, help="override the config's market count")
    ap.add_argument("--no-bbo", action="store_true", help="do not call get_bbos every step")
    ap.add_argument("--latency-steps", type=int, default=300)
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="target CPU time of the all-thread oracle leg")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds-more", type=float, default=5.0,
                    help="target CPU time of the oracle leg of each of configs 2, 4, 5 beside the headline")
    ap.add_argument("--no-more-configs", action="store_true",
                    help="with config 3: do not also run configs 2, 4 and 5 (reported under \"configs\")")
    ap.add_argument("--sweep", default="",
                    help="comma-separated market counts: quote-matches/s at config 3's shape for each "
                         "(one JSON line with the points; e.g. 1000,10000,30000,100000,300000,1048576,4194304)")
    ap.add_argument("--phases", default="ABCDRSG",
                    help="phases to run (A is always run; B latency, C events, D work counts, "
                         "R row layout, S multi-step, G graph replay)")
    ap.add_argument("--scatter-calibration", action="store_true",
                    help="only time scattered 4-byte writes, reads and atomic adds into a 1 GiB "
                         "buffer (the rate of scattered memory requests the device sustains)")
    ap.add_argument("--host-inputs", action="store_true",
                    help="generate the quotes with the host generator (numpy; the same values as the "
                         "device generator) and upload them step by step: for profiler runs that "
                         "should see no generator kernels")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of known size (for rocprof counter scaling)")
    return ap.parse_args()


def cpu_info():
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return model, avail


def pre_roll(args, run_steps: int) -> int:
    """Untimed steps before the warm-up: by default the timed steps are the last K
    of the config's run (W + K past its end is allowed: the generator is defined
    for every step)."""
    if args.start is not None:
        if args.start < 0:
            raise SystemExit("--start must be >= 0")
        return args.start
    return max(0, run_steps - args.warmup - args.steps)


def scatter_calibration():
    """Requests per second of scattered 4-byte accesses: 16M random offsets into a 1 GiB
    int32 buffer, written (index_put_), read (gather) and atomically added (index_add_),
    each timed with HIP events over 10 launches. Each access is one L1-to-L2 request
    (offsets are random, so no two accesses of a wavefront share a line)."""
    import torch
    n, k = 1 << 28, 1 << 24
    buf = torch.zeros(n, dtype=torch.int32, device="cuda")
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    idx = torch.randint(0, n, (k,), dtype=torch.int64, device="cuda", generator=g)
    val = torch.ones(k, dtype=torch.int32, device="cuda")
    out = {}
    for name, fn in (("write", lambda: buf.index_put_((idx,), val)),
                     ("read", lambda: torch.take(buf, idx)),
                     ("atomic_add", lambda: buf.index_add_(0, idx, val))):
        for _ in range(3):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(10):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        t = ev[0].elapsed_time(ev[1]) / 10 * 1e-3
        out[name] = {"us_per_launch": t * 1e6, "requests_per_s": k / t}
    print(json.dumps({"scatter_calibration": {"accesses_per_launch": k, "buffer_bytes": 4 * n, **out}}))


def copy_calibration():
    import torch
    n = 1 << 30  # 1 GiB
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": n, "launches": 10}))


def main():
    args = parse_args()
    if args.gpus != 1:
        msg = ("bench.py measures one GPU only: markets are independent and shard with no "
               "communication, so N GPUs would run N independent engines; --gpus must be 1")
        print(msg, file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration:
        return copy_calibration()
    if args.scatter_calibration:
        return scatter_calibration()
    if args.sweep:
        return bench_sweep(args)
    if args.config == 5:
        print(json.dumps(bench_game(args)), flush=True)
        return
    if args.config == 6:
        return bench_game_reference(args)
    result = bench_market(args, args.config)
    if args.config == 3 and not args.markets and not args.no_more_configs:
        result["configs"] = more_configs(args)
    print(json.dumps(result), flush=True)


def more_configs(args):
    """Configs 2, 4 and 5 of BASELINE.json, each over the end of its own run (the
    same --warmup / --steps window rule as the headline), reported beside it."""
    import torch
    out = {}
    for idx in (2, 4, 5):
        torch.cuda.empty_cache()
        log(f"---- config {idx} ----")
        out[f"config{idx}"] = bench_game(args, secondary=True) if idx == 5 else \
            bench_market(args, idx, secondary=True)
    return out


def bench_market(args, cfg_index: int, secondary: bool = False, markets: int = 0):
    """One VecMarket config over the timed window of its run; returns the result
    dict (the headline's JSON line, or an entry of its "configs")."""
    import numpy as np
    import torch
    from astra_cuda import order_matching as aom
    from astra_cuda.workloads import CONFIGS, DeviceQuoteStream

    cfg = CONFIGS[cfg_index]
    M = markets or args.markets or cfg.M
    W, K = args.warmup, args.steps
    S = pre_roll(args, cfg.steps)
    T0 = S + W          # first timed step
    T = T0 + K
    bbo = cfg.bbo_every_step and not args.no_bbo
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    phases = set(args.phases.upper()) | {"A"}
    if secondary:
        phases -= {"R", "S"}

    # ---- inputs: the counter-based generator on the device; the steps from the
    # warm-up on are generated up front and resident in HBM before timing, the
    # pre-roll's step by step ----
    t0 = time.perf_counter()
    if args.host_inputs:
        dq = HostInputs(cfg, np.arange(M), dev)
    else:
        dq = DeviceQuoteStream(cfg, None if M == cfg.M else np.arange(M), device=dev)
    shape = dict(num_markets=M, max_price_levels=cfg.L, max_active_orders_per_market=cfg.O,
                 max_active_fills_per_market=cfg.F, num_customers=cfg.C)
    market = aom.VecMarket(**shape, allow_extended_shapes=cfg.extended)
    fills = market.new_fill_batch()
    bbos = market.new_bbo_batch()

    def step(mk, q):
        mk.add_two_sided_quotes(*q, fills)
        if bbo:
            mk.get_bbos(bbos)

    for t in range(S):
        step(market, dq.step(t))
    dev_in = list(dq.steps(S, T))
    rows = {t: tuple(x[t - S] for x in dev_in) for t in range(S, T)}
    for t in range(S, T0):
        step(market, rows[t])
    torch.cuda.synchronize()
    where = "on the host" if args.host_inputs else "on the device"
    log(f"config {cfg.index}: {M} markets, pre-roll ({S} steps, inputs generated {where}) and "
        f"warm-up ({W} steps) in {time.perf_counter() - t0:.1f}s; timing steps [{T0}, {T})")
    # state at the start of the timed steps, for the replays B, C, D, R, S and G
    snaps = {p: market.clone() for p in "BCDRSG" if p in phases}
    torch.cuda.synchronize()

    # ---- A: throughput (the headline) ----
    torch.cuda.synchronize()
    a0 = time.perf_counter()
    for t in range(T0, T):
        step(market, rows[t])
    torch.cuda.synchronize()
    wall = time.perf_counter() - a0
    log(f"A: {K} steps in {wall * 1e3:.2f} ms")

    # ---- B: per-step latency (stream synced every step) and the host time of the
    # calls, through this package's binding and through the compiled one (a copy
    # of the same book) ----
    nlat = min(K, args.latency_steps) if "B" in phases else 0
    bindings = {}
    lat_ms = np.array([float("nan")])
    if nlat:
        from astra_cuda._C import order_matching as com
        cm = com.VecMarket(M, cfg.L, cfg.O, cfg.F, cfg.C) if not cfg.extended else None
        if cm is not None:
            cm._workspace.copy_(snaps["B"]._ws[:cm._workspace.numel()])
            cfills, cbbos = cm.new_fill_batch(), cm.new_bbo_batch()
        for name, mk in (("ctypes", snaps["B"]), ("compiled", cm)):
            if mk is None:
                continue
            f_, b_ = (fills, bbos) if name == "ctypes" else (cfills, cbbos)
            lat, host = [], []
            for t in range(T0, T0 + nlat):
                torch.cuda.synchronize()
                h0 = time.perf_counter()
                mk.add_two_sided_quotes(*rows[t], f_)
                h1 = time.perf_counter()
                if bbo:
                    mk.get_bbos(b_)
                torch.cuda.synchronize()
                lat.append(time.perf_counter() - h0)
                host.append(h1 - h0)
            bindings[name] = {"p50_step_latency_ms": float(np.percentile(lat, 50) * 1e3),
                              "p99_step_latency_ms": float(np.percentile(lat, 99) * 1e3),
                              "host_us_per_add_two_sided_quotes_p50": float(np.percentile(host, 50) * 1e6)}
            if name == "ctypes":
                lat_ms = np.array(lat) * 1e3
        del cm
        log("B: " + ", ".join(f"{k} p50 {v['p50_step_latency_ms'] * 1e3:.1f} us (host "
                              f"{v['host_us_per_add_two_sided_quotes_p50']:.1f} us per call)"
                              for k, v in bindings.items()))

    # ---- C: device time per kernel (HIP events on the launch stream) ----
    # The matching kernel of the K timed steps, replayed back to back (get_bbos
    # reads state only, so leaving it out changes no step), then K get_bbos.
    qm_ms, bbo_ms = wall / K * 1e3, 0.0
    if "C" in phases:
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda.synchronize()
        ev[0].record()
        for t in range(T0, T):
            snaps["C"].add_two_sided_quotes(*rows[t], fills)
        ev[1].record()
        if bbo:
            for t in range(T0, T):
                snaps["C"].get_bbos(bbos)
        ev[2].record()
        torch.cuda.synchronize()
        qm_ms = ev[0].elapsed_time(ev[1]) / K
        if bbo:
            bbo_ms = ev[1].elapsed_time(ev[2]) / K

    # ---- D: exact work counts for the algorithmic bytes ----
    counters = torch.zeros(11, dtype=torch.int64, device=dev)
    if "D" in phases:
        snaps["D"]._set_stats(counters)
        for t in range(T0, T):
            snaps["D"].add_two_sided_quotes(*rows[t], fills)
        torch.cuda.synchronize()
        snaps["D"]._set_stats(None)
    (n_ins, n_fill, n_empty, n_ovf, n_ff, n_pass, n_staged, n_cross, n_zruns,
     n_zrows, n_bbo_book) = (int(x) for x in counters.cpu().tolist())

    # ---- R: the same steps with the row layout of the FillBatch ----
    wall_rows = None
    if "R" in phases:
        rfills = snaps["R"].new_fill_batch(layout="rows")
        torch.cuda.synchronize()
        r0 = time.perf_counter()
        for t in range(T0, T):
            snaps["R"].add_two_sided_quotes(*rows[t], rfills)
            if bbo:
                snaps["R"].get_bbos(bbos)
        torch.cuda.synchronize()
        wall_rows = time.perf_counter() - r0
        log(f"R: {K} steps in {wall_rows * 1e3:.2f} ms with the row layout")

    # ---- S: the same K steps as ONE multi-step launch (every step's BBOs kept) ----
    multistep = None
    if "S" in phases:
        step_bbos = torch.empty((4, K, M), dtype=torch.int32, device=dev) if bbo else None
        ins = [x[T0 - S:T - S] for x in dev_in]
        sev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]

        def one_launch(mk, layout):
            sfills = mk.new_fill_batch(layout)
            torch.cuda.synchronize()
            s0 = time.perf_counter()
            sev[0].record()
            mk.add_two_sided_quotes_steps(*ins, sfills, step_bbos=step_bbos)
            sev[1].record()
            torch.cuda.synchronize()
            return time.perf_counter() - s0, sev[0].elapsed_time(sev[1]) / K

        mk_rows = snaps["S"].clone()
        wall_ms, dev_ms = one_launch(snaps["S"], "columns")
        wall_ms_rows, _ = one_launch(mk_rows, "rows")
        del mk_rows
        multistep = {"value": M * K / wall_ms, "ms_per_step": wall_ms / K * 1e3,
                     "device_ms_per_step": dev_ms, "steps_per_launch": K,
                     "value_rows_layout": M * K / wall_ms_rows,
                     "kernel": "quote_match_kernel (multi-step)"}
        log(f"S: {K} steps in one launch, {wall_ms * 1e3:.2f} ms ({wall_ms_rows * 1e3:.2f} ms with rows)")

    # ---- G: the same K steps captured in one HIP graph (add_two_sided_quotes +
    # get_bbos per step, through the drop-in API) and replayed once ----
    graph = None
    if "G" in phases:
        gm = snaps["G"]
        gfills, gbbos = gm.new_fill_batch(), gm.new_bbo_batch()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for t in range(T0, T):
                gm.add_two_sided_quotes(*rows[t], gfills)
                if bbo:
                    gm.get_bbos(gbbos)
        torch.cuda.synchronize()
        g0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        gwall = time.perf_counter() - g0
        del g
        graph = {"value": M * K / gwall, "ms_per_step": gwall / K * 1e3, "steps_per_graph": K,
                 "note": "the timed steps captured once (torch.cuda.graph) and replayed once; the "
                         "TID counter lives in device memory, so a replay advances it"}
        log(f"G: {K} steps as one graph replay in {gwall * 1e3:.2f} ms")
    log(f"work over {K} steps: inserts {n_ins}, fill rows {n_fill}, emptied {n_empty}, overflow {n_ovf}")

    # algorithmic bytes (per launch of the matching kernel): quotes in 20 B + fill_counts 4 B
    # per market; 32 B per accepted insert; 109 B per fill row; 8 B per emptied level.
    qm_bytes = (24.0 * M * K + 32.0 * n_ins + 109.0 * n_fill + 8.0 * n_empty) / K
    bbo_bytes = 24.0 * M  # 16 B out + 2 head-size reads of 4 B
    qm_avg_s = qm_ms * 1e-3
    achieved = qm_bytes / qm_avg_s / 1e9

    traffic, traffic_src = measured_traffic(cfg, M, bbo, (T0, T))
    requests = None
    if M == cfg.M and bbo == cfg.bbo_every_step:
        words = 1
        while words * 64 < cfg.L:
            words *= 2
        found = profile_requests(f"quote_match_kernel<{words}, false, false, false, false", (T0, T))
        if found:
            req, rates, src = found
            requests = {
                "per_launch": req,
                "per_s": sum(req.values()) / qm_avg_s,
                "device_scatter_rates_per_s": rates,
                "write_requests_at_device_rate_us": req["write"] / rates["write"] * 1e6,
                "source": src,
            }
    value = M * K / wall
    result = {
        "metric": "quote-matches/sec and market-steps/sec at 100k markets; p50 step latency",
        "value": value,
        "unit": "quote-matches/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": wall / K * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic",
        "config": {
            "workload": f"config{cfg.index}_{cfg.name}",
            "num_markets": M, "max_price_levels": cfg.L, "max_active_orders_per_market": cfg.O,
            "max_active_fills_per_market": cfg.F, "num_customers": cfg.C,
            "get_bbos_every_step": bbo, "run_steps": cfg.steps, "pre_roll_steps": S,
            "timed_steps": [T0, T], "parallelism": "single GPU, one lane per market",
        },
        "market_steps_per_s": K / wall,
        "value_rows_layout": (M * K / wall_rows) if wall_rows else None,
        "multistep": multistep,
        "graph_replay": graph,
        "p50_step_latency_ms": float(np.percentile(lat_ms, 50)),
        "p99_step_latency_ms": float(np.percentile(lat_ms, 99)),
        "max_step_latency_ms": float(lat_ms.max()),
        "binding": "ctypes (astra_cuda.order_matching)",
        "bindings": bindings or None,
        "device_ms_per_step": {"quote_match": float(qm_ms), "get_bbos": float(bbo_ms)},
        "work_per_step": {"inserts": n_ins / K, "fill_rows": n_fill / K, "levels_emptied": n_empty / K,
                          "overflow_markets": n_ovf / K, "crossing_markets": n_cross / K,
                          "loop_passes": n_pass / K, "staged_markets": n_staged / K,
                          "staged_zero_runs": n_zruns / K, "staged_zero_rows": n_zrows / K,
                          "bbo_sides_read_from_book": n_bbo_book / K,
                          "staged_counts_note": "staged_* come from the counting kernel, which "
                                                "stages serially (no helper wavefronts); the other "
                                                "counts are the work of any launch shape"},
        "roofline": {
            "kernel": "quote_match_kernel",
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic,
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": qm_bytes,
            "get_bbos_algorithmic_bytes_per_launch": bbo_bytes,
            "scattered_requests": requests,
        },
    }
    if secondary:
        for k in ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline", "dtype", "data"):
            result.pop(k)

    # ---- CPU baseline: the oracle on a bounded subset of the same workload ----
    del snaps, market, fills, bbos, dev_in, rows
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(args, cfg, M, T0, K, bbo,
                                              args.cpu_seconds_more if secondary else args.cpu_seconds)
    return result


def bench_sweep(args):
    """Quote-matches/s over market counts at config 3's shape (the reference's
    benchmark sweeps its market count the same way, benchmark_market.cc:256-268).
    Each point runs the same timed window as the headline (steps 980-999 with the
    driver's --steps 20 --warmup 5): A on the market itself; then on the same market
    the work counts of the next K steps (D) and the matching kernel's device time
    over the K steps after those (C), so that no copy of the book is needed at 4M
    markets (the book and the FillBatch take 183 GiB there). The three windows lie
    in the eviction regime of config 3 (the order ring wraps at step 512)."""
    import numpy as np
    import torch
    from astra_cuda import order_matching as aom
    from astra_cuda.workloads import CONFIGS, DeviceQuoteStream

    cfg = CONFIGS[3]
    W, K = args.warmup, args.steps
    S = pre_roll(args, cfg.steps)
    T0, T = S + W, S + W + K
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    points = []
    for M in [int(x) for x in args.sweep.split(",")]:
        torch.cuda.empty_cache()
        t0 = time.perf_counter()
        dq = DeviceQuoteStream(cfg, np.arange(M), device=dev)
        market = aom.VecMarket(M, cfg.L, cfg.O, cfg.F, cfg.C)
        fills, bbos = market.new_fill_batch(), market.new_bbo_batch()

        def step(q):
            market.add_two_sided_quotes(*q, fills)
            market.get_bbos(bbos)

        for t in range(T0):
            step(dq.step(t))
        window = [dq.step(t) for t in range(T0, T + 2 * K)]
        torch.cuda.synchronize()
        a0 = time.perf_counter()
        for q in window[:K]:
            step(q)
        torch.cuda.synchronize()
        wall = time.perf_counter() - a0
        counters = torch.zeros(11, dtype=torch.int64, device=dev)
        market._set_stats(counters)
        for q in window[K:2 * K]:
            market.add_two_sided_quotes(*q, fills)
        torch.cuda.synchronize()
        market._set_stats(None)
        n_ins, n_fill, n_empty = (int(x) for x in counters.cpu().tolist()[:3])
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        for q in window[2 * K:]:
            market.add_two_sided_quotes(*q, fills)
        ev[1].record()
        torch.cuda.synchronize()
        qm_ms = ev[0].elapsed_time(ev[1]) / K
        qm_bytes = (24.0 * M * K + 32.0 * n_ins + 109.0 * n_fill + 8.0 * n_empty) / K
        frac = qm_bytes / (qm_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
        pt = {"markets": M, "value": M * K / wall, "ms_per_step": wall / K * 1e3,
              "quote_match_device_ms": qm_ms, "roofline_frac": frac,
              "algorithmic_bytes_per_launch": qm_bytes,
              "windows": {"A": [T0, T], "D": [T, T + K], "C": [T + K, T + 2 * K]}}
        points.append(pt)
        log(f"sweep {M} markets: {pt['value']:.3e} quote-matches/s, {pt['ms_per_step']:.3f} ms/step, "
            f"kernel {qm_ms * 1e3:.1f} us, frac {frac:.4f} ({time.perf_counter() - t0:.1f}s)")
        del market, fills, bbos, window, dq
    print(json.dumps({"metric": "quote-matches/sec over market counts (config 3 shape)", "unit": "quote-matches/s",
                      "sweep": points, "config": {"workload": "config3_stress_100k shape", "timed_steps": [T0, T]}}),
          flush=True)


def bench_game(args, secondary: bool = False):
    """Config 5: one trading move of every env of the high-low game per step
    (HighLowTradingState::ApplyPlayerTrading: AddTwoSidedQuotes, GetBBOs,
    UpdateLastPrices and the per-player rewards and telemetry). The chance moves
    are applied before timing; the timed steps are the last K trading moves of
    one game, after S = players * steps_per_player - W - K untimed moves and W
    warm-up moves (--start sets S; S + W + K must not exceed the game)."""
    import numpy as np
    import torch
    import astra_cuda as astra
    from astra_cuda.workloads import GAME_CONFIG, GameStream

    cfg = GAME_CONFIG
    N = args.markets or cfg.envs
    P = cfg.players
    moves_total = P * cfg.steps_per_player
    W, K = args.warmup, args.steps
    S = pre_roll(args, moves_total)
    T0 = S + W
    if T0 + K > moves_total:
        print(f"config 5 has {moves_total} trading moves: start + warmup + steps must not exceed it",
              file=sys.stderr)
        sys.exit(2)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    t0 = time.perf_counter()
    gs = GameStream(cfg, np.arange(N))
    chance = gs.chance()
    host_moves = [gs.move(k) for k in range(T0 + K)]
    moves = [torch.from_numpy(m).to(dev) for m in host_moves]
    chance_d = [torch.from_numpy(c).to(dev) for c in chance]
    torch.cuda.synchronize()
    log(f"generated config 5 moves: {T0 + K} moves x {N} envs in {time.perf_counter() - t0:.1f}s; "
        f"timed moves [{T0}, {T0 + K})")
    astra.register_games()
    game = astra.load_game("high_low_trading", cfg.game_params(N, check_moves=True))
    state = game.new_initial_state()
    for c in chance_d:
        state.apply_action(c)
    for k in range(T0):
        state.apply_action(moves[k])
    torch.cuda.synchronize()
    snaps = [state.clone() for _ in range(5)]
    torch.cuda.synchronize()
    log(f"pre-roll ({S} moves) and warm-up ({W} moves) done; timing {K} moves")

    def timed(st, check):
        st.set_check_moves(check)
        torch.cuda.synchronize()
        a0 = time.perf_counter()
        for k in range(T0, T0 + K):
            st.apply_action(moves[k])
        torch.cuda.synchronize()
        return time.perf_counter() - a0

    wall = timed(state, True)                 # A: with the reference's input checks
    wall_unchecked = timed(snaps[0], False)   # A': checks deferred (no sync per move)
    log(f"A: {K} moves in {wall * 1e3:.2f} ms (checked), {wall_unchecked * 1e3:.2f} ms (unchecked)")
    # B: per-move latency, checked
    st = snaps[1]
    lat = []
    for k in range(T0, T0 + min(K, args.latency_steps)):
        torch.cuda.synchronize()
        h0 = time.perf_counter()
        st.apply_action(moves[k])
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - h0)
    lat_ms = np.array(lat) * 1e3
    # C: device time per move (one fused launch), unchecked moves back to back
    st = snaps[2]
    st.set_check_moves(False)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    torch.cuda.synchronize()
    ev[0].record()
    for k in range(T0, T0 + K):
        st.apply_action(moves[k])
    ev[1].record()
    torch.cuda.synchronize()
    step_ms = ev[0].elapsed_time(ev[1]) / K
    # D: work counts of the matching kernel
    st = snaps[3]
    st.set_check_moves(False)
    counters = torch.zeros(11, dtype=torch.int64, device=dev)
    st.market._set_stats(counters)
    for k in range(T0, T0 + K):
        st.apply_action(moves[k])
    torch.cuda.synchronize()
    st.market._set_stats(None)
    n_ins, n_fill, n_empty = (int(x) for x in counters.cpu().tolist()[:3])
    # G: the unchecked moves captured in one HIP graph and replayed once (the
    # move's kernel reads the TID counter from device memory; the acting player
    # and move number are kernel arguments, which the capture records in order)
    st = snaps[4]
    st.set_check_moves(False)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        for k in range(T0, T0 + K):
            st.apply_action(moves[k])
    torch.cuda.synchronize()
    g0 = time.perf_counter()
    gr.replay()
    torch.cuda.synchronize()
    gwall = time.perf_counter() - g0
    del gr
    log(f"G: {K} unchecked moves as one graph replay in {gwall * 1e3:.2f} ms")
    # algorithmic bytes per move: the matching kernel's (24 B per env + 32 per insert +
    # 109 per fill row + 8 per emptied level) plus the game's work fused into it:
    # reads of the move 16 B, contract value 4 B, last price 4 B and per player the
    # portfolio 8 B, target 4 B and reward since last action 4 B; writes of the BBO
    # 16 B, last price 4 B, telemetry 28 B and per player the portfolio snapshot
    # 8 B, telemetry 8 B, immediate reward 4 B and reward since last action 4 B.
    game_bytes = N * ((16 + 4 + 4 + 16 * P) + (16 + 4 + 28 + 24 * P))
    step_bytes = (24.0 * N * K + 32.0 * n_ins + 109.0 * n_fill + 8.0 * n_empty) / K + game_bytes
    achieved = step_bytes / (step_ms * 1e-3) / 1e9
    traffic, traffic_src = game_traffic(cfg, N, (T0, T0 + K))
    result = {
        "metric": "quote-matches/sec and market-steps/sec at 100k markets; p50 step latency",
        "value": N * K / wall,
        "unit": "quote-matches/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": wall / K * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic",
        "config": {
            "workload": f"config5_{cfg.name}", "envs": N, "players": P,
            "steps_per_player": cfg.steps_per_player, "max_contract_value": cfg.max_contract_value,
            "max_contracts_per_trade": cfg.max_contracts_per_trade,
            "market_shape_LOFC": list(cfg.market_shape), "move_checks": "one host wait per move (for the checks)",
            "run_moves": moves_total, "pre_roll_moves": S, "timed_moves": [T0, T0 + K],
            "parallelism": "single GPU, one lane per env",
        },
        "market_steps_per_s": K / wall,
        "value_unchecked": N * K / wall_unchecked,
        "ms_per_step_unchecked": wall_unchecked / K * 1e3,
        "graph_replay": {"value": N * K / gwall, "ms_per_step": gwall / K * 1e3, "steps_per_graph": K,
                         "note": "the timed moves, unchecked, captured once and replayed once"},
        "p50_step_latency_ms": float(np.percentile(lat_ms, 50)),
        "p99_step_latency_ms": float(np.percentile(lat_ms, 99)),
        "device_ms_per_step": {"fused_move_kernel": step_ms},
        "work_per_step": {"inserts": n_ins / K, "fill_rows": n_fill / K, "levels_emptied": n_empty / K},
        "roofline": {
            "kernel": "quote_match_kernel with the game move fused (one launch per move)", "bound": "hbm",
            "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": achieved / HBM_PEAK_GBS,
            "traffic": traffic, "traffic_source": traffic_src, "algorithmic_bytes_per_launch": step_bytes,
        },
    }
    if secondary:
        for k in ("metric", "n_gpus", "higher_is_better", "scaling", "vs_baseline", "dtype", "data"):
            result.pop(k)
    del snaps, state, st, moves
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = game_cpu_baseline(args, cfg, chance, host_moves, N, T0, K,
                                                   args.cpu_seconds_more if secondary else args.cpu_seconds)
    return result


# src/tests/README.md:142,144-145: the reference's best game figure, RTX 5090
REF_GAME_FPS_RTX5090 = 164_402_193
REF_GAME_ENVS = 262_144


def bench_game_reference(args):
    """The reference's own game benchmark (src/tests/benchmarks/high_low_benchmark.py:
    run_benchmark, :169-246, with its parameters, :305-314) on this engine: per
    episode reset, the four fixed chance moves and 40 trading steps of
    fill_observation_tensor + apply_action (input checks on) + fill_rewards +
    fill_rewards_since_last_action, then fill_returns; random trading actions
    (prices 1-10, sizes 0-1) pre-generated on the device. FPS = trading steps x
    envs / total wall time, as there (:233). One warm-up episode is not timed."""
    import numpy as np
    import torch
    import astra_cuda as astra

    N = args.markets or REF_GAME_ENVS
    P, T, V = 5, 8, 10
    params = {"steps_per_player": T, "max_contracts_per_trade": 1, "customer_max_size": 2,
              "max_contract_value": V, "players": P, "num_markets": N, "threads_per_block": 256,
              "device_id": 0}
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    astra.register_games()
    game = astra.load_game("high_low_trading", params)
    state = game.new_initial_state()
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    steps = T * P
    actions = torch.zeros((steps, N, 4), dtype=torch.int32, device=dev)
    actions[:, :, 0:2] = torch.randint(1, V + 1, (steps, N, 2), dtype=torch.int32, device=dev, generator=g)
    actions[:, :, 2:4] = torch.randint(0, 2, (steps, N, 2), dtype=torch.int32, device=dev, generator=g)
    cand = torch.zeros((N, 2), dtype=torch.int32, device=dev)
    cand[:, 0], cand[:, 1] = 3, 8
    settle = torch.arange(N, dtype=torch.int32, device=dev) % 2
    perm = torch.arange(P, dtype=torch.int32, device=dev).unsqueeze(0).repeat(N, 1)
    cust = torch.zeros((N, P - 3), dtype=torch.int32, device=dev)
    cust[:, 0] = -2
    cust[:, 1] = 2
    obs = torch.zeros(game.observation_tensor_shape(), dtype=torch.float32, device=dev)
    imm = torch.zeros((N, P), dtype=torch.float32, device=dev)
    mine = torch.zeros((N,), dtype=torch.float32, device=dev)
    ret = torch.zeros((N, P), dtype=torch.float32, device=dev)

    def episode(step_ms):
        state.reset()
        for a in (cand, settle, perm, cust):
            state.apply_action(a)
        k = 0
        while not state.is_terminal():
            player = state.current_player()
            h0 = time.perf_counter()
            state.fill_observation_tensor(obs)
            state.apply_action(actions[k])
            state.fill_rewards(imm)
            state.fill_rewards_since_last_action(mine, player)
            step_ms.append((time.perf_counter() - h0) * 1e3)
            k += 1
        state.fill_returns(ret)
        return k

    episode([])
    torch.cuda.synchronize()
    log(f"config 6: {N} envs, warm-up episode done; timing {args.episodes} episodes")
    step_ms = []
    t0 = time.perf_counter()
    total = sum(episode(step_ms) for _ in range(args.episodes))
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    fps = total * N / wall
    result = {
        "metric": "game env-steps/sec (the reference's high_low_benchmark.py workload)",
        "value": fps,
        "unit": "env-steps/s",
        "n_gpus": 1,
        "steps": total,
        "warmup": steps,
        "ms_per_step": wall / total * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int32",
        "data": "synthetic",
        "config": {"workload": "config6_reference_game_benchmark", "envs": N, "players": P,
                   "steps_per_player": T, "max_contract_value": V, "max_contracts_per_trade": 1,
                   "customer_max_size": 2, "episodes": args.episodes,
                   "parallelism": "single GPU, one lane per env"},
        "avg_step_ms": float(np.mean(step_ms)),
        "max_step_ms": float(np.max(step_ms)),
        "reference_published": {"value": REF_GAME_FPS_RTX5090, "envs": REF_GAME_ENVS,
                                "hardware": "NVIDIA GeForce RTX 5090",
                                "source": "src/tests/README.md:142,144-145",
                                "ratio": fps / REF_GAME_FPS_RTX5090},
    }
    print(json.dumps(result), flush=True)


def game_cpu_baseline(args, cfg, chance, host_moves, N, T0, K, seconds):
    """The game oracle (numpy state operations over the C market oracle, one
    thread) on the first envs of the same stream: the same untimed moves [0, T0),
    then the timed moves [T0, T0 + K)."""
    import numpy as np
    from oracle.high_low_oracle import OracleHighLow

    model, avail = cpu_info()

    def run(n, pre, steps):
        o = OracleHighLow(n, cfg.players, cfg.steps_per_player, cfg.max_contracts_per_trade,
                          cfg.customer_max_size, cfg.max_contract_value, market_shape=cfg.market_shape)
        for c in chance:
            o.apply_action(np.ascontiguousarray(c[:n]))
        for k in range(pre):
            o.apply_action(np.ascontiguousarray(host_moves[k][:n]))
        c0 = time.perf_counter()
        for k in range(pre, pre + steps):
            o.apply_action(np.ascontiguousarray(host_moves[k][:n]))
        return n * steps / (time.perf_counter() - c0)

    n0 = min(N, 1000)
    rate = run(n0, 0, min(T0 + K, 50))
    # envs such that the untimed moves and the timed window together take about
    # cpu_seconds
    n = int(min(N, max(500, rate * seconds / (T0 + K))))
    log(f"CPU leg: {n} envs, {T0} untimed + {K} timed moves")
    v = run(n, T0, K)
    return {"value": v, "unit": "quote-matches/s", "cores": 1, "kind": "port",
            "sample": f"envs 0..{n - 1} of the same config-5 stream: moves [0, {T0}) untimed, "
                      f"the timed moves [{T0}, {T0 + K})",
            "host_cpu": model, "host_cpus_available": avail}


def profile_traffic(prefix: str, kernel: str, window):
    """HBM bytes per launch of `kernel` over the launches of steps [window) from a
    committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary under profiles/ whose name
    starts with `prefix` (copy-calibrated), or (None, None) when no summary holds a
    figure for exactly that window (traffic depends on the book's state, so a
    figure from other steps would describe other work). `kernel` is the name up to
    its closing '>'; the matching kernel's last two template arguments, the fill rows
    a lane buffers (2 or 4) and the market wavefronts per helper wavefront (0, 2 or
    3), are the engine's choice for the grid and may follow."""
    import glob
    import re
    key = re.compile(r"traffic_bytes_per_launch\[void " + re.escape(kernel) + r"(, [24](, [0-3])?)?>\]\["
                     + f"{window[0]},{window[1]}" + r"\]:\s*(\S+)")
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", prefix + "*.md"))):
        with open(path) as f:
            for line in f:
                m = key.match(line)
                if m:
                    return float(m.group(3)), os.path.relpath(path, ROOT)
    return None, None


def profile_requests(kernel: str, window):
    """The matching kernel's scattered L1-to-L2 requests per launch (read, write, atomic)
    over steps [window) and the device's scattered-request rates per second (the
    scatter calibration), from a committed summary under profiles/, or None."""
    import glob
    import re
    key = re.compile(r"requests_per_launch\[void " + re.escape(kernel) + r"(, [24](, [0-3])?)?>\]\["
                     + f"{window[0]},{window[1]}" + r"\]: read (\S+) write (\S+) atomic (\S+)")
    cal = re.compile(r"scatter_calibration_requests_per_s: read (\S+) write (\S+) atomic (\S+)")
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_request_rate.md"))):
        req = rates = None
        with open(path) as f:
            for line in f:
                m = key.match(line)
                if m:
                    req = {k: float(m.group(i)) for k, i in (("read", 3), ("write", 4), ("atomic", 5))}
                c = cal.match(line)
                if c:
                    rates = {k: float(c.group(i)) for k, i in (("read", 1), ("write", 2), ("atomic", 3))}
        if req and rates:
            return req, rates, os.path.relpath(path, ROOT)
    return None


def measured_traffic(cfg, M, bbo, window):
    """HBM bytes per matching-kernel launch for this workload and window (see
    profile_traffic)."""
    if M != cfg.M or bbo != cfg.bbo_every_step:
        return None, None
    words = 1
    while words * 64 < cfg.L:
        words *= 2
    return profile_traffic(f"quote_match_config{cfg.index}_{cfg.name}_",
                           f"quote_match_kernel<{words}, false, false, false, false", window)


def game_traffic(cfg, N, window):
    """HBM bytes per fused game-move launch for this workload and window (see
    profile_traffic)."""
    if N != cfg.envs:
        return None, None
    return profile_traffic(f"game_move_config5_{cfg.name}_",
                           "quote_match_kernel<2, false, true, false, true", window)


def cpu_baseline(args, cfg, M, T0, K, bbo, seconds):
    """The C oracle on markets [0, mc) of the same stream (generated on the host by
    the numpy generator, which the device generator reproduces bit for bit):
    steps [0, T0) untimed, then the timed window [T0, T0 + K) on all host threads;
    then, from a copy of the state at T0, the first steps of the window on one
    thread. mc is sized so that the whole leg takes about `seconds`."""
    import numpy as np
    from astra_cuda.workloads import QuoteStream
    from oracle.oracle import OracleMarket

    model, avail = cpu_info()
    nthreads = max(1, avail)

    def sliced(mc, t1=None):
        return QuoteStream(cfg, np.arange(mc)).steps(0, T0 + K if t1 is None else t1)

    def steps(o, f, b, sl, t0, t1, threads, with_bbo):
        for t in range(t0, t1):
            o.add_two_sided_quotes(*(a[t] for a in sl), f, nthreads=threads)
            if with_bbo:
                o.get_bbos(b, nthreads=threads)

    # calibrate on a small sample, then size the sample so that the untimed steps
    # and the window together take about `seconds` on all threads
    mc0 = min(M, 2000)
    o = OracleMarket(mc0, cfg.L, cfg.O, cfg.F, cfg.C)
    f, b = o.new_fill_batch(), o.new_bbo_batch()
    n0 = min(T0 + K, 50)
    sl0 = sliced(mc0, n0)
    c0 = time.perf_counter()
    steps(o, f, b, sl0, 0, n0, nthreads, bbo)
    rate = mc0 * n0 / (time.perf_counter() - c0)
    del o, f, b, sl0
    mc = int(min(M, max(1000, rate * seconds / (T0 + K))))
    log(f"CPU leg: {mc} markets, {T0} untimed + {K} timed steps on {nthreads} threads")
    sl = sliced(mc)
    o = OracleMarket(mc, cfg.L, cfg.O, cfg.F, cfg.C)
    f, b = o.new_fill_batch(), o.new_bbo_batch()
    steps(o, f, b, sl, 0, T0, nthreads, False)  # get_bbos changes no state
    o1 = o.clone()
    c0 = time.perf_counter()
    steps(o, f, b, sl, T0, T0 + K, nthreads, bbo)
    v_all = mc * K / (time.perf_counter() - c0)
    del o
    # one thread: window steps one at a time until a third of cpu_seconds is spent
    k1, spent = 0, 0.0
    while k1 < K and spent < seconds / 3:
        c0 = time.perf_counter()
        steps(o1, f, b, sl, T0 + k1, T0 + k1 + 1, 1, bbo)
        spent += time.perf_counter() - c0
        k1 += 1
    v_one = mc * k1 / spent
    log(f"CPU leg: {mc} markets x {k1} steps on 1 thread")
    return {
        "value": v_all,
        "unit": "quote-matches/s",
        "cores": nthreads,
        "kind": "port",
        "sample": (f"markets 0..{mc - 1} of the same config-{cfg.index} stream: steps [0, {T0}) "
                   f"untimed, the timed steps [{T0}, {T0 + K})"
                   + (" with get_bbos every step" if bbo else "")),
        "single_thread_value": v_one,
        "single_thread_sample": f"markets 0..{mc - 1}, timed steps [{T0}, {T0 + k1})",
        "host_cpu": model,
        "host_cpus_available": avail,
    }


if __name__ == "__main__":
    main()
