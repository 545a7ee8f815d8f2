"""Drop-in calls captured in a HIP graph (torch.cuda.graph) and replayed (GPU).

The TID counter lives in the engine's workspace and the matching kernel moves it
on itself, so a captured add_two_sided_quotes replays with fresh TIDs (the
reference passes the host counter as a kernel argument, market.cu:520,531, which
a graph would freeze). Each test captures steps once, then replays them with new
quotes copied into the captured input tensors between replays (eager work and a
synchronisation between replays), and compares every replay with the oracle run
on the same quotes.
"""
import numpy as np
import pytest
import torch

from parity_util import DEV, compare_bbo, compare_fills, compare_portfolios, make_market

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def _setup(cfg_index, M, layout, **knobs):
    from astra_cuda.workloads import CONFIGS, QuoteStream
    from oracle.oracle import OracleMarket
    cfg = CONFIGS[cfg_index]
    qs = QuoteStream(cfg, np.arange(M))
    g = make_market(M, cfg.L, cfg.O, cfg.F, cfg.C, **knobs)
    gf, gb = g.new_fill_batch(layout), g.new_bbo_batch()
    o = OracleMarket(M, cfg.L, cfg.O, cfg.F, cfg.C)
    of, ob = o.new_fill_batch(), o.new_bbo_batch()
    return cfg, qs, g, gf, gb, o, of, ob


def _load(static, quotes):
    for dst, src in zip(static, quotes):
        dst.copy_(torch.from_numpy(np.ascontiguousarray(src, dtype=np.int32)))


@pytest.mark.parametrize("cfg_index,M,layout,knobs", [
    (2, 2000, "columns", {}),
    (2, 2000, "rows", {}),
    # the launch of a large grid: 64 markets per wavefront, helper wavefronts
    (3, 4000, "columns", {"per_wave": 64, "fill_rows": 4, "helpers": 2}),
])
def test_gpu_graph_of_one_step_replayed(cfg_index, M, layout, knobs):
    """One step (add_two_sided_quotes, get_bbos, update_last_prices) captured once,
    replayed for every step of the run; each replay is checked against the oracle."""
    cfg, qs, g, gf, gb, o, of, ob = _setup(cfg_index, M, layout, **knobs)
    steps = 600  # the ring of 1024 orders wraps at step 512
    static = [torch.zeros(M, dtype=torch.int32, device=DEV) for _ in range(5)]
    q0 = qs.step(0)  # (config 3's quotes come from a random walk: each step once, in order)
    _load(static, q0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g.add_two_sided_quotes(*static, gf)
        g.get_bbos(gb)
        gb.update_last_prices(gf)
    torch.cuda.synchronize()
    assert g.global_tid == 0  # capturing runs nothing
    _log(f"graph of one step: config {cfg_index}, {M} markets, {layout}, {knobs}")
    for t in range(steps):
        q = q0 if t == 0 else qs.step(t)
        if t:
            _load(static, q)
        graph.replay()
        o.add_two_sided_quotes(*q, of, nthreads=8)
        o.get_bbos(ob, nthreads=8)
        o.update_last_prices(ob, of)
        torch.cuda.synchronize()
        where = f"graph replay {t}"
        compare_fills(gf, of, cfg.F, where)
        compare_bbo(gb, ob, where)
        if t % 100 == 0 or t == steps - 1:
            compare_portfolios(g, o, where)
    assert g.global_tid == o.global_tid == 2 * steps


def test_gpu_graph_of_several_steps_replayed():
    """Four steps captured in one graph (each with input tensors of its own),
    replayed with the next four steps' quotes;
    after each replay the last step's fills and BBOs, the portfolios and the TID
    counter equal the oracle's after the same steps."""
    cfg, qs, g, gf, gb, o, of, ob = _setup(2, 1500, "columns")
    K, replays = 4, 150
    static = [[torch.zeros(1500, dtype=torch.int32, device=DEV) for _ in range(5)] for _ in range(K)]
    first = [qs.step(k) for k in range(K)]
    for k in range(K):
        _load(static[k], first[k])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for k in range(K):
            g.add_two_sided_quotes(*static[k], gf)
        g.get_bbos(gb)
    _log(f"graph of {K} steps, {replays} replays")
    for r in range(replays):
        for k in range(K):
            q = first[k] if r == 0 else qs.step(r * K + k)
            if r:
                _load(static[k], q)
            o.add_two_sided_quotes(*q, of, nthreads=8)
        o.get_bbos(ob, nthreads=8)
        graph.replay()
        torch.cuda.synchronize()
        where = f"replay {r}"
        compare_fills(gf, of, cfg.F, where)
        compare_bbo(gb, ob, where)
        compare_portfolios(g, o, where)
        assert g.global_tid == o.global_tid == 2 * K * (r + 1), where


def test_gpu_tid_counter_set_and_clone():
    """The TID counter can be set from the host (on the stream) and is copied
    with the book; the next call's rows carry it."""
    from astra_cuda import order_matching as aom
    g = aom.VecMarket(4, 16, 8, 8, 4)
    fills = g.new_fill_batch()
    one = torch.ones(4, dtype=torch.int32, device=DEV)
    g.global_tid = 1000
    assert g.global_tid == 1000
    c = g.clone()
    # market m: a bid of 1 at price 3 by customer 0, then an ask of 1 at 3 by customer 1
    g.add_two_sided_quotes(3 * one, one, 0 * one, 0 * one, 0 * one, fills)
    c.add_two_sided_quotes(3 * one, one, 0 * one, 0 * one, 0 * one, fills)
    assert g.global_tid == c.global_tid == 1002
    g.add_two_sided_quotes(0 * one, 0 * one, 3 * one, one, one, fills)
    torch.cuda.synchronize()
    assert fills.fill_counts.tolist() == [1, 1, 1, 1]
    assert fills.fill_tid[:, 0].tolist() == [1003] * 4        # the ask's TID: base 1002 + 1
    assert fills.fill_quote_tid[:, 0].tolist() == [1000] * 4  # the resting bid's
    assert g.global_tid == 1004 and c.global_tid == 1002
