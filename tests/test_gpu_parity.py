"""HIP engine vs the CPU oracle, bit-exact (GPU).

Everything goes through the drop-in API (astra_cuda.order_matching, i.e. the
C ABI in libastra_market.so). Bar: every fill field of every row a call wrote,
fill_counts, BBOs, last prices and portfolios are identical to the oracle's on
the same inputs, after every step.
"""
import numpy as np
import pytest
import torch

from kat_harness import load_kats, run_scenario
from parity_util import (DEV, GpuAdapter, GpuRowAdapter, compare_bbo, compare_fills, compare_portfolios,
                         run_parity, t32)
from quote_gen import EXT_CAP_CASES, drifting_window_gen

pytestmark = pytest.mark.gpu

SCENARIOS = load_kats()


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("sc", SCENARIOS, ids=[s["name"] for s in SCENARIOS])
@pytest.mark.parametrize("adapter", [GpuAdapter, GpuRowAdapter], ids=["columns", "rows"])
def test_gpu_kat(sc, adapter):
    _log(f"kat {sc['name']} {adapter.layout}")
    run_scenario(sc, adapter)


def test_gpu_library_is_the_in_tree_build():
    import astra_cuda._native as nat
    lib = nat.lib()
    assert lib._name.endswith("astra_cuda/libastra_market.so")


def _stream_gen(cfg_index, markets=None, M_override=None, seed=0):
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[cfg_index]
    qs = QuoteStream(cfg, markets, seed=seed)
    return cfg, qs.step


def test_gpu_config1_full_run():
    """Config 1 exactly as specified (64 markets x 1000 steps, ring wraps at step 512)."""
    cfg, gen = _stream_gen(1)
    _log("config 1: 64 x 1000")
    r = run_parity(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C, cfg.steps, gen, full_every=100, label="cfg1")
    # config 1 quotes never self-cross, but resting orders do cross later quotes
    assert r["fill_rows"] > 0


def test_gpu_config2_subset():
    cfg, gen = _stream_gen(2, np.arange(3000))
    _log("config 2 subset: 3000 x 400")
    r = run_parity(3000, cfg.L, cfg.O, cfg.F, cfg.C, 400, gen, full_every=200, label="cfg2")
    assert r["fill_rows"] > 3000


@pytest.mark.parametrize("stage_budget", [None, 1])
def test_gpu_config2_subset_after_many_wraps(stage_budget):
    """Config 2 markets 0..1999 for 3000 steps: the ring of 1024 orders wraps about
    six times, so crossing quotes walk chains of consumed orders (zero-size fills,
    levels emptied one after another) on the staged book's lean runs; with stage
    budget 1 every market that crosses twice in a call is finished staged. Every
    row of every step is compared with the oracle."""
    cfg, gen = _stream_gen(2, np.arange(2000))
    _log(f"config 2 subset: 2000 x 3000, stage budget {stage_budget}")
    r = run_parity(2000, cfg.L, cfg.O, cfg.F, cfg.C, 3000, gen, full_every=500, label="cfg2 wraps",
                   stage_budget=stage_budget)
    assert r["fill_rows"] > 2000


@pytest.mark.parametrize("cfg_index,M,steps,seed", [
    (3, 3000, 1000, 7), (3, 3000, 1000, 201), (2, 1500, 3000, 13), (4, 300, 2000, 99)])
def test_gpu_streams_with_other_seeds(cfg_index, M, steps, seed):
    """The config streams drawn with seeds other than their own (0): other books,
    other crossings and, after the ring wraps, other chains of consumed orders,
    every row of every step against the oracle."""
    cfg, gen = _stream_gen(cfg_index, np.arange(M), seed=seed)
    _log(f"config {cfg_index} stream, seed {seed}: {M} x {steps}")
    r = run_parity(M, cfg.L, cfg.O, cfg.F, cfg.C, steps, gen, full_every=250,
                   label=f"cfg{cfg_index} seed {seed}")
    assert r["fill_rows"] > M


@pytest.mark.parametrize("stage_budget,layout", [(None, "columns"), (1, "columns"), (None, "rows")])
def test_gpu_config3_subset_with_eviction(stage_budget, layout):
    """Config 3 markets 0..3999 for all 1000 steps (the ring of 1024 wraps after 512 steps).
    With stage_budget=1 every market that crosses twice in a call finishes on the
    LDS-staged path."""
    cfg, gen = _stream_gen(3, np.arange(4000))
    _log(f"config 3 subset: 4000 x 1000, stage budget {stage_budget}, {layout}")
    r = run_parity(4000, cfg.L, cfg.O, cfg.F, cfg.C, 1000, gen, bbo_every=1, full_every=250,
                   label="cfg3", stage_budget=stage_budget, layout=layout)
    assert r["fill_rows"] > 4000


@pytest.mark.parametrize("helpers,hand_lanes,stage_budget,layout,hand_queue", [
    (0, None, None, "columns", None), (3, 64, None, "columns", None), (3, 1, None, "columns", None),
    (2, 64, None, "rows", None), (3, 64, 1, "columns", None), (2, 2, 4, "rows", None),
    (2, 64, 1, "columns", 13), (3, 64, None, "columns", 1)])
def test_gpu_config3_subset_helpers(helpers, hand_lanes, stage_budget, layout, hand_queue):
    """Config 3 markets 0..3999 for all 1000 steps with 4 fill rows per lane and 64
    markets per wavefront, the launch shape of a large grid (a grid this small
    would otherwise run 32 per wavefront, without helpers): markets whose walks are
    long go to the helper
    wavefront of their workgroup (helpers 2 or 3) or, without helpers, are
    finished by their own wavefront after its loop. hand_lanes 64 hands off
    every zero-size walk, 1 only a lane left alone; stage budget 1 hands off
    every market that crosses twice; hand_queue 13 lets every slot of a
    workgroup fill (lanes then find no free slot and go on in global memory), 1
    hands off only to an idle helper."""
    cfg, gen = _stream_gen(3, np.arange(4000))
    _log(f"config 3 subset with helpers {helpers}, hand lanes {hand_lanes}, budget {stage_budget}, "
         f"{layout}, hand queue {hand_queue}")
    r = run_parity(4000, cfg.L, cfg.O, cfg.F, cfg.C, 1000, gen, bbo_every=1, full_every=250,
                   label="cfg3 helpers", stage_budget=stage_budget, layout=layout, fill_rows=4,
                   helpers=helpers, hand_lanes=hand_lanes, hand_queue=hand_queue, per_wave=64)
    assert r["fill_rows"] > 4000


@pytest.mark.parametrize("helpers,helper_polls", [(2, 1), (3, 1), (2, 8), (3, 64)])
def test_gpu_config3_subset_helpers_give_up(helpers, helper_polls):
    """The helper wavefronts' bounded wait, cut short from the host: after
    helper_polls idle polls a helper closes its workgroup's queue, finishes the
    markets already handed to it and leaves; lanes that would hand off later keep
    their markets and finish them in global memory. With 1 poll (about 0.1 us)
    every helper leaves before its wavefronts can hand anything off; with 8 and
    64 helpers leave in the middle of a call, some with markets in their queue.
    Every result must still equal the oracle's, and the give-ups are counted in
    the workspace."""
    from parity_util import helper_exits
    cfg, gen = _stream_gen(3, np.arange(4000))
    _log(f"config 3 subset, helpers {helpers} giving up after {helper_polls} idle polls")
    r = run_parity(4000, cfg.L, cfg.O, cfg.F, cfg.C, 1000, gen, bbo_every=1, full_every=250,
                   label=f"cfg3 helpers give up {helper_polls}", layout="columns", fill_rows=4,
                   helpers=helpers, per_wave=64, helper_polls=helper_polls)
    assert r["fill_rows"] > 4000
    exits = helper_exits(r["gpu"])
    _log(f"helper give-ups over 1000 calls: {exits}")
    if helper_polls == 1:
        # nearly every helper of every call (4000 markets: 63 market wavefronts in
        # 21 or 32 workgroups; a market wavefront needs two memory round trips
        # before it can end)
        assert exits >= 10000
    elif helper_polls == 8:
        assert exits > 0


@pytest.mark.parametrize("fill_rows,per_wave,stage_budget", [
    (None, None, None), (4, 64, None), (4, 64, 1)])
def test_gpu_config4_subset_deep_book(fill_rows, per_wave, stage_budget):
    """Config 4 shape (L=512: 8 mask words, O=F=4096, C=64) on 300 markets x 2000 steps;
    also with 4 fill rows per lane and 64 markets per wavefront, the launch of a large
    grid, where a staged book of 4096 orders reuses its wavefront's row buffer in LDS
    (stage budget 1: every market that crosses twice)."""
    cfg, gen = _stream_gen(4, np.arange(300))
    _log(f"config 4 subset: 300 x 2000, fill rows {fill_rows}, per wave {per_wave}, "
         f"stage budget {stage_budget}")
    r = run_parity(300, cfg.L, cfg.O, cfg.F, cfg.C, 2000, gen, bbo_every=5, full_every=500,
                   label="cfg4", fill_rows=fill_rows, per_wave=per_wave, stage_budget=stage_budget)
    assert r["fill_rows"] > 300


# (M, L, O, F, C, steps, seed): tiny rings and fill caps force eviction aliasing,
# self links, zero/negative fills and overflow; prices/sizes/customers include
# rejected and out-of-range values. L covers 1, 2, 4, 8 and 16 mask words.
ALIAS_CASES = [
    (257, 8, 1, 3, 3, 200, 11),
    (257, 8, 2, 4, 3, 200, 12),
    (300, 16, 3, 2, 4, 200, 13),
    (300, 70, 5, 6, 4, 300, 14),
    (300, 128, 7, 16, 5, 300, 15),
    (200, 200, 9, 5, 3, 300, 16),
    (200, 512, 6, 8, 70, 300, 17),
    (150, 1000, 11, 9, 3, 300, 18),
    (128, 128, 7, 16, 1024, 300, 19),  # C = 1024, the reference's customer cap
]


@pytest.mark.parametrize("stage_budget,layout,fill_rows,helpers", [
    (None, "columns", None, None), (1, "columns", None, None), (1, "rows", None, None),
    (1, "columns", 4, 0), (1, "columns", 4, 3), (None, "rows", 4, 2), (1, "rows", 4, 2)])
@pytest.mark.parametrize("M,L,O,F,C,steps,seed", ALIAS_CASES)
def test_gpu_aliasing_and_overflow(M, L, O, F, C, steps, seed, stage_budget, layout, fill_rows, helpers):
    _log(f"aliasing M={M} L={L} O={O} F={F} stage budget {stage_budget} {layout} fill rows {fill_rows} "
         f"helpers {helpers}")
    rng = np.random.default_rng(seed)
    hot = max(4, min(L, 24))  # concentrate prices so books cross often

    def gen(t):
        base = rng.integers(0, max(1, L - hot), 1)[0]
        bid = (base + rng.integers(-1, hot + 1, M)).astype(np.int32)
        ask = (base + rng.integers(-1, hot + 1, M)).astype(np.int32)
        bid[rng.random(M) < 0.02] = L  # rejected: price >= L
        ask[rng.random(M) < 0.02] = -1  # rejected here: negative price
        return (bid, rng.integers(-1, 8, M).astype(np.int32), ask,
                rng.integers(-1, 8, M).astype(np.int32), rng.integers(-1, C + 2, M).astype(np.int32))

    r = run_parity(M, L, O, F, C, steps, gen, full_every=50, label=f"alias L{L} O{O}",
                   stage_budget=stage_budget, layout=layout, fill_rows=fill_rows, helpers=helpers,
                   per_wave=None if helpers is None else 64)
    if O <= 3:
        assert r["overflows"] > 0


@pytest.mark.parametrize("name,M,L,O,F,C,steps", EXT_CAP_CASES, ids=[c[0] for c in EXT_CAP_CASES])
def test_gpu_extended_caps(name, M, L, O, F, C, steps):
    """The largest extended shape (16 mask words, slot indices up to 32767, 65,536 fill
    rows and customers), unstaged; "wrap" reuses every ring slot."""
    _log(f"extended caps {name}: M={M} L={L} O={O} F={F} C={C} x {steps} steps")
    every = 1 if steps < 1000 else 10
    r = run_parity(M, L, O, F, C, steps, drifting_window_gen(M, L, C, seed=21), bbo_every=every,
                   last_every=every, label=f"ext {name}")
    assert r["fill_rows"] > 0
    assert r["oracle"].order_next_slots.min() >= (O + 1000 if name == "wrap" else 2)


@pytest.mark.parametrize("per_wave,stage_budget", [(1, 1), (7, None), (32, 1), (33, None)])
def test_gpu_markets_per_wavefront(per_wave, stage_budget):
    """Fewer markets per wavefront than 64 (ASTRA_MARKET_PER_WAVE, read at creation):
    the same results, with staging (its cooperative copies use all 64 lanes)."""
    M, L, O, F, C, steps = 300, 16, 3, 4, 4, 150
    _log(f"per_wave {per_wave} stage budget {stage_budget}")
    rng = np.random.default_rng(per_wave)

    def gen(t):
        base = rng.integers(0, L - 12, 1)[0]
        bid = (base + rng.integers(-1, 13, M)).astype(np.int32)
        ask = (base + rng.integers(-1, 13, M)).astype(np.int32)
        return (bid, rng.integers(0, 8, M).astype(np.int32), ask, rng.integers(0, 8, M).astype(np.int32),
                rng.integers(0, C, M).astype(np.int32))

    r = run_parity(M, L, O, F, C, steps, gen, full_every=50, label=f"per_wave {per_wave}",
                   stage_budget=stage_budget, per_wave=per_wave)
    assert r["fill_rows"] > 0


def test_gpu_max_markets():
    """The reference's market cap, 2048 * 2048 = 4,194,304 markets (market.h:56), on a
    small book: launch geometry and 64-bit indexing at the largest grid, every output
    compared in full with the oracle over a few steps (eviction and overflow included)."""
    from astra_cuda import order_matching as aom
    M, L, O, F, C, steps = aom.MAX_MARKETS, 8, 2, 3, 4, 4
    _log(f"max markets M={M}")
    rng = np.random.default_rng(7)

    def gen(t):
        return (rng.integers(0, L, M).astype(np.int32), rng.integers(0, 6, M).astype(np.int32),
                rng.integers(0, L, M).astype(np.int32), rng.integers(0, 6, M).astype(np.int32),
                rng.integers(0, C, M).astype(np.int32))

    r = run_parity(M, L, O, F, C, steps, gen, full_every=1, label="max markets")
    assert r["fill_rows"] > 0 and r["overflows"] > 0


def test_gpu_reset_clear_clone_and_to_string():
    """Reset / ClearQuotes / copy constructor / ToString interleaved with trading."""
    from astra_cuda import order_matching as aom
    from oracle.oracle import OracleMarket
    M, L, O, F, C = 97, 40, 6, 12, 5
    rng = np.random.default_rng(7)
    g = aom.VecMarket(M, L, O, F, C)
    o = OracleMarket(M, L, O, F, C)
    gf, of = g.new_fill_batch(), o.new_fill_batch()
    gb, ob = g.new_bbo_batch(), o.new_bbo_batch()

    def step(gm, om, t):
        args = (rng.integers(0, L, M).astype(np.int32), rng.integers(0, 6, M).astype(np.int32),
                rng.integers(0, L, M).astype(np.int32), rng.integers(0, 6, M).astype(np.int32),
                rng.integers(0, C, M).astype(np.int32))
        gm.add_two_sided_quotes(*(t32(a) for a in args), gf)
        om.add_two_sided_quotes(*args, of)
        compare_fills(gf, of, F, f"step {t}")

    for t in range(300):
        step(g, o, t)
        if t % 37 == 5:
            mask = rng.random(M) < 0.3
            g.clear_quotes(torch.as_tensor(mask).to(DEV))
            o.clear_quotes(mask)
        if t == 150:
            g.reset()
            o.reset()
        if t % 25 == 0:
            g.get_bbos(gb)
            o.get_bbos(ob)
            compare_bbo(gb, ob, f"step {t}")
            compare_portfolios(g, o, f"step {t}")
            for m in (0, 1, M // 2, M - 1):
                assert g.to_string(m) == o.to_string(m), (t, m)
    assert g.to_string(M) == o.to_string(M)
    # copy constructor: the clone continues identically and independently
    g2, o2 = g.clone(), o.clone()
    assert g2.global_tid == o2.global_tid == g.global_tid
    for t in range(300, 340):
        step(g2, o2, t)
    compare_portfolios(g2, o2, "clone")
    g2.get_bbos(gb)
    o2.get_bbos(ob)
    compare_bbo(gb, ob, "clone")
    # the original is untouched by the clone's trading
    g.get_bbos(gb)
    o.get_bbos(ob)
    compare_bbo(gb, ob, "original after clone")
    compare_portfolios(g, o, "original after clone")


def test_gpu_portfolio_view_is_live_and_copy_to():
    from astra_cuda import order_matching as aom
    g = aom.VecMarket(3, 128, 64, 16)
    f = g.new_fill_batch()
    view = g.get_customer_portfolios()
    one = torch.ones(3, dtype=torch.int32, device=DEV)
    g.add_two_sided_quotes(one * 50, one * 10, one * 0, one * 0, one * 0, f)
    g.add_two_sided_quotes(one * 0, one * 0, one * 50, one * 4, one * 1, f)
    assert view.data_ptr() == g.get_customer_portfolios().data_ptr()
    assert view[:, 0].tolist() == [[4, -200]] * 3 and view[:, 1].tolist() == [[-4, 200]] * 3
    buf = torch.zeros(3, 16, 2, dtype=torch.int32, device=DEV)
    g.copy_customer_portfolios_to(buf)
    assert torch.equal(buf, view)
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        g.copy_customer_portfolios_to(torch.zeros(3, 15, 2, dtype=torch.int32, device=DEV))


def test_gpu_current_stream_is_used():
    """Work issued inside a torch stream context runs on that stream, in order."""
    from astra_cuda import order_matching as aom
    from oracle.oracle import OracleMarket
    M, L, O, F, C = 2000, 128, 64, 32, 16
    rng = np.random.default_rng(3)
    g = aom.VecMarket(M, L, O, F, C)
    o = OracleMarket(M, L, O, F, C)
    gf, of = g.new_fill_batch(), o.new_fill_batch()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        for t in range(50):
            args = [rng.integers(0, L, M), rng.integers(1, 9, M), rng.integers(0, L, M),
                    rng.integers(1, 9, M), rng.integers(0, C, M)]
            args = [a.astype(np.int32) for a in args]
            ins = [torch.as_tensor(a).to(DEV, non_blocking=False) for a in args]
            g.add_two_sided_quotes(*ins, gf)
            o.add_two_sided_quotes(*args, of)
        s.synchronize()
    compare_fills(gf, of, F, "stream")
    compare_portfolios(g, o, "stream")


def test_gpu_input_validation_errors():
    from astra_cuda import order_matching as aom
    g = aom.VecMarket(4, 128, 64, 16)
    f = g.new_fill_batch()
    ok = torch.zeros(4, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match=r"bid_px.size\(0\) == num_markets_"):
        g.add_two_sided_quotes(torch.zeros(5, dtype=torch.int32, device=DEV), ok, ok, ok, ok, f)
    with pytest.raises(RuntimeError, match="ask_px tensor must be on device 0"):
        g.add_two_sided_quotes(ok, ok, torch.zeros(4, dtype=torch.int32), ok, ok, f)
    with pytest.raises(RuntimeError, match="customer_ids tensor must be contiguous"):
        g.add_two_sided_quotes(ok, ok, ok, ok, torch.zeros(8, dtype=torch.int32, device=DEV)[::2], f)
    with pytest.raises(RuntimeError, match="must be int32"):
        g.add_two_sided_quotes(ok, ok.long(), ok, ok, ok, f)
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        aom.VecMarket(4, 129, 64, 16)  # market.cu:339
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        aom.VecMarket(4, 128, 64, 16, threads_per_block=0)  # market.cu:343
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        aom.VecMarket(4, 128, 64, 16, device_id=torch.cuda.device_count())  # market.cu:350
    with pytest.raises(RuntimeError, match="reset_indices"):
        g.clear_quotes(torch.zeros(4, dtype=torch.int32, device=DEV))
    # no state change from the rejected calls: TID still 0
    assert g.global_tid == 0


def test_gpu_row_layout_fill_batch():
    """FillBatch(layout="rows"): the fields are [M, F] views of one [M, F, 8] buffer with
    the dtypes of the reference; clone keeps the layout; assigning a field leaves it."""
    from astra_cuda import order_matching as aom
    M, F = 7, 5
    g = aom.VecMarket(M, 32, 16, F, 4)
    fr, fc = g.new_fill_batch(layout="rows"), g.new_fill_batch()
    assert fr.layout == "rows" and fc.layout == "columns"
    for f in aom.FillBatch.FIELDS:
        a, b = getattr(fr, f), getattr(fc, f)
        assert a.shape == b.shape and a.dtype == b.dtype, f
    one = torch.ones(M, dtype=torch.int32, device=DEV)
    for fills in (fr, fc):
        g2 = aom.VecMarket(M, 32, 16, F, 4)
        g2.add_two_sided_quotes(one * 10, one * 3, one * 20, one * 2, one * 0, fills)
        g2.add_two_sided_quotes(one * 20, one * 5, one * 10, one * 4, one * 1, fills)
    for f in aom.FillBatch.FIELDS:
        assert torch.equal(getattr(fr, f), getattr(fc, f)), f
    assert fr.fill_is_sell_quote.any() or not fc.fill_is_sell_quote.any()
    b1, b2 = g.new_bbo_batch(), g.new_bbo_batch()
    b1.update_last_prices(fr)
    b2.update_last_prices(fc)
    assert torch.equal(b1.last_prices, b2.last_prices) and b1.last_prices.tolist() == [20] * M
    cl = fr.clone()
    assert cl.layout == "rows" and torch.equal(cl.fill_prices, fr.fill_prices)
    assert cl.fill_prices.data_ptr() != fr.fill_prices.data_ptr()
    fr.fill_sizes = torch.zeros((M, F), dtype=torch.int32, device=DEV)
    assert fr.layout == "columns"
    with pytest.raises(RuntimeError, match="must be contiguous"):
        g.add_two_sided_quotes(one, one, one, one, one * 0, fr)
