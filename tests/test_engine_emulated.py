"""The engine's kernel bodies, compiled for the host, against the oracle (CPU only).

Same per-market code and data layout as the GPU build (see tests/emu_engine.py),
driven through the C ABI. These checks run without a GPU: logic, layout, the
mask/level/record bookkeeping under eviction aliasing, and the diagnostic work
counters. The GPU parity tests (test_gpu_*.py) repeat the parity checks on the
device build.
"""
import os

import numpy as np
import pytest

from emu_engine import EmuAdapter, EmuMarket, EmuRowAdapter
from kat_harness import FILL_FIELDS, load_kats, run_scenario
from quote_gen import EXT_CAP_CASES, drifting_window_gen
from oracle.oracle import OracleMarket

SCENARIOS = load_kats()


@pytest.mark.parametrize("sc", SCENARIOS, ids=[s["name"] for s in SCENARIOS])
@pytest.mark.parametrize("adapter", [EmuAdapter, EmuRowAdapter], ids=["columns", "rows"])
def test_emulated_kat(sc, adapter):
    run_scenario(sc, adapter)


def _compare(em, ef, eb, om, of, ob, F, where):
    assert np.array_equal(ef.fill_counts, of.fill_counts), where
    eff = np.where(of.fill_counts < 0, F, of.fill_counts)
    k = int(eff.max(initial=0))
    valid = np.arange(k)[None, :] < eff[:, None]
    for f in FILL_FIELDS:
        a, b = getattr(ef, f)[:, :k], getattr(of, f)[:, :k]
        assert np.array_equal(np.where(valid, a, 0), np.where(valid, b, 0)), (where, f)
    for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
        assert np.array_equal(getattr(eb, f), getattr(ob, f)), (where, f)
    assert np.array_equal(em.portfolios, om.customer_portfolios), where


def _emu(M, L, O, F, C, stage_budget=None, extended=None, fill_rows=None):
    """Emulated engine; stage_budget sets the passes before a market's book is staged
    (0: never), fill_rows (2 or 4) the fill rows a lane buffers before writing them
    (by default 2 for grids this small), both read by the engine when the market is
    created."""
    env = {"ASTRA_MARKET_STAGE_BUDGET": stage_budget, "ASTRA_MARKET_FILL_ROWS": fill_rows}
    old = {k: os.environ.get(k) for k in env}
    try:
        for k, v in env.items():
            if v is not None:
                os.environ[k] = str(v)
        return EmuMarket(M, L, O, F, C, extended=extended)
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v


def _run(M, L, O, F, C, steps, gen, with_stats=False, stage_budget=None, layout="columns",
         extended=None, fill_rows=None):
    em, om = _emu(M, L, O, F, C, stage_budget, extended, fill_rows), OracleMarket(M, L, O, F, C)
    ef, of = em.new_fill_batch(layout), om.new_fill_batch()
    eb, ob = em.new_bbo_batch(), om.new_bbo_batch()
    stats = np.zeros(11, np.int64)
    ostats = {"inserts": 0, "fills": 0, "levels_emptied": 0, "overflows": 0}
    if with_stats:
        em.set_stats(stats)
    for t in range(steps):
        args = gen(t)
        em.add_two_sided_quotes(*args, ef)
        c = om.add_two_sided_quotes(*args, of)
        for k in ostats:
            ostats[k] += c[k]
        em.update_last_prices(eb, ef)
        om.update_last_prices(ob, of)
        em.get_bbos(eb)
        om.get_bbos(ob)
        _compare(em, ef, eb, om, of, ob, F, f"step {t}")
    if with_stats:
        em.set_stats(None)
        assert stats.tolist()[:4] == [ostats["inserts"], ostats["fills"], ostats["levels_emptied"],
                                      ostats["overflows"]]
        ostats["fast_forwards"] = int(stats[4])
        ostats["staged"] = int(stats[6])
        ostats["zero_runs"] = int(stats[8])
        ostats["zero_rows"] = int(stats[9])
        ostats["crossing"] = int(stats[7])
        ostats["bbo_book_reads"] = int(stats[10])
    assert em.global_tid == om.global_tid
    ostats["last_fills"] = of
    return em, om, ostats


ALIAS_CASES = [
    (64, 8, 1, 3, 3, 150, 1),
    (64, 8, 2, 4, 3, 150, 2),
    (64, 16, 3, 2, 4, 150, 3),
    (64, 70, 5, 6, 4, 200, 4),
    (64, 128, 7, 16, 5, 200, 5),
    (48, 200, 9, 5, 3, 200, 6),
    (48, 512, 6, 8, 70, 200, 7),
    (32, 1000, 11, 9, 3, 200, 8),
    (64, 128, 7, 16, 1024, 200, 9),  # C = 1024, the reference's customer cap
]


@pytest.mark.parametrize("stage_budget,layout,fill_rows",
                         [(None, "columns", None), (0, "columns", None), (1, "columns", None),
                          (3, "columns", None), (None, "rows", None), (1, "rows", None),
                          (None, "columns", 4), (1, "rows", 4)])
@pytest.mark.parametrize("M,L,O,F,C,steps,seed", ALIAS_CASES)
def test_emulated_aliasing_vs_oracle(M, L, O, F, C, steps, seed, stage_budget, layout, fill_rows):
    rng = np.random.default_rng(seed)
    hot = max(4, min(L, 24))

    def gen(t):
        base = rng.integers(0, max(1, L - hot), 1)[0]
        bid = (base + rng.integers(-1, hot + 1, M)).astype(np.int32)
        ask = (base + rng.integers(-1, hot + 1, M)).astype(np.int32)
        bid[rng.random(M) < 0.02] = L
        ask[rng.random(M) < 0.02] = -1
        return (bid, rng.integers(-1, 8, M).astype(np.int32), ask,
                rng.integers(-1, 8, M).astype(np.int32), rng.integers(-1, C + 2, M).astype(np.int32))

    _, _, st = _run(M, L, O, F, C, steps, gen, with_stats=True, stage_budget=stage_budget, layout=layout,
                    fill_rows=fill_rows)
    # tiny rings exercise both overflow routes: the repeating-state fast-forward
    # and the ordinary F-th fill (with O = 1 every overflow repeats)
    assert st["fast_forwards"] > 0
    if O > 1:
        assert st["overflows"] > st["fast_forwards"]


@pytest.mark.parametrize("name,M,L,O,F,C,steps", EXT_CAP_CASES, ids=[c[0] for c in EXT_CAP_CASES])
def test_emulated_extended_caps(name, M, L, O, F, C, steps):
    M = min(M, 16)
    _, om, st = _run(M, L, O, F, C, steps, drifting_window_gen(M, L, C, seed=21), with_stats=True)
    assert st["fills"] > 0
    # the slot counter counts every accepted insert (slot = counter % O)
    assert om.order_next_slots.min() >= (O + 1000 if name == "wrap" else 2)


def test_emulated_config1_full_run():
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[1]
    qs = QuoteStream(cfg)
    _, _, st = _run(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C, cfg.steps, qs.step, with_stats=True)
    assert st["fills"] > 0


@pytest.mark.parametrize("stage_budget,layout,fill_rows", [(None, "columns", None), (1, "columns", None),
                                                           (1, "rows", None), (None, "columns", 4)])
def test_emulated_config3_and_4_samples(stage_budget, layout, fill_rows):
    from astra_cuda.workloads import CONFIGS, QuoteStream
    for idx, M, steps in ((3, 300, 700), (4, 60, 400)):
        cfg = CONFIGS[idx]
        qs = QuoteStream(cfg, np.arange(M))
        _, _, st = _run(M, cfg.L, cfg.O, cfg.F, cfg.C, steps, qs.step, with_stats=True,
                        stage_budget=stage_budget, layout=layout, fill_rows=fill_rows)
        # A best level's head size is left for get_bbos to read from the book
        # only where the call's matching loop moved that side to a head whose
        # record it did not read (the next call reads and caches it): at most
        # two sides per crossing market, and far fewer than the 2 M per step a
        # cache that never refills would leave.
        assert 0 < st["bbo_book_reads"] <= 2 * st["crossing"], (idx, st)


def test_emulated_reset_clear_clone_to_string():
    M, L, O, F, C = 41, 40, 6, 12, 5
    rng = np.random.default_rng(9)
    em, om = EmuMarket(M, L, O, F, C), OracleMarket(M, L, O, F, C)
    ef, of = em.new_fill_batch(), om.new_fill_batch()
    eb, ob = em.new_bbo_batch(), om.new_bbo_batch()

    def step(e, o):
        args = (rng.integers(0, L, M).astype(np.int32), rng.integers(0, 6, M).astype(np.int32),
                rng.integers(0, L, M).astype(np.int32), rng.integers(0, 6, M).astype(np.int32),
                rng.integers(0, C, M).astype(np.int32))
        e.add_two_sided_quotes(*args, ef)
        o.add_two_sided_quotes(*args, of)

    for t in range(300):
        step(em, om)
        if t % 37 == 5:
            mask = rng.random(M) < 0.3
            em.clear_quotes(mask)
            om.clear_quotes(mask)
        if t == 150:
            em.reset()
            om.reset()
        em.get_bbos(eb)
        om.get_bbos(ob)
        _compare(em, ef, eb, om, of, ob, F, f"step {t}")
        if t % 10 == 0:
            for m in range(M):
                assert em.to_string(m) == om.to_string(m), (t, m)
    assert em.to_string(M) == om.to_string(M) and em.to_string(-1) == om.to_string(-1)
    e2, o2 = em.clone(), om.clone()
    for t in range(40):
        step(e2, o2)
        e2.get_bbos(eb)
        o2.get_bbos(ob)
        _compare(e2, ef, eb, o2, of, ob, F, f"clone step {t}")
    # the original did not move
    em.get_bbos(eb)
    om.get_bbos(ob)
    assert np.array_equal(eb.best_bid_prices, ob.best_bid_prices)
    assert np.array_equal(em.portfolios, om.customer_portfolios)


def test_emulated_zero_sized_shapes():
    # M = 0 and F = 0 and L = 0 are accepted by the reference constructor
    em = EmuMarket(0, 128, 16, 16, 4)
    em.add_two_sided_quotes(*(np.zeros(0, np.int32) for _ in range(5)), em.new_fill_batch())
    assert em.global_tid == 2
    em = EmuMarket(3, 128, 16, 0, 4)  # F = 0: the first crossing overflows
    f = em.new_fill_batch()
    one = np.ones(3, np.int32)
    em.add_two_sided_quotes(one * 5, one * 2, one * 5, one * 2, one * 0, f)
    assert f.fill_counts.tolist() == [-1, -1, -1]
    em = EmuMarket(3, 0, 16, 4, 4)  # L = 0: nothing is ever inserted
    f = em.new_fill_batch()
    em.add_two_sided_quotes(one * 0, one * 2, one * 0, one * 2, one * 0, f)
    b = em.new_bbo_batch()
    em.get_bbos(b)
    assert f.fill_counts.tolist() == [0, 0, 0] and b.best_bid_prices.tolist() == [-1, -1, -1]


# Markets of the config-3 stream whose books, after the order ring wraps, walk long
# runs of zero-size fills (consumed orders that slot reuse has linked into live
# lists): at O = 1024 runs of up to about 110 rows, and market 115 at O = F = 4096
# (extended shape) a run of 631 rows at step 2457, which spans ten flushes of the
# staged walk's 64-row buffer.
LONG_WALK_MARKETS = [115, 21099, 72837, 22178, 66430, 46789, 23615, 89995, 93998, 90015]


@pytest.mark.parametrize("stage_budget", [None, 1, 3, 0])
def test_emulated_zero_size_runs_after_the_wrap(stage_budget):
    """The config-3 stream past the ring wrap against the oracle, with markets
    staged after the default number of passes, after 1 and 3, and never."""
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[3]
    qs = QuoteStream(cfg, np.array(LONG_WALK_MARKETS + list(range(54)), np.int64))
    M = len(LONG_WALK_MARKETS) + 54
    _, _, st = _run(M, cfg.L, cfg.O, cfg.F, cfg.C, cfg.steps, qs.step, with_stats=True,
                    stage_budget=stage_budget)
    if stage_budget == 0:
        assert st["staged"] == 0 and st["zero_runs"] == 0
    else:
        assert st["zero_runs"] > 20 and st["zero_rows"] > 3 * st["zero_runs"]


def test_emulated_zero_size_run_of_631_rows():
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[3]
    O = F = 4096
    qs = QuoteStream(cfg, np.array([115, 0, 1, 2], np.int64))
    _, _, st = _run(4, cfg.L, O, F, cfg.C, 2458, qs.step, with_stats=True)
    # the last step's rows of market 0 (stream market 115), compared above, hold the run
    of = st["last_fills"]
    n = int(of.fill_counts[0])
    run = best = 0
    for v in of.fill_sizes[0, :n]:
        run = run + 1 if v == 0 else 0
        best = max(best, run)
    assert best == 631
    assert st["zero_rows"] >= 631
