"""The multi-step call (astra_market_add_two_sided_quotes_steps) on the host
emulation build (CPU only): one call of K steps must leave exactly what K single
calls leave (the whole engine workspace byte for byte except the head-size
cache, which the multi-step call fills more of; the fill batch including rows
beyond the last count; the TID counter), and its per-step fill counts and BBOs
must be the oracle's step by step."""
import os

import numpy as np
import pytest

from emu_engine import EmuMarket
from oracle.oracle import OracleMarket
from ws_layout import normalized

BBO = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes")


def _emu(M, L, O, F, C, stage_budget):
    old = os.environ.get("ASTRA_MARKET_STAGE_BUDGET")
    if stage_budget is not None:
        os.environ["ASTRA_MARKET_STAGE_BUDGET"] = str(stage_budget)
    try:
        return EmuMarket(M, L, O, F, C)
    finally:
        if old is None:
            os.environ.pop("ASTRA_MARKET_STAGE_BUDGET", None)
        else:
            os.environ["ASTRA_MARKET_STAGE_BUDGET"] = old


def _fields(fills):
    return {f: np.array(getattr(fills, f)) for f in fills.FIELDS}


def run_multistep(M, L, O, F, C, gen, chunks, layout, stage_budget):
    single = _emu(M, L, O, F, C, stage_budget)
    multi = single.clone()
    om = OracleMarket(M, L, O, F, C)
    fs, fm, fo = single.new_fill_batch(layout), multi.new_fill_batch(layout), om.new_fill_batch()
    ob = om.new_bbo_batch()
    t = 0
    for K in chunks:
        qs = [gen(t + k) for k in range(K)]
        stacked = [np.stack([q[i] for q in qs]) if K else np.zeros((0, M), np.int32) for i in range(5)]
        counts = np.full((K, M), -7, np.int32)
        bbos = np.full((4, K, M), -7, np.int32)
        multi.add_two_sided_quotes_steps(*stacked, fm, counts, bbos)
        for k in range(K):
            single.add_two_sided_quotes(*qs[k], fs)
            om.add_two_sided_quotes(*qs[k], fo)
            om.get_bbos(ob)
            assert np.array_equal(counts[k], fo.fill_counts), (t + k, "counts")
            for j, f in enumerate(BBO):
                assert np.array_equal(bbos[j, k], getattr(ob, f)), (t + k, f)
        t += K
        assert multi.global_tid == single.global_tid == om.global_tid, t
        assert np.array_equal(normalized(multi.ws, M, L, O, C), normalized(single.ws, M, L, O, C)), \
            f"workspace after step {t}"
        a, b = _fields(fm), _fields(fs)
        for f in a:
            assert np.array_equal(a[f], b[f]), (t, f)
        assert np.array_equal(multi.portfolios, om.customer_portfolios), t
    return t


ALIAS_CASES = [  # M, L, O, F, C, seed: tiny rings, overflow, aliasing
    (64, 8, 1, 3, 3, 1),
    (64, 16, 3, 2, 4, 3),
    (64, 128, 7, 16, 5, 5),
    (48, 512, 6, 8, 70, 7),
]


@pytest.mark.parametrize("stage_budget,layout", [(None, "columns"), (1, "columns"), (1, "rows"),
                                                 (0, "rows")])
@pytest.mark.parametrize("M,L,O,F,C,seed", ALIAS_CASES)
def test_multistep_aliasing(M, L, O, F, C, seed, stage_budget, layout):
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

    assert run_multistep(M, L, O, F, C, gen, [1, 7, 0, 30, 2, 40], layout, stage_budget) == 80


@pytest.mark.parametrize("stage_budget,layout", [(None, "columns"), (1, "rows")])
def test_multistep_config3_sample(stage_budget, layout):
    """Config 3's stream (ring wrap after 512 steps, so eviction) on 120 markets."""
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[3]
    qs = QuoteStream(cfg, np.arange(120))
    run_multistep(120, cfg.L, cfg.O, cfg.F, cfg.C, qs.step, [300, 1, 299, 100], layout, stage_budget)


def test_multistep_errors():
    from emu_engine import _check, lib
    em = EmuMarket(4, 8, 4, 4, 2)
    f = em.new_fill_batch()
    z = np.zeros((0, 4), np.int32)
    em.add_two_sided_quotes_steps(z, z, z, z, z, f)  # zero steps: nothing happens
    assert em.global_tid == 0
    with pytest.raises(RuntimeError, match="steps must be >= 0"):
        _check(lib().astra_market_add_two_sided_quotes_steps(em.h, -1, *([None] * 17), None))
    q = np.ones((2, 4), np.int32)
    with pytest.raises(RuntimeError, match="NULL input"):
        _check(lib().astra_market_add_two_sided_quotes_steps(em.h, 2, q.ctypes.data, *([None] * 16),
                                                             None))
    assert em.global_tid == 0
