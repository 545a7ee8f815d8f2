"""astra_market_add_two_sided_quotes_steps on the GPU, through
VecMarket.add_two_sided_quotes_steps: one launch of K steps against K single
calls of the drop-in path on a clone of the same engine (the whole workspace
byte for byte except the head-size cache, which the multi-step launch fills more
of; every fill-batch field including rows beyond the last count, the
TID counter, every step's fill counts and BBOs), and against the oracle at small
sizes."""
import numpy as np
import pytest
import torch

from oracle.oracle import OracleMarket
from parity_util import DEV, compare_fills, make_market, t32
from ws_layout import normalized

pytestmark = pytest.mark.gpu

BBO = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes")


def _run(M, L, O, F, C, stream, warm, chunks, layout, stage_budget=None, oracle=False, **knobs):
    print(f"multistep M={M} L={L} O={O} F={F} C={C} warm={warm} chunks={chunks} layout={layout} "
          f"budget={stage_budget} {knobs}", flush=True)
    single = make_market(M, L, O, F, C, stage_budget=stage_budget, **knobs)
    fs = single.new_fill_batch(layout)
    bs = single.new_bbo_batch()
    om = OracleMarket(M, L, O, F, C) if oracle else None
    if om is not None:
        fo, ob = om.new_fill_batch(), om.new_bbo_batch()
    for t in range(warm):
        q = stream(t)
        single.add_two_sided_quotes(*(t32(a) for a in q), fs)
        if om is not None:
            om.add_two_sided_quotes(*q, fo)
    multi = single.clone()
    fm = multi.new_fill_batch(layout)
    if layout == "rows":  # the same stale rows to start from
        fm._rows.copy_(fs._rows)
        fm.fill_counts.copy_(fs.fill_counts)
    else:
        for f in fs.FIELDS:
            getattr(fm, f).copy_(getattr(fs, f))
    t = warm
    for K in chunks:
        qs = [stream(t + k) for k in range(K)]
        stacked = [t32(np.stack([q[i] for q in qs]) if K else np.zeros((0, M), np.int32))
                   for i in range(5)]
        counts = torch.full((K, M), -7, dtype=torch.int32, device=DEV)
        bbos = torch.full((4, K, M), -7, dtype=torch.int32, device=DEV)
        multi.add_two_sided_quotes_steps(*stacked, fm, step_fill_counts=counts, step_bbos=bbos)
        for k in range(K):
            single.add_two_sided_quotes(*(t32(a) for a in qs[k]), fs)
            single.get_bbos(bs)
            assert torch.equal(counts[k], fs.fill_counts), (t + k, "counts")
            for j, f in enumerate(BBO):
                assert torch.equal(bbos[j, k], getattr(bs, f)), (t + k, f)
            if om is not None:
                om.add_two_sided_quotes(*qs[k], fo)
                om.get_bbos(ob)
                assert np.array_equal(counts[k].cpu().numpy(), fo.fill_counts), (t + k, "oracle counts")
                for j, f in enumerate(BBO):
                    assert np.array_equal(bbos[j, k].cpu().numpy(), getattr(ob, f)), (t + k, f)
        t += K
        torch.cuda.synchronize()
        assert multi.global_tid == single.global_tid, t
        assert torch.equal(normalized(multi._ws, M, L, O, C), normalized(single._ws, M, L, O, C)), \
            f"workspace after step {t}"
        if layout == "rows":
            assert torch.equal(fm._rows, fs._rows), t
        for f in fs.FIELDS:
            assert torch.equal(getattr(fm, f), getattr(fs, f)), (t, f)
        if om is not None:
            assert np.array_equal(multi.get_customer_portfolios().cpu().numpy(), om.customer_portfolios)
            if K:  # the last step's rows, field by field
                compare_fills(fm, fo, F, f"multi-step launch ending at step {t}")
    bm = multi.new_bbo_batch()
    multi.get_bbos(bm)  # the BBO cache a later get_bbos reads is the last step's
    for f in BBO:
        assert torch.equal(getattr(bm, f), getattr(bs, f)), f


# per_wave: markets per wavefront (7 and 32 leave lanes of each wavefront idle through
# every step, and 7 splits the markets over 46 wavefronts).
@pytest.mark.parametrize("stage_budget,layout,knobs", [
    (None, "columns", {}), (1, "rows", {}), (0, "columns", {}),
    (1, "columns", {"per_wave": 32}), (1, "rows", {"per_wave": 7})])
def test_gpu_multistep_aliasing_vs_oracle(stage_budget, layout, knobs):
    M, L, O, F, C = 320, 16, 3, 2, 4
    rng = np.random.default_rng(11)

    def gen(t):
        base = rng.integers(0, L - 12, 1)[0]
        bid = (base + rng.integers(-1, 13, M)).astype(np.int32)
        ask = (base + rng.integers(-1, 13, M)).astype(np.int32)
        bid[rng.random(M) < 0.02] = L
        ask[rng.random(M) < 0.02] = -1
        return (bid, rng.integers(-1, 8, M).astype(np.int32), ask,
                rng.integers(-1, 8, M).astype(np.int32), rng.integers(-1, C + 2, M).astype(np.int32))

    cache = {}

    def stream(t):  # the same quotes for both engines and the oracle
        if t not in cache:
            cache[t] = gen(t)
        return cache[t]

    _run(M, L, O, F, C, stream, 5, [1, 9, 0, 40, 64], layout, stage_budget, oracle=True, **knobs)


@pytest.mark.parametrize("idx,M,warm,chunks,layout", [
    (3, 100_000, 520, [1, 63, 150], "columns"),   # full config 3, ring wrapped (eviction)
    (3, 100_000, 0, [200], "rows"),
    (4, 20_000, 100, [1, 120], "columns"),        # full config 4 (W = 8)
    (2, 10_000, 0, [1, 99], "rows"),
])
def test_gpu_multistep_configs(idx, M, warm, chunks, layout):
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[idx]
    qs = QuoteStream(cfg, np.arange(M))
    cache = {}

    def stream(t):
        if t not in cache:
            cache.clear()
            cache[t] = qs.step(t)
        return cache[t]

    _run(M, cfg.L, cfg.O, cfg.F, cfg.C, stream, warm, chunks, layout)


@pytest.mark.parametrize("idx,M,warm,chunks,layout,knobs", [
    (3, 4000, 500, [20, 1, 39], "columns", {}),          # past the ring wrap (step 512)
    (3, 4000, 500, [60], "rows", {"per_wave": 16}),
    (2, 3000, 2000, [20, 20], "columns", {}),            # the ring wrapped about 4 times
    (4, 1500, 300, [25, 25], "columns", {}),             # W = 8, extended shape
])
def test_gpu_multistep_configs_vs_oracle(idx, M, warm, chunks, layout, knobs):
    """Launches of several steps at the config shapes, with thousands of markets and
    after the order ring has wrapped, against the oracle step by step (fill counts
    and BBOs of every step, the last step's rows, portfolios), besides the single
    calls."""
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[idx]
    qs = QuoteStream(cfg, np.arange(M))
    cache = {}

    def stream(t):
        if t not in cache:
            cache[t] = qs.step(t)
        return cache[t]

    _run(M, cfg.L, cfg.O, cfg.F, cfg.C, stream, warm, chunks, layout, oracle=True, **knobs)
