"""Config 3 at full size (100,000 markets x 1000 steps) against the oracle (GPU).

Per step, the fill rows each call wrote (gathered by (market, row) index),
fill_counts and the four BBO arrays are reduced to weighted sums (a checksum per step; the list of them is the run's
checksum of checksums) on each side, the GPU side in torch on the device, the
oracle side in numpy. Weights are < 2^20 and all values here are small, so the
int64 sums never overflow and both sides compute the same exact integers; a
single differing value changes its sum. Portfolios are compared in full.
"""
import os
import time

import numpy as np
import pytest
import torch

from parity_util import DEV, effective_counts

pytestmark = pytest.mark.gpu

FIELDS = ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
          "fill_quote_sizes", "fill_tid", "fill_quote_tid")
BBO = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes")
_P = (1 << 20) - 3


def _rows(eff, xp):
    """(market, k) of every fill row the last call wrote: k < eff[market]."""
    if xp is torch:
        m = torch.repeat_interleave(torch.arange(eff.shape[0], device=DEV), eff.to(torch.int64))
        start = torch.cumsum(eff.to(torch.int64), 0) - eff.to(torch.int64)
        k = torch.arange(m.shape[0], device=DEV) - torch.repeat_interleave(start, eff.to(torch.int64))
    else:
        m = np.repeat(np.arange(eff.shape[0]), eff)
        start = np.cumsum(eff) - eff
        k = np.arange(m.shape[0]) - np.repeat(start, eff)
    return m, k


def _fill_digest(arrays, eff, xp):
    m, k = _rows(eff, xp)
    w0 = (m * 2654435761 + k * 40503) % _P + 1
    out = []
    for i, a in enumerate(arrays):
        v = a[m, k]
        v = v.to(torch.int64) if xp is torch else v.astype(np.int64)
        out.append(int((v * ((w0 + i * 97) % _P + 1)).sum()))
    return out


def _vec_digest(v, salt, xp):
    M = v.shape[0]
    m = torch.arange(M, dtype=torch.int64, device=DEV) if xp is torch else np.arange(M, dtype=np.int64)
    w = (m * 2654435761 + (salt + 50) * 97) % _P + 1
    v = v.to(torch.int64) if xp is torch else v.astype(np.int64)
    return int((v * w).sum())


def test_gpu_config3_full_size_checksums():
    from astra_cuda import order_matching as aom
    from astra_cuda.workloads import CONFIGS, QuoteStream
    from oracle.oracle import OracleMarket
    cfg = CONFIGS[3]
    M, F = cfg.M, cfg.F
    nthreads = max(1, min(16, os.cpu_count() or 1))
    print(f"config 3 full size: {M} markets x {cfg.steps} steps, oracle threads {nthreads}", flush=True)
    g = aom.VecMarket(**cfg.shape_kwargs())
    gf, gb = g.new_fill_batch(), g.new_bbo_batch()
    o = OracleMarket(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C)
    of, ob = o.new_fill_batch(), o.new_bbo_batch()
    qs = QuoteStream(cfg)
    t0 = time.time()
    total_rows = 0
    overflow = 0
    for t in range(cfg.steps):
        args = qs.step(t)
        g.add_two_sided_quotes(*(torch.as_tensor(a).to(DEV) for a in args), gf)
        g.get_bbos(gb)
        o.add_two_sided_quotes(*args, of, nthreads=nthreads)
        o.get_bbos(ob, nthreads=nthreads)
        oc = of.fill_counts
        gc = gf.fill_counts
        assert _vec_digest(gc, 0, torch) == _vec_digest(oc, 0, np), f"step {t}: fill_counts"
        eff_o = effective_counts(oc, F)
        eff_g = torch.where(gc < 0, torch.full_like(gc, F), gc)
        dg = _fill_digest([getattr(gf, f) for f in FIELDS], eff_g, torch)
        do = _fill_digest([getattr(of, f) for f in FIELDS], eff_o, np)
        assert dg == do, f"step {t}: fill digests differ {dg} vs {do}"
        for i, f in enumerate(BBO):
            assert _vec_digest(getattr(gb, f), i + 1, torch) == _vec_digest(getattr(ob, f), i + 1, np), \
                f"step {t}: {f}"
        total_rows += int(eff_o.sum())
        overflow += int((oc < 0).sum())
        if t % 100 == 0 or t == cfg.steps - 1:
            assert np.array_equal(g.get_customer_portfolios().cpu().numpy(), o.customer_portfolios), \
                f"step {t}: portfolios"
            print(f"  step {t}: ok, {total_rows} fill rows so far, {time.time() - t0:.1f}s", flush=True)
    assert total_rows > cfg.M  # the workload trades
    assert overflow > 0  # ring reuse drives some books into the overflow state
