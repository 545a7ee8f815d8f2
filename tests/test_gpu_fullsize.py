"""Configs 2, 3 and 4 at full size and full length, and config 5 (the game step) at
full size and length, against the oracle (GPU).

Markets (configs 2-4): per step, the fill rows each call wrote (gathered by
(market, row) index), fill_counts and the four BBO arrays are reduced to weighted
sums (a checksum per step; the list of them is the run's checksum of checksums) on
each side, the GPU side in torch on the device, the oracle side in numpy. Weights
are < 2^20 and all values here are small, so the int64 sums never overflow and
both sides compute the same exact integers; a single differing value changes its
sum. Portfolios are compared in full every 100 steps and at the end. Config 2
runs 10,000 steps (its order ring wraps about 20 times), config 3 1,000 (wraps
at step 512), config 4 2,000 (4,000 inserts per market, no wrap).

The game (config 5, 10,000 envs, 1,000 fused moves, the ring wrapping at move 512)
is compared array for array with the game oracle after every move (the per-env
state, fill batch and BBO), and its [N,P,T,6] / [N,P*T,3] telemetry every 100
moves and at the end.
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


@pytest.mark.parametrize("idx", [2, 3, 4])
def test_gpu_full_size_checksums(idx):
    from astra_cuda import order_matching as aom
    from astra_cuda.workloads import CONFIGS, QuoteStream
    from oracle.oracle import OracleMarket
    cfg = CONFIGS[idx]
    M, F = cfg.M, cfg.F
    nthreads = max(1, min(16, os.cpu_count() or 1))
    print(f"config {idx} full size: {M} markets x {cfg.steps} steps, oracle threads {nthreads}", flush=True)
    g = aom.VecMarket(**cfg.shape_kwargs(), allow_extended_shapes=cfg.extended)
    gf, gb = g.new_fill_batch(), g.new_bbo_batch()
    o = OracleMarket(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C)
    of, ob = o.new_fill_batch(), o.new_bbo_batch()
    qs = QuoteStream(cfg)
    t0 = time.time()
    total_rows = 0
    overflow = 0
    chunk = 500
    every = max(100, cfg.steps // 10)
    for c0 in range(0, cfg.steps, chunk):
        host = qs.steps(c0, min(cfg.steps, c0 + chunk))
        dev = [torch.as_tensor(a).to(DEV) for a in host]
        for j in range(host[0].shape[0]):
            t = c0 + j
            g.add_two_sided_quotes(*(d[j] for d in dev), gf)
            g.get_bbos(gb)
            o.add_two_sided_quotes(*(a[j] for a in host), of, nthreads=nthreads)
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
            if t % every == 0 or t == cfg.steps - 1:
                assert np.array_equal(g.get_customer_portfolios().cpu().numpy(), o.customer_portfolios), \
                    f"step {t}: portfolios"
                print(f"  step {t}: ok, {total_rows} fill rows so far, {time.time() - t0:.1f}s", flush=True)
    assert g.global_tid == o.global_tid == 2 * cfg.steps
    assert total_rows > cfg.M  # the workload trades
    if idx in (2, 3):
        assert overflow > 0  # ring reuse drives some books into the overflow state


def test_gpu_config5_game_full_length():
    """Config 5: 10,000 envs of the high-low game, 1,000 fused trading moves
    (with the reference's input checks) against the game oracle."""
    import astra_cuda as astra
    from astra_cuda.workloads import GAME_CONFIG, GameStream
    from oracle.high_low_oracle import OracleHighLow
    cfg = GAME_CONFIG
    N, P = cfg.envs, cfg.players
    print(f"config 5 full length: {N} envs x {P * cfg.steps_per_player} moves", flush=True)
    astra.register_games()
    s = astra.load_game("high_low_trading", cfg.game_params(N, check_moves=True)).new_initial_state()
    o = OracleHighLow(N, P, cfg.steps_per_player, cfg.max_contracts_per_trade, cfg.customer_max_size,
                      cfg.max_contract_value, market_shape=cfg.market_shape)
    gs = GameStream(cfg, np.arange(N))
    for c in gs.chance():
        o.apply_action(c)
        s.apply_action(torch.as_tensor(c).to(DEV))
    t0 = time.time()
    per_move = ("player_last_positions", "immediate_rewards", "rewards_since_last_action")
    bbo = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices")
    moves = P * cfg.steps_per_player
    overflow = 0
    for k in range(moves):
        mv = gs.move(k)
        o.apply_action(mv)
        s.apply_action(torch.as_tensor(mv).to(DEV))
        for name in per_move:
            assert np.array_equal(getattr(o, name), getattr(s, name).cpu().numpy()), (k, name)
        for f in bbo:
            assert np.array_equal(getattr(o.bbo, f), getattr(s.bbo_batch, f).cpu().numpy()), (k, f)
        assert np.array_equal(o.fills.fill_counts, s.fill_batch.fill_counts.cpu().numpy()), k
        for f in FIELDS:  # the whole batch: rows past a count are what earlier moves left
            assert np.array_equal(np.asarray(getattr(o.fills, f)),
                                  getattr(s.fill_batch, f).cpu().numpy()), (k, f)
        assert np.array_equal(o.market.customer_portfolios, s.market.get_customer_portfolios().cpu().numpy()), k
        overflow += int((o.fills.fill_counts < 0).sum())
        if k % 100 == 0 or k == moves - 1:
            assert np.array_equal(o.player_contract_over_time, s.player_contract_over_time.cpu().numpy()), k
            assert np.array_equal(o.market_contract_over_time, s.market_contract_over_time.cpu().numpy()), k
            print(f"  move {k}: ok, {time.time() - t0:.1f}s", flush=True)
    assert s.is_terminal() and o.is_terminal()
    ret = torch.zeros((N, P), dtype=torch.float32, device=DEV)
    s.fill_returns(ret)
    assert np.array_equal(o.fill_returns(), ret.cpu().numpy())
    assert s.market.global_tid == o.market.global_tid == 2 * moves
