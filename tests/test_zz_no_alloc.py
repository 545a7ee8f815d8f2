"""astra_high_low_trade_scratch, the allocation-free trading move (no counterpart in
the reference), against astra_high_low_trade through the C ABI: two identical games,
one moved by each entry point, must hold identical state after every move, for two
games in a row (the second smaller, so the per-device scratch holds what the first
left), and a move that fails a check must return the same error through both and
change nothing. Moves of two markets on two streams (one failing its checks while
the other goes on) must each match the ordinary entry point; the scratch's words
are per market (64 per GPU); and after the first call on a device the entry point
allocates no device memory (GPU)."""
import ctypes
import gc

import numpy as np
import pytest
import torch

from high_low_cases import random_game

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
STATE = ("player_last_positions", "_pcot", "_mcot", "immediate_rewards", "rewards_since_last_action",
         "target_positions", "contract_values")


def _t(a):
    return torch.as_tensor(np.ascontiguousarray(a)).to(DEV)


def _games(N, seed, P=5, T=4, S=5, cM=5, V=30):
    import astra_cuda as astra
    astra.register_games()
    prm = dict(num_markets=N, players=P, steps_per_player=T, max_contracts_per_trade=S,
               customer_max_size=cM, max_contract_value=V)
    game = astra.load_game("high_low_trading", prm)
    a, b = game.new_initial_state(), game.new_initial_state()
    # b moves through the allocation-free entry point; its own error word is not
    # handed over at all
    b._trade_fn = b._lib.astra_high_low_trade_scratch
    b._trade.errors = None
    chance, moves = random_game(np.random.default_rng(seed), N, P, T, S, cM, V)
    for c in chance:
        a.apply_action(_t(c))
        b.apply_action(_t(c))
    return a, b, moves


def _same(a, b, where):
    torch.cuda.synchronize()
    for name in STATE:
        assert torch.equal(getattr(a, name), getattr(b, name)), (where, name)
    assert torch.equal(a.market._ws, b.market._ws), where
    assert torch.equal(a.fill_batch.fill_counts, b.fill_batch.fill_counts), where
    assert torch.equal(a.fill_batch._rows, b.fill_batch._rows), where
    for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
        assert torch.equal(getattr(a.bbo_batch, f), getattr(b.bbo_batch, f)), (where, f)
    assert a.market.global_tid == b.market.global_tid, where
    assert a.move_number() == b.move_number(), where


def test_scratch_trade_matches_trade_on_two_games_in_a_row():
    for N, seed in ((3000, 11), (700, 12)):
        print(f"no-alloc trade: {N} envs, seed {seed}", flush=True)
        a, b, moves = _games(N, seed)
        for k, mv in enumerate(moves[:12]):
            a.apply_action(_t(mv))
            b.apply_action(_t(mv))
            _same(a, b, f"N={N} move {k}")
        # a failed check: the same error through both, nothing changed in either
        bad = moves[12].copy()
        bad[N // 2, 2] = 99  # bid size above max_contracts_per_trade
        before = {n: getattr(b, n).clone() for n in STATE}
        ws = b.market._ws.clone()
        errs = []
        for s in (a, b):
            with pytest.raises(RuntimeError) as e:
                s.apply_action(_t(bad))
            errs.append(str(e.value))
        assert errs[0] == errs[1] and "max(bid_sizes)" in errs[0] and "GetMaxContractsPerTrade" in errs[0]
        _same(a, b, f"N={N} after the failed check")
        assert torch.equal(b.market._ws, ws)
        for n, v in before.items():
            assert torch.equal(getattr(b, n), v), n
        # and the next good move goes through both
        a.apply_action(_t(moves[12]))
        b.apply_action(_t(moves[12]))
        _same(a, b, f"N={N} move 12")


def test_scratch_moves_of_two_markets_on_two_streams():
    """Market A moves on one stream, market B on another; A's move fails its checks
    and B's next move is issued right after, while A's (aborting) move kernel may
    still be queued. Each market has a scratch word of its own, so each state must
    match the same moves made through the ordinary entry point."""
    ref_a, scr_a, moves_a = _games(900, 21)
    ref_b, scr_b, moves_b = _games(1300, 22)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for k in range(6):
        with torch.cuda.stream(s1):
            scr_a.apply_action(_t(moves_a[k]))
        with torch.cuda.stream(s2):
            scr_b.apply_action(_t(moves_b[k]))
        ref_a.apply_action(_t(moves_a[k]))
        ref_b.apply_action(_t(moves_b[k]))
    bad = moves_a[6].copy()
    bad[1, 0] = 0  # a bid price of 0 fails min(bid_prices) > 0
    with torch.cuda.stream(s1):
        with pytest.raises(RuntimeError) as e:
            scr_a.apply_action(_t(bad))
    assert "min(bid_prices)" in str(e.value)
    with torch.cuda.stream(s2):
        scr_b.apply_action(_t(moves_b[6]))
    with pytest.raises(RuntimeError):
        ref_a.apply_action(_t(bad))
    ref_b.apply_action(_t(moves_b[6]))
    _same(ref_a, scr_a, "A after its failed move")
    _same(ref_b, scr_b, "B after its move beside A's failed one")
    # and both go on
    with torch.cuda.stream(s1):
        scr_a.apply_action(_t(moves_a[6]))
    with torch.cuda.stream(s2):
        scr_b.apply_action(_t(moves_b[7]))
    ref_a.apply_action(_t(moves_a[6]))
    ref_b.apply_action(_t(moves_b[7]))
    _same(ref_a, scr_a, "A move 6")
    _same(ref_b, scr_b, "B move 7")


def test_scratch_words_are_per_market_and_returned_on_destroy():
    """At most 64 live markets per GPU hold a scratch word; the next one's move
    reports that, and moves again once a market holding a word is gone."""
    gc.collect()
    held, failed, moves = [], None, None
    for i in range(66):
        _, b, mv = _games(2, 100 + i)
        try:
            b.apply_action(_t(mv[0]))
        except RuntimeError as e:
            assert "scratch words" in str(e)
            failed, moves = b, mv
            break
        held.append(b)
    assert failed is not None and len(held) <= 64
    print(f"scratch words held by this test's markets: {len(held)}", flush=True)
    del held[0]
    gc.collect()
    failed.apply_action(_t(moves[0]))
    torch.cuda.synchronize()


def test_scratch_trade_allocates_no_device_memory():
    """After the device's first call (the set-up: the scratch's device address and
    its events), moves through the entry point leave the device's free memory
    exactly as it was. The moves are uploaded first; the entry point is called
    through the C ABI directly, so nothing else runs between the two readings."""
    from astra_cuda import _native
    _, b, moves = _games(2000, 31)
    lib = _native.lib()
    dev_moves = [_t(m) for m in moves]
    stream = torch.cuda.current_stream().cuda_stream
    t = b._trade
    P = b.num_players()

    def move(k):
        t.move = dev_moves[k].data_ptr()
        t.player = k % P
        t.trade_move_number = k
        assert lib.astra_high_low_trade_scratch(b.market._h, ctypes.byref(t), stream) == 0, \
            _native.last_error()

    move(0)  # set-up (if no earlier call on this device made it)
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for k in range(1, len(dev_moves)):
        move(k)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, (free0, free1)


def test_scratch_trade_rejects_unchecked_moves_and_missing_host_word():
    from astra_cuda import _native
    a, b, moves = _games(64, 13)
    lib = _native.lib()
    t = b._trade
    t.move = _t(moves[0]).data_ptr()
    t.player = b.current_player()
    t.trade_move_number = 0
    t.check = 0
    assert lib.astra_high_low_trade_scratch(b.market._h, ctypes.byref(t), None) != 0
    assert "check must be 1" in _native.last_error()
    t.check = 1
    host = t.errors_host
    t.errors_host = None
    assert lib.astra_high_low_trade_scratch(b.market._h, ctypes.byref(t), None) != 0
    assert "errors_host" in _native.last_error()
    t.errors_host = host
