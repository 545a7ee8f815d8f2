"""The high-low game's move kernels (csrc/high_low.hip), compiled for the host,
against the game oracle (CPU only). The chance-move set-up is copied from the
oracle; every trading move then runs through astra_high_low_trade and every
state array is compared; observations through astra_high_low_observation."""
import numpy as np
import pytest

from emu_engine import EmuHighLow
from high_low_cases import HAND_GAME, random_game
from oracle.high_low_oracle import MAX_CHANCE_NODES, OracleHighLow

STATE = ("player_last_positions", "player_contract_over_time", "market_contract_over_time",
         "immediate_rewards", "rewards_since_last_action")


def _setup(o, e):
    e.contract_values[:] = o.contract_values
    e.contract_high_settle[:] = o.contract_high_settle
    e.player_permutation[:] = o.player_permutation
    e.target_positions[:] = o.target_positions


def _compare(o, e, where):
    for name in STATE:
        assert np.array_equal(getattr(o, name), getattr(e, name)), (where, name)
    assert np.array_equal(o.market.customer_portfolios, e.market.portfolios), where
    for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
        assert np.array_equal(getattr(o.bbo, f), getattr(e.bbo, f)), (where, f)
    assert np.array_equal(o.fills.fill_counts, e.fills.fill_counts), where


def _play(N, P, T, S, cM, V, shape, seed, obs_every=3, layout="columns", stage_budget=None):
    import os
    rng = np.random.default_rng(seed)
    o = OracleHighLow(N, P, T, S, cM, V, market_shape=shape)
    old = os.environ.get("ASTRA_MARKET_STAGE_BUDGET")
    if stage_budget is not None:  # read when the market is created
        os.environ["ASTRA_MARKET_STAGE_BUDGET"] = str(stage_budget)
    try:
        e = EmuHighLow(N, P, T, S, cM, V, (o.L, o.O, o.F, o.C), layout)
    finally:
        if stage_budget is not None:
            if old is None:
                del os.environ["ASTRA_MARKET_STAGE_BUDGET"]
            else:
                os.environ["ASTRA_MARKET_STAGE_BUDGET"] = old
    chance, moves = random_game(rng, N, P, T, S, cM, V)
    for c in chance:
        o.apply_action(c)
    _setup(o, e)
    for k, mv in enumerate(moves):
        player = o.current_player()
        o.apply_action(mv)
        assert e.trade(mv, player, k) == 0
        _compare(o, e, f"move {k}")
        if k % obs_every == 0 and k + 1 < T * P:
            cr = (o.move_number - MAX_CHANCE_NODES) // P
            for p in range(P):
                assert np.array_equal(o.fill_observation_tensor(p), e.observation(p, cr)), (k, p)


@pytest.mark.parametrize("N,P,T,S,cM,V,shape,seed", [
    (37, 4, 3, 5, 5, 30, None, 1),          # the game's own market shape
    (64, 5, 6, 5, 5, 30, None, 2),
    (50, 5, 8, 3, 4, 20, (21, 12, 6, 5), 3),  # a ring of 12 wraps: slot reuse
    (40, 6, 4, 5, 5, 127, (128, 1024, 10, 16), 4),  # the config-5 shape (C > players)
    (37, 7, 4, 5, 5, 30, None, 8),          # 7 and 10 (the most) players
    (33, 10, 3, 5, 5, 30, None, 9),
])
@pytest.mark.parametrize("layout", ["columns", "rows"])
def test_emulated_game_vs_oracle(N, P, T, S, cM, V, shape, seed, layout):
    _play(N, P, T, S, cM, V, shape, seed, layout=layout)


@pytest.mark.parametrize("N,P,T,S,cM,V,shape,seed", [
    (40, 8, 3, 5, 5, 30, None, 5),     # 8 and 9 players
    (40, 9, 3, 5, 5, 30, None, 6),
    (50, 5, 8, 3, 4, 20, (21, 12, 6, 5), 7),
])
def test_emulated_game_staged_and_player_counts(N, P, T, S, cM, V, shape, seed):
    """Every market that crosses twice finished from its staged book (stage budget 1),
    with more players than the default games have."""
    _play(N, P, T, S, cM, V, shape, seed, layout="rows", stage_budget=1)


def test_emulated_hand_game():
    prm = HAND_GAME["params"]
    o = OracleHighLow(**prm)
    e = EmuHighLow(1, prm["players"], prm["steps_per_player"], prm["max_contracts_per_trade"],
                   prm["customer_max_size"], prm["max_contract_value"], (o.L, o.O, o.F, o.C))
    for c in HAND_GAME["chance"]:
        o.apply_action(c)
    _setup(o, e)
    for k, mv in enumerate(HAND_GAME["moves"]):
        player = o.current_player()
        o.apply_action(np.array([mv], np.int32))
        assert e.trade(np.array([mv], np.int32), player, k) == 0
        assert e.immediate_rewards[0].tolist() == HAND_GAME["immediate"][k]
        assert e.rewards_since_last_action[0].tolist() == HAND_GAME["since_last"][k]
        assert e.market_contract_over_time[0, k].tolist() == HAND_GAME["market_rows"][k]
        if k == HAND_GAME["obs_after"]:
            assert e.observation(HAND_GAME["obs_player"], 1)[0].tolist() == HAND_GAME["obs"]
        for after, player, want in HAND_GAME["more_obs"]:
            if k == after:  # current round after move k of 4 players: (k + 1) // 4
                assert e.observation(player, (k + 1) // 4)[0].tolist() == want, (after, player)


@pytest.mark.parametrize("host_word", [True, False], ids=["errors_host", "no_errors_host"])
def test_emulated_checks_flag_and_stop(host_word):
    N, P, T, S, cM, V = 6, 4, 2, 5, 5, 30
    o = OracleHighLow(N, P, T, S, cM, V)
    e = EmuHighLow(N, P, T, S, cM, V, (o.L, o.O, o.F, o.C))
    if not host_word:
        e.errors_host = None
    mv = np.tile(np.array([[12, 18, 2, 1]], np.int32), (N, 1))
    mv[2, 2] = S + 1     # bid size above max_contracts_per_trade
    mv[4, 0] = 0         # bid price not > 0
    e.trade(np.tile(np.array([[12, 18, 2, 1]], np.int32), (N, 1)), 0, 0, check=1)  # a good move first
    e.errors[0] = 0
    names = ("player_last_positions", "player_contract_over_time", "market_contract_over_time",
             "immediate_rewards", "rewards_since_last_action")
    before = {n: getattr(e, n).copy() for n in names}
    ws, tid = e.market.ws.copy(), e.market.global_tid
    fills = {f: np.array(getattr(e.fills, f)).copy() for f in e.fills.FIELDS}
    bbo = {f: getattr(e.bbo, f).copy() for f in e.bbo.FIELDS}
    rc = e.trade(mv, 1, 1, check=1)
    assert rc != 0
    assert e.errors[0] == (1 << 0) | (1 << 6)
    # nothing changed: the book, the TID counter, fills, BBOs and every state array
    assert np.array_equal(e.market.ws, ws) and e.market.global_tid == tid
    for f, v in fills.items():
        assert np.array_equal(np.array(getattr(e.fills, f)), v), f
    for f, v in bbo.items():
        assert np.array_equal(getattr(e.bbo, f), v), f
    for n, v in before.items():
        assert np.array_equal(getattr(e, n), v), n
    e.errors[0] = 0
    assert e.trade(mv, 1, 1, check=0) == 0  # no check: trades, flag kept for the caller
    assert e.errors[0] == (1 << 0) | (1 << 6) and e.market.global_tid == tid + 2


@pytest.mark.parametrize("N,P", [(1, 4), (37, 7), (33, 10), (0, 5)])
def test_emulated_rewards_entry_point(N, P):
    """astra_high_low_rewards (FillRewards / FillRewardsSinceLastAction,
    high_low_trading.cc:331-343): int32 -> float32, all words or one player's column."""
    from emu_engine import lib
    rng = np.random.default_rng(N * 31 + P)
    src = rng.integers(-(1 << 30), 1 << 30, size=(N, P), dtype=np.int32)
    dst = np.full((N, P), np.nan, np.float32)
    assert lib().astra_high_low_rewards(src.ctypes.data, N, P, -1, dst.ctypes.data, None) == 0
    assert np.array_equal(dst, src.astype(np.float32))
    for p in (0, P - 1):
        col = np.full(N, np.nan, np.float32)
        assert lib().astra_high_low_rewards(src.ctypes.data, N, P, p, col.ctypes.data, None) == 0
        assert np.array_equal(col, src[:, p].astype(np.float32))
    assert lib().astra_high_low_rewards(src.ctypes.data, N, P, P, dst.ctypes.data, None) != 0


def test_emulated_scratch_trade_entry_point():
    """astra_high_low_trade_scratch (the allocation-free move, no counterpart in the
    reference) on the host build: random games against the oracle through it, two
    games in a row, the second smaller; its own error word unused; a failed check
    returns the error and changes nothing; unchecked moves and a missing host word
    are refused."""
    from emu_engine import lib
    for N, seed in ((40, 21), (9, 22)):
        P, T, S, cM, V = 5, 4, 5, 5, 30
        rng = np.random.default_rng(seed)
        o = OracleHighLow(N, P, T, S, cM, V)
        e = EmuHighLow(N, P, T, S, cM, V, (o.L, o.O, o.F, o.C))
        e.errors = None
        chance, moves = random_game(rng, N, P, T, S, cM, V)
        for c in chance:
            o.apply_action(c)
        _setup(o, e)
        for k, mv in enumerate(moves[:8]):
            player = o.current_player()
            o.apply_action(mv)
            assert e.trade(mv, player, k, entry="astra_high_low_trade_scratch") == 0
            _compare(o, e, f"N={N} move {k}")
        bad = moves[8].copy()
        bad[N // 2, 3] = S + 1
        ws, tid = e.market.ws.copy(), e.market.global_tid
        assert e.trade(bad, o.current_player(), 8, entry="astra_high_low_trade_scratch") != 0
        assert "ask_sizes" in lib().astra_last_error().decode()
        assert np.array_equal(e.market.ws, ws) and e.market.global_tid == tid
        _compare(o, e, f"N={N} after the failed check")
    assert e.trade(moves[8], 3, 8, check=0, entry="astra_high_low_trade_scratch") != 0
    assert "check must be 1" in lib().astra_last_error().decode()
    e.errors_host = None
    assert e.trade(moves[8], 3, 8, entry="astra_high_low_trade_scratch") != 0
    assert "errors_host" in lib().astra_last_error().decode()
