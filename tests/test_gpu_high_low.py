"""The high-low trading game on the HIP engine (astra_cuda.load_game) against the
game oracle, bit-exact (GPU)."""
import contextlib

import numpy as np
import pytest
import torch

from high_low_cases import HAND_GAME, random_game
from oracle.high_low_oracle import MAX_CHANCE_NODES, OracleHighLow

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _t(a):
    return torch.as_tensor(np.ascontiguousarray(a)).to(DEV)


@contextlib.contextmanager
def _engine_knobs(stage_budget=None, per_wave=None, fill_rows=None):
    """Engine knobs for the markets created inside the block (a game creates its market
    with each new state): the loop passes before a book is staged in LDS, envs per
    wavefront of the fused move and fill rows a lane buffers (64 and 4 is the launch
    of a large game, such as the reference benchmark's 262,144 envs)."""
    import os
    env = {"ASTRA_MARKET_STAGE_BUDGET": stage_budget, "ASTRA_MARKET_PER_WAVE": per_wave,
           "ASTRA_MARKET_FILL_ROWS": fill_rows}
    old = {k: os.environ.get(k) for k in env}
    for k, v in env.items():
        if v is not None:
            os.environ[k] = str(v)
    try:
        yield
    finally:
        for k, v in env.items():
            if v is None:
                continue
            if old[k] is None:
                del os.environ[k]
            else:
                os.environ[k] = old[k]


def _game(params):
    import astra_cuda as astra
    astra.register_games()
    return astra.load_game("high_low_trading", params)


def _compare(o, s, where):
    for name in ("player_last_positions", "player_contract_over_time", "market_contract_over_time",
                 "immediate_rewards", "rewards_since_last_action", "target_positions", "contract_values"):
        assert np.array_equal(getattr(o, name), getattr(s, name).cpu().numpy()), (where, name)
    P = o.P
    assert np.array_equal(o.market.customer_portfolios, s.market.get_customer_portfolios().cpu().numpy()), where
    for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
        assert np.array_equal(getattr(o.bbo, f), getattr(s.bbo_batch, f).cpu().numpy()), (where, f)
    rb = torch.zeros((o.N, P), dtype=torch.float32, device=DEV)
    s.fill_rewards(rb)
    assert np.array_equal(o.fill_rewards(), rb.cpu().numpy()), where
    one = torch.zeros((o.N,), dtype=torch.float32, device=DEV)
    for p in range(P):
        s.fill_rewards_since_last_action(one, p)
        assert np.array_equal(o.fill_rewards_since_last_action(p), one.cpu().numpy()), (where, p)


def _params(N, P, T, S, cM, V, shape):
    p = dict(num_markets=N, players=P, steps_per_player=T, max_contracts_per_trade=S,
             customer_max_size=cM, max_contract_value=V)
    if shape is not None:
        p.update(market_price_levels=shape[0], market_orders=shape[1], market_fills=shape[2],
                 market_customers=shape[3])
    return p


@pytest.mark.parametrize("N,P,T,S,cM,V,shape,seed,budget,knobs", [
    (500, 5, 4, 5, 5, 30, None, 1, None, {}),
    (300, 4, 6, 3, 4, 20, (21, 12, 6, 4), 2, None, {}),         # ring of 12: slot reuse
    (2000, 5, 3, 5, 5, 127, (128, 1024, 10, 16), 3, None, {}),  # the config-5 shape
    (300, 8, 3, 5, 5, 30, None, 4, 1, {}),     # 8 and 9 players, staging forced
    (300, 9, 3, 5, 5, 30, None, 5, 1, {}),
    (300, 5, 8, 3, 4, 20, (21, 12, 6, 5), 6, 1, {}),
    (37, 7, 4, 5, 5, 30, None, 7, None, {}),   # 7 players: the observation's tile of 64 envs, ragged
    (33, 10, 3, 5, 5, 30, None, 8, None, {}),  # 10 (the most): the per-element observation kernel
    # the fused move as a large game launches it: 64 envs per wavefront, 4 fill rows
    (2000, 5, 3, 5, 5, 127, (128, 1024, 10, 16), 9, None, {"per_wave": 64, "fill_rows": 4}),
    (300, 5, 8, 3, 4, 20, (21, 12, 6, 5), 10, 1, {"per_wave": 64, "fill_rows": 4}),
])
def test_gpu_game_vs_oracle(N, P, T, S, cM, V, shape, seed, budget, knobs):
    print(f"game N={N} P={P} T={T} shape={shape} stage budget {budget} {knobs}", flush=True)
    rng = np.random.default_rng(seed)
    o = OracleHighLow(N, P, T, S, cM, V, market_shape=shape)
    g = _game(_params(N, P, T, S, cM, V, shape))
    with _engine_knobs(stage_budget=budget, **knobs):
        s = g.new_initial_state()
    chance, moves = random_game(rng, N, P, T, S, cM, V)
    for c in chance:
        assert s.is_chance_node() and s.current_player() == -1
        o.apply_action(c)
        s.apply_action(_t(c))
    values = torch.zeros(g.observation_tensor_shape(), dtype=torch.float32, device=DEV)
    for k, mv in enumerate(moves):
        assert s.current_player() == o.current_player() == k % P
        if k % 2 == 0:  # the rollout loop's observation of the acting player
            assert s.fill_observation_tensor(values) == k % P
            assert np.array_equal(o.fill_observation_tensor(k % P), values.cpu().numpy()), k
        o.apply_action(mv)
        assert s.apply_action(_t(mv)) == k % P
        _compare(o, s, f"move {k}")
        if k == len(moves) // 2:  # a clone continues identically
            s2, o2 = s.clone(), o  # o keeps going; compare the clone at the end
            clone_at = k
    assert s.is_terminal() and o.is_terminal()
    ret = torch.zeros((N, P), dtype=torch.float32, device=DEV)
    s.fill_returns(ret)
    assert np.array_equal(o.fill_returns(), ret.cpu().numpy())
    info = s.expose_info()
    assert np.array_equal(info["players"].cpu().numpy(), o.player_contract_over_time)
    # a copy in the reference's layout, not a view of the env-minor storage
    assert info["players"].is_contiguous() and info["players"].shape == (o.N, o.P, o.T, 6)
    assert np.array_equal(info["market"].cpu().numpy(), o.market_contract_over_time)
    assert info["market"].is_contiguous() and info["market"].shape == (o.N, o.P * o.T, 3)
    for mv in moves[clone_at + 1:]:
        s2.apply_action(_t(mv))
    _compare(o, s2, "clone")
    s.reset()
    assert s.move_number() == 0 and not s.player_contract_over_time.any()
    assert not s.market.get_customer_portfolios().any()


def test_gpu_hand_game():
    g = _game(HAND_GAME["params"])
    s = g.new_initial_state()
    for c in HAND_GAME["chance"]:
        s.apply_action(_t(c))
    values = torch.zeros(g.observation_tensor_shape(), dtype=torch.float32, device=DEV)
    for k, mv in enumerate(HAND_GAME["moves"]):
        s.apply_action(_t(np.array([mv], np.int32)))
        assert s.immediate_rewards[0].tolist() == HAND_GAME["immediate"][k]
        assert s.rewards_since_last_action[0].tolist() == HAND_GAME["since_last"][k]
        assert s.market_contract_over_time[0, k].tolist() == HAND_GAME["market_rows"][k]
        if k in HAND_GAME["portfolios_after"]:
            assert s.market.get_customer_portfolios()[0].tolist() == HAND_GAME["portfolios_after"][k]
        if k == HAND_GAME["obs_after"]:
            s.fill_observation_tensor(HAND_GAME["obs_player"], values)
            assert values[0].tolist() == HAND_GAME["obs"]
        for after, player, want in HAND_GAME["more_obs"]:
            if k == after:
                s.fill_observation_tensor(player, values)
                assert values[0].tolist() == want, (after, player)
    ret = torch.zeros((1, 4), dtype=torch.float32, device=DEV)
    s.fill_returns(ret)
    assert ret[0].tolist() == HAND_GAME["returns"]


def test_gpu_move_checks():
    prm = dict(HAND_GAME["params"], num_markets=5)
    s = _game(prm).new_initial_state()
    for c in HAND_GAME["chance"]:
        s.apply_action(_t(np.repeat(c, 5, axis=0)))
    bad = np.tile(np.array([[12, 18, 2, 1]], np.int32), (5, 1))
    bad[3, 3] = 6  # ask size above max_contracts_per_trade
    names = ("player_last_positions", "player_contract_over_time", "market_contract_over_time",
             "immediate_rewards", "rewards_since_last_action")
    before = {n: getattr(s, n).clone() for n in names}
    ws = s.market._ws.clone()
    with pytest.raises(RuntimeError, match="Astra Fatal Error.*ask_sizes"):
        s.apply_action(_t(bad))
    assert s.move_number() == MAX_CHANCE_NODES and s.market.global_tid == 0
    assert torch.equal(s.market._ws, ws)  # the move kernel ran and left every env as it was
    for n, v in before.items():
        assert torch.equal(getattr(s, n), v), n
    s.apply_action(_t(np.tile(np.array([[12, 18, 2, 1]], np.int32), (5, 1))))  # good move goes through
    assert s.move_number() == MAX_CHANCE_NODES + 1
    # unchecked: no sync per move; check_errors reports afterwards
    s2 = _game(dict(prm, check_moves=False)).new_initial_state()
    for c in HAND_GAME["chance"]:
        s2.apply_action(_t(np.repeat(c, 5, axis=0)))
    s2.apply_action(_t(bad))
    with pytest.raises(RuntimeError, match="ask_sizes <= max_contracts_per_trade"):
        s2.check_errors()
    s2.check_errors()  # cleared
    # a failed unchecked move, then checks switched on: the switch reports it and
    # clears the word, so the next good checked move goes through
    s2.apply_action(_t(bad))
    with pytest.raises(RuntimeError, match="ask_sizes <= max_contracts_per_trade"):
        s2.set_check_moves(True)
    mv = s2.move_number()
    s2.apply_action(_t(np.tile(np.array([[12, 18, 2, 1]], np.int32), (5, 1))))
    assert s2.move_number() == mv + 1


def test_gpu_move_checks_many_blocks():
    """The check kernel over 300,000 envs (1024 blocks, several envs per thread): the
    last block publishes the OR of every block's bits; a failed check anywhere stops
    the move, the message names the first failed check in the reference's order, and
    the calls after it (the block counter reset) behave."""
    N = 300_000
    prm = dict(HAND_GAME["params"], num_markets=N)
    s = _game(prm).new_initial_state()
    for c in HAND_GAME["chance"]:
        s.apply_action(_t(np.repeat(c, N, axis=0)))
    good = np.tile(np.array([[12, 18, 2, 1]], np.int32), (N, 1))
    s.apply_action(_t(good))
    bad = good.copy()
    bad[N - 1, 3] = 6  # ask size above max in the last env
    with pytest.raises(RuntimeError, match="max\\(ask_sizes\\)"):
        s.apply_action(_t(bad))
    bad[0, 1] = 0      # ask price not > 0 in the first env: earlier in the reference's order
    with pytest.raises(RuntimeError, match="min\\(ask_prices\\)"):
        s.apply_action(_t(bad))
    assert s.move_number() == MAX_CHANCE_NODES + 1 and s.market.global_tid == 2
    s.apply_action(_t(good))
    assert s.move_number() == MAX_CHANCE_NODES + 2 and s.market.global_tid == 4


def test_gpu_text_renderings():
    """to_string / observation_string / information_state_string: the hand-derived
    text, and the oracle's on a random game (every few moves, several envs)."""
    from high_low_cases import HAND_PRIVATE_TEXT, HAND_PUBLIC_TEXT, HAND_SETUP_TEXT, HAND_TEXT_AFTER
    from oracle.high_low_oracle import oracle_information_state_string, oracle_to_string
    s = _game(HAND_GAME["params"]).new_initial_state()
    assert s.observation_string(0) == ("********** Private Information **********\nPrivate info pending...\n"
                                       "***************************\n")
    for c in HAND_GAME["chance"]:
        s.apply_action(_t(c))
    for mv in HAND_GAME["moves"][:HAND_TEXT_AFTER + 1]:
        s.apply_action(_t(np.array([mv], np.int32)))
    book = s.market.to_string(0)
    assert s.to_string(0) == HAND_SETUP_TEXT + HAND_PUBLIC_TEXT + book
    assert str(s) == s.to_string(0)
    for p, priv in HAND_PRIVATE_TEXT.items():
        exp = ("********** Private Information **********\n" + priv +
               "******************************************\n\n" + HAND_PUBLIC_TEXT + book)
        assert s.observation_string(p, 0) == exp
        assert s.information_state_string(p) == exp
    # random game against the oracle
    N, P, T, S, cM, V = 40, 5, 3, 5, 5, 30
    rng = np.random.default_rng(9)
    o = OracleHighLow(N, P, T, S, cM, V)
    s = _game(_params(N, P, T, S, cM, V, None)).new_initial_state()
    chance, moves = random_game(rng, N, P, T, S, cM, V)
    for k, c in enumerate(chance):
        o.apply_action(c)
        s.apply_action(_t(c))
        assert s.to_string(k) == oracle_to_string(o, k)
    for k, mv in enumerate(moves):
        o.apply_action(mv)
        s.apply_action(_t(mv))
        if k % 4 == 0 or k == len(moves) - 1:
            for idx in (0, 7, N - 1):
                assert s.to_string(idx) == oracle_to_string(o, idx), (k, idx)
                for p in range(P):
                    assert s.observation_string(p, idx) == oracle_information_state_string(o, p, idx), (k, idx, p)


@pytest.mark.parametrize("N,P", [(1, 4), (37, 7), (33, 10), (262144, 5)])
def test_gpu_rewards_entry_point(N, P):
    """astra_high_low_rewards against torch's int32 -> float32 copy_: the 16-byte path
    (aligned buffers, word counts with a tail of 1-3), the one-word path (a buffer that
    starts one float into its allocation) and one player's column."""
    from astra_cuda import _native
    print(f"rewards N={N} P={P}", flush=True)
    lib = _native.lib()
    g = torch.Generator().manual_seed(N + P)
    src = torch.randint(-(1 << 30), 1 << 30, (N, P), dtype=torch.int32, generator=g).to(DEV)
    want = src.float()
    for off in (0, 1):
        raw = torch.full((N * P + 4,), float("nan"), dtype=torch.float32, device=DEV)
        dst = raw[off:off + N * P]
        assert lib.astra_high_low_rewards(src.data_ptr(), N, P, -1, dst.data_ptr(), None) == 0
        torch.cuda.synchronize()
        assert torch.equal(dst.view(N, P), want), off
        assert torch.isnan(raw[off + N * P:]).all()  # nothing written past the end
    for p in (0, P - 1):
        col = torch.full((N,), float("nan"), dtype=torch.float32, device=DEV)
        assert lib.astra_high_low_rewards(src.data_ptr(), N, P, p, col.data_ptr(), None) == 0
        torch.cuda.synchronize()
        assert torch.equal(col, want[:, p]), p
