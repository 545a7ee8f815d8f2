"""The high-low game oracle (oracle/high_low_oracle.py) against hand-derived values
and identities of the reward formula (CPU only)."""
import numpy as np
import pytest

from high_low_cases import HAND_GAME, random_game
from oracle.high_low_oracle import GameError, OracleHighLow


def _play_hand(o):
    for c in HAND_GAME["chance"]:
        o.apply_action(c)
    out = []
    for k, mv in enumerate(HAND_GAME["moves"]):
        o.apply_action(np.array([mv], np.int32))
        out.append((o.immediate_rewards[0].tolist(), o.rewards_since_last_action[0].tolist(),
                    o.market.customer_portfolios[0].tolist(), o.market_contract_over_time[0, k].tolist()))
        if k == HAND_GAME["obs_after"]:
            obs = o.fill_observation_tensor(HAND_GAME["obs_player"])[0].tolist()
        for after, player, want in HAND_GAME["more_obs"]:
            if k == after:
                assert o.fill_observation_tensor(player)[0].tolist() == want, (after, player)
    return out, obs


def test_oracle_hand_game():
    o = OracleHighLow(**{k: v for k, v in HAND_GAME["params"].items()})
    assert (o.L, o.O, o.F, o.C) == (31, 16, 10, 4)  # high_low_trading.cc:57-69
    out, obs = _play_hand(o)
    for k, (imm, since, pf, mrow) in enumerate(out):
        assert imm == HAND_GAME["immediate"][k], k
        assert since == HAND_GAME["since_last"][k], k
        assert mrow == HAND_GAME["market_rows"][k], k
        if k in HAND_GAME["portfolios_after"]:
            assert pf == HAND_GAME["portfolios_after"][k], k
    assert o.is_terminal() and o.current_player() == -4
    assert o.fill_returns()[0].tolist() == HAND_GAME["returns"]
    assert obs == pytest.approx(HAND_GAME["obs"], abs=0, rel=0)
    info = o.expose_info()
    assert info["players"][0, 3, 0].tolist() == [26, 24, 2, 1, 1, -25]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reward_telescopes_to_returns(seed):
    """Without penalties (no crossing quote of one's own, no zero size), each player's
    immediate rewards over a game sum to FillReturns + |target| * V for a customer:
    the position term telescopes from |0 - target| and the cash term from 0, and the
    last move adds the settlement (high_low_trading.cc:290-328 against :344-373)."""
    rng = np.random.default_rng(seed)
    N, P, T, S, cM, V = 40, 5, 4, 5, 5, 30
    o = OracleHighLow(N, P, T, S, cM, V)
    chance, _ = random_game(rng, N, P, T, S, cM, V)
    for c in chance:
        o.apply_action(c)
    total = np.zeros((N, P), np.int64)
    for _ in range(T * P):
        bid = rng.integers(1, V, N)
        ask = np.minimum(bid + rng.integers(1, 4, N), V)
        bid = np.minimum(bid, ask - 1)
        mv = np.stack([bid, ask, rng.integers(1, S + 1, N), rng.integers(1, S + 1, N)], 1).astype(np.int32)
        o.apply_action(mv)
        total += o.immediate_rewards
    ret = o.fill_returns().astype(np.int64)
    bonus = (o.target_positions != 0) * np.abs(o.target_positions) * V
    assert np.array_equal(total, ret + bonus)
    # and the cash moved by the market sums to zero across players in every env
    assert not o.market.customer_portfolios[:, :, 1].astype(np.int64).sum(axis=1).any()


def test_input_checks_stop_before_trading():
    o = OracleHighLow(3, 4, 2, 5, 5, 30)
    for c in HAND_GAME["chance"]:
        o.apply_action(np.repeat(c, 3, axis=0))
    bad = np.array([[12, 18, 2, 1], [12, 31, 2, 1], [12, 18, 2, 1]], np.int32)  # ask price > V
    with pytest.raises(GameError, match="ask_prices <= max_contract_value"):
        o.apply_action(bad)
    assert o.move_number == 4 and o.market.global_tid == 0


def test_oracle_text_renderings():
    from high_low_cases import (HAND_PRIVATE_TEXT, HAND_PUBLIC_TEXT, HAND_SETUP_TEXT, HAND_TEXT_AFTER)
    from oracle.high_low_oracle import oracle_information_state_string, oracle_to_string
    o = OracleHighLow(**HAND_GAME["params"])
    pending = oracle_information_state_string(o, 0, 0)
    assert pending == ("********** Private Information **********\nPrivate info pending...\n"
                       "***************************\n")
    for c in HAND_GAME["chance"]:
        o.apply_action(c)
    for k, mv in enumerate(HAND_GAME["moves"][:HAND_TEXT_AFTER + 1]):
        o.apply_action(np.array([mv], np.int32))
    book = o.market.to_string(0)
    assert oracle_to_string(o, 0) == HAND_SETUP_TEXT + HAND_PUBLIC_TEXT + book
    for p, priv in HAND_PRIVATE_TEXT.items():
        assert oracle_information_state_string(o, p, 0) == (
            "********** Private Information **********\n" + priv +
            "******************************************\n\n" + HAND_PUBLIC_TEXT + book)


def test_oracle_reset_replays_identically():
    """DoReset (:375-394) returns to the initial state: the hand game after a reset
    gives the same rewards, portfolios, market rows, observation and returns."""
    o = OracleHighLow(**{k: v for k, v in HAND_GAME["params"].items()})
    first = _play_hand(o)
    ret = o.fill_returns().copy()
    o.reset()
    assert o.move_number == 0 and o.current_player() == -1 and not o.is_terminal()
    assert not o.market.customer_portfolios.any() and o.market.global_tid == 0
    assert _play_hand(o) == first
    assert np.array_equal(o.fill_returns(), ret)


def test_game_keeps_the_reference_market_caps():
    """A game whose derived market exceeds the reference's VecMarket caps
    (max_contract_value = 200 gives 201 price levels; market.cu:338-342) raises the
    reference's constructor error, as the reference's game does; the non-reference
    parameter market_extended_shapes lifts the caps (the constructor then gets as
    far as the device check, since this test runs without a GPU)."""
    import pytest
    import astra_cuda as astra
    astra.register_games()
    prm = dict(num_markets=4, players=5, steps_per_player=2, max_contract_value=200)
    with pytest.raises(RuntimeError, match="L <= ASTRA_PRICE_LEVELS"):
        astra.load_game("high_low_trading", prm).new_initial_state()
    import torch
    if torch.cuda.device_count() == 0:
        with pytest.raises(RuntimeError, match="device_id < device_count"):
            astra.load_game("high_low_trading", dict(prm, market_extended_shapes=True)).new_initial_state()


def test_observation_cases_tell_the_round_selections_apart():
    """The hand observations pin the round selection (:559-584): for each case,
    every other plausible choice of rounds (the current round for all players,
    the previous one for all, or the wrap-around split at the observing player;
    a round index of -1 reads the last round, as torch's negative indexing would)
    that differs from the reference's choice gives a vector other than the hand
    one. (For player 0 the wrap-around split is the previous round for all: the
    same choice as its own branch.)"""
    o = OracleHighLow(**{k: v for k, v in HAND_GAME["params"].items()})
    for c in HAND_GAME["chance"]:
        o.apply_action(c)
    cases = HAND_GAME["more_obs"] + [(HAND_GAME["obs_after"], HAND_GAME["obs_player"], HAND_GAME["obs"])]
    P = o.P
    checked = 0
    for k, mv in enumerate(HAND_GAME["moves"]):
        o.apply_action(np.array([mv], np.int32))
        for after, player, want in cases:
            if k != after:
                continue
            cr = (o.move_number - 4) // P
            if cr == 0 or player == P - 1:
                ref = [cr] * P
            elif player == 0:
                ref = [cr - 1] * P
            else:
                ref = [cr if p < player else cr - 1 for p in range(P)]
            pcot = o.player_contract_over_time[0]
            base = o.fill_observation_tensor(player)[0]
            assert base.tolist() == want
            for rounds in ([cr] * P, [cr - 1] * P, [cr if p < player else cr - 1 for p in range(P)]):
                if rounds == ref:
                    continue
                v = base.copy()
                v[7:7 + 6 * P] = np.concatenate([pcot[p, rounds[p]] for p in range(P)]).astype(np.float32)
                assert v.tolist() != want, (after, player, rounds)
                checked += 1
    assert checked >= 5
