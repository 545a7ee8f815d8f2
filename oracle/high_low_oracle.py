"""CPU oracle of the high-low trading game's vectorised state (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline; the
product never calls it.

Restates nlyu1/astra-cuda src/games/high_low_trading/high_low_trading.cc in
numpy, one env per row, int32 arithmetic with two's-complement wrap (numpy int32
arrays wrap like torch's int32 kernels), on top of the C market oracle
(oracle/market_oracle.c) for the order matching:

* chance moves: candidate values (:136-149), high/low settle (:151-173),
  permutation (:175-195), customer sizes (:197-226);
* the trading move (:247-329), including its input checks (:260-271);
* FillRewards / FillRewardsSinceLastAction / FillReturns (:331-373);
* DoReset (:375-394), IsTerminal (:465-467), ExposeInfo (:475-485);
* FillObservationTensor (:510-602) in float32;
* the text renderings ToString (:398-466), InformationStateString (:620-680) and
  PublicInformationString (:682-804), as module functions.

What pins each part (tests/test_high_low_oracle.py; values worked out on paper in
tests/high_low_cases.py, not by running any implementation): the chance moves, the
trading move, every reward, portfolio and market row, the returns, ExposeInfo and
four observations, one for each branch of the round selection (:559-584: round 0,
player 0, the last player, a middle player, each shown to differ from what the
other branches would give), by the hand-derived four-player game; the reward formula also by an
identity (without penalties a player's rewards over a game sum to its return plus
|target|*V for a customer); the input checks by a hand case; the text renderings by
hand-written text; DoReset by replaying the hand game after a reset; the order
matching underneath by the market oracle's own pins (oracle/market_oracle.c). No function
here is left unpinned.

The market shape defaults to the game's own (:57-69): L = max_contract_value + 1,
O = players * steps_per_player * 2, F = min(O, 2 * max_contracts_per_trade),
C = players; a harness may pass another (L, O, F, C) with C >= players, as the
config-5 benchmark does (customers >= players never trade, and the snapshot of
last positions covers customers 0..players-1).
"""
from __future__ import annotations

import math

import numpy as np

from oracle.oracle import OracleMarket

MAX_CHANCE_NODES = 4  # high_low_trading.h:127-133


class GameError(RuntimeError):
    pass


def _check(cond, what):
    if not cond:
        raise GameError(what)


def _i32(a):
    return np.asarray(a).astype(np.int64).astype(np.uint32).view(np.int32)


class OracleHighLow:
    def __init__(self, num_markets, players=5, steps_per_player=20, max_contracts_per_trade=5,
                 customer_max_size=5, max_contract_value=30, market_shape=None):
        self.N, self.P, self.T = int(num_markets), int(players), int(steps_per_player)
        self.S, self.cM, self.V = int(max_contracts_per_trade), int(customer_max_size), int(max_contract_value)
        if market_shape is None:  # high_low_trading.cc:57-69
            O = self.P * self.T * 2
            market_shape = (self.V + 1, O, min(O, self.S * 2), self.P)
        self.L, self.O, self.F, self.C = (int(x) for x in market_shape)
        assert self.C >= self.P
        self.market = OracleMarket(self.N, self.L, self.O, self.F, self.C)
        self.fills = self.market.new_fill_batch()
        self.bbo = self.market.new_bbo_batch()
        N, P, T = self.N, self.P, self.T
        z = lambda *s: np.zeros(s, np.int32)  # noqa: E731
        self.contract_values = z(N, 3)
        self.contract_high_settle = np.zeros(N, bool)
        self.player_permutation = z(N, P)
        self.inv_permutation = z(N, P)
        self.target_positions = z(N, P)
        self.player_last_positions = z(N, P, 2)
        self.player_contract_over_time = z(N, P, T, 6)
        self.market_contract_over_time = z(N, P * T, 3)
        self.immediate_rewards = z(N, P)
        self.rewards_since_last_action = z(N, P)
        self.move_number = 0

    # ---- core State (src/core/core.cc:15-20, core.h:278, 427) ----
    def max_game_length(self):
        return MAX_CHANCE_NODES + self.T * self.P

    def current_player(self):
        if self.is_terminal():
            return -4  # kTerminalPlayerId
        if self.move_number < MAX_CHANCE_NODES:
            return -1  # kChancePlayerId
        return (self.move_number - MAX_CHANCE_NODES) % self.P

    def is_terminal(self):
        return self.move_number >= self.max_game_length()

    def apply_action(self, move):
        player = self.current_player()
        move = np.asarray(move, np.int32)
        _check(move.shape[0] == self.N, "move.size(0) == num_envs_")
        mn = self.move_number
        if mn == 0:
            self._candidate_values(move)
        elif mn == 1:
            self._high_low_settle(move)
        elif mn == 2:
            self._permutation(move)
        elif mn == 3:
            self._customer_size(move)
        else:
            self._trading(move)
        self.move_number += 1
        return player

    # ---- chance moves ----
    def _candidate_values(self, move):  # :136-149
        _check(move.ndim == 2 and move.shape[1] == 2, "candidate values shape")
        _check(move.min() >= 1 and move.max() <= self.V, "candidate values range")
        self.contract_values[:, 0:2] = move

    def _high_low_settle(self, move):  # :151-173
        _check(move.ndim == 1, "settle shape")
        _check(move.min() >= 0 and move.max() <= 1, "settle range")
        self.contract_high_settle = move.astype(bool)
        mx = np.maximum(self.contract_values[:, 0], self.contract_values[:, 1])
        mn = np.minimum(self.contract_values[:, 0], self.contract_values[:, 1])
        self.contract_values[:, 2] = _i32(move.astype(np.int64) * mx + (1 - move.astype(np.int64)) * mn)

    def _permutation(self, move):  # :175-195
        _check(move.ndim == 2 and move.shape[1] == self.P, "permutation shape")
        _check(move.min() >= 0 and move.max() < self.P, "permutation range")
        self.player_permutation = move.copy()
        self.inv_permutation = np.argsort(move, axis=1, kind="stable").astype(np.int32)

    def _customer_size(self, move):  # :197-226
        _check(move.ndim == 2 and move.shape[1] == self.P - 3, "customer size shape")
        a = np.abs(move)
        _check(a.max() <= self.cM, "customer size max")
        _check(a.min() > 0, "customer size zero")
        idx = self.inv_permutation[:, 3:]
        np.put_along_axis(self.target_positions, idx.astype(np.int64), move.astype(np.int32), axis=1)

    # ---- the trading move (:247-329) ----
    def _trading(self, move):
        P, V = self.P, self.V
        player = self.current_player()
        tmn = self.move_number - MAX_CHANCE_NODES
        pmn = tmn // P
        _check(move.ndim == 2 and move.shape[1] == 4, "move.size(1) == 4")
        self.player_last_positions[:] = self.market.customer_portfolios[:, :P, :]
        bid_px = np.ascontiguousarray(move[:, 0])
        ask_px = np.ascontiguousarray(move[:, 1])
        bid_sz = np.ascontiguousarray(move[:, 2])
        ask_sz = np.ascontiguousarray(move[:, 3])
        _check(bid_px.min() > 0, "bid_prices > 0")
        _check(ask_px.min() > 0, "ask_prices > 0")
        _check(bid_px.max() <= V, "bid_prices <= max_contract_value")
        _check(ask_px.max() <= V, "ask_prices <= max_contract_value")
        _check(bid_sz.min() >= 0, "bid_sizes >= 0")
        _check(ask_sz.min() >= 0, "ask_sizes >= 0")
        _check(bid_sz.max() <= self.S, "bid_sizes <= max_contracts_per_trade")
        _check(ask_sz.max() <= self.S, "ask_sizes <= max_contracts_per_trade")
        cust = np.full(self.N, player, np.int32)
        self.market.add_two_sided_quotes(bid_px, bid_sz, ask_px, ask_sz, cust, self.fills)
        self.rewards_since_last_action[:, player] = 0
        cur = self.market.customer_portfolios[:, :P, :].astype(np.int64)
        last = self.player_last_positions.astype(np.int64)
        self.market.get_bbos(self.bbo)
        self.market.update_last_prices(self.bbo, self.fills)
        cash_diff = cur[:, :, 1] - last[:, :, 1]
        self.player_contract_over_time[:, player, pmn, 0:4] = move
        self.player_contract_over_time[:, :, pmn, 4:6] = cur
        self.market_contract_over_time[:, tmn, 0] = self.bbo.best_bid_prices
        self.market_contract_over_time[:, tmn, 1] = self.bbo.best_ask_prices
        self.market_contract_over_time[:, tmn, 2] = self.bbo.last_prices
        tgt = self.target_positions.astype(np.int64)
        prev_diff = np.abs(_i32(last[:, :, 0] - tgt)).astype(np.int64)
        cur_diff = np.abs(_i32(cur[:, :, 0] - tgt)).astype(np.int64)
        is_c = (tgt != 0).astype(np.int64)
        imm = _i32(_i32(is_c * _i32(prev_diff - cur_diff)) * V).astype(np.int64)
        imm = _i32(imm + _i32(cash_diff)).astype(np.int64)
        b, a = bid_sz.astype(np.int64), ask_sz.astype(np.int64)
        pen = _i32(_i32(np.minimum(b, a) + 1) * np.maximum(_i32(bid_px.astype(np.int64) - ask_px + 1), 0))
        pen = _i32(pen.astype(np.int64) * V).astype(np.int64)
        imm[:, player] = _i32(imm[:, player] - pen)
        bid_cheap = (bid_sz == 0).astype(np.int64) * (bid_px != 1).astype(np.int64) * V
        ask_cheap = (ask_sz == 0).astype(np.int64) * (ask_px != V).astype(np.int64) * V
        imm[:, player] = _i32(imm[:, player] - bid_cheap)
        imm[:, player] = _i32(imm[:, player] - ask_cheap)
        if tmn == self.T * P - 1:
            imm = _i32(imm + _i32(cur[:, :, 0] * self.contract_values[:, 2:3].astype(np.int64))).astype(np.int64)
        self.immediate_rewards = _i32(imm)
        self.rewards_since_last_action = _i32(self.rewards_since_last_action.astype(np.int64) + imm)

    # ---- reward and return reads (:331-373) ----
    def fill_rewards(self):
        return self.immediate_rewards.astype(np.float32)

    def fill_rewards_since_last_action(self, player):
        return self.rewards_since_last_action[:, player].astype(np.float32)

    def fill_returns(self):
        pf = self.market.customer_portfolios[:, :self.P, :].astype(np.int64)
        r = pf[:, :, 1] + _i32(pf[:, :, 0] * self.contract_values[:, 2:3].astype(np.int64))
        is_c = (self.target_positions != 0).astype(np.int64)
        diff = np.abs(_i32(pf[:, :, 0] - self.target_positions.astype(np.int64))).astype(np.int64)
        r = _i32(r + _i32(_i32(-is_c * diff) * self.V))
        return r.astype(np.float32)

    def reset(self):  # core.h:427, :375-394
        self.move_number = 0
        for a in (self.contract_values, self.player_permutation, self.inv_permutation,
                  self.target_positions, self.player_last_positions, self.player_contract_over_time,
                  self.market_contract_over_time, self.immediate_rewards, self.rewards_since_last_action):
            a[...] = 0
        self.contract_high_settle = np.zeros(self.N, bool)
        self.market.reset()
        for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
            getattr(self.bbo, f)[...] = 0
        for f in ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
                  "fill_quote_sizes", "fill_tid", "fill_quote_tid", "fill_counts"):
            getattr(self.fills, f)[...] = 0

    def expose_info(self):  # :475-485
        _check(self.is_terminal(), "ExposeInfo called on non-terminal state")
        return {"players": self.player_contract_over_time.copy(),
                "market": self.market_contract_over_time.copy(),
                "target_positions": self.target_positions.copy()}

    # ---- FillObservationTensor (:510-602) ----
    def observation_shape(self):
        return (self.N, 6 + 1 + 6 * self.P + 5)

    def fill_observation_tensor(self, player):
        _check(0 <= player < self.P, "player range")
        _check(self.move_number >= MAX_CHANCE_NODES, "observation before trading")
        P = self.P
        v = np.zeros(self.observation_shape(), np.float32)
        perm = self.player_permutation[:, player]
        v[:, 0] = ((perm == 0) | (perm == 1)).astype(np.float32)
        v[:, 1] = (perm == 2).astype(np.float32)
        v[:, 2] = (perm > 2).astype(np.float32)
        angle = 2.0 * math.pi * player / P
        v[:, 3] = np.float32(math.sin(angle))
        v[:, 4] = np.float32(math.cos(angle))
        m0, m1, m2, mc = perm == 0, perm == 1, perm == 2, perm > 2
        v[m0, 5] = self.contract_values[m0, 0].astype(np.float32)
        v[m1, 5] = self.contract_values[m1, 1].astype(np.float32)
        v[m2, 5] = self.contract_high_settle[m2].astype(np.float32)
        v[mc, 5] = self.target_positions[mc, player].astype(np.float32)
        ctm = max(0, self.move_number - MAX_CHANCE_NODES)
        cr = ctm // P
        v[:, 6] = np.float32(cr) / np.float32(self.T)
        pcot = self.player_contract_over_time
        if cr == 0 or player == P - 1:
            data = pcot[:, :, cr, :].reshape(self.N, P * 6)
        elif player == 0:
            data = pcot[:, :, cr - 1, :].reshape(self.N, P * 6)
        else:
            data = np.concatenate([pcot[:, :player, cr, :], pcot[:, player:, cr - 1, :]], axis=1)
            data = data.reshape(self.N, P * 6)
        v[:, 7:7 + 6 * P] = data.astype(np.float32)
        o = 7 + 6 * P
        v[:, o] = self.bbo.best_bid_prices.astype(np.float32)
        v[:, o + 1] = self.bbo.best_ask_prices.astype(np.float32)
        v[:, o + 2] = self.bbo.best_bid_sizes.astype(np.float32)
        v[:, o + 3] = self.bbo.best_ask_sizes.astype(np.float32)
        v[:, o + 4] = self.bbo.last_prices.astype(np.float32)
        return v


# ---- text renderings (high_low_trading.cc:398-466, 603-804), numpy restatement ----
def _roles_line(perm_row):
    names = []
    for i, r in enumerate(perm_row):
        names.append(f"P{i}=" + ("ValueCheater" if r in (0, 1) else "HighLowCheater" if r == 2 else "Customer"))
    return "Player permutation: Player roles: " + ", ".join(names) + "\n"


def oracle_to_string(o: OracleHighLow, index: int) -> str:
    out = ["********** Game setup **********\n"]
    mn = o.move_number
    if mn >= 1:
        out.append(f"Contract values: {o.contract_values[index, 0]}, {o.contract_values[index, 1]}\n")
    if mn >= 2:
        out.append("Contract high settle: " + ("High" if o.contract_high_settle[index] else "Low") + "\n")
    if mn >= 3:
        out.append(_roles_line(o.player_permutation[index]))
    if mn >= 4:
        for i in range(o.P):
            t = int(o.target_positions[index, i])
            out.append(f"Player {i} target position: " + ("No requirement" if t == 0 else str(t)) + "\n")
    out.append("********************************\n\n")
    if mn >= MAX_CHANCE_NODES:
        out.append(oracle_public_information(o, index))
    return "".join(out)


def oracle_public_information(o: OracleHighLow, index: int) -> str:
    out = ["********** Game Configuration **********\n",
           f"Environment: {index} / {o.N}\n", f"Steps per player: {o.T}\n",
           f"Max contracts per trade: {o.S}\n", f"Customer max size: {o.cM}\n",
           f"Max contract value: {o.V}\n", f"Number of players: {o.P}\n",
           "****************************************\n\n", "********** Player Positions **********\n"]
    pf = o.market.customer_portfolios
    for i in range(o.P):
        out.append(f"Player {i} position: [{pf[index, i, 0]} contracts, {pf[index, i, 1]} cash]\n")
    out.append("**************************************\n\n")
    out.append("********** Quotes & Market Movement **********\n")
    f = o.fills
    n = int(f.fill_counts[index])
    out.append(f"Number of fills in the last round: {n}\n")
    for i in range(max(n, 0)):
        sell = bool(f.fill_is_sell_quote[index, i])
        out.append(f"Order fill: id={f.fill_customer_ids[index, i]} {'bought' if sell else 'sold'} "
                   f"{f.fill_sizes[index, i]} contracts at px={f.fill_prices[index, i]} on t={f.fill_tid[index, i]}. "
                   f"Quote: id={f.fill_quoter_ids[index, i]} {'sale' if sell else 'bid'} sz={f.fill_quote_sizes[index, i]}, "
                   f"submitted t={f.fill_quote_tid[index, i]}\n")
    ctm = max(0, o.move_number - MAX_CHANCE_NODES)
    cr, pin = ctm // o.P, ctm % o.P
    pc = o.player_contract_over_time
    for rnd in range(0, min(cr, o.T - 1) + 1):
        if rnd > cr:
            break
        for p in range(o.P if rnd < cr else pin):
            bp, ap, bs, az = (int(x) for x in pc[index, p, rnd, :4])
            if bp > 0 or ap > 0:
                out.append(f"Player {p} quote: {bp} @ {ap} [{bs} x {az}]\n")
    out.append("\n--- Market Movement ---\n")
    mc = o.market_contract_over_time
    for t in range(min(ctm, o.P * o.T)):
        bb, ba, lp = (int(x) for x in mc[index, t])
        out.append(f"Time {t}: Bid: {'none' if bb == -1 else bb} @ Ask: {'none' if ba == -1 else ba}"
                   + (f", Last: {lp}" if lp != -1 else "") + "\n")
    out.append("***********************************\n\n")
    out.append("********** Current Market **********\n")
    out.append(o.market.to_string(index))
    return "".join(out)


def oracle_information_state_string(o: OracleHighLow, player: int, index: int) -> str:
    out = ["********** Private Information **********\n"]
    if o.move_number >= MAX_CHANCE_NODES:
        perm = int(o.player_permutation[index, player])
        role = "ValueCheater" if perm in (0, 1) else "HighLowCheater" if perm == 2 else "Customer"
        out.append(f"My role: {role}\n")
        if perm in (0, 1):
            out.append(f"Candidate contract value: {o.contract_values[index, perm]}\n")
        elif perm == 2:
            out.append("Settlement will be: " + ("High" if o.contract_high_settle[index] else "Low") + "\n")
        else:
            t = int(o.target_positions[index, player])
            _check(t != 0, "Not supposed to happen. Customer roles should be assigned")
            out.append(f"My target position: {t}\n")
        out.append("******************************************\n\n")
        out.append(oracle_public_information(o, index))
    else:
        out.append("Private info pending...\n")
        out.append("***************************\n")
    return "".join(out)
