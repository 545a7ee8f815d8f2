"""The high-low trading game on the MI355X engine.

Mirrors nlyu1/astra-cuda src/games/high_low_trading/high_low_trading.{h,cc}
(``HighLowTradingGame``, ``HighLowTradingState``) with the method names of the
reference's core bindings (src/pybind/core/core_bindings.cc:33-115), so code
written against ``astra.load_game("high_low_trading", params)`` runs unchanged.
One state holds ``num_markets`` independent envs, each a VecMarket market.

The trading move (ApplyPlayerTrading, high_low_trading.cc:247-329) and
FillObservationTensor (:510-602) run as the HIP kernels of
include/astra_high_low.h: one launch of the matching kernel with the game's
work fused, plus a check launch and one host wait, for the checks only, while
the move kernel runs (the reference makes eight syncs); a move that fails a
check changes nothing and raises. ``check_moves=False`` drops the check and the
wait, and
``check_errors()`` then reports any move that failed a check. FillRewards and
FillRewardsSinceLastAction (:331-343) convert into a float32 buffer on a HIP
kernel too. The chance moves (:136-226), returns and reset are the reference's
tensor operations.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import torch

from . import _native
from .order_matching import VecMarket, _check, _fatal, _raw_stream

MAX_CHANCE_NODES = 4            # high_low_trading.h:127-133
CHANCE_PLAYER_ID = -1           # src/core/core.h kChancePlayerId
TERMINAL_PLAYER_ID = -4         # src/core/core.h kTerminalPlayerId

# high_low_trading.h:19-26 and the parameter specification (high_low_trading.cc:36-45)
DEFAULT_PARAMETERS = {
    "steps_per_player": 20,
    "max_contracts_per_trade": 5,
    "customer_max_size": 5,
    "max_contract_value": 30,
    "players": 5,
    "num_markets": 32768,
    "threads_per_block": 128,
    "device_id": 0,
}
# Not in the reference: override the market shape the game derives (:57-69), for
# game-shaped benchmarks on larger books. num_customers must be >= players.
# A shape beyond the reference's VecMarket caps (L <= 128, O <= 1024, F <= 1024,
# C <= 1024) raises the reference's constructor error (market.cu:338-342) unless
# market_extended_shapes is true.
MARKET_SHAPE_PARAMETERS = ("market_price_levels", "market_orders", "market_fills", "market_customers",
                           "market_extended_shapes")


def _assert(cond: bool, what: str):
    if not cond:
        _fatal(f"high_low_trading.py {what}")


class HighLowTradingGame:
    """HighLowTradingGame (high_low_trading.h:117-153)."""

    short_name = "high_low_trading"

    def __init__(self, params: dict | None = None):
        params = dict(params or {})
        unknown = set(params) - set(DEFAULT_PARAMETERS) - set(MARKET_SHAPE_PARAMETERS) - {"check_moves"}
        if unknown:
            _fatal(f"Unknown parameter(s) for high_low_trading: {sorted(unknown)}")
        self._params = {**DEFAULT_PARAMETERS, **params}
        p = self._params
        self.steps_per_player = int(p["steps_per_player"])
        self.max_contracts_per_trade = int(p["max_contracts_per_trade"])
        self.customer_max_size = int(p["customer_max_size"])
        self.max_contract_value = int(p["max_contract_value"])
        self.players = int(p["players"])
        self.num_markets = int(p["num_markets"])
        self.threads_per_block = int(p["threads_per_block"])
        self.device_id = int(p["device_id"])
        self.check_moves = bool(p.get("check_moves", True))
        orders = self.players * self.steps_per_player * 2  # :57-69
        self.market_shape = (
            int(p.get("market_price_levels", self.max_contract_value + 1)),
            int(p.get("market_orders", orders)),
            int(p.get("market_fills", min(orders, self.max_contracts_per_trade * 2))),
            int(p.get("market_customers", self.players)),
        )
        if self.market_shape[3] < self.players:
            _fatal("high_low_trading.py market_customers >= players")
        self.market_extended_shapes = bool(p.get("market_extended_shapes", False))

    # core_bindings.cc:93-115
    def new_initial_state(self) -> "HighLowTradingState":
        return HighLowTradingState(self)

    def get_parameters(self) -> dict:
        return {k: v for k, v in self._params.items()}

    def num_players(self) -> int:
        return self.players

    def max_chance_nodes_in_history(self) -> int:
        return MAX_CHANCE_NODES

    def max_game_length(self) -> int:  # high_low_trading.h:124-126
        return MAX_CHANCE_NODES + self.steps_per_player * self.players

    def max_move_number(self) -> int:
        return self.max_game_length()

    def observation_tensor_shape(self) -> list:  # :506-508
        return [self.num_markets, 6 + 1 + 6 * self.players + 5]

    def information_state_tensor_shape(self):  # :491-493
        _fatal("InformationStateTensorShape not implemented")

    NumPlayers = num_players
    MaxGameLength = max_game_length
    MaxChanceNodesInHistory = max_chance_nodes_in_history
    ObservationTensorShape = observation_tensor_shape
    NewInitialState = new_initial_state

    def __repr__(self):
        return f"high_low_trading({self._params})"


class HighLowTradingState:
    """HighLowTradingState (high_low_trading.h:30-115)."""

    def __init__(self, game: HighLowTradingGame, _clone_of: "HighLowTradingState | None" = None):
        self._game = game
        N, P, T = game.num_markets, game.players, game.steps_per_player
        self._N, self._P, self._T = N, P, T
        self._dev = torch.device("cuda", game.device_id)
        if _clone_of is None:
            L, O, F, C = game.market_shape
            self.market = VecMarket(N, L, O, F, C, game.device_id, game.threads_per_block,
                                    allow_extended_shapes=game.market_extended_shapes)
            i32 = dict(dtype=torch.int32, device=self._dev)
            self.contract_values = torch.zeros((N, 3), **i32)
            self.contract_high_settle = torch.zeros((N,), dtype=torch.bool, device=self._dev)
            self.player_permutation = torch.zeros((N, P), **i32)
            self.inv_permutation = torch.zeros((N, P), **i32)
            self.target_positions = torch.zeros((N, P), **i32)
            self.player_last_positions = torch.zeros((N, P, 2), **i32)
            # player_contract_over_time, stored env-minor (see the property below)
            self._pcot = torch.zeros((T, P, 6, N), **i32)
            # market_contract_over_time, stored env-minor (see the property below)
            self._mcot = torch.zeros((P * T, 3, N), **i32)
            self.immediate_rewards = torch.zeros((N, P), **i32)
            self.rewards_since_last_action = torch.zeros((N, P), **i32)
            self.bbo_batch = self.market.new_bbo_batch()
            # the fills stay inside the state, so the row layout (one 32-byte write
            # per fill) costs callers nothing
            self.fill_batch = self.market.new_fill_batch(layout="rows")
            self._move_number = 0
        else:  # copy constructor (high_low_trading.cc:104-123)
            o = _clone_of
            self.market = o.market.clone()
            for name in ("contract_values", "contract_high_settle", "player_permutation",
                         "inv_permutation", "target_positions", "player_last_positions",
                         "_pcot", "_mcot",
                         "immediate_rewards", "rewards_since_last_action"):
                setattr(self, name, getattr(o, name).clone())
            self.bbo_batch = o.bbo_batch.clone()
            self.fill_batch = o.fill_batch.clone()
            self._move_number = o._move_number
        self._errors = torch.zeros((1,), dtype=torch.int32, device=self._dev)
        # the checked move's error word lands here (pinned) for the one host wait
        self._errors_host = torch.zeros((1,), dtype=torch.int32, pin_memory=True)
        self._lib = _native.lib()
        # the C entry point of a trading move (astra_high_low_trade)
        self._trade_fn = self._lib.astra_high_low_trade
        self._trade = self._make_trade_args()

    @property
    def player_contract_over_time(self) -> torch.Tensor:
        """The reference's [N,P,T,6] tensor (bid_px, ask_px, bid_sz, ask_sz, contracts,
        cash per player and round, high_low_trading.h:109) as a view. The storage is
        [T,P,6,N], env-minor, so that the move's stores and the observation's loads of
        consecutive envs touch adjacent words."""
        return self._pcot.permute(3, 1, 0, 2)

    @property
    def market_contract_over_time(self) -> torch.Tensor:
        """The reference's [N,P*T,3] tensor (best bid, best ask, last price after each
        trading move, high_low_trading.h:110) as a view of [P*T,3,N] storage, env-minor
        like player_contract_over_time."""
        return self._mcot.permute(2, 0, 1)

    def _make_trade_args(self):
        g = self._game
        t = _native.HLTrade()
        fb, bb = self.fill_batch, self.bbo_batch
        ptrs = {
            "player_last_positions": self.player_last_positions,
            "target_positions": self.target_positions, "contract_values": self.contract_values,
            "player_contract_over_time": self._pcot,
            "market_contract_over_time": self._mcot,
            "immediate_rewards": self.immediate_rewards,
            "rewards_since_last_action": self.rewards_since_last_action,
            "errors": self._errors,
        }
        ptrs["fill_counts"] = fb.fill_counts
        if fb._rows is not None:
            ptrs["fill_rows"] = fb._rows
        else:
            for f in ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
                      "fill_quote_sizes", "fill_tid", "fill_quote_tid"):
                ptrs[f] = getattr(fb, f)
        for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
            ptrs[f] = getattr(bb, f)
        for k, v in ptrs.items():
            assert v.is_contiguous() and v.device == self._dev, k
            setattr(t, k, v.data_ptr())
        t.errors_host = self._errors_host.data_ptr()
        t.players, t.steps_per_player = self._P, self._T
        t.max_contracts_per_trade, t.max_contract_value = g.max_contracts_per_trade, g.max_contract_value
        t.check = 1 if g.check_moves else 0
        return t

    # ---- core State (src/core/core.h, core.cc:15-20) ----
    def current_player(self) -> int:  # :125-134
        if self.is_terminal():
            return TERMINAL_PLAYER_ID
        if self._move_number < MAX_CHANCE_NODES:
            return CHANCE_PLAYER_ID
        return (self._move_number - MAX_CHANCE_NODES) % self._P

    def is_terminal(self) -> bool:  # :465-467
        return self._move_number >= self._game.max_game_length()

    def is_chance_node(self) -> bool:
        return self.current_player() == CHANCE_PLAYER_ID

    def is_player_node(self) -> bool:
        return self.current_player() >= 0

    def is_simultaneous_node(self) -> bool:
        return False

    def is_player_acting(self, player: int) -> bool:
        return self.current_player() == player

    def move_number(self) -> int:
        return self._move_number

    def is_initial_state(self) -> bool:
        return self._move_number == 0

    def num_players(self) -> int:
        return self._P

    def get_game(self) -> HighLowTradingGame:
        return self._game

    def apply_action(self, action_id: torch.Tensor) -> int:
        """ApplyAction (core.cc:15-20) -> DoApplyAction (:228-245)."""
        player = self.current_player()
        move = action_id
        _assert(move.size(0) == self._N, f"move.size(0) == num_envs_\nmove.size(0) = {move.size(0)}, "
                                         f"num_envs_ = {self._N}")
        mn = self._move_number
        if mn == 0:
            self._apply_candidate_values(move)
        elif mn == 1:
            self._apply_high_low_settle(move)
        elif mn == 2:
            self._apply_permutation(move)
        elif mn == 3:
            self._apply_customer_size(move)
        else:
            self._apply_player_trading(move)
        self._move_number += 1
        return player

    def child(self, action):
        c = self.clone()
        c.apply_action(action)
        return c

    def clone(self) -> "HighLowTradingState":
        return HighLowTradingState(self._game, _clone_of=self)

    def reset(self) -> None:
        """Reset (core.h:427) -> DoReset (:375-394)."""
        self._move_number = 0
        for t in (self.contract_values, self.contract_high_settle, self.player_permutation,
                  self.inv_permutation, self.target_positions, self.player_last_positions,
                  self._pcot, self._mcot,
                  self.immediate_rewards, self.rewards_since_last_action):
            t.zero_()
        self.market.reset()
        self.bbo_batch.reset()
        self.fill_batch.reset()

    # ---- chance moves (:136-226), tensor operations as in the reference ----
    def _apply_candidate_values(self, move):
        _assert(move.dim() == 2, f"move.dim() == 2\nmove.dim() = {move.dim()}")
        _assert(move.size(1) == 2, f"move.size(1) == 2\nmove.size(1) = {move.size(1)}")
        lo, hi = int(torch.min(move).item()), int(torch.max(move).item())
        _assert(lo >= 1, f"min_val >= 1\nmin_val = {lo}")
        _assert(hi <= self._game.max_contract_value, f"max_val <= GetGame()->GetMaxContractValue()\nmax_val = {hi}")
        self.contract_values[:, 0:2] = move

    def _apply_high_low_settle(self, move):
        _assert(move.dim() == 1, f"move.dim() == 1\nmove.dim() = {move.dim()}")
        lo, hi = int(torch.min(move).item()), int(torch.max(move).item())
        _assert(lo >= 0, f"min_val >= 0\nmin_val = {lo}")
        _assert(hi <= 1, f"max_val <= 1\nmax_val = {hi}")
        self.contract_high_settle.copy_(move.to(torch.bool))
        mx = torch.max(self.contract_values[:, 0], self.contract_values[:, 1])
        mn = torch.min(self.contract_values[:, 0], self.contract_values[:, 1])
        self.contract_values[:, 2] = move * mx + (1 - move) * mn

    def _apply_permutation(self, move):
        _assert(move.dim() == 2, f"move.dim() == 2\nmove.dim() = {move.dim()}")
        _assert(move.size(1) == self._P, f"move.size(1) == num_players_\nmove.size(1) = {move.size(1)}")
        lo, hi = int(torch.min(move).item()), int(torch.max(move).item())
        _assert(lo >= 0, f"min_val >= 0\nmin_val = {lo}")
        _assert(hi < self._P, f"max_val < num_players_\nmax_val = {hi}")
        self.player_permutation.copy_(move)
        self.inv_permutation.copy_(move.argsort(dim=1))

    def _apply_customer_size(self, move):
        _assert(move.dim() == 2, f"move.dim() == 2\nmove.dim() = {move.dim()}")
        _assert(move.size(1) == self._P - 3, f"move.size(1) == num_players_ - 3\nmove.size(1) = {move.size(1)}")
        a = torch.abs(move)
        _assert(int(torch.max(a).item()) <= self._game.customer_max_size,
                "torch::max(abs_move).item<int>() <= GetGame()->GetCustomerMaxSize()")
        _assert(int(torch.min(a).item()) > 0, "torch::min(abs_move).item<int>() > 0")
        idx = self.inv_permutation[:, 3:]
        self.target_positions.scatter_(1, idx.to(torch.int64), move.to(self.target_positions.dtype))

    # ---- the trading move (:247-329) on the HIP kernels ----
    def _apply_player_trading(self, move):
        player = self.current_player()
        tmn = self._move_number - MAX_CHANCE_NODES
        _assert(move.dim() == 2 and move.size(1) == 4, f"move.size(1) == 4\nmove.size(1) = {move.size(-1)}")
        if move.dtype != torch.int32:
            _fatal(f"move tensor must be int32, got {move.dtype}")
        if move.device != self._dev:
            _fatal(f"move tensor must be on device {self._game.device_id}")
        move = move.contiguous()
        t = self._trade
        t.move = move.data_ptr()
        t.player = player
        t.trade_move_number = tmn
        rc = self._trade_fn(self.market._h, ctypes.byref(t),
                                           _raw_stream(self._game.device_id))
        self._last_move = move  # keep the buffer alive while the kernels may read it
        if rc:
            self._errors.zero_()
            _fatal(_native.last_error())

    def set_check_moves(self, check: bool) -> None:
        """Switch the per-move input checks (one host wait per move) on or off.
        Switching them on first reports (raises, like check_errors) any unchecked
        move since the last check_errors() that failed a check, and clears the
        error word, so the next checked move sees only its own checks."""
        was = self._trade.check
        self._trade.check = 1 if check else 0
        if check and not was:
            self.check_errors()

    def check_errors(self) -> None:
        """With check_moves=False: raise if any move since the last call failed the
        reference's input checks (high_low_trading.cc:264-271). Synchronises."""
        bits = int(self._errors.item())
        if bits:
            self._errors.zero_()
            names = ("bid_prices > 0", "ask_prices > 0", "bid_prices <= max_contract_value",
                     "ask_prices <= max_contract_value", "bid_sizes >= 0", "ask_sizes >= 0",
                     "bid_sizes <= max_contracts_per_trade", "ask_sizes <= max_contracts_per_trade")
            _fatal("high_low_trading.py moves failed: " + ", ".join(n for i, n in enumerate(names) if bits >> i & 1))

    # ---- rewards and returns (:331-373) ----
    def fill_rewards(self, reward_buffer: torch.Tensor) -> None:
        _assert(reward_buffer.dim() == 2 and reward_buffer.size(0) == self._N and reward_buffer.size(1) == self._P,
                "reward_buffer shape == [num_envs, num_players]")
        self._rewards_to(reward_buffer, self.immediate_rewards, -1)

    def fill_rewards_since_last_action(self, reward_buffer: torch.Tensor, player_id: int) -> None:
        _assert(reward_buffer.dim() == 1 and reward_buffer.size(0) == self._N,
                "reward_buffer shape == [num_envs]")
        if 0 <= player_id < self._P:
            self._rewards_to(reward_buffer, self.rewards_since_last_action, player_id)
        else:  # the reference's index error
            reward_buffer.copy_(self.rewards_since_last_action[:, player_id])

    def _rewards_to(self, buf: torch.Tensor, src: torch.Tensor, player: int) -> None:
        """buf.copy_(src, or its column `player`) on the HIP kernel for a contiguous
        float32 buffer on the game's device; torch's copy_ for any other buffer."""
        if buf.dtype == torch.float32 and buf.is_contiguous() and buf.device == self._dev:
            _check(self._lib.astra_high_low_rewards(src.data_ptr(), self._N, self._P, player,
                                                    buf.data_ptr(), _raw_stream(self._game.device_id)))
        else:
            buf.copy_(src if player < 0 else src[:, player])

    def fill_returns(self, returns_buffer: torch.Tensor) -> None:
        _assert(returns_buffer.dim() == 2 and returns_buffer.size(0) == self._N and returns_buffer.size(1) == self._P,
                "returns_buffer shape == [num_envs, num_players]")
        returns_buffer.zero_()
        is_customer = self.target_positions != 0
        pf = self.market.get_customer_portfolios()[:, :self._P]
        returns_buffer.add_(pf[:, :, 1])
        returns_buffer.addcmul_(pf[:, :, 0], self.contract_values[:, 2].unsqueeze(-1))
        diff = torch.abs(pf[:, :, 0] - self.target_positions)
        returns_buffer.add_(-is_customer.to(torch.int32) * diff * self._game.max_contract_value)

    # ---- FillObservationTensor (:510-602) on the HIP kernel ----
    def fill_observation_tensor(self, *args):
        """fill_observation_tensor(player, values) or fill_observation_tensor(values) -> player
        (core_bindings.cc:77-82)."""
        if len(args) == 1:
            values, player, ret = args[0], self.current_player(), True
        else:
            player, values = args
            ret = False
        g = self._game
        _assert(0 <= player < self._P, f"player >= 0 && player < NumPlayers()\nplayer = {player}")
        _assert(self._move_number >= MAX_CHANCE_NODES, "MoveNumber() >= MaxChanceNodesInHistory()")
        shape = g.observation_tensor_shape()
        _assert(list(values.shape) == shape, f"values.sizes() == {shape}\nvalues.sizes() = {list(values.shape)}")
        if values.dtype != torch.float32 or not values.is_contiguous() or values.device != self._dev:
            _fatal("values must be a contiguous float32 tensor on the game's device")
        ctm = max(0, self._move_number - MAX_CHANCE_NODES)
        cr = ctm // self._P
        _assert(cr < self._T, f"current_round < steps_per_player\ncurrent_round = {cr}")
        angle = 2.0 * math.pi * player / self._P
        o = _native.HLObservation()
        o.values = values.data_ptr()
        o.player_permutation = self.player_permutation.data_ptr()
        o.contract_values = self.contract_values.data_ptr()
        o.contract_high_settle = self.contract_high_settle.data_ptr()
        o.target_positions = self.target_positions.data_ptr()
        o.player_contract_over_time = self._pcot.data_ptr()
        bb = self.bbo_batch
        o.best_bid_prices = bb.best_bid_prices.data_ptr()
        o.best_ask_prices = bb.best_ask_prices.data_ptr()
        o.best_bid_sizes = bb.best_bid_sizes.data_ptr()
        o.best_ask_sizes = bb.best_ask_sizes.data_ptr()
        o.last_prices = bb.last_prices.data_ptr()
        o.num_envs, o.players, o.steps_per_player = self._N, self._P, self._T
        o.player, o.current_round = player, cr
        o.player_sin = float(np.float32(math.sin(angle)))
        o.player_cos = float(np.float32(math.cos(angle)))
        o.round_fraction = float(np.float32(cr) / np.float32(self._T))
        _check(self._lib.astra_high_low_observation(ctypes.byref(o), _raw_stream(g.device_id)))
        return player if ret else None

    def fill_information_state_tensor(self, *args):  # :495-500: not implemented in the reference
        _fatal("FillInformationStateTensor not implemented")

    def expose_info(self) -> dict:  # :475-485
        if not self.is_terminal():
            _fatal("ExposeInfo called on non-terminal state")
        cf = torch.contiguous_format  # copies in the reference's layout, not views of the storage
        return {"players": self.player_contract_over_time.clone(memory_format=cf),
                "market": self.market_contract_over_time.clone(memory_format=cf),
                "target_positions": self.target_positions.clone()}

    # ---- text renderings (:398-466, :603-804); copies the tensors to the host ----
    def to_string(self, index: int = 0) -> str:
        """ToString (:398-466)."""
        self._check_index(index)
        mn = self._move_number
        out = ["********** Game setup **********\n"]
        if mn >= 1:
            cv = self.contract_values[index].tolist()
            out.append(f"Contract values: {cv[0]}, {cv[1]}\n")
        if mn >= 2:
            out.append("Contract high settle: " + ("High" if bool(self.contract_high_settle[index]) else "Low") + "\n")
        if mn >= 3:
            roles = [f"P{i}=" + ("ValueCheater" if r in (0, 1) else "HighLowCheater" if r == 2 else "Customer")
                     for i, r in enumerate(self.player_permutation[index].tolist())]
            out.append("Player permutation: Player roles: " + ", ".join(roles) + "\n")
        if mn >= 4:
            for i, t in enumerate(self.target_positions[index].tolist()):
                out.append(f"Player {i} target position: " + ("No requirement" if t == 0 else str(t)) + "\n")
        out.append("********************************\n\n")
        if mn >= MAX_CHANCE_NODES:
            out.append(self._public_information_string(index))
        return "".join(out)

    def information_state_string(self, player: int | None = None, index: int = 0) -> str:
        """InformationStateString (:620-680). Called with one positional argument it
        is the player, as the reference binding resolves its two overloads
        (core_bindings.cc:59-64); without a player it uses the current player."""
        if player is None:
            player = self.current_player()
        player, index = int(player), int(index)
        _assert(0 <= player < self._P, f"player >= 0 && player < NumPlayers()\nplayer = {player}")
        self._check_index(index)
        out = ["********** Private Information **********\n"]
        if self._move_number >= MAX_CHANCE_NODES:
            perm = int(self.player_permutation[index, player])
            role = "ValueCheater" if perm in (0, 1) else "HighLowCheater" if perm == 2 else "Customer"
            out.append(f"My role: {role}\n")
            if perm in (0, 1):
                out.append(f"Candidate contract value: {int(self.contract_values[index, perm])}\n")
            elif perm == 2:
                out.append("Settlement will be: " + ("High" if bool(self.contract_high_settle[index]) else "Low") + "\n")
            else:
                t = int(self.target_positions[index, player])
                if t == 0:
                    _fatal("Not supposed to happen. Customer roles should be assigned")
                out.append(f"My target position: {t}\n")
            out.append("******************************************\n\n")
            out.append(self._public_information_string(index))
        else:
            out.append("Private info pending...\n")
            out.append("***************************\n")
        return "".join(out)

    observation_string = information_state_string  # ObservationString (:502-504)

    def _public_information_string(self, index: int) -> str:
        """PublicInformationString (:682-804)."""
        g = self._game
        out = ["********** Game Configuration **********\n", f"Environment: {index} / {self._N}\n",
               f"Steps per player: {self._T}\n", f"Max contracts per trade: {g.max_contracts_per_trade}\n",
               f"Customer max size: {g.customer_max_size}\n", f"Max contract value: {g.max_contract_value}\n",
               f"Number of players: {self._P}\n", "****************************************\n\n",
               "********** Player Positions **********\n"]
        pf = self.market.get_customer_portfolios()[index].tolist()
        for i in range(self._P):
            out.append(f"Player {i} position: [{pf[i][0]} contracts, {pf[i][1]} cash]\n")
        out.append("**************************************\n\n")
        out.append("********** Quotes & Market Movement **********\n")
        fb = self.fill_batch
        n = int(fb.fill_counts[index])
        out.append(f"Number of fills in the last round: {n}\n")
        if n > 0:
            cols = {f: getattr(fb, f)[index, :n].tolist() for f in (
                "fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
                "fill_quote_sizes", "fill_tid", "fill_quote_tid")}
            for i in range(n):
                sell = bool(cols["fill_is_sell_quote"][i])
                out.append(f"Order fill: id={cols['fill_customer_ids'][i]} {'bought' if sell else 'sold'} "
                           f"{cols['fill_sizes'][i]} contracts at px={cols['fill_prices'][i]} on "
                           f"t={cols['fill_tid'][i]}. Quote: id={cols['fill_quoter_ids'][i]} "
                           f"{'sale' if sell else 'bid'} sz={cols['fill_quote_sizes'][i]}, "
                           f"submitted t={cols['fill_quote_tid'][i]}\n")
        ctm = max(0, self._move_number - MAX_CHANCE_NODES)
        cr, pin = ctm // self._P, ctm % self._P
        pc = self.player_contract_over_time[index].tolist()
        for rnd in range(0, min(cr, self._T - 1) + 1):
            for p in range(self._P if rnd < cr else pin):
                bp, ap, bs, az = pc[p][rnd][:4]
                if bp > 0 or ap > 0:
                    out.append(f"Player {p} quote: {bp} @ {ap} [{bs} x {az}]\n")
        out.append("\n--- Market Movement ---\n")
        mc = self.market_contract_over_time[index].tolist()
        for t in range(min(ctm, self._P * self._T)):
            bb, ba, lp = mc[t]
            out.append(f"Time {t}: Bid: {'none' if bb == -1 else bb} @ Ask: {'none' if ba == -1 else ba}"
                       + (f", Last: {lp}" if lp != -1 else "") + "\n")
        out.append("***********************************\n\n")
        out.append("********** Current Market **********\n")
        out.append(self.market.to_string(index))
        return "".join(out)

    def _check_index(self, index: int) -> None:
        _assert(0 <= index < self._N, f"index >= 0 && index < num_envs_\nindex = {index}")

    def __str__(self):
        return self.to_string(0)

    __repr__ = __str__

    def get_contract_value(self) -> torch.Tensor:  # :469-473
        _assert(self._move_number >= 2, "MoveNumber() >= 2")
        return self.contract_values[:, 2]

    # C++ method names
    CurrentPlayer = current_player
    IsTerminal = is_terminal
    ApplyAction = apply_action
    MoveNumber = move_number
    FillRewards = fill_rewards
    FillRewardsSinceLastAction = fill_rewards_since_last_action
    FillReturns = fill_returns
    FillObservationTensor = fill_observation_tensor
    Clone = clone
    Reset = reset
    ToString = to_string
    InformationStateString = information_state_string
    ObservationString = observation_string
