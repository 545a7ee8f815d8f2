"""Deterministic synthetic quote streams for the benchmark configurations.

Every random draw is a pure function of (seed, step, market, field): SplitMix64
of a packed 64-bit counter, so a config can be regenerated for any step range
and any subset of markets, on any host, bit for bit. Only integer arithmetic and
IEEE double +,-,*,/ (correctly rounded everywhere) are used, so the streams do
not depend on a libm.

Counter layout (bits): seed 56-63 | field 48-55 | step 24-47 | market 0-23.

Configurations (the BASELINE.json ``configs`` list, 1-based):
  1. CPU reference run: 64 markets, L=128, O=F=1024, C=16, 1000 steps;
     customer = step mod 16; bid ~ U[0,63]; ask = min(bid + U[1,63], 127);
     sizes U[1,10].
  2. README shape: 10,000 markets, 10,000 steps; bid/ask prices independently
     U[0,127]; sizes U[1,10]; customer U[0,15]; get_bbos every step.
  3. Stress: 100,000 markets, 1000 steps; per-market mid random walk
     mid <- clip(mid + U[-3,3], 0, 127) from 64; spread s ~ U[0,8];
     bid = clip(mid - s//2, 0, 127); ask = clip(bid + s, 0, 127);
     sizes geometric(p=0.3) on {1,2,...} capped at 50; customer U[0,15].
  4. Deep book: 20,000 markets, L=512, O=F=4096, C=64, 2000 steps; prices
     clip(round(N(256, 40)), 0, 511) from a 16-term Irwin-Hall sum; sizes
     U[1,100]; customer U[0,63].
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)

# field ids
F_BID_PX, F_ASK_PX, F_BID_SZ, F_ASK_SZ, F_CUST, F_MID, F_SPREAD = range(7)
F_NORMAL_BASE = 16  # 16 + k: Irwin-Hall terms for bid (k < 16) and ask (16 <= k < 32)


def splitmix64(x: np.ndarray) -> np.ndarray:
    """SplitMix64 finaliser of x + golden gamma (uint64, wrapping)."""
    with np.errstate(over="ignore"):
        z = x + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def draws(seed: int, field: int, step: int, markets: np.ndarray) -> np.ndarray:
    """uint64 hash per market for (seed, field, step)."""
    if not (0 <= seed < 256 and 0 <= field < 256 and 0 <= step < (1 << 24)):
        raise ValueError("seed/field/step out of the counter layout")
    base = np.uint64((seed << 56) | (field << 48) | (step << 24))
    return splitmix64(base | markets.astype(np.uint64))


def uniform(seed, field, step, markets, lo: int, hi: int) -> np.ndarray:
    """Integers in [lo, hi] (inclusive)."""
    h = draws(seed, field, step, markets)
    return (np.int64(lo) + (h % np.uint64(hi - lo + 1)).astype(np.int64)).astype(np.int32)


# geometric(p) on {1, 2, ...}: P(K > k) = (1-p)^k. K = 1 + #{k >= 1 : u >= 1 - (1-p)^k},
# u = h / 2^64, with thresholds computed by repeated multiplication in double.
def _geometric_thresholds(p: float, cap: int) -> np.ndarray:
    q, th = 1.0, []
    for _ in range(1, cap):
        q *= (1.0 - p)
        th.append(int((1.0 - q) * 2.0 ** 53) << 11)  # 53-bit fraction, scaled to 2^64
    return np.array(th, dtype=np.uint64)


_GEOM_03_50 = _geometric_thresholds(0.3, 50)


def geometric(seed, field, step, markets, thresholds=_GEOM_03_50) -> np.ndarray:
    h = draws(seed, field, step, markets)
    return (1 + np.searchsorted(thresholds, h, side="right")).astype(np.int32)


def normal_irwin_hall(seed, field0, step, markets, mean: float, sd: float) -> np.ndarray:
    """Approximately N(mean, sd): sum of 16 uniform 16-bit integers, standardised, rounded."""
    acc = np.zeros(markets.shape, dtype=np.int64)
    for k in range(16):
        acc += (draws(seed, field0 + k, step, markets) >> np.uint64(48)).astype(np.int64)
    mu = 16 * 32767.5
    sigma = (16 * (65536.0 ** 2 - 1) / 12.0) ** 0.5
    z = (acc.astype(np.float64) - mu) / sigma
    return np.floor(mean + sd * z + 0.5).astype(np.int64)


@dataclass(frozen=True)
class Config:
    index: int
    name: str
    M: int
    L: int
    O: int
    F: int
    C: int
    steps: int
    bbo_every_step: bool
    extended: bool = False

    def shape_kwargs(self) -> dict:
        return dict(num_markets=self.M, max_price_levels=self.L, max_active_orders_per_market=self.O,
                    max_active_fills_per_market=self.F, num_customers=self.C)


CONFIGS = {
    1: Config(1, "cpu_reference_run", 64, 128, 1024, 1024, 16, 1000, False),
    2: Config(2, "readme_shape", 10_000, 128, 1024, 1024, 16, 10_000, True),
    3: Config(3, "stress_100k", 100_000, 128, 1024, 1024, 16, 1000, True),
    4: Config(4, "deep_book", 20_000, 512, 4096, 4096, 64, 2000, True, extended=True),
}


class QuoteStream:
    """Generates the per-step inputs of one config for a subset of markets.

    ``steps(t0, t1)`` returns five int32 arrays of shape [t1 - t0, len(markets)]
    (bid_px, bid_sz, ask_px, ask_sz, customer_ids). Config 3's random-walk mid is
    carried across calls, so steps must be requested in order from 0.
    """

    def __init__(self, cfg: Config, markets: np.ndarray | None = None, seed: int = 0):
        self.cfg = cfg
        self.seed = seed
        self.markets = np.arange(cfg.M, dtype=np.int64) if markets is None else np.asarray(markets, np.int64)
        self._mid = np.full(self.markets.shape, 64, dtype=np.int64)
        self._next_step = 0

    def step(self, t: int):
        c, s, mk = self.cfg, self.seed, self.markets
        if c.index == 1:
            bid = uniform(s, F_BID_PX, t, mk, 0, 63)
            ask = np.minimum(bid.astype(np.int64) + uniform(s, F_ASK_PX, t, mk, 1, 63), 127).astype(np.int32)
            bsz = uniform(s, F_BID_SZ, t, mk, 1, 10)
            asz = uniform(s, F_ASK_SZ, t, mk, 1, 10)
            cust = np.full(mk.shape, t % 16, dtype=np.int32)
        elif c.index == 2:
            bid = uniform(s, F_BID_PX, t, mk, 0, 127)
            ask = uniform(s, F_ASK_PX, t, mk, 0, 127)
            bsz = uniform(s, F_BID_SZ, t, mk, 1, 10)
            asz = uniform(s, F_ASK_SZ, t, mk, 1, 10)
            cust = uniform(s, F_CUST, t, mk, 0, 15)
        elif c.index == 3:
            if t != self._next_step:
                raise ValueError("config 3 steps must be generated in order")
            self._mid = np.clip(self._mid + uniform(s, F_MID, t, mk, -3, 3), 0, 127)
            spread = uniform(s, F_SPREAD, t, mk, 0, 8).astype(np.int64)
            b = np.clip(self._mid - spread // 2, 0, 127)
            bid = b.astype(np.int32)
            ask = np.clip(b + spread, 0, 127).astype(np.int32)
            bsz = geometric(s, F_BID_SZ, t, mk)
            asz = geometric(s, F_ASK_SZ, t, mk)
            cust = uniform(s, F_CUST, t, mk, 0, 15)
        elif c.index == 4:
            bid = np.clip(normal_irwin_hall(s, F_NORMAL_BASE, t, mk, 256.0, 40.0), 0, 511).astype(np.int32)
            ask = np.clip(normal_irwin_hall(s, F_NORMAL_BASE + 16, t, mk, 256.0, 40.0), 0, 511).astype(np.int32)
            bsz = uniform(s, F_BID_SZ, t, mk, 1, 100)
            asz = uniform(s, F_ASK_SZ, t, mk, 1, 100)
            cust = uniform(s, F_CUST, t, mk, 0, 63)
        else:
            raise ValueError(f"no generator for config {c.index}")
        self._next_step = t + 1
        return bid, bsz, ask, asz, cust

    def steps(self, t0: int, t1: int):
        out = [np.empty((t1 - t0, len(self.markets)), dtype=np.int32) for _ in range(5)]
        for i, t in enumerate(range(t0, t1)):
            for arr, v in zip(out, self.step(t)):
                arr[i] = v
        return tuple(out)


# ---- config 5: the high-low trading game step ----
F_GAME_CAND, F_GAME_HL, F_GAME_PERM, F_GAME_CUST, F_GAME_MOVE = 64, 66, 67, 80, 96  # 80+j, 96+c


@dataclass(frozen=True)
class GameConfig:
    """Config 5: 10,000 envs of the high-low game, 5 players, 200 steps per player
    (1,000 trading moves), on a market of 128 levels, 1,024 orders and 16 customers
    (the shape BASELINE names; the game's own sizing would be smaller). Prices are
    U[1, max_contract_value], sizes U[0, max_contracts_per_trade]: a random policy
    over the legal actions."""
    index: int = 5
    name: str = "game_step_10k"
    envs: int = 10_000
    players: int = 5
    steps_per_player: int = 200
    max_contracts_per_trade: int = 5
    customer_max_size: int = 5
    max_contract_value: int = 127
    market_shape: tuple = (128, 1024, 10, 16)

    def game_params(self, envs: int | None = None, check_moves: bool = True) -> dict:
        L, O, F, C = self.market_shape
        return dict(num_markets=envs or self.envs, players=self.players,
                    steps_per_player=self.steps_per_player,
                    max_contracts_per_trade=self.max_contracts_per_trade,
                    customer_max_size=self.customer_max_size,
                    max_contract_value=self.max_contract_value, market_price_levels=L,
                    market_orders=O, market_fills=F, market_customers=C, check_moves=check_moves)


GAME_CONFIG = GameConfig()


class GameStream:
    """Chance moves (as the reference's env.py:42-56 draws them) and trading moves
    [N, 4] = (bid_px, ask_px, bid_sz, ask_sz) for envs ``envs``, from the counter
    generator."""

    def __init__(self, cfg: GameConfig = GAME_CONFIG, envs: np.ndarray | None = None, seed: int = 0):
        self.cfg, self.seed = cfg, seed
        self.envs = np.arange(cfg.envs, dtype=np.int64) if envs is None else np.asarray(envs, np.int64)

    def chance(self):
        c, s, e = self.cfg, self.seed, self.envs
        V, P, cM = c.max_contract_value, c.players, c.customer_max_size
        cand = np.stack([uniform(s, F_GAME_CAND + j, 0, e, 1, V) for j in range(2)], 1)
        hl = uniform(s, F_GAME_HL, 0, e, 0, 1)
        keys = np.stack([draws(s, F_GAME_PERM, j, e) for j in range(P)], 1)
        perm = np.argsort(keys, axis=1, kind="stable").astype(np.int32)
        cs = np.stack([uniform(s, F_GAME_CUST + j, 0, e, -cM, cM - 1) for j in range(P - 3)], 1)
        cs[cs >= 0] += 1
        return [cand.astype(np.int32), hl.astype(np.int32), perm, cs.astype(np.int32)]

    def move(self, k: int):
        c, s, e = self.cfg, self.seed, self.envs
        V, S = c.max_contract_value, c.max_contracts_per_trade
        return np.stack([uniform(s, F_GAME_MOVE + 0, k, e, 1, V), uniform(s, F_GAME_MOVE + 1, k, e, 1, V),
                         uniform(s, F_GAME_MOVE + 2, k, e, 0, S), uniform(s, F_GAME_MOVE + 3, k, e, 0, S)],
                        1).astype(np.int32)


# ---- the same streams generated by torch, on the device (or the CPU) ----
#
# Bit for bit the numpy generator above: SplitMix64 in int64 arithmetic (which
# wraps like uint64 for +, * and ^), logical shifts by masking, unsigned modulo
# from the halved value, unsigned order for the geometric thresholds by flipping
# the sign bit, and float64 +,-,*,/ (IEEE, correctly rounded) for the normal
# draws. Used where generating on the host would dominate (large market counts);
# tests/test_workloads_torch.py checks it against the numpy streams.

def _i64(u: int) -> int:
    """The int64 with the bits of uint64 u."""
    u &= (1 << 64) - 1
    return u - (1 << 64) if u >= (1 << 63) else u


_T_GOLDEN, _T_C1, _T_C2 = _i64(0x9E3779B97F4A7C15), _i64(0xBF58476D1CE4E5B9), _i64(0x94D049BB133111EB)
_T_SIGN = _i64(1 << 63)


def _lsr(z, k: int):
    return (z >> k) & ((1 << (64 - k)) - 1)


def t_splitmix64(x):
    z = x + _T_GOLDEN
    z = (z ^ _lsr(z, 30)) * _T_C1
    z = (z ^ _lsr(z, 27)) * _T_C2
    return z ^ _lsr(z, 31)


def t_draws(seed: int, field: int, step: int, markets):
    """int64 tensor with the bits of draws(seed, field, step, markets)."""
    if not (0 <= seed < 256 and 0 <= field < 256 and 0 <= step < (1 << 24)):
        raise ValueError("seed/field/step out of the counter layout")
    return t_splitmix64(markets | _i64((seed << 56) | (field << 48) | (step << 24)))


def t_umod(h, n: int):
    """Unsigned h mod n for int64 h holding uint64 bits (n < 2^62)."""
    return ((_lsr(h, 1) % n) * 2 + (h & 1)) % n


def t_uniform(seed, field, step, markets, lo: int, hi: int):
    import torch
    return (lo + t_umod(t_draws(seed, field, step, markets), hi - lo + 1)).to(torch.int32)


def t_geometric(seed, field, step, markets, thresholds=_GEOM_03_50):
    import torch
    th = torch.tensor([_i64(int(v)) ^ _T_SIGN for v in thresholds], dtype=torch.int64,
                      device=markets.device)
    h = t_draws(seed, field, step, markets) ^ _T_SIGN
    return (1 + torch.searchsorted(th, h, right=True)).to(torch.int32)


def t_normal_irwin_hall(seed, field0, step, markets, mean: float, sd: float):
    import torch
    acc = torch.zeros_like(markets)
    for k in range(16):
        acc += _lsr(t_draws(seed, field0 + k, step, markets), 48)
    mu = 16 * 32767.5
    sigma = (16 * (65536.0 ** 2 - 1) / 12.0) ** 0.5
    z = (acc.to(torch.float64) - mu) / sigma
    return torch.floor(mean + sd * z + 0.5).to(torch.int64)


class DeviceQuoteStream:
    """QuoteStream's per-step inputs as int32 tensors on `device` (config 3's
    random-walk mid lives there too, so steps come in order from 0)."""

    def __init__(self, cfg: Config, markets=None, seed: int = 0, device="cuda"):
        import torch
        self.cfg, self.seed = cfg, seed
        if markets is None:
            self.markets = torch.arange(cfg.M, dtype=torch.int64, device=device)
        else:
            self.markets = torch.as_tensor(np.asarray(markets, np.int64)).to(device)
        self._mid = torch.full(self.markets.shape, 64, dtype=torch.int64, device=self.markets.device)
        self._next_step = 0

    def step(self, t: int):
        import torch
        c, s, mk = self.cfg, self.seed, self.markets
        if c.index == 1:
            bid = t_uniform(s, F_BID_PX, t, mk, 0, 63)
            ask = torch.clamp(bid.to(torch.int64) + t_uniform(s, F_ASK_PX, t, mk, 1, 63), max=127).to(torch.int32)
            bsz = t_uniform(s, F_BID_SZ, t, mk, 1, 10)
            asz = t_uniform(s, F_ASK_SZ, t, mk, 1, 10)
            cust = torch.full(mk.shape, t % 16, dtype=torch.int32, device=mk.device)
        elif c.index == 2:
            bid = t_uniform(s, F_BID_PX, t, mk, 0, 127)
            ask = t_uniform(s, F_ASK_PX, t, mk, 0, 127)
            bsz = t_uniform(s, F_BID_SZ, t, mk, 1, 10)
            asz = t_uniform(s, F_ASK_SZ, t, mk, 1, 10)
            cust = t_uniform(s, F_CUST, t, mk, 0, 15)
        elif c.index == 3:
            if t != self._next_step:
                raise ValueError("config 3 steps must be generated in order")
            self._mid = torch.clamp(self._mid + t_uniform(s, F_MID, t, mk, -3, 3), 0, 127)
            spread = t_uniform(s, F_SPREAD, t, mk, 0, 8).to(torch.int64)
            b = torch.clamp(self._mid - spread // 2, 0, 127)
            bid = b.to(torch.int32)
            ask = torch.clamp(b + spread, 0, 127).to(torch.int32)
            bsz = t_geometric(s, F_BID_SZ, t, mk)
            asz = t_geometric(s, F_ASK_SZ, t, mk)
            cust = t_uniform(s, F_CUST, t, mk, 0, 15)
        elif c.index == 4:
            bid = torch.clamp(t_normal_irwin_hall(s, F_NORMAL_BASE, t, mk, 256.0, 40.0), 0, 511).to(torch.int32)
            ask = torch.clamp(t_normal_irwin_hall(s, F_NORMAL_BASE + 16, t, mk, 256.0, 40.0), 0, 511).to(torch.int32)
            bsz = t_uniform(s, F_BID_SZ, t, mk, 1, 100)
            asz = t_uniform(s, F_ASK_SZ, t, mk, 1, 100)
            cust = t_uniform(s, F_CUST, t, mk, 0, 63)
        else:
            raise ValueError(f"no generator for config {c.index}")
        self._next_step = t + 1
        return bid, bsz, ask, asz, cust

    def steps(self, t0: int, t1: int):
        """Five int32 [t1 - t0, M] tensors, row k = step t0 + k."""
        import torch
        rows = [self.step(t) for t in range(t0, t1)]
        return tuple(torch.stack([r[i] for r in rows]) for i in range(5))


def t_game_move(cfg: GameConfig, k: int, envs, seed: int = 0):
    """GameStream.move(k) as an int32 [N, 4] tensor on envs' device."""
    import torch
    V, S = cfg.max_contract_value, cfg.max_contracts_per_trade
    return torch.stack([t_uniform(seed, F_GAME_MOVE + 0, k, envs, 1, V),
                        t_uniform(seed, F_GAME_MOVE + 1, k, envs, 1, V),
                        t_uniform(seed, F_GAME_MOVE + 2, k, envs, 0, S),
                        t_uniform(seed, F_GAME_MOVE + 3, k, envs, 0, S)], 1).contiguous()
