"""numpy/ctypes front end of the C oracle (``market_oracle.c``).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker or the timed CPU baseline; the product never routes through it.

``OracleMarket`` mirrors the reference ``VecMarket`` surface
(nlyu1/astra-cuda src/order_matching/market.h:121-350) on host numpy arrays:
``new_fill_batch``/``new_bbo_batch`` (market.cu:420-456),
``add_two_sided_quotes`` (market.cu:458-571), ``get_bbos`` (market.cu:573-597),
``update_last_prices`` (market.cu:798-825), ``reset``/``clear_quotes``
(market.cu:693-756), ``to_string`` (market.cu:599-691) and ``clone``
(market.cu:385-411). The reference's internal state arrays are exposed as
numpy views so tests can check invariants on them.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# ASTRA_ORACLE_LIB: another build of the same source (the Makefile's `sanitize`
# target) for a sanitizer run of the test suite
_LIB_PATH = os.environ.get("ASTRA_ORACLE_LIB") or os.path.join(_HERE, "libmarket_oracle.so")

_i32p = ctypes.POINTER(ctypes.c_int32)
_u8p = ctypes.POINTER(ctypes.c_uint8)


class _OmMarket(ctypes.Structure):
    _fields_ = [
        ("num_markets", ctypes.c_int32),
        ("max_price_levels", ctypes.c_int32),
        ("max_orders", ctypes.c_int32),
        ("max_fills", ctypes.c_int32),
        ("num_customers", ctypes.c_int32),
        ("global_tid", ctypes.c_int32),
        ("bid_heads", _i32p),
        ("ask_heads", _i32p),
        ("bid_tails", _i32p),
        ("ask_tails", _i32p),
        ("order_prices", _i32p),
        ("order_sizes", _i32p),
        ("order_customer_ids", _i32p),
        ("order_tid", _i32p),
        ("order_is_bid", _u8p),
        ("order_next", _i32p),
        ("order_next_slots", _i32p),
        ("customer_portfolios", _i32p),
    ]


class OmCounters(ctypes.Structure):
    _fields_ = [
        ("inserts", ctypes.c_int64),
        ("fills", ctypes.c_int64),
        ("levels_emptied", ctypes.c_int64),
        ("overflows", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        return {k: int(getattr(self, k)) for k, _ in self._fields_}


_lib = None


def build(force: bool = False) -> str:
    """Compile the oracle with its Makefile (gcc). Returns the library path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.POINTER(_OmMarket)
        L.om_create.restype = P
        L.om_create.argtypes = [ctypes.c_int32] * 5
        L.om_clone.restype = P
        L.om_clone.argtypes = [P]
        L.om_destroy.restype = None
        L.om_destroy.argtypes = [P]
        L.om_add_two_sided_quotes.restype = None
        L.om_add_two_sided_quotes.argtypes = (
            [P] + [_i32p] * 5 + [_i32p] * 4 + [_u8p] + [_i32p] * 4
            + [ctypes.c_int, ctypes.POINTER(OmCounters)]
        )
        L.om_get_bbos.restype = None
        L.om_get_bbos.argtypes = [P] + [_i32p] * 4 + [ctypes.c_int]
        L.om_update_last_prices.restype = None
        L.om_update_last_prices.argtypes = [_i32p, _i32p, _i32p, ctypes.c_int32, ctypes.c_int32]
        L.om_reset.restype = None
        L.om_reset.argtypes = [P]
        L.om_clear_quotes.restype = None
        L.om_clear_quotes.argtypes = [P, _u8p]
        L.om_to_string.restype = ctypes.c_size_t
        L.om_to_string.argtypes = [P, ctypes.c_int32, ctypes.c_char_p, ctypes.c_size_t]
        _lib = L
    return _lib


def _p32(a: np.ndarray):
    assert a.dtype == np.int32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_i32p)


def _p8(a: np.ndarray):
    assert a.dtype in (np.uint8, np.bool_) and a.flags.c_contiguous
    return a.ctypes.data_as(_u8p)


@dataclass
class OracleFills:
    """FillBatch (market.h:64-92) on host memory, zero-initialised (market.cu:428-436)."""

    fill_prices: np.ndarray
    fill_sizes: np.ndarray
    fill_customer_ids: np.ndarray
    fill_quoter_ids: np.ndarray
    fill_is_sell_quote: np.ndarray  # bool
    fill_quote_sizes: np.ndarray
    fill_tid: np.ndarray
    fill_quote_tid: np.ndarray
    fill_counts: np.ndarray

    FIELDS = (
        "fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids",
        "fill_is_sell_quote", "fill_quote_sizes", "fill_tid", "fill_quote_tid", "fill_counts",
    )


@dataclass
class OracleBBO:
    """BBOBatch (market.h:95-119), all five fields zero-initialised (market.cu:448-453)."""

    best_bid_prices: np.ndarray
    best_bid_sizes: np.ndarray
    best_ask_prices: np.ndarray
    best_ask_sizes: np.ndarray
    last_prices: np.ndarray

    FIELDS = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes")


class OracleMarket:
    """Host-side restatement of VecMarket, backed by ``market_oracle.c``."""

    def __init__(self, num_markets, max_price_levels, max_active_orders_per_market,
                 max_active_fills_per_market, num_customers=16, _handle=None):
        self.M = int(num_markets)
        self.L = int(max_price_levels)
        self.O = int(max_active_orders_per_market)
        self.F = int(max_active_fills_per_market)
        self.C = int(num_customers)
        self._lib = lib()
        self._h = _handle if _handle is not None else self._lib.om_create(
            self.M, self.L, self.O, self.F, self.C)
        if not self._h:
            raise MemoryError("om_create failed")
        s = self._h.contents
        M, L, O, C = self.M, self.L, self.O, self.C

        def view(ptr, shape, dt=np.int32):
            n = int(np.prod(shape))
            if n == 0:
                return np.zeros(shape, dtype=dt)
            arr = np.ctypeslib.as_array(ptr, shape=(n,))
            return arr.view(dt).reshape(shape)

        self.bid_heads = view(s.bid_heads, (M, L))
        self.ask_heads = view(s.ask_heads, (M, L))
        self.bid_tails = view(s.bid_tails, (M, L))
        self.ask_tails = view(s.ask_tails, (M, L))
        self.order_prices = view(s.order_prices, (M, O))
        self.order_sizes = view(s.order_sizes, (M, O))
        self.order_customer_ids = view(s.order_customer_ids, (M, O))
        self.order_tid = view(s.order_tid, (M, O))
        self.order_next = view(s.order_next, (M, O))
        self.order_next_slots = view(s.order_next_slots, (M,))
        self.customer_portfolios = view(s.customer_portfolios, (M, C, 2))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            self._lib.om_destroy(h)
            self._h = None

    @property
    def global_tid(self) -> int:
        return int(self._h.contents.global_tid)

    def clone(self) -> "OracleMarket":
        return OracleMarket(self.M, self.L, self.O, self.F, self.C, _handle=self._lib.om_clone(self._h))

    def new_fill_batch(self) -> OracleFills:
        z = lambda: np.zeros((self.M, self.F), dtype=np.int32)
        return OracleFills(z(), z(), z(), z(), np.zeros((self.M, self.F), dtype=np.bool_), z(), z(),
                           z(), np.zeros((self.M,), dtype=np.int32))

    def new_bbo_batch(self) -> OracleBBO:
        z = lambda: np.zeros((self.M,), dtype=np.int32)
        return OracleBBO(z(), z(), z(), z(), z())

    def add_two_sided_quotes(self, bid_px, bid_sz, ask_px, ask_sz, customer_ids, fills: OracleFills,
                             nthreads: int = 1) -> dict:
        ins = [np.ascontiguousarray(x, dtype=np.int32) for x in (bid_px, bid_sz, ask_px, ask_sz, customer_ids)]
        for x in ins:
            if x.shape != (self.M,):
                raise ValueError(f"input shape {x.shape} != ({self.M},)")
        c = OmCounters()
        self._lib.om_add_two_sided_quotes(
            self._h, *[_p32(x) for x in ins],
            _p32(fills.fill_prices), _p32(fills.fill_sizes), _p32(fills.fill_customer_ids),
            _p32(fills.fill_quoter_ids), _p8(fills.fill_is_sell_quote), _p32(fills.fill_quote_sizes),
            _p32(fills.fill_tid), _p32(fills.fill_quote_tid), _p32(fills.fill_counts),
            int(nthreads), ctypes.byref(c))
        return c.as_dict()

    def get_bbos(self, bbo: OracleBBO, nthreads: int = 1) -> None:
        self._lib.om_get_bbos(self._h, _p32(bbo.best_bid_prices), _p32(bbo.best_bid_sizes),
                              _p32(bbo.best_ask_prices), _p32(bbo.best_ask_sizes), int(nthreads))

    def update_last_prices(self, bbo: OracleBBO, fills: OracleFills) -> None:
        self._lib.om_update_last_prices(_p32(bbo.last_prices), _p32(fills.fill_counts),
                                        _p32(fills.fill_prices), self.M, self.F)

    def reset(self) -> None:
        self._lib.om_reset(self._h)

    def clear_quotes(self, reset_indices) -> None:
        r = np.ascontiguousarray(reset_indices, dtype=np.bool_)
        if r.shape != (self.M,):
            raise ValueError("reset_indices must have shape [num_markets]")
        self._lib.om_clear_quotes(self._h, r.ctypes.data_as(_u8p))

    def to_string(self, market_id: int) -> str:
        n = self._lib.om_to_string(self._h, int(market_id), None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        self._lib.om_to_string(self._h, int(market_id), buf, n + 1)
        return buf.value.decode()

    def get_customer_portfolios(self) -> np.ndarray:
        return self.customer_portfolios
