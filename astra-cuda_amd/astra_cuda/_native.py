"""ctypes binding of ``libastra_market.so`` (C ABI in include/astra_market.h).

torch is imported first so that the library's libamdhip64.so.7 dependency
resolves to the HIP runtime torch already loaded: one runtime, shared streams.
There is no fallback: if the library is missing, importing this module fails.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

from .build import LIB_PATH

_c_i32 = ctypes.c_int32
_c_int = ctypes.c_int
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t

# name -> (restype, argtypes)
PROTOTYPES = {
    "astra_last_error": (ctypes.c_char_p, []),
    "astra_market_workspace_size": (_c_int, [_c_i32] * 6 + [ctypes.POINTER(_sz)]),
    "astra_market_create": (_c_int, [_c_i32] * 5 + [_c_int, _c_i32, _c_i32, _vp, _sz, _vp,
                                                    ctypes.POINTER(_vp)]),
    "astra_market_destroy": (_c_int, [_vp]),
    "astra_market_clone": (_c_int, [_vp, _vp, _sz, _vp, ctypes.POINTER(_vp)]),
    "astra_market_add_two_sided_quotes": (_c_int, [_vp] + [_vp] * 5 + [_vp] * 9 + [_vp]),
    "astra_market_get_bbos": (_c_int, [_vp] + [_vp] * 4 + [_vp]),
    "astra_update_last_prices": (_c_int, [_vp, _vp, _vp, _c_i32, _c_i32, _vp]),
    "astra_market_add_two_sided_quotes_rows": (_c_int, [_vp] + [_vp] * 5 + [_vp, _vp, _vp]),
    "astra_update_last_prices_rows": (_c_int, [_vp, _vp, _vp, _c_i32, _c_i32, _vp]),
    "astra_market_add_two_sided_quotes_steps": (_c_int, [_vp, _c_i32] + [_vp] * 5 + [_vp] * 12 + [_vp]),
    "astra_fill_i32": (_c_int, [_vp, ctypes.c_int64, _c_i32, _vp]),
    "astra_market_reset": (_c_int, [_vp, _vp]),
    "astra_market_clear_quotes": (_c_int, [_vp, _vp, _vp]),
    "astra_market_portfolios": (_c_int, [_vp, ctypes.POINTER(_vp)]),
    "astra_market_to_string": (_c_int, [_vp, _c_i32, ctypes.c_char_p, _sz, ctypes.POINTER(_sz),
                                        _vp]),
    "astra_market_set_stats": (_c_int, [_vp, _vp]),
    "astra_market_get_tid": (_c_int, [_vp, ctypes.POINTER(_c_i32), _vp]),
    "astra_market_set_tid": (_c_int, [_vp, _c_i32, _vp]),
    "astra_market_shape": (_c_int, [_vp] + [ctypes.POINTER(_c_i32)] * 5),
    "astra_high_low_trade": (_c_int, [_vp, _vp, _vp]),
    "astra_high_low_trade_scratch": (_c_int, [_vp, _vp, _vp]),
    "astra_high_low_observation": (_c_int, [_vp, _vp]),
    "astra_high_low_rewards": (_c_int, [_vp, ctypes.c_int64, _c_i32, _c_i32, _vp, _vp]),
}


class HLTrade(ctypes.Structure):
    """astra_hl_trade (include/astra_high_low.h)."""
    _fields_ = [(n, _vp) for n in (
        "move", "player_last_positions", "target_positions", "contract_values",
        "player_contract_over_time", "market_contract_over_time", "immediate_rewards",
        "rewards_since_last_action", "fill_prices", "fill_sizes", "fill_customer_ids",
        "fill_quoter_ids", "fill_is_sell_quote", "fill_quote_sizes", "fill_tid", "fill_quote_tid",
        "fill_counts", "best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes",
        "last_prices", "fill_rows", "errors", "errors_host")] + [(n, _c_i32) for n in (
        "players", "steps_per_player", "max_contracts_per_trade", "max_contract_value", "player",
        "trade_move_number", "check")]


class HLObservation(ctypes.Structure):
    """astra_hl_observation (include/astra_high_low.h)."""
    _fields_ = [(n, _vp) for n in (
        "values", "player_permutation", "contract_values", "contract_high_settle",
        "target_positions", "player_contract_over_time", "best_bid_prices", "best_ask_prices",
        "best_bid_sizes", "best_ask_sizes", "last_prices")] + [(n, _c_i32) for n in (
        "num_envs", "players", "steps_per_player", "player", "current_round")] + [
        (n, ctypes.c_float) for n in ("player_sin", "player_cos", "round_fraction")]

_lib = None


def lib() -> ctypes.CDLL:
    """Load the engine library (once). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP engine first "
                "(python astra-cuda_amd/astra_cuda/build.py or __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    msg = lib().astra_last_error()
    return msg.decode(errors="replace") if msg else ""
