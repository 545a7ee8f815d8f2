"""The C-ABI library loads, exports what include/*.h declares, and validates
shapes like the reference constructor (CPU only: no device calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", h) for h in sorted(os.listdir(os.path.join(ROOT, "include")))
           if h.endswith(".h")]


def _ensure_built():
    from astra_cuda.build import LIB_PATH, build
    if not os.path.exists(LIB_PATH):
        build()
    return LIB_PATH


def _declared():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(astra_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = _declared()
    for must in ("astra_market_create", "astra_market_add_two_sided_quotes", "astra_market_get_bbos",
                 "astra_update_last_prices", "astra_market_reset", "astra_market_clear_quotes",
                 "astra_market_clone", "astra_market_to_string", "astra_market_portfolios",
                 "astra_market_shape", "astra_high_low_trade",
                 "astra_high_low_observation"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_ensure_built())
    missing = [n for n in _declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_python_prototypes_cover_header():
    from astra_cuda._native import PROTOTYPES
    assert sorted(PROTOTYPES) == _declared()


def _ws(*shape, flags=0):
    from astra_cuda import _native
    n = ctypes.c_size_t(0)
    rc = _native.lib().astra_market_workspace_size(*shape, flags, ctypes.byref(n))
    return rc, n.value, _native.last_error()


def test_workspace_size_and_reference_caps():
    rc, n, _ = _ws(10, 128, 1024, 512, 16)
    assert rc == 0 and n > 0
    # market.cu:338-342: L <= 128, O <= 1024, F <= 1024, C <= 1024
    for shape, text in (((10, 129, 1024, 512, 16), "max_price_levels <= ASTRA_PRICE_LEVELS"),
                        ((10, 128, 1025, 512, 16), "<= ASTRA_MAX_ACTIVE_ORDERS_PER_MARKET"),
                        ((10, 128, 1024, 1025, 16), "<= ASTRA_MAX_ACTIVE_FILLS_PER_MARKET"),
                        ((10, 128, 1024, 512, 1025), "<= ASTRA_MAX_CUSTOMERS"),
                        ((2048 * 2048 + 1, 128, 16, 16, 16), "<= ASTRA_MAX_MARKETS")):
        rc, _, msg = _ws(*shape)
        assert rc == 1, shape
        assert text.split()[-1] in msg and "=" in msg, msg


def test_extended_shapes_flag():
    rc, _, _ = _ws(20000, 512, 4096, 4096, 64)
    assert rc == 1
    rc, n, _ = _ws(20000, 512, 4096, 4096, 64, flags=1)
    assert rc == 0
    # records dominate: 16 bytes per order slot
    assert n >= 20000 * 4096 * 16


def test_constants_match_reference():
    from astra_cuda import order_matching as aom  # market.h:56-61, test_vec_market.py:36-39
    assert aom.MAX_MARKETS == 2048 * 2048
    assert aom.PRICE_LEVELS == 128
    assert aom.MAX_ACTIVE_ORDERS_PER_MARKET == 1024
    assert aom.MAX_ACTIVE_FILLS_PER_MARKET == 1024
    assert aom.NULL_INDEX == -1
    assert aom.MAX_CUSTOMERS == 1024


def test_no_device_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from astra_cuda import order_matching as aom
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        aom.VecMarket(4, 128, 16, 16)


@pytest.mark.parametrize("shape", [(10, 128, 1024, 512, 16), (7, 70, 5, 3, 4), (3, 1024, 32768, 8, 65536),
                                   (0, 8, 1, 1, 1)])
def test_test_side_workspace_layout_matches_the_engine(shape):
    """tests/ws_layout.py (used to compare workspaces) describes the engine's layout."""
    from ws_layout import layout
    M, L, O, F, C = shape
    rc, n, _ = _ws(*shape, flags=1)
    assert rc == 0 and layout(M, L, O, C)["total"][1] == n


def test_compiled_binding_has_the_reference_module_surface():
    """astra_cuda._C.order_matching exposes what market_bindings.cc:14-73 binds: the
    three classes, their tensor fields, the methods with the reference's keyword
    names, and the six constants (import only: no device calls on the CPU)."""
    from astra_cuda.build import binding_path, build_binding
    if not os.path.exists(binding_path()):
        build_binding()
    from astra_cuda._C import order_matching as com
    for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes"):
        assert isinstance(getattr(com.BBOBatch, f), property)
    for f in ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
              "fill_quote_sizes", "fill_tid", "fill_quote_tid", "fill_counts"):
        assert isinstance(getattr(com.FillBatch, f), property)
    for m in ("new_fill_batch", "new_bbo_batch", "add_two_sided_quotes", "get_bbos", "to_string",
              "get_customer_portfolios"):
        assert callable(getattr(com.VecMarket, m))
    doc = com.VecMarket.__init__.__doc__
    for kw in ("num_markets", "max_price_levels", "max_active_orders_per_market",
               "max_active_fills_per_market"):
        assert kw + ":" in doc, kw
    for kw, default in (("num_customers", 16), ("device_id", 0), ("threads_per_block", 64)):
        assert re.search(kw + r": [\w.]+ = " + str(default), doc), kw
    assert "bid_px" in com.VecMarket.add_two_sided_quotes.__doc__ and "fills" in \
        com.VecMarket.add_two_sided_quotes.__doc__
    assert (com.MAX_MARKETS, com.PRICE_LEVELS, com.MAX_ACTIVE_ORDERS_PER_MARKET, com.MAX_ACTIVE_FILLS_PER_MARKET,
            com.NULL_INDEX, com.MAX_CUSTOMERS) == (2048 * 2048, 128, 1024, 1024, -1, 1024)
