"""astra_cuda -- MI355X-native drop-in for nlyu1/astra-cuda's order-matching module.

``import astra_cuda; astra_cuda.order_matching.VecMarket`` works as with the
reference pybind module (src/pybind/bindings.cc:16-24). The engine is the HIP
library ``libastra_market.so`` next to this file (built by ``astra_cuda.build``).
``register_games()`` / ``load_game("high_low_trading", params)`` give the
reference's high-low trading game on the same engine (core_bindings.cc:24-32).
"""
__version__ = "0.0.2"  # bindings.cc:10

from . import order_matching  # noqa: E402,F401
from .games import load_game, register_games, registered_names  # noqa: E402,F401
