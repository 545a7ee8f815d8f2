"""astra_cuda -- MI355X-native drop-in for nlyu1/astra-cuda's order-matching module.

``import astra_cuda; astra_cuda.order_matching.VecMarket`` works as with the
reference pybind module (src/pybind/bindings.cc:16-24). The engine is the HIP
library ``libastra_market.so`` next to this file (built by ``astra_cuda.build``).
"""
__version__ = "0.0.2"  # bindings.cc:10

from . import order_matching  # noqa: E402,F401
