"""Game registry: ``register_games``, ``load_game``, ``registered_names``
(src/pybind/core/core_bindings.cc:24-32, src/core/core.cc GameRegistrar).

Only the high-low trading game is on this engine's path.
"""
from __future__ import annotations

_REGISTRY = {}


def register_games() -> None:
    """RegisterGames: make the built-in games loadable by name."""
    from .high_low_trading import HighLowTradingGame
    _REGISTRY[HighLowTradingGame.short_name] = HighLowTradingGame


def registered_names() -> list:
    return sorted(_REGISTRY)


def load_game(name: str, params: dict | None = None):
    """GameRegistrar::CreateByName."""
    if name not in _REGISTRY:
        from .order_matching import _fatal
        _fatal(f"Unknown game '{name}'. Available games are: {', '.join(registered_names())}")
    return _REGISTRY[name](params)
