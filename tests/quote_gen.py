"""Quote generators and shapes shared by the emulated (CPU) and GPU parity tests."""
from __future__ import annotations

import numpy as np


def drifting_window_gen(M, L, C, seed, hot=24):
    """Quotes in a window of `hot` levels that random-walks over all L levels (so
    every mask word is used), sizes 0-7 (0 is rejected), customers mostly 0-7 with
    some at C-1 (the last valid id) and at C (out of range: no portfolio change)."""
    rng = np.random.default_rng(seed)
    state = {"base": (L - hot) // 2}

    def gen(t):
        state["base"] = int(np.clip(state["base"] + rng.integers(-2, 3), 0, L - hot))
        base = state["base"]
        bid = (base + rng.integers(0, hot, M)).astype(np.int32)
        ask = (base + rng.integers(0, hot, M)).astype(np.int32)
        cust = rng.integers(0, 8, M).astype(np.int32)
        cust[rng.random(M) < 0.1] = C - 1
        cust[rng.random(M) < 0.05] = C
        return bid, rng.integers(0, 8, M).astype(np.int32), ask, rng.integers(0, 8, M).astype(np.int32), cust

    return gen


# The largest shape ASTRA_FLAG_EXTENDED_SHAPES accepts: L=1024 (16 mask words),
# O=32768 (slot 32767 is the last index below the 0xFFFF NULL), F=65536, C=65536.
# Books this big are never staged in LDS. "wrap" runs past 16,384 steps, so the ring
# hands out every slot up to 32767 and then reuses them (7 in 8 quotes are accepted);
# its F is small so that overflowing markets stay cheap to compare.
# (name, M, L, O, F, C, steps)
EXT_CAP_CASES = [("caps", 100, 1024, 32768, 65536, 65536, 300),
                 ("wrap", 70, 1024, 32768, 64, 65536, 22_000)]
