"""Shared helpers for the GPU parity tests: the HIP engine (through the drop-in
``astra_cuda.order_matching`` API) against the CPU oracle on the same inputs."""
from __future__ import annotations

import numpy as np
import torch

from kat_harness import BBO_FIELDS, FILL_FIELDS

DEV = "cuda:0"


def t32(a) -> torch.Tensor:
    return torch.as_tensor(np.ascontiguousarray(a, dtype=np.int32)).to(DEV)


class GpuAdapter:
    """KAT adapter over astra_cuda.order_matching (the product path)."""
    layout = "columns"

    def __init__(self, shape):
        from astra_cuda import order_matching as aom
        ext = shape["L"] > 128 or shape["O"] > 1024 or shape["F"] > 1024 or shape["C"] > 1024
        self.mk = aom.VecMarket(shape["M"], shape["L"], shape["O"], shape["F"], shape["C"],
                                allow_extended_shapes=ext)
        self.fills = self.mk.new_fill_batch(self.layout)
        self.bbo = self.mk.new_bbo_batch()

    def quote(self, bid_px, bid_sz, ask_px, ask_sz, cust):
        self.mk.add_two_sided_quotes(t32(bid_px), t32(bid_sz), t32(ask_px), t32(ask_sz), t32(cust),
                                     self.fills)

    def bbos(self):
        self.mk.get_bbos(self.bbo)

    def update_last(self):
        self.bbo.update_last_prices(self.fills)

    def reset(self):
        self.mk.reset()

    def bbo_reset(self):
        self.bbo.reset()

    def new_bbo(self):
        self.bbo = self.mk.new_bbo_batch()

    def array(self, name):
        if name == "portfolio":
            return self.mk.get_customer_portfolios().cpu().numpy()
        if name in BBO_FIELDS:
            return getattr(self.bbo, name).cpu().numpy()
        return getattr(self.fills, name).cpu().numpy()

    def to_string(self, m):
        return self.mk.to_string(m)


class GpuRowAdapter(GpuAdapter):
    layout = "rows"


class GpuCompiledAdapter(GpuAdapter):
    """KAT adapter over the compiled binding astra_cuda._C.order_matching (the
    reference's pybind surface: reference caps, the per-field FillBatch)."""
    layout = "compiled"

    def __init__(self, shape):
        from astra_cuda._C import order_matching as com
        self.mk = com.VecMarket(shape["M"], shape["L"], shape["O"], shape["F"], shape["C"])
        self.fills = self.mk.new_fill_batch()
        self.bbo = self.mk.new_bbo_batch()


def effective_counts(counts: np.ndarray, F: int) -> np.ndarray:
    """Number of fill rows written by the last call (F for an overflowed market)."""
    return np.where(counts < 0, F, counts)


def compare_fills(gpu_fills, ora_fills, F: int, where: str, full: bool = False) -> int:
    """Compare the rows written by the last call (or the full arrays when ``full``).
    Returns the number of fill rows compared."""
    gc = gpu_fills.fill_counts.cpu().numpy()
    oc = ora_fills.fill_counts
    if not np.array_equal(gc, oc):
        bad = np.nonzero(gc != oc)[0][:5]
        raise AssertionError(f"{where}: fill_counts differ at markets {bad.tolist()}: "
                             f"gpu {gc[bad].tolist()} oracle {oc[bad].tolist()}")
    eff = effective_counts(oc, F)
    kmax = F if full else int(eff.max(initial=0))
    if kmax == 0:
        return 0
    valid = np.arange(kmax)[None, :] < eff[:, None]
    for f in FILL_FIELDS:
        g = getattr(gpu_fills, f)[:, :kmax].cpu().numpy()
        o = getattr(ora_fills, f)[:, :kmax]
        if full:
            ok = np.array_equal(g, o)
        else:
            ok = np.array_equal(np.where(valid, g, 0), np.where(valid, o, 0))
        if not ok:
            diff = np.argwhere((g != o) & (True if full else valid))[:5]
            raise AssertionError(f"{where}: {f} differs at {diff.tolist()}: "
                                 f"gpu {[g[tuple(d)] for d in diff]} oracle {[o[tuple(d)] for d in diff]}")
    return int(eff.sum())


def compare_bbo(gpu_bbo, ora_bbo, where: str):
    for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
        g = getattr(gpu_bbo, f).cpu().numpy()
        o = getattr(ora_bbo, f)
        if not np.array_equal(g, o):
            bad = np.nonzero(g != o)[0][:5]
            raise AssertionError(f"{where}: {f} differs at {bad.tolist()}: gpu {g[bad].tolist()} "
                                 f"oracle {o[bad].tolist()}")


def compare_portfolios(gpu_mk, ora_mk, where: str):
    g = gpu_mk.get_customer_portfolios().cpu().numpy()
    o = ora_mk.customer_portfolios
    if not np.array_equal(g, o):
        bad = np.argwhere(g != o)[:5]
        raise AssertionError(f"{where}: portfolios differ at {bad.tolist()}")


def make_market(M, L, O, F, C, extended=None, stage_budget=None, per_wave=None, fill_rows=None,
                helpers=None, hand_lanes=None, hand_queue=None, helper_polls=None):
    """VecMarket through the drop-in API. stage_budget (read by the engine when the
    market is created) sets the loop passes before a market's book is staged in
    LDS; 1 forces the staged path for every market that crosses twice. per_wave
    (likewise) sets the markets per wavefront of the matching kernel, fill_rows
    (2 or 4) the fill rows a lane buffers before writing them, helpers the market
    wavefronts per helper wavefront (0: none; 2 or 3) where the launch uses
    helpers (4 fill rows, staged books), hand_lanes how few lanes must still loop
    for a zero-size walk to go to the helper, hand_queue how many markets one helper
    may hold at once, helper_polls the idle polls after which a helper gives up
    waiting (closing its queue)."""
    import os
    from astra_cuda import order_matching as aom
    if extended is None:
        extended = L > 128 or O > 1024 or F > 1024 or C > 1024
    env = {"ASTRA_MARKET_STAGE_BUDGET": stage_budget, "ASTRA_MARKET_PER_WAVE": per_wave,
           "ASTRA_MARKET_FILL_ROWS": fill_rows, "ASTRA_MARKET_HELPERS": helpers,
           "ASTRA_MARKET_HAND_LANES": hand_lanes, "ASTRA_MARKET_HAND_QUEUE": hand_queue,
           "ASTRA_MARKET_HELPER_POLLS": helper_polls}
    old = {k: os.environ.get(k) for k in env}
    for k, v in env.items():
        if v is not None:
            os.environ[k] = str(v)
    try:
        return aom.VecMarket(M, L, O, F, C, allow_extended_shapes=extended)
    finally:
        for k, v in env.items():
            if v is None:
                continue
            if old[k] is None:
                del os.environ[k]
            else:
                os.environ[k] = old[k]


def run_parity(M, L, O, F, C, steps, gen, *, bbo_every=1, full_every=0, last_every=1,
               extended=None, nthreads=8, label="", stage_budget=None, layout="columns",
               per_wave=None, fill_rows=None, helpers=None, hand_lanes=None, hand_queue=None,
               helper_polls=None):
    """Drive GPU engine and oracle with the same inputs; compare after every step.
    layout "columns" / "rows" picks the FillBatch layout of astra_cuda.order_matching;
    "compiled" runs the compiled binding astra_cuda._C.order_matching instead.

    ``gen(t)`` returns (bid_px, bid_sz, ask_px, ask_sz, cust) int32 arrays of shape [M].
    Returns summary statistics (fill rows compared, overflows seen).
    """
    from oracle.oracle import OracleMarket
    if layout == "compiled":  # the compiled binding (reference caps, per-field FillBatch)
        from astra_cuda._C import order_matching as com
        g = com.VecMarket(M, L, O, F, C)
        gf, gb = g.new_fill_batch(), g.new_bbo_batch()
    else:
        g = make_market(M, L, O, F, C, extended, stage_budget, per_wave, fill_rows, helpers, hand_lanes,
                        hand_queue, helper_polls)
        gf, gb = g.new_fill_batch(layout), g.new_bbo_batch()
    o = OracleMarket(M, L, O, F, C)
    of, ob = o.new_fill_batch(), o.new_bbo_batch()
    rows = overflows = 0
    for t in range(steps):
        args = gen(t)
        where = f"{label} step {t}"
        g.add_two_sided_quotes(*(t32(a) for a in args), gf)
        o.add_two_sided_quotes(*args, of, nthreads=nthreads)
        full = bool(full_every) and (t % full_every == full_every - 1 or t == steps - 1)
        rows += compare_fills(gf, of, F, where, full=full)
        overflows += int((of.fill_counts < 0).sum())
        if last_every and t % last_every == 0:
            gb.update_last_prices(gf)
            o.update_last_prices(ob, of)
        if bbo_every and t % bbo_every == 0:
            g.get_bbos(gb)
            o.get_bbos(ob, nthreads=nthreads)
            compare_bbo(gb, ob, where)
        if t % 50 == 0 or t == steps - 1:
            compare_portfolios(g, o, where)
    assert g.global_tid == o.global_tid
    return {"fill_rows": rows, "overflows": overflows, "gpu": g, "oracle": o}


def helper_exits(mk) -> int:
    """Helper wavefronts that gave up waiting so far (the second control word at the
    start of the engine's workspace)."""
    torch.cuda.synchronize()
    return int(mk._ws[4:8].view(torch.int32).item())
