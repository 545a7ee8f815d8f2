"""Runs the known-answer scenarios of ``tests/golden/kats.json`` against an engine.

An *adapter* wraps one engine (the CPU oracle or the HIP engine behind
``astra_cuda.order_matching``) behind a handful of calls, so the same scenario
file checks both. Expected values in the fixture come from the reference's own
tests or from hand traces of market.cu, never from the oracle.
"""
from __future__ import annotations

import json
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

FILL_FIELDS = ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids",
               "fill_is_sell_quote", "fill_quote_sizes", "fill_tid", "fill_quote_tid")
BBO_FIELDS = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices")


def load_kats():
    with open(os.path.join(GOLDEN, "kats.json")) as f:
        return json.load(f)["scenarios"]


class OracleAdapter:
    """Adapter over ``oracle.oracle.OracleMarket`` (host numpy arrays)."""

    def __init__(self, shape):
        from oracle.oracle import OracleMarket
        self.mk = OracleMarket(shape["M"], shape["L"], shape["O"], shape["F"], shape["C"])
        self.fills = self.mk.new_fill_batch()
        self.bbo = self.mk.new_bbo_batch()

    def quote(self, bid_px, bid_sz, ask_px, ask_sz, cust):
        self.mk.add_two_sided_quotes(bid_px, bid_sz, ask_px, ask_sz, cust, self.fills)

    def bbos(self):
        self.mk.get_bbos(self.bbo)

    def update_last(self):
        self.mk.update_last_prices(self.bbo, self.fills)

    def reset(self):
        self.mk.reset()

    def bbo_reset(self):
        for f in BBO_FIELDS:
            getattr(self.bbo, f)[:] = 0

    def new_bbo(self):
        self.bbo = self.mk.new_bbo_batch()

    def array(self, name) -> np.ndarray:
        if name == "portfolio":
            return np.array(self.mk.get_customer_portfolios())
        if name in BBO_FIELDS:
            return np.array(getattr(self.bbo, name))
        return np.array(getattr(self.fills, name))

    def to_string(self, m) -> str:
        return self.mk.to_string(m)


def run_scenario(sc, adapter_cls):
    """Execute one scenario; raises AssertionError with context on the first mismatch."""
    ad = adapter_cls(sc["shape"])
    for i, op in enumerate(sc["ops"]):
        kind = op["op"]
        if kind == "quote":
            ad.quote(*(np.array(op[k], dtype=np.int32) for k in ("bid_px", "bid_sz", "ask_px", "ask_sz", "cust")))
        elif kind == "bbos":
            ad.bbos()
        elif kind == "update_last":
            ad.update_last()
        elif kind == "reset":
            ad.reset()
        elif kind == "bbo_reset":
            ad.bbo_reset()
        elif kind == "new_bbo":
            ad.new_bbo()
        elif kind == "check":
            for chk in op["checks"]:
                _check(ad, chk, f"{sc['name']} op#{i}")
        else:
            raise ValueError(f"unknown op {kind}")
    return ad


def _check(ad, chk, where):
    k = chk["kind"]
    if k in ("eq", "gt"):
        arr = ad.array(chk["array"])
        got = arr[tuple(chk["index"])]
        got = bool(got) if arr.dtype == np.bool_ else int(got)
        exp = chk["value"]
        if k == "eq":
            assert got == exp, f"{where}: {chk['array']}{chk['index']} = {got}, expected {exp}"
        else:
            assert got > exp, f"{where}: {chk['array']}{chk['index']} = {got}, expected > {exp}"
    elif k == "fill":
        m, j = chk["market"], chk["k"]
        got = [ad.array(f)[m, j] for f in FILL_FIELDS]
        got = [bool(v) if i == 4 else int(v) for i, v in enumerate(got)]
        assert got == chk["value"], f"{where}: fill[{m},{j}] = {got}, expected {chk['value']}"
    elif k == "sum_sizes":
        m = chk["market"]
        n = int(ad.array("fill_counts")[m])
        s = int(ad.array("fill_sizes")[m, :max(n, 0)].sum())
        assert s == chk["value"], f"{where}: sum of fill sizes of market {m} = {s}, expected {chk['value']}"
    elif k == "contains":
        txt = ad.to_string(chk["market"])
        assert chk["value"] in txt, f"{where}: {chk['value']!r} not in {txt!r}"
    elif k == "text":
        txt = ad.to_string(chk["market"])
        assert txt == chk["value"], f"{where}: to_string = {txt!r}, expected {chk['value']!r}"
    else:
        raise ValueError(f"unknown check kind {k}")
