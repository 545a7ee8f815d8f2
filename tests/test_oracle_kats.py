"""The CPU oracle against the reference's known answers (CPU only).

Pins ``oracle/market_oracle.c`` with the asserts of the reference's own tests
(src/tests/integration/test_vec_market.py, src/tests/unit_tests/market_tests.cu
where they agree with market.cu) and with hand traces of market.cu
(eviction aliasing, same-slot alias, fill overflow), all in tests/golden/kats.json.
The independent pure-Python model in ``oracle/naive.py`` must pass them too.
"""
import numpy as np
import pytest

from kat_harness import OracleAdapter, load_kats, run_scenario

SCENARIOS = load_kats()


@pytest.mark.parametrize("sc", SCENARIOS, ids=[s["name"] for s in SCENARIOS])
def test_oracle_kat(sc):
    run_scenario(sc, OracleAdapter)


class NaiveAdapter:
    """The same scenarios through oracle/naive.py (an independent second model)."""

    def __init__(self, shape):
        from oracle.naive import NaiveVecMarket
        self.shape = shape
        self.mk = NaiveVecMarket(shape["M"], shape["L"], shape["O"], shape["F"], shape["C"])
        M, F = shape["M"], shape["F"]
        self.f = {k: np.zeros((M, F), dtype=np.int32) for k in
                  ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids",
                   "fill_quote_sizes", "fill_tid", "fill_quote_tid")}
        self.f["fill_is_sell_quote"] = np.zeros((M, F), dtype=np.bool_)
        self.f["fill_counts"] = np.zeros((M,), dtype=np.int32)
        self.new_bbo()

    def quote(self, *args):
        counts, fills = self.mk.step(*args)
        keys = [("fill_prices", "price"), ("fill_sizes", "size"), ("fill_customer_ids", "taker"),
                ("fill_quoter_ids", "quoter"), ("fill_is_sell_quote", "is_sell_quote"),
                ("fill_quote_sizes", "quote_size"), ("fill_tid", "tid"), ("fill_quote_tid", "quote_tid")]
        for m, (c, fl) in enumerate(zip(counts, fills)):
            self.f["fill_counts"][m] = c
            for j, fd in enumerate(fl):
                for arr, key in keys:
                    self.f[arr][m, j] = fd[key]

    def bbos(self):
        for m, book in enumerate(self.mk.books):
            bp, bs, ap, as_ = book.bbo()
            self.b["best_bid_prices"][m], self.b["best_bid_sizes"][m] = bp, bs
            self.b["best_ask_prices"][m], self.b["best_ask_sizes"][m] = ap, as_

    def update_last(self):
        for m in range(self.shape["M"]):
            c = self.f["fill_counts"][m]
            if c > 0:
                self.b["last_prices"][m] = self.f["fill_prices"][m, c - 1]

    def reset(self):
        from oracle.naive import NaiveVecMarket
        s = self.shape
        old = self.mk
        self.mk = NaiveVecMarket(s["M"], s["L"], s["O"], s["F"], s["C"])
        # Reset keeps the order pool contents (market.cu:704-706); only lists,
        # counters, portfolios and the TID restart.
        for nb, ob in zip(self.mk.books, old.books):
            for slot_new, slot_old in zip(nb.slots, ob.slots):
                slot_new.update(slot_old, nxt=-1)

    def bbo_reset(self):
        for v in self.b.values():
            v[:] = 0

    def new_bbo(self):
        M = self.shape["M"]
        self.b = {k: np.zeros((M,), dtype=np.int32) for k in
                  ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices")}

    def array(self, name):
        if name == "portfolio":
            return np.array([b.pf for b in self.mk.books], dtype=np.int64)
        if name in self.b:
            return self.b[name]
        return self.f[name]

    def to_string(self, m):
        pytest.skip("the naive model has no to_string")


@pytest.mark.parametrize("sc", [s for s in SCENARIOS if s["name"] != "string_representation"],
                         ids=[s["name"] for s in SCENARIOS if s["name"] != "string_representation"])
def test_naive_kat(sc):
    run_scenario(sc, NaiveAdapter)
