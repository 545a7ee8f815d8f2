"""C oracle vs the independent Python model on small random books (CPU only).

Tiny L/O/F make ring eviction, stale heads, self-links, zero/negative-size
fills and fill overflow frequent; prices and sizes include rejected values
(negative, >= L, <= 0) and customer ids include ids >= C. Every observable
output and the level/order state is compared after every step.
"""
import numpy as np
import pytest

from oracle.naive import NaiveVecMarket
from oracle.oracle import OracleMarket

CASES = [
    # (M, L, O, F, C, steps, seed)
    (6, 8, 1, 3, 3, 80, 1),
    (6, 8, 2, 4, 3, 80, 2),
    (6, 8, 3, 2, 4, 80, 3),
    (5, 12, 5, 6, 4, 120, 4),
    (4, 16, 7, 16, 5, 150, 5),
    (4, 70, 9, 5, 3, 150, 6),   # L > 64: two mask words on the GPU side
    (3, 130, 4, 8, 3, 150, 7),  # L > 128
]


def _inputs(rng, M, L, C):
    bid_px = rng.integers(-1, L + 1, M).astype(np.int32)
    ask_px = rng.integers(-1, L + 1, M).astype(np.int32)
    bid_sz = rng.integers(-1, 6, M).astype(np.int32)
    ask_sz = rng.integers(-1, 6, M).astype(np.int32)
    cust = rng.integers(0, C + 2, M).astype(np.int32)
    return bid_px, bid_sz, ask_px, ask_sz, cust


@pytest.mark.parametrize("M,L,O,F,C,steps,seed", CASES)
def test_oracle_matches_naive(M, L, O, F, C, steps, seed):
    rng = np.random.default_rng(seed)
    ora = OracleMarket(M, L, O, F, C)
    fills = ora.new_fill_batch()
    bbo = ora.new_bbo_batch()
    nv = NaiveVecMarket(M, L, O, F, C)
    seen_overflow = seen_negative_fill = 0
    for t in range(steps):
        args = _inputs(rng, M, L, C)
        ora.add_two_sided_quotes(*args, fills)
        counts, nfills = nv.step(*args)
        assert list(fills.fill_counts) == counts, f"step {t}"
        for m in range(M):
            n = F if counts[m] < 0 else counts[m]
            seen_overflow += counts[m] < 0
            for k in range(n):
                f = nfills[m][k]
                got = (fills.fill_prices[m, k], fills.fill_sizes[m, k], fills.fill_customer_ids[m, k],
                       fills.fill_quoter_ids[m, k], bool(fills.fill_is_sell_quote[m, k]),
                       fills.fill_quote_sizes[m, k], fills.fill_tid[m, k], fills.fill_quote_tid[m, k])
                exp = (f["price"], f["size"], f["taker"], f["quoter"], f["is_sell_quote"],
                       f["quote_size"], f["tid"], f["quote_tid"])
                assert tuple(int(x) if not isinstance(x, bool) else x for x in got) == exp, (t, m, k)
                seen_negative_fill += f["size"] <= 0
        ora.get_bbos(bbo)
        for m, book in enumerate(nv.books):
            assert (bbo.best_bid_prices[m], bbo.best_bid_sizes[m], bbo.best_ask_prices[m],
                    bbo.best_ask_sizes[m]) == book.bbo(), (t, m)
            assert ora.customer_portfolios[m].tolist() == book.pf, (t, m)
            assert ora.bid_heads[m].tolist() == [h for h, _ in book.lv["bid"]], (t, m)
            assert ora.bid_tails[m].tolist() == [tl for _, tl in book.lv["bid"]], (t, m)
            assert ora.ask_heads[m].tolist() == [h for h, _ in book.lv["ask"]], (t, m)
            assert ora.ask_tails[m].tolist() == [tl for _, tl in book.lv["ask"]], (t, m)
            assert ora.order_sizes[m].tolist() == [s["size"] for s in book.slots], (t, m)
            assert ora.order_next[m].tolist() == [s["nxt"] for s in book.slots], (t, m)
    if O <= 3:
        # the small rings must actually have produced the aliasing cases
        assert seen_overflow > 0 and seen_negative_fill > 0
