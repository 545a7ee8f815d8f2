"""Invariants of the matching semantics, checked on the oracle (CPU only).

Each property follows from the reference kernel (src/order_matching/market.cu)
without restating its steps, so a dropped term, a wrong sign, a swapped operand or
a wrong priority in the oracle fails here even where no known-answer test reaches:

* contracts and cash sum to zero per market (every fill moves q and p*q between a
  buyer and a seller, market.cu:221-232);
* without ring wrap-around, the resting size linked from the level heads equals
  the previous one plus the accepted insert sizes minus twice the filled size
  (:237-238), and every order record is on exactly one list or has size 0;
* after a call that did not overflow, the book is uncrossed (loop exit, :145-146);
* fill_counts lies in [-1, F] (:187-195);
* the quote (resting) side of each fill has the smaller TID (:172), and the fill
  price is the quote's price level, between the crossing bid and ask (:174);
* a BBO side is (NULL, 0) exactly when no level of that side has a head, and
  otherwise the best level with its head's size (:280-320);
* the TID counter advances by 2 per call (:512).
"""
import numpy as np
import pytest

from oracle.oracle import OracleMarket

NULL = -1


def _walk(heads, nxt, sizes, O):
    """Sizes of every order on a level list (bounded walk) and the slots seen."""
    total, seen = 0, []
    for h in heads:
        s, n = int(h), 0
        while s != NULL and n <= O:
            total += int(sizes[s])
            seen.append(s)
            s = int(nxt[s])
            n += 1
    return total, seen


def _best(heads_row, bid):
    lv = np.nonzero(heads_row != NULL)[0]
    if lv.size == 0:
        return NULL
    return int(lv.max() if bid else lv.min())


def _quotes(rng, M, L, C, t, sizes_hi=9):
    base = rng.integers(2, L - 2)
    bid = np.clip(base + rng.integers(-3, 4, M), 0, L - 1).astype(np.int32)
    ask = np.clip(base + rng.integers(-3, 4, M), 0, L - 1).astype(np.int32)
    return (bid, rng.integers(1, sizes_hi, M).astype(np.int32), ask,
            rng.integers(1, sizes_hi, M).astype(np.int32), rng.integers(0, C, M).astype(np.int32))


@pytest.mark.parametrize("M,L,O,F,C,steps,seed,wraps", [
    (40, 16, 512, 64, 5, 200, 1, False),
    (40, 64, 512, 8, 7, 200, 2, False),   # small F: overflowing calls too
    (40, 12, 6, 16, 4, 200, 3, True),     # tiny ring: slot reuse and stale links
])
def test_oracle_invariants(M, L, O, F, C, steps, seed, wraps):
    rng = np.random.default_rng(seed)
    om = OracleMarket(M, L, O, F, C)
    fills, bbo = om.new_fill_batch(), om.new_bbo_batch()
    prev_live = np.zeros(M, np.int64)
    for t in range(steps):
        args = _quotes(rng, M, L, C, t)
        bid_px, bid_sz, ask_px, ask_sz, _ = args
        om.add_two_sided_quotes(*args, fills)
        om.get_bbos(bbo)
        assert om.global_tid == 2 * (t + 1)
        counts = fills.fill_counts
        assert counts.min() >= -1 and counts.max() <= F
        pf = om.customer_portfolios.astype(np.int64)
        assert not pf[:, :, 0].sum(axis=1).any(), f"step {t}: contracts do not sum to zero"
        assert not pf[:, :, 1].sum(axis=1).any(), f"step {t}: cash does not sum to zero"
        for m in range(M):
            n = F if counts[m] < 0 else int(counts[m])
            tid, qtid = fills.fill_tid[m, :n], fills.fill_quote_tid[m, :n]
            assert (qtid <= tid).all(), f"step {t} market {m}: quote side is not the earlier TID"
            bb = _best(om.bid_heads[m], True)
            ba = _best(om.ask_heads[m], False)
            # BBO
            if bb == NULL:
                assert bbo.best_bid_prices[m] == NULL and bbo.best_bid_sizes[m] == 0
            else:
                assert bbo.best_bid_prices[m] == bb
                assert bbo.best_bid_sizes[m] == om.order_sizes[m, om.bid_heads[m, bb]]
            if ba == NULL:
                assert bbo.best_ask_prices[m] == NULL and bbo.best_ask_sizes[m] == 0
            else:
                assert bbo.best_ask_prices[m] == ba
                assert bbo.best_ask_sizes[m] == om.order_sizes[m, om.ask_heads[m, ba]]
            if wraps:
                continue
            # no slot reuse: every row is a real trade between two crossing orders
            sz = fills.fill_sizes[m, :n]
            assert (sz > 0).all()
            px = fills.fill_prices[m, :n]
            prices = om.order_prices[m]
            slot_of_tid = {int(om.order_tid[m, s]): s for s in range(O) if om.order_tid[m, s] or s == 0}
            for k in range(n):
                qs = slot_of_tid[int(qtid[k])]
                ts = slot_of_tid[int(tid[k])]
                assert px[k] == prices[qs], f"step {t} market {m}: fill price is not the quote's level"
                buy_px, sell_px = (prices[ts], prices[qs]) if fills.fill_is_sell_quote[m, k] else \
                    (prices[qs], prices[ts])
                assert sell_px <= px[k] <= buy_px
            if counts[m] >= 0:
                assert bb == NULL or ba == NULL or bb < ba, f"step {t} market {m}: book left crossed"
            live_b, seen_b = _walk(om.bid_heads[m], om.order_next[m], om.order_sizes[m], O)
            live_a, seen_a = _walk(om.ask_heads[m], om.order_next[m], om.order_sizes[m], O)
            seen = seen_b + seen_a
            assert len(seen) == len(set(seen)), "an order is on two lists"
            off_list = np.setdiff1d(np.arange(int(om.order_next_slots[m])), np.array(seen, dtype=np.int64))
            assert not om.order_sizes[m, off_list].any(), "an unlinked order still has size"
            ins = (int(bid_sz[m]) if bid_px[m] < L else 0) + (int(ask_sz[m]) if ask_px[m] < L else 0)
            if counts[m] >= 0:
                assert live_b + live_a == prev_live[m] + ins - 2 * int(sz.sum())
            prev_live[m] = live_b + live_a
        if not wraps:
            assert int(om.order_next_slots.max()) < O  # the ring never wrapped


def test_invariant_checks_catch_a_planted_sign_error():
    """A portfolio update with the seller's sign flipped (planted in a copy of the
    oracle's output, on the CPU) must break the zero-sum invariant."""
    rng = np.random.default_rng(5)
    om = OracleMarket(8, 16, 64, 16, 3)
    fills = om.new_fill_batch()
    for t in range(20):
        om.add_two_sided_quotes(*_quotes(rng, 8, 16, 3, t), fills)
    pf = om.customer_portfolios.astype(np.int64).copy()
    assert not pf[:, :, 0].sum(axis=1).any()
    m = int(np.nonzero(np.abs(pf[:, :, 0]).sum(axis=1))[0][0])
    seller = int(np.argmin(pf[m, :, 0]))
    pf[m, seller, 0] = -pf[m, seller, 0]
    assert pf[:, :, 0].sum(axis=1).any()
