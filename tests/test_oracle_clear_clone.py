"""ClearQuotes and the copy constructor of the oracle, pinned by what they must mean
(CPU only).

ClearQuotes (market.cu:718-756) empties the selected markets' books and keeps their
portfolios and the TID counter. What follows is fixed without restating its steps:
a cleared market must from then on behave exactly like a freshly constructed
book fed the same quotes with the same TID counter (its fills, BBOs and text; its
portfolio moving by the same amounts), through as many ring wrap-arounds as the
test runs, while every market not selected goes on exactly as if nothing had been
cleared. The copy constructor (market.cu:385-411) must give an independent book
that evolves exactly like its source under the same quotes, every state array
equal after every step, and not at all when only the source moves.

Right after the clear, a cleared market's level heads and tails and its ring
position must also equal a fresh book's: the ring position alone cannot show in
any output (with every list empty, starting the ring at another slot only
relabels the slots: each insert still evicts the one O inserts before it).

Each check is shown to catch a plausible mistake planted in the oracle's state
(a clear that leaves the ring position where it was, or one level's head, or
zeroes the portfolios, or clears a market not selected; a copy that misses the
ring positions or the TID counter, or shares the source's arrays).
"""
import numpy as np
import pytest

from oracle.oracle import OracleMarket

M, L, O, F, C = 40, 24, 6, 12, 5
STATE = ("bid_heads", "ask_heads", "bid_tails", "ask_tails", "order_prices", "order_sizes",
         "order_customer_ids", "order_tid", "order_next", "order_next_slots", "customer_portfolios")
FILL_FIELDS = ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
               "fill_quote_sizes", "fill_tid", "fill_quote_tid")


def _stream(seed, steps):
    """Quotes around a drifting mid (about half cross), with rejected prices and
    zero or negative sizes now and then; a small ring (O = 6) wraps every 3 steps."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(steps):
        base = rng.integers(0, L - 10)
        bid = (base + rng.integers(-1, 11, M)).astype(np.int32)
        ask = (base + rng.integers(-1, 11, M)).astype(np.int32)
        bid[rng.random(M) < 0.03] = L
        out.append((bid, rng.integers(-1, 7, M).astype(np.int32), ask,
                    rng.integers(-1, 7, M).astype(np.int32), rng.integers(0, C, M).astype(np.int32)))
    return out


def _step(o, q):
    f, b = o.new_fill_batch(), o.new_bbo_batch()
    o.add_two_sided_quotes(*q, f)
    o.get_bbos(b)
    o.update_last_prices(b, f)
    return f, b


def _rows(f, m):
    n = int(f.fill_counts[m])
    n = F if n < 0 else n
    return int(f.fill_counts[m]), [tuple(int(getattr(f, k)[m, i]) for k in FILL_FIELDS) for i in range(n)]


def _bbo(b, m):
    return tuple(int(getattr(b, k)[m]) for k in ("best_bid_prices", "best_bid_sizes", "best_ask_prices",
                                                   "best_ask_sizes"))


def _set_tid(o, tid):
    o._h.contents.global_tid = tid


def _clear_check(seed, t0, k, plant=None):
    """Run t0 steps, clear a random half of the markets, run k more; return the
    list of mismatches against a fresh book (cleared markets) and against an
    uncleared replay (the others)."""
    qs = _stream(seed, t0 + k)
    o, keep = OracleMarket(M, L, O, F, C), OracleMarket(M, L, O, F, C)
    for q in qs[:t0]:
        _step(o, q)
        _step(keep, q)
    mask = np.random.default_rng(seed + 1).random(M) < 0.5
    pf0 = o.customer_portfolios.copy()
    ring0 = o.order_next_slots.copy()
    heads0 = o.bid_heads.copy()
    if plant == "a market not selected cleared":
        mask_used = mask.copy()
        mask_used[int(np.nonzero(~mask & (heads0 != -1).any(1))[0][0])] = True
    else:
        mask_used = mask
    o.clear_quotes(mask_used)
    if plant == "ring position kept":
        o.order_next_slots[mask] = ring0[mask]
    elif plant == "one head kept":
        m = int(np.nonzero(mask & (heads0 != -1).any(1))[0][0])
        p = int(np.nonzero(heads0[m] != -1)[0][0])
        o.bid_heads[m, p] = heads0[m, p]
    elif plant == "portfolios zeroed":
        o.customer_portfolios[mask] = 0
    fresh = OracleMarket(M, L, O, F, C)
    _set_tid(fresh, o.global_tid)
    bad = []
    for name in ("bid_heads", "ask_heads", "bid_tails", "ask_tails", "order_next_slots"):
        if not np.array_equal(getattr(o, name)[mask], getattr(fresh, name)[mask]):
            bad.append((-1, -1, name))
    for t, q in enumerate(qs[t0:]):
        fo, bo = _step(o, q)
        ff, bf = _step(fresh, q)
        fk, bk = _step(keep, q)
        for m in range(M):
            ref_f, ref_b, ref_o = (ff, bf, fresh) if mask[m] else (fk, bk, keep)
            if _rows(fo, m) != _rows(ref_f, m) or _bbo(bo, m) != _bbo(ref_b, m):
                bad.append((t, m, "fills/bbo"))
            if o.to_string(m) != ref_o.to_string(m):
                bad.append((t, m, "text"))
            if bo.last_prices[m] != ref_b.last_prices[m]:
                bad.append((t, m, "last price"))
            if mask[m]:
                delta = (o.customer_portfolios[m].astype(np.int64) - pf0[m]).astype(np.int32)
                if not np.array_equal(delta, fresh.customer_portfolios[m]):
                    bad.append((t, m, "portfolio"))
            elif not np.array_equal(o.customer_portfolios[m], keep.customer_portfolios[m]):
                bad.append((t, m, "portfolio"))
        if not o.global_tid == fresh.global_tid == keep.global_tid:
            bad.append((t, -1, "tid"))
    return bad, int(mask.sum())


@pytest.mark.parametrize("seed,t0", [(1, 5), (2, 11), (3, 40)])
def test_cleared_market_is_a_fresh_book(seed, t0):
    bad, n = _clear_check(seed, t0, 3 * O)
    assert n > 5
    assert bad == []


@pytest.mark.parametrize("plant", ["ring position kept", "one head kept", "portfolios zeroed",
                                   "a market not selected cleared"])
def test_clear_check_catches_planted_mistakes(plant):
    bad, _ = _clear_check(2, 11, 3 * O, plant=plant)
    assert bad, plant
    if plant != "ring position kept":  # the others show in the outputs, not only the state
        assert any(t >= 0 for t, _, _ in bad), plant


def test_clear_with_no_market_selected_changes_nothing():
    qs = _stream(7, 20)
    o, keep = OracleMarket(M, L, O, F, C), OracleMarket(M, L, O, F, C)
    for q in qs[:10]:
        _step(o, q)
        _step(keep, q)
    o.clear_quotes(np.zeros(M, np.bool_))
    for q in qs[10:]:
        fo, _ = _step(o, q)
        fk, _ = _step(keep, q)
        assert all(_rows(fo, m) == _rows(fk, m) for m in range(M))
    for name in STATE:
        assert np.array_equal(getattr(o, name), getattr(keep, name)), name


def _clone_check(seed, t0, k, plant=None):
    """Run t0 steps, copy, run the same k steps on both; every state array, fill row,
    BBO, text and the TID counter must agree after every step."""
    qs = _stream(seed, t0 + k)
    o = OracleMarket(M, L, O, F, C)
    for q in qs[:t0]:
        _step(o, q)
    c = o.clone()
    if plant == "ring positions not copied":
        c.order_next_slots[:] = 0
    elif plant == "TID counter not copied":
        _set_tid(c, 0)
    bad = []
    for t, q in enumerate(qs[t0:]):
        fo, bo = _step(o, q)
        fc, bc = _step(c, q)
        for name in STATE:
            if not np.array_equal(getattr(o, name), getattr(c, name)):
                bad.append((t, name))
        for m in range(M):
            if _rows(fo, m) != _rows(fc, m) or _bbo(bo, m) != _bbo(bc, m) or o.to_string(m) != c.to_string(m):
                bad.append((t, m))
        if o.global_tid != c.global_tid:
            bad.append((t, "tid"))
    return bad, o, c, qs


@pytest.mark.parametrize("seed,t0", [(4, 2), (5, 13), (6, 50)])
def test_copy_evolves_like_its_source(seed, t0):
    bad, _, _, _ = _clone_check(seed, t0, 2 * O)
    assert bad == []


@pytest.mark.parametrize("plant", ["ring positions not copied", "TID counter not copied"])
def test_copy_check_catches_planted_mistakes(plant):
    bad, _, _, _ = _clone_check(5, 13, 2 * O, plant=plant)
    assert bad, plant


def test_copy_is_independent_of_its_source():
    """Moving only the source changes nothing in the copy (a copy sharing the
    source's arrays would change with it), and the other way round."""
    qs = _stream(8, 30)
    o = OracleMarket(M, L, O, F, C)
    for q in qs[:10]:
        _step(o, q)
    c = o.clone()
    snap = {name: getattr(c, name).copy() for name in STATE}
    tid = c.global_tid
    for q in qs[10:20]:
        _step(o, q)
    assert any(not np.array_equal(getattr(o, name), snap[name]) for name in STATE)
    for name in STATE:
        assert np.array_equal(getattr(c, name), snap[name]), name
    assert c.global_tid == tid
    # the copy then replays the source's ten steps and ends where the source is
    for q in qs[10:20]:
        _step(c, q)
    for name in STATE:
        assert np.array_equal(getattr(c, name), getattr(o, name)), name
