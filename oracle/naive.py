"""An independently written pure-Python model of one VecMarket market.

TEST INFRASTRUCTURE ONLY (same rules as ``oracle.py``). It exists to cross-check
``market_oracle.c`` by brute force on tiny random books: it is written in a
different shape (one object per market, Python lists, explicit helper methods,
64-bit Python ints masked to int32) so that a slip in either implementation
shows up as a disagreement.

Semantics modelled (nlyu1/astra-cuda src/order_matching/market.cu):
- insertion appends to the tail of the level's FIFO list and reuses ring slots
  without unlinking them (:17-100);
- matching repeatedly crosses the head of the best bid level with the head of
  the best ask level while best_bid >= best_ask (:102-278): the earlier TID is
  the resting quote and sets the price (its order's stored price), the size is
  min of the two remaining sizes, a side whose remaining size becomes exactly 0
  pops its head, and an emptied level triggers a new best-price search;
- the F+1-th fill of one call sets the count to -1 and stops (:187-195).
"""
from __future__ import annotations

NULL = -1


def i32(x: int) -> int:
    """Wrap a Python int to a signed 32-bit value."""
    x &= 0xFFFFFFFF
    return x - (1 << 32) if x >= (1 << 31) else x


class NaiveBook:
    def __init__(self, L: int, O: int, F: int, C: int):
        self.L, self.O, self.F, self.C = L, O, F, C
        # per side: level -> [head, tail]
        self.lv = {"bid": [[NULL, NULL] for _ in range(L)], "ask": [[NULL, NULL] for _ in range(L)]}
        # order slots: dicts so every field is explicit
        self.slots = [dict(price=0, size=0, cust=0, tid=0, nxt=NULL) for _ in range(O)]
        self.counter = 0
        self.pf = [[0, 0] for _ in range(C)]

    # ---- insertion -------------------------------------------------------
    def _take_slot(self) -> int:
        s = self.counter % self.O
        self.counter += 1
        return s

    def submit(self, side: str, price: int, size: int, cust: int, tid: int) -> bool:
        if size <= 0 or price >= self.L or price < 0:
            return False
        s = self._take_slot()
        self.slots[s] = dict(price=price, size=size, cust=cust, tid=tid, nxt=NULL)
        level = self.lv[side][price]
        prev_tail = level[1]
        level[1] = s
        if prev_tail == NULL:
            level[0] = s
        else:
            self.slots[prev_tail]["nxt"] = s
        return True

    # ---- best prices -----------------------------------------------------
    def best(self, side: str) -> int:
        levels = range(self.L - 1, -1, -1) if side == "bid" else range(self.L)
        for p in levels:
            if self.lv[side][p][0] != NULL:
                return p
        return -1 if side == "bid" else self.L

    # ---- matching --------------------------------------------------------
    def _pop_if_done(self, side: str, price: int, slot: int) -> bool:
        """Pop the level head if that order is exhausted; True if the level emptied."""
        if self.slots[slot]["size"] != 0:
            return False
        nxt = self.slots[slot]["nxt"]
        self.lv[side][price][0] = nxt
        if nxt == NULL:
            self.lv[side][price][1] = NULL
            return True
        return False

    def match(self, fills_out: list) -> int:
        """Run the crossing loop; append fill tuples; return the fill count or -1."""
        bb, ba = self.best("bid"), self.best("ask")
        n = 0
        while bb >= 0 and ba < self.L and bb >= ba:
            b = self.lv["bid"][bb][0]
            a = self.lv["ask"][ba][0]
            if b == NULL or a == NULL:
                break
            B, A = dict(self.slots[b]), dict(self.slots[a])  # snapshots before the fill
            bid_rests = B["tid"] < A["tid"]
            quote, taker = (B, A) if bid_rests else (A, B)
            px = quote["price"]
            q = min(B["size"], A["size"])
            if n >= self.F:
                return -1
            fills_out.append(dict(price=px, size=q, taker=taker["cust"], quoter=quote["cust"],
                                  is_sell_quote=not bid_rests, quote_size=quote["size"],
                                  tid=taker["tid"], quote_tid=quote["tid"]))
            if 0 <= B["cust"] < self.C and 0 <= A["cust"] < self.C:
                notional = i32(px * q)
                buyer, seller = self.pf[B["cust"]], self.pf[A["cust"]]
                buyer[0] = i32(buyer[0] + q)
                buyer[1] = i32(buyer[1] - notional)
                seller[0] = i32(seller[0] - q)
                seller[1] = i32(seller[1] + notional)
            n += 1
            self.slots[b]["size"] = i32(self.slots[b]["size"] - q)
            self.slots[a]["size"] = i32(self.slots[a]["size"] - q)
            if self._pop_if_done("bid", bb, b):
                bb = self.best("bid")
            if self._pop_if_done("ask", ba, a):
                ba = self.best("ask")
        return n

    def bbo(self):
        bb, ba = self.best("bid"), self.best("ask")
        out = [NULL, 0, NULL, 0]
        if bb >= 0:
            out[0], out[1] = bb, self.slots[self.lv["bid"][bb][0]]["size"]
        if ba < self.L:
            out[2], out[3] = ba, self.slots[self.lv["ask"][ba][0]]["size"]
        return tuple(out)


class NaiveVecMarket:
    """Lock-step collection of NaiveBook with the reference's host TID rule (+2 per call)."""

    def __init__(self, M: int, L: int, O: int, F: int, C: int):
        self.books = [NaiveBook(L, O, F, C) for _ in range(M)]
        self.tid = 0

    def step(self, bid_px, bid_sz, ask_px, ask_sz, cust):
        """Returns (counts, fills) where fills[m] is the list of fill dicts of market m."""
        counts, fills = [], []
        for m, book in enumerate(self.books):
            book.submit("bid", int(bid_px[m]), int(bid_sz[m]), int(cust[m]), self.tid)
            book.submit("ask", int(ask_px[m]), int(ask_sz[m]), int(cust[m]), i32(self.tid + 1))
            out: list = []
            counts.append(book.match(out))
            fills.append(out)
        self.tid = i32(self.tid + 2)
        return counts, fills
