"""``astra_cuda.order_matching`` -- drop-in for the reference pybind submodule.

Mirrors nlyu1/astra-cuda src/pybind/order_matching/market_bindings.cc:14-73
(``VecMarket``, ``FillBatch``, ``BBOBatch`` and the six constants) and the C++
surface the reference game also uses (``Reset``, ``ClearQuotes``,
``CopyCustomerPortfoliosTo``, the copy constructor, ``FillBatch::Reset``,
``BBOBatch::Reset`` / ``UpdateLastPrices``; market.h:64-350). All tensors are
PyTorch-ROCm tensors on the engine's device; every computation runs in the HIP
kernels of ``libastra_market.so`` on the caller's current stream, and no call
synchronises except ``to_string``.

Errors follow the reference's AstraFatalError convention
(src/utils/astra_utils.cc:13-18): the message is printed to stderr and raised
as ``RuntimeError("Astra Fatal Error: ...")``.
"""
from __future__ import annotations

import ctypes
import sys

import torch

from . import _native

# market.h:56-61 (exposed at market_bindings.cc:67-72)
MAX_MARKETS = 2048 * 2048
PRICE_LEVELS = 128
MAX_ACTIVE_ORDERS_PER_MARKET = 1024
MAX_ACTIVE_FILLS_PER_MARKET = 1024
NULL_INDEX = -1
MAX_CUSTOMERS = 1024

_FLAG_EXTENDED_SHAPES = 1

try:
    _raw_stream = torch._C._cuda_getCurrentRawStream
except AttributeError:  # pragma: no cover - older torch
    def _raw_stream(index):
        return torch.cuda.current_stream(index).cuda_stream


def _fatal(msg: str):
    """AstraFatalError: print to stderr, raise RuntimeError."""
    text = "Astra Fatal Error: " + msg
    print(text + "\n", file=sys.stderr, flush=True)
    raise RuntimeError(text)


def _check(rc: int) -> None:
    if rc != 0:
        _fatal(_native.last_error())


def _device_index(device) -> int:
    if isinstance(device, torch.device):
        return 0 if device.index is None else int(device.index)
    if isinstance(device, str):
        d = torch.device(device)
        return 0 if d.index is None else int(d.index)
    return int(device)


def _ptr(t):
    return t.data_ptr()


class FillBatch:
    """Per-market fills of one call (market.h:64-92), reused across calls.

    ``fill_prices, fill_sizes, fill_customer_ids`` (taker), ``fill_quoter_ids``,
    ``fill_quote_sizes``, ``fill_tid`` (taker), ``fill_quote_tid``: int32
    ``[M, F]``; ``fill_is_sell_quote``: bool ``[M, F]``; ``fill_counts``: int32
    ``[M]`` (``-1`` marks a market that ran out of fill slots). Only
    ``[m, :fill_counts[m]]`` is written by a call; later entries keep older values.

    Layout: by default (``"columns"``) each field is its own contiguous tensor, as in
    the reference. ``VecMarket.new_fill_batch(layout="rows")`` keeps the eight
    per-row fields side by side in one int32 ``[M, F, 8]`` buffer and exposes them
    as strided ``[M, F]`` views with the same values (a row is then one 32-byte
    write for the engine); assigning a field replaces the layout by "columns".
    """

    FIELDS = ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids",
              "fill_is_sell_quote", "fill_quote_sizes", "fill_tid", "fill_quote_tid",
              "fill_counts")
    __slots__ = FIELDS + ("_pack", "_rows")

    def __init__(self):
        for f in self.FIELDS:
            object.__setattr__(self, f, None)
        object.__setattr__(self, "_pack", None)
        object.__setattr__(self, "_rows", None)

    def __setattr__(self, name, value):
        object.__setattr__(self, name, value)
        if name in FillBatch.FIELDS:
            object.__setattr__(self, "_pack", None)
            if name != "fill_counts":
                object.__setattr__(self, "_rows", None)

    def _set_rows(self, rows: torch.Tensor, counts: torch.Tensor) -> None:
        """Point the eight row fields at views of ``rows`` (int32 [M, F, 8])."""
        for i, f in enumerate(self.FIELDS[:8]):
            v = rows.view(torch.uint8)[:, :, 16].view(torch.bool) if f == "fill_is_sell_quote" else rows[:, :, i]
            object.__setattr__(self, f, v)
        object.__setattr__(self, "fill_counts", counts)
        object.__setattr__(self, "_rows", rows)
        object.__setattr__(self, "_pack", None)

    @property
    def layout(self) -> str:
        return "rows" if self._rows is not None else "columns"

    def _pointers(self, M: int, F: int, device: torch.device):
        """Validated device pointers (cached until a field is reassigned): the nine
        fields, or ("rows", rows, fill_counts) for the row layout."""
        pack = self._pack
        if pack is not None and pack[0] == (M, F, device):
            return pack[1]
        rows = self._rows
        if rows is not None:
            fc = self.fill_counts
            if tuple(rows.shape) != (M, F, 8) or rows.dtype != torch.int32 or not rows.is_contiguous():
                _fatal(f"fills row buffer must be int32 [{M}, {F}, 8]")
            if not isinstance(fc, torch.Tensor) or tuple(fc.shape) != (M,) or fc.dtype != torch.int32 \
                    or not fc.is_contiguous():
                _fatal(f"fills.fill_counts must be a contiguous int32 tensor of shape [{M}]")
            if rows.device != device or fc.device != device:
                _fatal(f"fills tensors must be on device {device.index}")
            ptrs = ("rows", rows.data_ptr(), fc.data_ptr())
            object.__setattr__(self, "_pack", ((M, F, device), ptrs))
            return ptrs
        ptrs = []
        for f in self.FIELDS:
            t = getattr(self, f)
            if not isinstance(t, torch.Tensor):
                _fatal(f"fills.{f} is not a tensor")
            shape = (M,) if f == "fill_counts" else (M, F)
            dtype = torch.bool if f == "fill_is_sell_quote" else torch.int32
            if tuple(t.shape) != shape or t.dtype != dtype:
                _fatal(f"fills.{f} must be {dtype} of shape {list(shape)}, got {t.dtype} {list(t.shape)}")
            if t.device != device:
                _fatal(f"fills.{f} tensor must be on device {device.index}")
            if not t.is_contiguous():
                _fatal(f"fills.{f} tensor must be contiguous")
            ptrs.append(t.data_ptr())
        ptrs = tuple(ptrs)
        object.__setattr__(self, "_pack", ((M, F, device), ptrs))
        return ptrs

    def reset(self) -> None:
        """FillBatch::Reset (market.cu:758-760): fill_counts to 0."""
        fc = self.fill_counts
        with torch.cuda.device(fc.device):
            _check(_native.lib().astra_fill_i32(fc.data_ptr(), fc.numel(), 0,
                                                _raw_stream(fc.device.index)))

    Reset = reset

    def clone(self) -> "FillBatch":
        """Copy constructor (market.h:80-89): every tensor cloned (the layout kept)."""
        out = FillBatch()
        if self._rows is not None:
            out._set_rows(self._rows.clone(), self.fill_counts.clone())
            return out
        for f in self.FIELDS:
            setattr(out, f, getattr(self, f).clone())
        return out

    __copy__ = clone

    def __deepcopy__(self, memo):
        return self.clone()


class BBOBatch:
    """Best bid/offer per market (market.h:95-119): int32 ``[M]`` tensors.

    ``last_prices`` is C++-only in the reference binding (market_bindings.cc:18-22);
    it is exposed here as well, with ``reset()`` and ``update_last_prices()``.
    """

    FIELDS = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes")
    __slots__ = FIELDS + ("last_prices", "_pack")

    def __init__(self):
        for f in self.FIELDS + ("last_prices",):
            object.__setattr__(self, f, None)
        object.__setattr__(self, "_pack", None)

    def __setattr__(self, name, value):
        object.__setattr__(self, name, value)
        if name in BBOBatch.FIELDS:
            object.__setattr__(self, "_pack", None)

    def _pointers(self, M: int, device: torch.device):
        pack = self._pack
        if pack is not None and pack[0] == (M, device):
            return pack[1]
        ptrs = []
        for f in self.FIELDS:
            t = getattr(self, f)
            if not isinstance(t, torch.Tensor) or tuple(t.shape) != (M,) or t.dtype != torch.int32:
                _fatal(f"bbos.{f} must be an int32 tensor of shape [{M}]")
            if t.device != device:
                _fatal(f"bbos.{f} tensor must be on device {device.index}")
            if not t.is_contiguous():
                _fatal(f"bbos.{f} tensor must be contiguous")
            ptrs.append(t.data_ptr())
        ptrs = tuple(ptrs)
        object.__setattr__(self, "_pack", ((M, device), ptrs))
        return ptrs

    def reset(self) -> None:
        """BBOBatch::Reset (market.cu:788-796): all five tensors to 0."""
        for f in self.FIELDS + ("last_prices",):
            t = getattr(self, f)
            with torch.cuda.device(t.device):
                _check(_native.lib().astra_fill_i32(t.data_ptr(), t.numel(), 0,
                                                    _raw_stream(t.device.index)))

    Reset = reset

    def update_last_prices(self, fills: FillBatch) -> None:
        """BBOBatch::UpdateLastPrices (market.cu:798-825): last fill price where count > 0."""
        lp, fc, fp = self.last_prices, fills.fill_counts, fills.fill_prices
        if fills._rows is not None:
            rows = fills._rows
            M, F = int(rows.shape[0]), int(rows.shape[1])
            if rows.device != lp.device or fc.device != lp.device or lp.shape[0] != M:
                _fatal("UpdateLastPrices: fills and last_prices must match in device and markets")
            with torch.cuda.device(lp.device):
                _check(_native.lib().astra_update_last_prices_rows(
                    lp.data_ptr(), fc.data_ptr(), rows.data_ptr(), M, F, _raw_stream(lp.device.index)))
            return
        if fc.device != lp.device:  # market.cu:801-802
            _fatal(f"fills.fill_counts.device() == last_prices.device()\n"
                   f"fills.fill_counts.device() = {fc.device}, last_prices.device() = {lp.device}")
        if fp.device != lp.device:
            _fatal(f"fills.fill_prices.device() == last_prices.device()\n"
                   f"fills.fill_prices.device() = {fp.device}, last_prices.device() = {lp.device}")
        M, F = int(fc.shape[0]), int(fp.shape[1])
        for t, dt in ((lp, torch.int32), (fc, torch.int32), (fp, torch.int32)):
            if t.dtype != dt or not t.is_contiguous():
                _fatal("UpdateLastPrices needs contiguous int32 tensors")
        if lp.shape[0] != M or fp.shape[0] != M:
            _fatal("UpdateLastPrices: inconsistent number of markets")
        with torch.cuda.device(lp.device):
            _check(_native.lib().astra_update_last_prices(lp.data_ptr(), fc.data_ptr(), fp.data_ptr(),
                                                          M, F, _raw_stream(lp.device.index)))

    UpdateLastPrices = update_last_prices

    def clone(self) -> "BBOBatch":
        """Copy constructor (market.h:107-112)."""
        out = BBOBatch()
        for f in self.FIELDS + ("last_prices",):
            setattr(out, f, getattr(self, f).clone())
        return out

    __copy__ = clone

    def __deepcopy__(self, memo):
        return self.clone()


class VecMarket:
    """Vectorised double-auction markets on one MI355X (market.h:121-350).

    ``VecMarket(num_markets, max_price_levels, max_active_orders_per_market,
    max_active_fills_per_market, num_customers=16, device_id=0,
    threads_per_block=64)`` with the reference's keyword names
    (market_bindings.cc:36-43). ``device`` is accepted as an alias of
    ``device_id``. ``allow_extended_shapes=True`` lifts the reference caps
    (L <= 128, O <= 1024, F <= 1024, C <= 1024) to L <= 1024, O <= 32768,
    F <= 65536, C <= 65536; without it, the reference's checks apply.
    ``threads_per_block`` is validated (0 < tpb <= 1024) and, as in the
    reference, does not change any result.
    """

    def __init__(self, num_markets, max_price_levels, max_active_orders_per_market,
                 max_active_fills_per_market, num_customers=16, device_id=0,
                 threads_per_block=64, *, device=None, allow_extended_shapes=False,
                 _clone_of=None):
        self._h = None
        lib = _native.lib()
        if device is not None:
            device_id = _device_index(device)
        self._M = int(num_markets)
        self._L = int(max_price_levels)
        self._O = int(max_active_orders_per_market)
        self._F = int(max_active_fills_per_market)
        self._C = int(num_customers)
        self._device_index = int(device_id)
        self._tpb = int(threads_per_block)
        self._flags = _FLAG_EXTENDED_SHAPES if allow_extended_shapes else 0
        nbytes = ctypes.c_size_t(0)
        _check(lib.astra_market_workspace_size(self._M, self._L, self._O, self._F, self._C,
                                               self._flags, ctypes.byref(nbytes)))
        ndev = torch.cuda.device_count()
        if not 0 <= self._device_index < ndev:  # market.cu:349-350
            _fatal(f"order_matching.py device_id < device_count\n"
                   f"device_id = {self._device_index}, device_count = {ndev}")
        self._device = torch.device("cuda", self._device_index)
        with torch.cuda.device(self._device):
            self._ws = torch.empty(max(int(nbytes.value), 256), dtype=torch.uint8, device=self._device)
            stream = _raw_stream(self._device_index)
            h = ctypes.c_void_p()
            if _clone_of is None:
                _check(lib.astra_market_create(self._M, self._L, self._O, self._F, self._C,
                                               self._device_index, self._tpb, self._flags,
                                               self._ws.data_ptr(), self._ws.numel(), stream,
                                               ctypes.byref(h)))
            else:
                _check(lib.astra_market_clone(_clone_of._h, self._ws.data_ptr(), self._ws.numel(),
                                              stream, ctypes.byref(h)))
        self._h = h
        pf = ctypes.c_void_p()
        _check(lib.astra_market_portfolios(self._h, ctypes.byref(pf)))
        off = int(pf.value) - self._ws.data_ptr()
        n = self._M * self._C * 2 * 4
        self._portfolios = self._ws[off:off + n].view(torch.int32).view(self._M, self._C, 2)
        self._lib = lib

    # -- lifetime ----------------------------------------------------------

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                self._lib.astra_market_destroy(h)  # syncs the device (market.cu:413-418)
            except Exception:
                pass
            self._h = None

    def clone(self) -> "VecMarket":
        """Deep copy (copy constructor, market.cu:385-411), TID counter included."""
        return VecMarket(self._M, self._L, self._O, self._F, self._C, self._device_index, self._tpb,
                         allow_extended_shapes=bool(self._flags), _clone_of=self)

    __copy__ = clone

    def __deepcopy__(self, memo):
        return self.clone()

    # -- batches -----------------------------------------------------------

    def new_fill_batch(self, layout: str = "columns") -> FillBatch:
        """NewFillBatch (market.cu:420-439): zero-initialised tensors. ``layout="rows"``
        (not in the reference) stores the eight row fields in one [M, F, 8] buffer
        and exposes strided views of it (see FillBatch)."""
        b = FillBatch()
        M, F, dev = self._M, self._F, self._device
        if layout == "rows":
            b._set_rows(torch.zeros((M, F, 8), dtype=torch.int32, device=dev),
                        torch.zeros((M,), dtype=torch.int32, device=dev))
            return b
        if layout != "columns":
            _fatal(f"unknown fill batch layout {layout!r} (columns or rows)")
        for f in FillBatch.FIELDS:
            if f == "fill_counts":
                setattr(b, f, torch.zeros((M,), dtype=torch.int32, device=dev))
            elif f == "fill_is_sell_quote":
                setattr(b, f, torch.zeros((M, F), dtype=torch.bool, device=dev))
            else:
                setattr(b, f, torch.zeros((M, F), dtype=torch.int32, device=dev))
        return b

    def new_bbo_batch(self) -> BBOBatch:
        """NewBBOBatch (market.cu:441-456): all five tensors zero (not NULL)."""
        b = BBOBatch()
        for f in BBOBatch.FIELDS + ("last_prices",):
            setattr(b, f, torch.zeros((self._M,), dtype=torch.int32, device=self._device))
        return b

    # -- hot path ----------------------------------------------------------

    def add_two_sided_quotes(self, bid_px, bid_sz, ask_px, ask_sz, customer_ids, fills):
        """AddTwoSidedQuotes + MatchAllMarkets (market.cu:458-571).

        Inputs are int32 ``[M]`` contiguous tensors on the engine's device. Each
        market inserts its bid (TID = counter) and then its ask (TID = counter+1)
        when ``size > 0`` and ``0 <= price < L``, matches, and writes the fills;
        the TID counter then advances by 2. Asynchronous.
        """
        M = self._M
        names = ("bid_px", "bid_sz", "ask_px", "ask_sz", "customer_ids")
        ts = (bid_px, bid_sz, ask_px, ask_sz, customer_ids)
        for name, t in zip(names, ts):  # market.cu:467-471
            if t.size(0) != M:
                _fatal(f"order_matching.py {name}.size(0) == num_markets_\n"
                       f"{name}.size(0) = {t.size(0)}, num_markets_ = {M}")
        dev = self._device
        for name, t in zip(names, ts):  # market.cu:474-504
            if t.device != dev:
                _fatal(f"{name} tensor must be on device {self._device_index}")
            if not t.is_contiguous():
                _fatal(f"{name} tensor must be contiguous")
            if t.dtype != torch.int32:
                _fatal(f"{name} tensor must be int32, got {t.dtype}")
        fp = fills._pointers(M, self._F, dev)
        if fp[0] == "rows":
            rc = self._lib.astra_market_add_two_sided_quotes_rows(
                self._h, bid_px.data_ptr(), bid_sz.data_ptr(), ask_px.data_ptr(), ask_sz.data_ptr(),
                customer_ids.data_ptr(), fp[1], fp[2], _raw_stream(self._device_index))
        else:
            rc = self._lib.astra_market_add_two_sided_quotes(
                self._h, bid_px.data_ptr(), bid_sz.data_ptr(), ask_px.data_ptr(), ask_sz.data_ptr(),
                customer_ids.data_ptr(), *fp, _raw_stream(self._device_index))
        if rc:
            _fatal(_native.last_error())

    AddTwoSidedQuotes = add_two_sided_quotes

    def add_two_sided_quotes_steps(self, bid_px, bid_sz, ask_px, ask_sz, customer_ids, fills,
                                   step_fill_counts=None, step_bbos=None) -> None:
        """``steps`` consecutive add_two_sided_quotes calls in one launch (not in the
        reference): the inputs are int32 ``[steps, M]`` tensors, row k being step k's
        quotes. Afterwards the engine, ``fills`` and the BBOs that get_bbos reads are
        exactly as after the single calls. ``step_fill_counts`` (int32 ``[steps, M]``)
        receives every step's fill counts and ``step_bbos`` (int32 ``[4, steps, M]``:
        best bid price, bid size, ask price, ask size) every step's get_bbos.
        Asynchronous."""
        M = self._M
        names = ("bid_px", "bid_sz", "ask_px", "ask_sz", "customer_ids")
        ts = (bid_px, bid_sz, ask_px, ask_sz, customer_ids)
        if bid_px.dim() != 2:
            _fatal("order_matching.py bid_px must be [steps, num_markets]")
        steps = bid_px.size(0)
        dev = self._device
        for name, t in zip(names, ts):
            if tuple(t.shape) != (steps, M):
                _fatal(f"order_matching.py {name} must be [{steps}, {M}], got {list(t.shape)}")
            if t.device != dev:
                _fatal(f"{name} tensor must be on device {self._device_index}")
            if not t.is_contiguous():
                _fatal(f"{name} tensor must be contiguous")
            if t.dtype != torch.int32:
                _fatal(f"{name} tensor must be int32, got {t.dtype}")
        for name, t, shape in (("step_fill_counts", step_fill_counts, (steps, M)),
                               ("step_bbos", step_bbos, (4, steps, M))):
            if t is None:
                continue
            if tuple(t.shape) != shape or t.dtype != torch.int32 or not t.is_contiguous() \
                    or t.device != dev:
                _fatal(f"{name} must be a contiguous int32 tensor of shape {list(shape)} on device "
                       f"{self._device_index}")
        fp = fills._pointers(M, self._F, dev)
        if fp[0] == "rows":
            fields, rows, counts = (None,) * 8, fp[1], fp[2]
        else:
            fields, rows, counts = fp[:8], None, fp[8]
        rc = self._lib.astra_market_add_two_sided_quotes_steps(
            self._h, steps, *(t.data_ptr() for t in ts), *fields, rows, counts,
            None if step_fill_counts is None else step_fill_counts.data_ptr(),
            None if step_bbos is None else step_bbos.data_ptr(), _raw_stream(self._device_index))
        if rc:
            _fatal(_native.last_error())

    def get_bbos(self, bbos: BBOBatch) -> None:
        """GetBBOs (market.cu:573-597): best level and its head order's size per side,
        ``(NULL_INDEX, 0)`` for an empty side. Asynchronous."""
        bp = bbos._pointers(self._M, self._device)
        rc = self._lib.astra_market_get_bbos(self._h, *bp, _raw_stream(self._device_index))
        if rc:
            _fatal(_native.last_error())

    GetBBOs = get_bbos

    # -- the rest of the reference surface ------------------------------------

    def to_string(self, market_id: int) -> str:
        """ToString (market.cu:599-691); synchronises the current stream."""
        lib = self._lib
        need = ctypes.c_size_t(0)
        cap = 1 << 16
        while True:
            buf = ctypes.create_string_buffer(cap)
            _check(lib.astra_market_to_string(self._h, int(market_id), buf, cap, ctypes.byref(need),
                                              _raw_stream(self._device_index)))
            if need.value < cap:
                return buf.value.decode()
            cap = int(need.value) + 1

    ToString = to_string

    def get_customer_portfolios(self) -> torch.Tensor:
        """Live int32 ``[M, C, 2]`` view (contracts, cash) of the portfolios (market.h:294-296)."""
        return self._portfolios

    GetCustomerPortfolios = get_customer_portfolios

    def copy_customer_portfolios_to(self, buffer: torch.Tensor) -> None:
        """CopyCustomerPortfoliosTo (market.h:285-292): blocking copy into ``buffer``."""
        for got, exp, what in ((buffer.dim(), 3, "buffer.dim()"), (buffer.size(0), self._M, "buffer.size(0)"),
                               (buffer.size(1), self._C, "buffer.size(1)"), (buffer.size(2), 2, "buffer.size(2)")):
            if got != exp:
                _fatal(f"order_matching.py {what} == {exp}\n{what} = {got}")
        buffer.copy_(self._portfolios, non_blocking=False)

    CopyCustomerPortfoliosTo = copy_customer_portfolios_to

    def reset(self) -> None:
        """Reset (market.cu:693-716): empty books, zero portfolios, TID counter 0."""
        with torch.cuda.device(self._device):
            _check(self._lib.astra_market_reset(self._h, _raw_stream(self._device_index)))

    Reset = reset

    def clear_quotes(self, reset_indices: torch.Tensor) -> None:
        """ClearQuotes (market.cu:718-756): empty the books of the selected markets;
        portfolios and the TID counter are kept."""
        r = reset_indices
        if r.dim() != 1:
            _fatal(f"order_matching.py reset_indices.dim() == 1\nreset_indices.dim() = {r.dim()}, 1 = 1")
        if r.size(0) != self._M:
            _fatal(f"order_matching.py reset_indices.size(0) == num_markets_\n"
                   f"reset_indices.size(0) = {r.size(0)}, num_markets_ = {self._M}")
        if r.dtype != torch.bool:
            _fatal(f"order_matching.py reset_indices.dtype() == torch::kBool\n"
                   f"reset_indices.dtype() = {r.dtype}, torch::kBool = torch.bool")
        if r.device != self._device:
            _fatal(f"reset_indices tensor must be on device {self._device_index}")
        r = r.contiguous()
        with torch.cuda.device(self._device):
            _check(self._lib.astra_market_clear_quotes(self._h, r.data_ptr(),
                                                       _raw_stream(self._device_index)))

    ClearQuotes = clear_quotes

    # -- introspection (not in the reference binding) -------------------------

    def _set_stats(self, counters) -> None:
        """Diagnostic: accumulate per-call work counts into an int64 [11] device tensor
        (inserts, fill rows, emptied levels, overflowed markets, fast-forwarded
        overflows, loop passes, staged markets, crossing markets, zero-size runs
        listed on a staged book and their rows, best levels whose head size the
        next get_bbos reads from the book); None switches it off."""
        if counters is None:
            _check(self._lib.astra_market_set_stats(self._h, None))
            return
        if (counters.dtype != torch.int64 or counters.numel() < 11 or counters.device != self._device
                or not counters.is_contiguous()):
            _fatal("stats counters must be a contiguous int64 tensor of >= 11 elements on the engine's device")
        self._stats_ref = counters
        _check(self._lib.astra_market_set_stats(self._h, counters.data_ptr()))

    @property
    def num_markets(self) -> int:
        return self._M

    @property
    def global_tid(self) -> int:
        """The TID counter (market.h:338): base TID of the next call. It lives in
        device memory (the matching kernel moves it on), so reading it
        synchronises the current stream."""
        v = ctypes.c_int32(0)
        with torch.cuda.device(self._device):
            _check(self._lib.astra_market_get_tid(self._h, ctypes.byref(v), _raw_stream(self._device_index)))
        return int(v.value)

    @global_tid.setter
    def global_tid(self, tid: int) -> None:
        with torch.cuda.device(self._device):
            _check(self._lib.astra_market_set_tid(self._h, int(tid), _raw_stream(self._device_index)))
