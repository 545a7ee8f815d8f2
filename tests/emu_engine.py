"""The engine's own per-market code, compiled for the host, behind the same C ABI.

``csrc/*.hip`` built with ``-DASTRA_HOST_EMULATION --cuda-host-only`` runs
every kernel body (the same __host__ __device__ functions the GPU runs) as a
plain loop over host memory. ``EmuMarket`` drives that build through the
prototypes of ``astra_cuda._native`` with numpy buffers standing in for device
memory, so the CPU test suite checks the engine's logic, data layout and
bounds against the oracle without a GPU. Test infrastructure only.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
BUILD_DIR = os.path.join(HERE, "_build")
EMU_LIB = os.path.join(BUILD_DIR, "libastra_market_emu.so")
CSRC = os.path.join(ROOT, "astra-cuda_amd", "csrc")
SRCS = [os.path.join(CSRC, f) for f in ("market.hip", "high_low.hip")]
DEPS = SRCS + [os.path.join(CSRC, "runtime.h"), os.path.join(CSRC, "game_move.h"),
               os.path.join(ROOT, "include", "astra_market.h"),
               os.path.join(ROOT, "include", "astra_high_low.h")]

_lib = None


# ASTRA_EMU_SANITIZE=1 builds (and loads) the library with AddressSanitizer and
# UndefinedBehaviorSanitizer on the host code; the Python process must then run
# with the sanitizer runtime preloaded (see sanitize_env()).
SANITIZE = os.environ.get("ASTRA_EMU_SANITIZE", "") not in ("", "0")
if SANITIZE:
    EMU_LIB = os.path.join(BUILD_DIR, "libastra_market_emu_asan.so")
SAN_FLAGS = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
             "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer"]


def sanitize_env() -> dict:
    """Environment for a process that loads the sanitized build: the clang
    AddressSanitizer runtime preloaded (it carries the UBSan handlers too)."""
    from astra_cuda.build import hipcc
    clang = os.path.join(os.path.dirname(os.path.realpath(hipcc())), "..", "llvm", "bin", "clang")
    rt = subprocess.run([clang, "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True,
                        text=True, check=True).stdout.strip()
    return {"LD_PRELOAD": rt, "ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1",
            "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1", "ASTRA_EMU_SANITIZE": "1"}


def build(force: bool = False) -> str:
    if not force and os.path.exists(EMU_LIB) and \
            os.path.getmtime(EMU_LIB) >= max(os.path.getmtime(d) for d in DEPS):
        return EMU_LIB
    os.makedirs(BUILD_DIR, exist_ok=True)
    from astra_cuda.build import hipcc
    tmp = f"{EMU_LIB}.{os.getpid()}.tmp"
    opt = ["-O1", *SAN_FLAGS] if SANITIZE else ["-O2"]
    cmd = [hipcc(), "-DASTRA_HOST_EMULATION", "--cuda-host-only", *opt, "-g", "-std=c++17",
           "-fPIC", "-shared", f"-I{os.path.join(ROOT, 'include')}", *SRCS, "-o", tmp]
    subprocess.run(cmd, check=True, capture_output=True)
    os.replace(tmp, EMU_LIB)  # atomic: parallel test workers each build their own copy
    return EMU_LIB


def lib():
    global _lib
    if _lib is None:
        from astra_cuda._native import PROTOTYPES
        L = ctypes.CDLL(build())
        for name, (res, args) in PROTOTYPES.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        _lib = L
    return _lib


def _check(rc):
    if rc:
        raise RuntimeError("Astra Fatal Error: " + lib().astra_last_error().decode())


def _aligned(nbytes: int) -> np.ndarray:
    raw = np.zeros(nbytes + 256, dtype=np.uint8)
    off = (-raw.ctypes.data) % 256
    return raw[off:off + nbytes]


class EmuFills:
    FIELDS = ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids",
              "fill_is_sell_quote", "fill_quote_sizes", "fill_tid", "fill_quote_tid", "fill_counts")

    def __init__(self, M, F):
        for f in self.FIELDS:
            if f == "fill_counts":
                setattr(self, f, np.zeros((M,), np.int32))
            elif f == "fill_is_sell_quote":
                setattr(self, f, np.zeros((M, F), np.bool_))
            else:
                setattr(self, f, np.zeros((M, F), np.int32))

    def ptrs(self):
        return [getattr(self, f).ctypes.data for f in self.FIELDS]


class EmuRowFills:
    """A FillBatch in the row layout: int32 [M, F, 8] rows plus fill_counts; the
    fields read as views of the rows."""
    FIELDS = EmuFills.FIELDS

    def __init__(self, M, F):
        self.rows = np.zeros((M, F, 8), np.int32)
        self.fill_counts = np.zeros((M,), np.int32)

    def __getattr__(self, name):
        if name in self.FIELDS[:8]:
            v = self.rows[:, :, self.FIELDS.index(name)]
            return v.astype(np.bool_) if name == "fill_is_sell_quote" else v
        raise AttributeError(name)


class EmuBBO:
    FIELDS = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices")

    def __init__(self, M):
        for f in self.FIELDS:
            setattr(self, f, np.zeros((M,), np.int32))


class EmuMarket:
    def __init__(self, M, L, O, F, C, extended=None, _src=None):
        self.M, self.L, self.O, self.F, self.C = M, L, O, F, C
        if extended is None:
            extended = L > 128 or O > 1024 or F > 1024 or C > 1024
        self.flags = 1 if extended else 0
        n = ctypes.c_size_t()
        _check(lib().astra_market_workspace_size(M, L, O, F, C, self.flags, ctypes.byref(n)))
        self.ws = _aligned(max(int(n.value), 256))
        h = ctypes.c_void_p()
        if _src is None:
            _check(lib().astra_market_create(M, L, O, F, C, 0, 64, self.flags, self.ws.ctypes.data,
                                             self.ws.nbytes, None, ctypes.byref(h)))
        else:
            _check(lib().astra_market_clone(_src.h, self.ws.ctypes.data, self.ws.nbytes, None,
                                            ctypes.byref(h)))
        self.h = h
        p = ctypes.c_void_p()
        _check(lib().astra_market_portfolios(self.h, ctypes.byref(p)))
        off = p.value - self.ws.ctypes.data
        self.portfolios = self.ws[off:off + M * C * 8].view(np.int32).reshape(M, C, 2)

    def __del__(self):
        if getattr(self, "h", None):
            lib().astra_market_destroy(self.h)
            self.h = None

    def clone(self):
        return EmuMarket(self.M, self.L, self.O, self.F, self.C, bool(self.flags), _src=self)

    def new_fill_batch(self, layout="columns"):
        return EmuRowFills(self.M, self.F) if layout == "rows" else EmuFills(self.M, self.F)

    def new_bbo_batch(self):
        return EmuBBO(self.M)

    def add_two_sided_quotes(self, bid_px, bid_sz, ask_px, ask_sz, cust, fills):
        ins = [np.ascontiguousarray(a, np.int32) for a in (bid_px, bid_sz, ask_px, ask_sz, cust)]
        if isinstance(fills, EmuRowFills):
            _check(lib().astra_market_add_two_sided_quotes_rows(
                self.h, *[a.ctypes.data for a in ins], fills.rows.ctypes.data, fills.fill_counts.ctypes.data,
                None))
            return
        _check(lib().astra_market_add_two_sided_quotes(self.h, *[a.ctypes.data for a in ins],
                                                        *fills.ptrs(), None))

    def add_two_sided_quotes_steps(self, bid_px, bid_sz, ask_px, ask_sz, cust, fills,
                                   step_counts=None, step_bbos=None):
        ins = [np.ascontiguousarray(a, np.int32) for a in (bid_px, bid_sz, ask_px, ask_sz, cust)]
        steps = ins[0].shape[0]
        if isinstance(fills, EmuRowFills):
            fields, rows, counts = [None] * 8, fills.rows.ctypes.data, fills.fill_counts.ctypes.data
        else:
            p = fills.ptrs()
            fields, rows, counts = p[:8], None, p[8]
        _check(lib().astra_market_add_two_sided_quotes_steps(
            self.h, steps, *[a.ctypes.data for a in ins], *fields, rows, counts,
            None if step_counts is None else step_counts.ctypes.data,
            None if step_bbos is None else step_bbos.ctypes.data, None))

    def get_bbos(self, b):
        _check(lib().astra_market_get_bbos(self.h, b.best_bid_prices.ctypes.data,
                                           b.best_bid_sizes.ctypes.data, b.best_ask_prices.ctypes.data,
                                           b.best_ask_sizes.ctypes.data, None))

    def update_last_prices(self, b, fills):
        if isinstance(fills, EmuRowFills):
            _check(lib().astra_update_last_prices_rows(b.last_prices.ctypes.data, fills.fill_counts.ctypes.data,
                                                       fills.rows.ctypes.data, self.M, self.F, None))
            return
        _check(lib().astra_update_last_prices(b.last_prices.ctypes.data, fills.fill_counts.ctypes.data,
                                              fills.fill_prices.ctypes.data, self.M, self.F, None))

    def reset(self):
        _check(lib().astra_market_reset(self.h, None))

    def clear_quotes(self, mask):
        m = np.ascontiguousarray(mask, np.bool_)
        _check(lib().astra_market_clear_quotes(self.h, m.ctypes.data, None))

    def to_string(self, market_id):
        need = ctypes.c_size_t()
        buf = ctypes.create_string_buffer(1 << 16)
        _check(lib().astra_market_to_string(self.h, int(market_id), buf, 1 << 16, ctypes.byref(need), None))
        if need.value >= (1 << 16):
            buf = ctypes.create_string_buffer(need.value + 1)
            _check(lib().astra_market_to_string(self.h, int(market_id), buf, need.value + 1,
                                                ctypes.byref(need), None))
        return buf.value.decode()

    def set_stats(self, counters):
        _check(lib().astra_market_set_stats(self.h, None if counters is None else counters.ctypes.data))

    @property
    def global_tid(self):
        v = ctypes.c_int32()
        _check(lib().astra_market_get_tid(self.h, ctypes.byref(v), None))
        return v.value


class EmuAdapter:
    """KAT adapter (tests/kat_harness.py) over the emulation build."""

    layout = "columns"

    def __init__(self, shape):
        self.mk = EmuMarket(shape["M"], shape["L"], shape["O"], shape["F"], shape["C"])
        self.fills = self.mk.new_fill_batch(self.layout)
        self.bbo = self.mk.new_bbo_batch()

    def quote(self, *args):
        self.mk.add_two_sided_quotes(*args, self.fills)

    def bbos(self):
        self.mk.get_bbos(self.bbo)

    def update_last(self):
        self.mk.update_last_prices(self.bbo, self.fills)

    def reset(self):
        self.mk.reset()

    def bbo_reset(self):
        for f in EmuBBO.FIELDS:
            getattr(self.bbo, f)[:] = 0

    def new_bbo(self):
        self.bbo = self.mk.new_bbo_batch()

    def array(self, name):
        if name == "portfolio":
            return self.mk.portfolios.copy()
        if name in EmuBBO.FIELDS:
            return getattr(self.bbo, name).copy()
        return np.array(getattr(self.fills, name))

    def to_string(self, m):
        return self.mk.to_string(m)


class EmuRowAdapter(EmuAdapter):
    layout = "rows"


class EmuHighLow:
    """The high-low game's move kernels (csrc/high_low.hip) on the emulation build,
    with numpy arrays as the state tensors (high_low_trading.h:85-115). The setup
    arrays (contract values, settle flags, permutation, targets) are set directly."""

    def __init__(self, N, P, T, S, cM, V, market_shape, layout="columns"):
        from astra_cuda._native import HLObservation, HLTrade
        self.N, self.P, self.T, self.S, self.cM, self.V = N, P, T, S, cM, V
        L, O, F, C = market_shape
        self.market = EmuMarket(N, L, O, F, C)
        self.fills = self.market.new_fill_batch(layout)
        self.bbo = self.market.new_bbo_batch()
        z = lambda *s: np.zeros(s, np.int32)  # noqa: E731
        self.contract_values = z(N, 3)
        self.contract_high_settle = np.zeros(N, np.uint8)
        self.player_permutation = z(N, P)
        self.target_positions = z(N, P)
        self.player_last_positions = z(N, P, 2)
        self._pcot = z(T, P, 6, N)  # env-minor, as the C ABI keeps it
        self._mcot = z(P * T, 3, N)  # env-minor, as the C ABI keeps it
        self.immediate_rewards = z(N, P)
        self.rewards_since_last_action = z(N, P)
        self.errors = z(1)
        self.errors_host = z(1)
        self._HLTrade, self._HLObservation = HLTrade, HLObservation

    @property
    def player_contract_over_time(self):
        """[N,P,T,6] view of the env-minor [T,P,6,N] storage."""
        return np.transpose(self._pcot, (3, 1, 0, 2))

    @property
    def market_contract_over_time(self):
        """[N,P*T,3] view of the env-minor [P*T,3,N] storage."""
        return np.transpose(self._mcot, (2, 0, 1))

    def trade(self, move, player, tmn, check=1, entry="astra_high_low_trade"):
        self.move = np.ascontiguousarray(move, np.int32)
        t = self._HLTrade()
        ptr = lambda a: a.ctypes.data  # noqa: E731
        for name in ("player_last_positions", "target_positions", "contract_values",
                     "immediate_rewards", "rewards_since_last_action", "errors", "errors_host"):
            a = getattr(self, name)
            setattr(t, name, None if a is None else ptr(a))
        t.player_contract_over_time = ptr(self._pcot)
        t.market_contract_over_time = ptr(self._mcot)
        t.move = ptr(self.move)
        if isinstance(self.fills, EmuRowFills):
            t.fill_rows, t.fill_counts = ptr(self.fills.rows), ptr(self.fills.fill_counts)
        else:
            for f in EmuFills.FIELDS:
                setattr(t, f, ptr(getattr(self.fills, f)))
        for f in EmuBBO.FIELDS:
            setattr(t, f, ptr(getattr(self.bbo, f)))
        t.players, t.steps_per_player = self.P, self.T
        t.max_contracts_per_trade, t.max_contract_value = self.S, self.V
        t.player, t.trade_move_number, t.check = player, tmn, check
        return getattr(lib(), entry)(self.market.h, ctypes.byref(t), None)

    def observation(self, player, current_round):
        import math
        v = np.zeros((self.N, 6 + 1 + 6 * self.P + 5), np.float32)
        o = self._HLObservation()
        ptr = lambda a: a.ctypes.data  # noqa: E731
        o.values = ptr(v)
        o.player_permutation = ptr(self.player_permutation)
        o.contract_values = ptr(self.contract_values)
        o.contract_high_settle = ptr(self.contract_high_settle)
        o.target_positions = ptr(self.target_positions)
        o.player_contract_over_time = ptr(self._pcot)
        o.best_bid_prices, o.best_ask_prices = ptr(self.bbo.best_bid_prices), ptr(self.bbo.best_ask_prices)
        o.best_bid_sizes, o.best_ask_sizes = ptr(self.bbo.best_bid_sizes), ptr(self.bbo.best_ask_sizes)
        o.last_prices = ptr(self.bbo.last_prices)
        o.num_envs, o.players, o.steps_per_player = self.N, self.P, self.T
        o.player, o.current_round = player, current_round
        angle = 2.0 * math.pi * player / self.P
        o.player_sin, o.player_cos = float(np.float32(math.sin(angle))), float(np.float32(math.cos(angle)))
        o.round_fraction = float(np.float32(current_round) / np.float32(self.T))
        _check(lib().astra_high_low_observation(ctypes.byref(o), None))
        return v
