"""The committed config-1 digest (tests/golden/config1_digest.json) against the
oracle and the host-emulated engine (CPU), and against the HIP engine (GPU)."""
import json
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from make_config1_digest import BBO, DUMP_STEPS, FIELDS, run, step_digest, step_dump  # noqa: E402

GOLDEN = json.load(open(os.path.join(HERE, "golden", "config1_digest.json")))["steps"]
DUMPS = {d["step"]: d for d in json.load(open(os.path.join(HERE, "golden", "config1_dumps.json")))["dumps"]}


def test_oracle_reproduces_config1_digest():
    dumps = []
    assert run(dumps=dumps) == GOLDEN
    assert sorted(DUMPS) == list(DUMP_STEPS)
    for d in dumps:
        assert d == DUMPS[d["step"]], d["step"]


def test_config1_dumps_match_their_digests():
    """The full dumps and the digests were written from the same run."""
    from astra_cuda.workloads import CONFIGS
    F = CONFIGS[1].F
    for t, d in DUMPS.items():
        counts = np.array(d["fill_counts"], np.int32)
        M = counts.shape[0]
        fills = {f: np.zeros((M, F), np.int32) for f in FIELDS}
        for m, rows in d["rows"].items():
            r = np.array(rows, np.int32)
            for i, f in enumerate(FIELDS):
                fills[f][int(m), :len(r)] = r[:, i]
        bbo = {f: np.array(v, np.int32) for f, v in d["bbo"].items()}
        assert step_digest(counts, fills, bbo, np.array(d["portfolios"], np.int32), F) == GOLDEN[t], t


def _drive(mk, fills, bbo, arrays, steps=None):
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[1]
    qs = QuoteStream(cfg)
    out = []
    for t in range(cfg.steps if steps is None else steps):
        arrays["quote"](qs.step(t))
        arrays["after"]()
        f, b, pf = arrays["read"]()
        out.append(step_digest(f["fill_counts"], f, b, pf, cfg.F))
        if t in DUMPS:  # in full, so a mismatch names its field and market
            d = step_dump(t, f["fill_counts"], f, b, pf, cfg.F)
            for key in ("fill_counts", "rows", "bbo", "portfolios"):
                assert d[key] == DUMPS[t][key], (t, key)
        if out[-1] != GOLDEN[t]:
            raise AssertionError(f"step {t}: digest {out[-1]} != golden {GOLDEN[t]}")
    return out


def test_emulated_engine_reproduces_config1_digest():
    from astra_cuda.workloads import CONFIGS
    from emu_engine import EmuMarket
    cfg = CONFIGS[1]
    em = EmuMarket(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C)
    ef, eb = em.new_fill_batch(), em.new_bbo_batch()

    def after():
        em.update_last_prices(eb, ef)
        em.get_bbos(eb)

    def read():
        f = {k: getattr(ef, k) for k in FIELDS + ("fill_counts",)}
        return f, {k: getattr(eb, k) for k in BBO}, em.portfolios

    _drive(em, ef, eb, {"quote": lambda a: em.add_two_sided_quotes(*a, ef), "after": after, "read": read})


@pytest.mark.gpu
def test_gpu_engine_reproduces_config1_digest():
    import torch
    from astra_cuda import order_matching as aom
    from astra_cuda.workloads import CONFIGS
    cfg = CONFIGS[1]
    print("config 1 digest on the GPU", flush=True)
    g = aom.VecMarket(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C)
    gf, gb = g.new_fill_batch(), g.new_bbo_batch()

    def quote(a):
        g.add_two_sided_quotes(*(torch.as_tensor(np.ascontiguousarray(x)).to("cuda:0") for x in a), gf)

    def after():
        gb.update_last_prices(gf)
        g.get_bbos(gb)

    def read():
        f = {k: getattr(gf, k).cpu().numpy() for k in FIELDS + ("fill_counts",)}
        b = {k: getattr(gb, k).cpu().numpy() for k in BBO}
        return f, b, g.get_customer_portfolios().cpu().numpy()

    _drive(g, gf, gb, {"quote": quote, "after": after, "read": read})
