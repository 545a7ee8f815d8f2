"""Write tests/golden/config1_digest.json: a per-step digest of every output of
the config-1 run (64 markets x 1000 steps) on the oracle, and
tests/golden/config1_dumps.json: every output in full at a few steps.

Per step: SHA-256 (first 16 hex digits) over fill_counts, the rows each market
wrote (k < count, or F for an overflowed market) of all eight fill fields, the
four BBO arrays after get_bbos, last prices after update_last_prices, and the
portfolios. The fixture pins the oracle against later edits; the GPU tests
compare the engine with the oracle step by step.

    python tests/golden/make_config1_digest.py
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "astra-cuda_amd")]

FIELDS = ("fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids", "fill_is_sell_quote",
          "fill_quote_sizes", "fill_tid", "fill_quote_tid")
BBO = ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices")


def step_digest(counts, fills, bbo, portfolios, F):
    h = hashlib.sha256()
    h.update(np.ascontiguousarray(counts, dtype=np.int32).tobytes())
    eff = np.where(counts < 0, F, counts)
    for m in range(counts.shape[0]):
        for f in FIELDS:
            h.update(np.ascontiguousarray(fills[f][m, :eff[m]], dtype=np.int32).tobytes())
    for f in BBO:
        h.update(np.ascontiguousarray(bbo[f], dtype=np.int32).tobytes())
    h.update(np.ascontiguousarray(portfolios, dtype=np.int32).tobytes())
    return h.hexdigest()[:16]


# Steps dumped in full (tests/golden/config1_dumps.json): the first, one before and
# the one at which the order ring (O = 1024, two inserts per step) starts to wrap,
# one in the middle of each half, and the last.
DUMP_STEPS = (0, 255, 511, 512, 767, 999)


def step_dump(t, counts, fills, bbo, portfolios, F):
    """Every output of step t: fill_counts, the rows each market wrote (eight fields
    per row), the BBO arrays and last prices, and the portfolios."""
    counts = np.asarray(counts)
    eff = np.where(counts < 0, F, counts)
    rows = {}
    for m in range(counts.shape[0]):
        if eff[m]:
            rows[str(m)] = np.stack([np.asarray(fills[f][m, :eff[m]]).astype(np.int64) for f in FIELDS],
                                    1).tolist()
    return {"step": t, "fill_counts": counts.astype(np.int64).tolist(), "rows": rows,
            "bbo": {f: np.asarray(bbo[f]).astype(np.int64).tolist() for f in BBO},
            "portfolios": np.asarray(portfolios).astype(np.int64).tolist()}


def run(steps=None, dumps=None):
    """Step digests of the oracle's config-1 run; full dumps of DUMP_STEPS go to
    `dumps` (a list) when given."""
    from astra_cuda.workloads import CONFIGS, QuoteStream
    from oracle.oracle import OracleMarket
    cfg = CONFIGS[1]
    qs = QuoteStream(cfg)
    om = OracleMarket(cfg.M, cfg.L, cfg.O, cfg.F, cfg.C)
    of, ob = om.new_fill_batch(), om.new_bbo_batch()
    out = []
    for t in range(cfg.steps if steps is None else steps):
        om.add_two_sided_quotes(*qs.step(t), of)
        om.update_last_prices(ob, of)
        om.get_bbos(ob)
        fills, bbo = {f: getattr(of, f) for f in FIELDS}, {f: getattr(ob, f) for f in BBO}
        out.append(step_digest(of.fill_counts, fills, bbo, om.customer_portfolios, cfg.F))
        if dumps is not None and t in DUMP_STEPS:
            dumps.append(step_dump(t, of.fill_counts, fills, bbo, om.customer_portfolios, cfg.F))
    return out


if __name__ == "__main__":
    dumps = []
    d = run(dumps=dumps)
    with open(os.path.join(HERE, "config1_digest.json"), "w") as f:
        json.dump({"about": "per-step output digest of config 1 (64 x 1000) on the oracle; "
                            "see make_config1_digest.py", "steps": d}, f, indent=0)
    with open(os.path.join(HERE, "config1_dumps.json"), "w") as f:
        json.dump({"about": "every output of config 1 (64 x 1000) on the oracle at steps "
                            f"{list(DUMP_STEPS)}; see make_config1_digest.py", "dumps": dumps},
                  f, separators=(",", ":"))
    print(f"wrote {len(d)} step digests and {len(dumps)} full dumps")
