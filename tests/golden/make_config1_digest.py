"""Write tests/golden/config1_digest.json: a per-step digest of every output of
the config-1 run (64 markets x 1000 steps) on the oracle.

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


def run(steps=None):
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
        out.append(step_digest(of.fill_counts, {f: getattr(of, f) for f in FIELDS},
                               {f: getattr(ob, f) for f in BBO}, om.customer_portfolios, cfg.F))
    return out


if __name__ == "__main__":
    d = run()
    with open(os.path.join(HERE, "config1_digest.json"), "w") as f:
        json.dump({"about": "per-step output digest of config 1 (64 x 1000) on the oracle; "
                            "see make_config1_digest.py", "steps": d}, f, indent=0)
    print(f"wrote {len(d)} step digests")
