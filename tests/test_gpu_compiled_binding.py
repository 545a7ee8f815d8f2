"""The compiled binding astra_cuda._C.order_matching (csrc/bindings.cpp: the
reference's market_bindings.cc surface over the C ABI, validation in C++) against
the CPU oracle, bit-exact, and its errors and surface (GPU)."""
import numpy as np
import pytest
import torch

from kat_harness import load_kats, run_scenario
from parity_util import DEV, GpuCompiledAdapter, compare_fills, compare_portfolios, run_parity

pytestmark = pytest.mark.gpu
SCENARIOS = load_kats()


def _log(msg):
    print(msg, flush=True)


def _com():
    from astra_cuda._C import order_matching as com
    return com


def test_gpu_compiled_binding_is_the_in_tree_build():
    import astra_cuda._C as C
    from astra_cuda.build import binding_path
    assert C.__file__ == binding_path()


@pytest.mark.parametrize("sc", SCENARIOS, ids=[s["name"] for s in SCENARIOS])
def test_gpu_compiled_kat(sc):
    _log(f"kat {sc['name']} compiled")
    run_scenario(sc, GpuCompiledAdapter)


@pytest.mark.parametrize("cfg_index,M,steps", [(1, 64, 1000), (2, 3000, 300), (3, 4000, 700)])
def test_gpu_compiled_parity(cfg_index, M, steps):
    from astra_cuda.workloads import CONFIGS, QuoteStream
    cfg = CONFIGS[cfg_index]
    qs = QuoteStream(cfg, np.arange(M))
    _log(f"compiled binding: config {cfg_index}, {M} x {steps}")
    r = run_parity(M, cfg.L, cfg.O, cfg.F, cfg.C, steps, qs.step, bbo_every=1, full_every=100,
                   layout="compiled", label=f"compiled cfg{cfg_index}")
    assert r["fill_rows"] > M


def test_gpu_compiled_validation_errors(capfd):
    com = _com()
    g = com.VecMarket(4, 128, 64, 16)
    f = g.new_fill_batch()
    ok = torch.zeros(4, dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match=r"bid_px.size\(0\) == num_markets_"):
        g.add_two_sided_quotes(torch.zeros(5, dtype=torch.int32, device=DEV), ok, ok, ok, ok, f)
    with pytest.raises(RuntimeError, match="ask_px tensor must be on device 0"):
        g.add_two_sided_quotes(ok, ok, torch.zeros(4, dtype=torch.int32), ok, ok, f)
    with pytest.raises(RuntimeError, match="customer_ids tensor must be contiguous"):
        g.add_two_sided_quotes(ok, ok, ok, ok, torch.zeros(8, dtype=torch.int32, device=DEV)[::2], f)
    with pytest.raises(RuntimeError, match="must be int32"):
        g.add_two_sided_quotes(ok, ok.long(), ok, ok, ok, f)
    f.fill_sizes = torch.zeros((4, 15), dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="fills.fill_sizes"):
        g.add_two_sided_quotes(ok, ok, ok, ok, ok, f)
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        com.VecMarket(4, 129, 64, 16)  # market.cu:339
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        com.VecMarket(4, 128, 64, 16, threads_per_block=0)  # market.cu:343
    with pytest.raises(RuntimeError, match="Astra Fatal Error"):
        com.VecMarket(4, 128, 64, 16, device_id=torch.cuda.device_count())  # market.cu:350
    with pytest.raises(RuntimeError, match="reset_indices"):
        g.clear_quotes(torch.zeros(4, dtype=torch.int32, device=DEV))
    assert "Astra Fatal Error: " in capfd.readouterr().err  # printed as well (astra_utils.cc:14-16)
    assert g.global_tid == 0


def test_gpu_compiled_surface_matches_the_ctypes_binding():
    """Reset, clear_quotes, clone, to_string, the live portfolio view, copy_to,
    the batches' reset / update_last_prices and the current stream: the compiled
    binding and astra_cuda.order_matching give the same results on the same calls."""
    from astra_cuda import order_matching as aom
    com = _com()
    M, L, O, F, C = 500, 32, 16, 8, 6
    rng = np.random.default_rng(5)
    a, b = aom.VecMarket(M, L, O, F, C), com.VecMarket(M, L, O, F, C)
    fa, fb = a.new_fill_batch(), b.new_fill_batch()
    ba, bb = a.new_bbo_batch(), b.new_bbo_batch()
    s = torch.cuda.Stream()
    for t in range(60):
        q = [torch.as_tensor(x.astype(np.int32)).to(DEV) for x in
             (rng.integers(-1, L + 1, M), rng.integers(-1, 6, M), rng.integers(-1, L + 1, M),
              rng.integers(-1, 6, M), rng.integers(-1, C + 1, M))]
        if t == 20:
            sel = torch.as_tensor(rng.integers(0, 2, M).astype(bool)).to(DEV)
            a.clear_quotes(sel)
            b.clear_quotes(sel)
        if t == 40:
            a, b = a.clone(), b.clone()
        with torch.cuda.stream(s):
            a.add_two_sided_quotes(*q, fa)
            b.add_two_sided_quotes(*q, fb)
            a.get_bbos(ba)
            b.get_bbos(bb)
            ba.update_last_prices(fa)
            bb.update_last_prices(fb)
        s.synchronize()
        for f in ("fill_counts", "fill_prices", "fill_sizes", "fill_customer_ids", "fill_quoter_ids",
                  "fill_is_sell_quote", "fill_quote_sizes", "fill_tid", "fill_quote_tid"):
            assert torch.equal(getattr(fa, f), getattr(fb, f)), (t, f)
        for f in ("best_bid_prices", "best_bid_sizes", "best_ask_prices", "best_ask_sizes", "last_prices"):
            assert torch.equal(getattr(ba, f), getattr(bb, f)), (t, f)
        assert torch.equal(a.get_customer_portfolios(), b.get_customer_portfolios()), t
    assert a.global_tid == b.global_tid == 120
    for m in (0, 7, 499):
        assert a.to_string(m) == b.to_string(m)
    buf = torch.empty((M, C, 2), dtype=torch.int32, device=DEV)
    b.copy_customer_portfolios_to(buf)
    assert torch.equal(buf, a.get_customer_portfolios())
    view = b.get_customer_portfolios()
    b.reset()
    torch.cuda.synchronize()
    assert not view.any() and b.global_tid == 0  # the view is live
    bb.reset()
    fb.reset()
    torch.cuda.synchronize()
    assert not bb.last_prices.any() and not fb.fill_counts.any()
