"""bench.py reads `roofline.traffic` from the committed rocprofv3 summaries under
profiles/ by kernel name and step window: the names it asks for must be the ones
those summaries hold (a kernel's template arguments are part of its name), and
a figure is used only for exactly the steps it was measured on. CPU only."""
import os
import sys
import types

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (stdlib imports only at module level)
from astra_cuda.workloads import CONFIGS, GAME_CONFIG  # noqa: E402

# the driver's command: bench.py --steps 20 --warmup 5
DRIVER = types.SimpleNamespace(start=None, warmup=5, steps=20)


def _window(run_steps):
    t0 = bench.pre_roll(DRIVER, run_steps) + DRIVER.warmup
    return (t0, t0 + DRIVER.steps)


def test_driver_window_is_the_end_of_the_run():
    assert _window(CONFIGS[3].steps) == (980, 1000)   # config 3: ring wrapped at step 512
    default = types.SimpleNamespace(start=None, warmup=100, steps=900)
    assert bench.pre_roll(default, CONFIGS[3].steps) == 0
    assert bench.pre_roll(types.SimpleNamespace(start=7, warmup=5, steps=20), 1000) == 7


def test_matching_kernel_traffic_is_found_for_config3_driver_window():
    cfg = CONFIGS[3]
    traffic, src = bench.measured_traffic(cfg, cfg.M, cfg.bbo_every_step, _window(cfg.steps))
    assert src.startswith("profiles/quote_match_config3_stress_100k_"), src
    assert traffic is not None and traffic > 0
    # every summary that holds a figure for this window holds the same one
    with open(os.path.join(ROOT, "profiles", "quote_match_config3_stress_100k_hbm_traffic.md")) as f:
        assert f"]: {int(traffic)}" in f.read()


def test_game_move_traffic_is_found_for_config5_driver_window():
    moves = GAME_CONFIG.players * GAME_CONFIG.steps_per_player
    traffic, src = bench.game_traffic(GAME_CONFIG, GAME_CONFIG.envs, _window(moves))
    assert src == "profiles/game_move_config5_game_step_10k_kernel_trace.md"
    assert traffic is not None and traffic > 0


def test_other_workloads_and_windows_report_no_traffic():
    cfg = CONFIGS[3]
    w = _window(cfg.steps)
    assert bench.measured_traffic(cfg, cfg.M // 2, cfg.bbo_every_step, w) == (None, None)
    assert bench.measured_traffic(cfg, cfg.M, cfg.bbo_every_step, (5, 25)) == (None, None)
    assert bench.game_traffic(GAME_CONFIG, GAME_CONFIG.envs + 1, w) == (None, None)


def test_matching_kernel_traffic_is_found_for_configs_2_and_4_driver_windows():
    for idx, name in ((2, "readme_shape"), (4, "deep_book")):
        cfg = CONFIGS[idx]
        traffic, src = bench.measured_traffic(cfg, cfg.M, cfg.bbo_every_step, _window(cfg.steps))
        assert src == f"profiles/quote_match_config{idx}_{name}_window.md", src
        assert traffic is not None and traffic > 0


def test_profile_summary_idle_counts_only_time_no_kernel_ran():
    import profile_summary as ps
    # matching kernel 70 ns, a 2 ns gap, bbo 4 ns, a 4 ns gap, matching again (times in ns)
    disp = {"void quote_match_kernel<2>": [(0, 70), (80, 70), (160, 70)],
            "bbo_kernel": [(72, 4), (152, 4)]}
    line = ps.idle(disp, "void quote_match_kernel", 0, 3)
    assert "0.23 us, of which no kernel ran 0.01 us" in line  # 230 ns span, 12 ns idle
    # overlapping spans are counted once
    disp = {"a": [(0, 100), (50, 100)], "b": [(120, 10)]}
    assert "no kernel ran 0.00 us" in ps.idle(disp, "a", 0, 2)


def test_matching_kernel_requests_are_found_for_config3_driver_window():
    """The scattered-request counts and the device's scatter rates of the committed
    request-rate summary, for exactly the driver's window."""
    cfg = CONFIGS[3]
    found = bench.profile_requests("quote_match_kernel<2, false, false, false, false", _window(cfg.steps))
    assert found is not None
    req, rates, src = found
    assert src.startswith("profiles/quote_match_config3_stress_100k_")
    assert set(req) == set(rates) == {"read", "write", "atomic"}
    assert all(v > 0 for v in req.values()) and all(v > 0 for v in rates.values())
    assert bench.profile_requests("quote_match_kernel<2, false, false, false, false", (100, 1000)) is None
