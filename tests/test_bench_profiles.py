"""bench.py reads `roofline.traffic` from the committed rocprofv3 summaries under
profiles/ by kernel name: the names it asks for must be the ones those summaries
hold (a kernel's template arguments are part of its name). CPU only."""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402  (stdlib imports only at module level)
from astra_cuda.workloads import CONFIGS, GAME_CONFIG  # noqa: E402


def test_matching_kernel_traffic_is_found_for_config3():
    cfg = CONFIGS[3]
    traffic, src = bench.measured_traffic(cfg, cfg.M, cfg.bbo_every_step)
    assert src == "profiles/quote_match_config3_stress_100k_hbm_traffic.md"
    assert traffic is not None and traffic > 0


def test_game_move_traffic_is_found_for_config5():
    traffic, src = bench.game_traffic(GAME_CONFIG, GAME_CONFIG.envs)
    assert src == "profiles/game_move_config5_game_step_10k_kernel_trace.md"
    assert traffic is not None and traffic > 0


def test_other_workloads_report_no_traffic():
    cfg = CONFIGS[3]
    assert bench.measured_traffic(cfg, cfg.M // 2, cfg.bbo_every_step) == (None, None)
    assert bench.game_traffic(GAME_CONFIG, GAME_CONFIG.envs + 1) == (None, None)
