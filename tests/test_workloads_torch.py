"""The torch generator (DeviceQuoteStream, t_game_move) reproduces the numpy
counter-based streams of astra_cuda.workloads bit for bit (run here on the CPU:
int64 wrap-around, logical shifts, unsigned modulo, unsigned threshold order and
float64 arithmetic are the same on the device)."""
import numpy as np
import pytest
import torch

from astra_cuda.workloads import (CONFIGS, GAME_CONFIG, DeviceQuoteStream, GameStream, QuoteStream, draws,
                                  t_draws, t_game_move, t_umod, uniform)


def test_draws_and_unsigned_modulo_match_numpy():
    mk = np.array([0, 1, 2, 77, 4095, 100_000, 4_194_303, (1 << 24) - 1], dtype=np.int64)
    tm = torch.as_tensor(mk)
    for seed, field, step in ((0, 0, 0), (0, 3, 999), (7, 96, 12345), (255, 255, (1 << 24) - 1)):
        h = draws(seed, field, step, mk)
        th = t_draws(seed, field, step, tm)
        assert np.array_equal(th.numpy().view(np.uint64), h)
        for n in (1, 2, 7, 128, 1000, 1 << 31, (1 << 62) - 1):
            assert np.array_equal(t_umod(th, n).numpy(), (h % np.uint64(n)).astype(np.int64)), n


@pytest.mark.parametrize("cfg_index", [1, 2, 3, 4])
def test_device_quote_stream_matches_numpy(cfg_index):
    cfg = CONFIGS[cfg_index]
    mk = np.unique(np.concatenate([np.arange(200), np.random.default_rng(cfg_index).integers(0, cfg.M, 300)]))
    ref = QuoteStream(cfg, mk)
    dev = DeviceQuoteStream(cfg, mk, device="cpu")
    for t in range(40):
        a, b = ref.step(t), dev.step(t)
        for x, y in zip(a, b):
            assert y.dtype == torch.int32
            assert np.array_equal(x, y.numpy()), (cfg_index, t)
    # far steps (independent configs; config 3 walks on in order)
    if cfg_index != 3:
        for t in (999, cfg.steps - 1, 123_456):
            for x, y in zip(ref.step(t), dev.step(t)):
                assert np.array_equal(x, y.numpy()), (cfg_index, t)


def test_device_stream_covers_the_largest_market_ids():
    cfg = CONFIGS[3]
    mk = np.arange(4_194_304 - 500, 4_194_304)
    ref, dev = QuoteStream(cfg, mk), DeviceQuoteStream(cfg, mk, device="cpu")
    for t in range(5):
        for x, y in zip(ref.step(t), dev.step(t)):
            assert np.array_equal(x, y.numpy())


def test_game_moves_match_numpy():
    envs = np.arange(0, 10_000, 7)
    gs = GameStream(GAME_CONFIG, envs)
    te = torch.as_tensor(envs.astype(np.int64))
    for k in (0, 1, 999):
        assert np.array_equal(gs.move(k), t_game_move(GAME_CONFIG, k, te).numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("cfg_index", [2, 3, 4])
def test_gpu_device_quote_stream_matches_numpy(cfg_index):
    """The same streams generated on the MI355X (bench.py's inputs)."""
    cfg = CONFIGS[cfg_index]
    mk = np.arange(0, cfg.M, 37)
    ref = QuoteStream(cfg, mk)
    dev = DeviceQuoteStream(cfg, mk, device="cuda:0")
    for t in range(30):
        for x, y in zip(ref.step(t), dev.step(t)):
            assert np.array_equal(x, y.cpu().numpy()), (cfg_index, t)


@pytest.mark.gpu
def test_gpu_game_moves_match_numpy():
    envs = np.arange(10_000)
    gs = GameStream(GAME_CONFIG, envs)
    te = torch.as_tensor(envs.astype(np.int64)).to("cuda:0")
    for k in (0, 5, 999):
        assert np.array_equal(gs.move(k), t_game_move(GAME_CONFIG, k, te).cpu().numpy())
