"""Host bookkeeping of the KHQ step (no GPU): split count, compression
cadence, window bounds (ref:src/khq/runtime.mojo:211-222, 454-613)."""
import pytest

from khq.layer import CHUNK, RING, KhqOptions, plan_step, split_count


def test_split_count():
    assert split_count(0, 16) == 1
    assert split_count(1000, 1) == 1
    assert split_count(7, 16) == 1        # c_len // 8 == 0 -> 1
    assert split_count(64, 16) == 8       # capped by c_len // 8
    assert split_count(384, 16) == 16
    assert split_count(32640, 32) == 32
    assert split_count(32640, 64) == 64


def test_options_env(monkeypatch):
    monkeypatch.setenv("BONSAI_KHQ_SPLITS", "16")
    assert KhqOptions.from_env().splits == 16    # full int parse ("16" is not "1")
    monkeypatch.setenv("BONSAI_KHQ_SPLITS", "100")
    assert KhqOptions.from_env().splits == 32    # reference clamp
    assert KhqOptions.from_env(max_splits=64).splits == 64
    monkeypatch.setenv("BONSAI_KHQ_SPLITS", "0")
    assert KhqOptions.from_env().splits == 1
    monkeypatch.setenv("BONSAI_KHQ_SPLITS", "x")
    assert KhqOptions.from_env().splits == 16
    monkeypatch.delenv("BONSAI_KHQ_SPLITS")
    assert KhqOptions.from_env().splits == 16    # code default (README says 8)


def test_cadence():
    """Event k fires at write_pos 256 + 128 (k - 1) and leaves boundary 128 k
    with a raw window of 128 (the deploy cadence gate)."""
    b, w = 0, 0
    events = []
    for t in range(2000):
        b, w, ev, c_len, win_len, win_start = plan_step(b, w, cap=4096)
        assert c_len == b and win_len == w - b and win_start == b % RING
        assert 1 <= win_len <= RING
        if ev is not None:
            events.append((w, b, win_len))
    assert events[0] == (256, 128, 128)
    for k, (wp, bd, win) in enumerate(events, start=1):
        assert wp == 256 + 128 * (k - 1) and bd == 128 * k and win == 128


def test_config2_state():
    b, w = 0, 0
    for _ in range(512):
        b, w, *_ = plan_step(b, w, cap=4096)
    assert (b, w) == (384, 512)


def test_capacity_stops_compression():
    b, w = 0, 0
    over = None
    for t in range(1000):
        b, w, ev, c_len, win_len, _ = plan_step(b, w, cap=512)
        if win_len > RING and over is None:
            over = w
    assert b == 512 and over == 512 + RING + 1
