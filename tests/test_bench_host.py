"""Host-side logic of bench.py (no GPU): the one-GPU contract, the spin-up
loop, the weight-set rotation and the algorithmic byte / flop counts that
the roofline blocks divide by."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert p.returncode == 2
    assert "one GPU only" in p.stderr


class FakeForwards:
    """call(n): n forwards of `per` seconds each (host time advanced by hand)."""

    def __init__(self, per, clock):
        self.per, self.clock, self.calls = per, clock, []

    def __call__(self, n):
        self.calls.append(n)
        self.clock[0] += n * self.per
        return n * self.per


def test_spin_up_sizes_calls_and_stops(monkeypatch):
    clock = [0.0]
    monkeypatch.setattr(bench.time, "time", lambda: clock[0])
    f = FakeForwards(per=10e-6, clock=clock)
    bench.spin_up(f, iters=20, seconds=0.3)
    # one call of `iters` forwards to time them, then calls of >= 50 ms of work
    assert f.calls[0] == 20
    assert all(n == 5000 for n in f.calls[1:])
    assert clock[0] >= 0.3 and clock[0] < 0.3 + 0.05 + 1e-9


def test_spin_up_long_forwards_keep_iters(monkeypatch):
    clock = [0.0]
    monkeypatch.setattr(bench.time, "time", lambda: clock[0])
    f = FakeForwards(per=1.3e-3, clock=clock)  # C4-sized forwards
    bench.spin_up(f, iters=10, seconds=0.3)
    assert f.calls[0] == 10 and all(n == 38 for n in f.calls[1:])


def test_spin_up_zero_seconds_runs_nothing():
    f = FakeForwards(per=1e-5, clock=[0.0])
    bench.spin_up(f, iters=20, seconds=0)
    assert f.calls == []


def test_weight_sets_stream_past_the_last_level_cache():
    # the headline's 77 sets: the down matrix of every set is 7.8 MB
    assert bench.mxfp4_bytes(7168, 2048) == 7168 * 1024 + 7168 * 64
    assert bench.sets_for(bench.mxfp4_bytes(7168, 2048)) == 77
    n = bench.sets_for(bench.fmt_bytes(4, 4096, 14336))
    assert n * bench.fmt_bytes(4, 4096, 14336) >= 600e6 > (n - 1) * bench.fmt_bytes(4, 4096, 14336)


@pytest.mark.parametrize("name,expect", [
    # decode GEMV at C1 T=1: gate and up weights + E8M0 scales, x in, mid out
    ("gemv_mxfp4_gate_up_swiglu", ("hbm", 15_616_000)),
    ("gemv_mxfp4_down", ("hbm", 7_817_216)),
    # GEMM steps: 2*T*H*2I for a gate/up step, 2*T*H*I for one GEMM
    ("gemm_q_mxfp4_gate_up_swiglu", ("mfma", 2 * 1 * 7168 * 2 * 2048)),
    ("gemm_q_mxfp4_down", ("mfma", 2 * 1 * 7168 * 2048)),
    # prologues and fix-up passes are never the roofline kernel
    ("split_x_f8x2", (None, 0)),
    ("w4a4_prologue", (None, 0)),
])
def test_kernel_work(name, expect):
    assert bench.kernel_work(name, 1, 7168, 2048) == expect


def test_format_row_bytes():
    # INT4 g32: nibbles + an f16 scale per 32; 8-bit: codes + an f32 row scale
    assert bench.fmt_bytes(4, 14336, 4096) == 14336 * 2048 + 14336 * 128 * 2
    assert bench.fmt_bytes(1, 14336, 4096) == 14336 * 4096 + 14336 * 4
