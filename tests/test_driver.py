"""The command-line host driver (counterpart of the reference's MetalFP41Probe
executable, Sources/MetalFP41Probe/main.swift): flag surface, error path
(`error: <message>` on stderr, exit 1, main.swift:83-88) and, on the GPU, the
full probe ending in PASS with the reference checksum 403573 on the fused
MXFP4 row (README.md:292-294)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "mpp-4.1-fp4-fp8-block_amd", "lib", "mxfp4_probe")

needs_driver = pytest.mark.skipif(not os.path.exists(DRIVER), reason="driver not built (run build())")


def run(*args, timeout=120):
    return subprocess.run([DRIVER, *args], capture_output=True, text=True, timeout=timeout)


@needs_driver
@pytest.mark.parametrize("args,message", [
    (["--mlp-benchmark", "--mlp-hidden=100"],
     "MLP hidden and intermediate sizes must be multiples of 16 for packed FP4 weights."),
    (["--mlp-benchmark", "--mlp-tokens=0"], "MLP sizes and iterations must be positive."),
    (["--mlp-benchmark", "--mlp-iterations=-2"], "MLP sizes and iterations must be positive."),
    (["--benchmark", "--k=100"], "Matmul K/depth must be a multiple of 16 for packed FP4 groups."),
    (["--benchmark", "--m=0"], "Matmul sizes and iterations must be positive."),
    (["--benchmark", "--iterations=-1"], "Matmul sizes and iterations must be positive."),
])
def test_driver_rejects_bad_arguments(args, message):
    # checked before the device is opened (main.swift:592-597), so this runs anywhere
    r = run(*args)
    assert r.returncode == 1
    assert r.stderr.strip() == f"error: {message}"


@needs_driver
@pytest.mark.gpu
def test_driver_mlp_benchmark_on_gpu():
    r = run("--mlp-benchmark", "--mlp-iterations=2", "--skip-tensor", timeout=300)
    print(r.stdout[-3000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr
    out = r.stdout
    for name in ("FP4 E2M1", "FP8 E4M3", "FP8 E5M2"):
        assert f"[ok] {name}" in out
    assert "bytes:    FF DE BC 9A 10 32 54 76" in out          # E2M1 KAT bytes
    assert "bytes:    FE FE D8 B0 00 20 58 7E" in out          # E4M3 KAT bytes
    assert "shape: tokens=128, hidden=1024, intermediate=4096" in out
    assert out.rstrip().endswith("PASS")
    # reference fused-row checksum over the reference LCG data
    m = re.search(r"reference epilogue\): h_mxfp4_f:\n.*\n\s+checksum: ([-0-9.e+]+) over 32 samples", out)
    assert m, out
    assert abs(float(m.group(1)) - 403573) / 403573 < 2e-5
    for row in ("W4A4", "scaled MFMA", "FP8 E5M2 weights", "INT4 weights", "W8A8 MLP", "relative slowdown"):
        assert row in out


@needs_driver
@pytest.mark.gpu
def test_driver_accum_probe_on_gpu():
    """--accum-probe (runAccumulatorProbe, main.swift:1523-1713): the table
    rows behind the reference's published findings (README.md:342-352)."""
    r = run("--accum-probe", "--skip-tensor", timeout=300)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr
    out = r.stdout
    assert "Accumulator precision/overflow probe" in out
    assert "    1818 | 65448 | 65440 | 65448" in out       # one RNE rounding to half
    assert "    256 | 65536 | inf | 65536" in out          # FP8 x FP8 overflow in half only
    assert "    131072 | 131072 | inf | 131072" in out    # f32 accumulation, exact
    assert "    65504 | 65504 | 65504 | 65504" in out
    assert "non-uniform" not in out
    assert out.rstrip().endswith("PASS")


@needs_driver
@pytest.mark.gpu
def test_driver_matmul_benchmark_on_gpu():
    """--benchmark --fp4-group-sweep (runBigMatmulBenchmark, main.swift:380-584)
    at 256^3 on the reference's LCG data; the INT4 x INT4 row is exact integer
    arithmetic, so its checksum is pinned by numpy on the same bytes."""
    import numpy as np
    import oracle as O
    s = 256
    r = run("--benchmark", "--fp4-group-sweep", f"--matmul-size={s}", "--iterations=2", "--skip-tensor", timeout=300)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, r.stderr
    out = r.stdout
    # g8 and g16 are one kernel here: the sweep prints each kernel once
    for row in ("FP4 E2M1 g8/g16 -> FP32 accumulate", "half x FP4 E2M1 g8/g16 -> half accumulate",
                "half x INT4 -> half accumulate", "INT8 x half -> half accumulate",
                "INT4 x INT4 -> INT32 accumulate", "relative slowdown"):
        assert row in out, row
    assert "E2M1 g8 ->" not in out and "E2M1 g16 ->" not in out, out
    a = O.lcg_bytes(0x12345678, s * s // 2).reshape(s, s // 2)
    b = O.lcg_bytes(0x87654321, s * s // 2).reshape(s, s // 2)

    def i4(x):
        x = x.astype(np.int64)
        v = np.empty((x.shape[0], x.shape[1] * 2), np.int64)
        v[:, 0::2], v[:, 1::2] = ((x & 15) ^ 8) - 8, ((x >> 4) ^ 8) - 8
        return v

    c = (i4(a) @ i4(b).T).reshape(-1)
    step = max(1, c.size // 32)
    want = f"{int(c[::step].sum())} over {len(c[::step])} samples"
    m = re.search(r"INT4 x INT4 -> INT32 accumulate:\n.*\n\s+checksum: (.*)", out)
    assert m and m.group(1).strip() == want, (m and m.group(1), want)
    assert out.rstrip().endswith("PASS")
