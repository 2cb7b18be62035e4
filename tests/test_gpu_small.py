"""GPU parity of the few-tile MXFP4 GEMMs (mx_gemm_small.hip) against the
CPU oracle.

These kernels take the fused MLP's GEMMs at BASELINE configs[0]-like shapes
(at most 128 tokens; gate/up at hidden = 1024, down at intermediate % 1024 up
to 4096 with hidden % 32 up to 2048) and mx_mxfp4_matmul at such shapes.
Semantics are the fused rows' (MXFP4Kernels.metal:138-173, dequantize then
f32 accumulate, swiglu_float / swiglu_half): BASELINE tolerance for the MLP,
1e-3 of rms for the f32 matmul, E8M0 bytes 255 / 0 with the reference's
+inf / 0.0 meaning, and deterministic results (the K quarters are added in a
fixed order).
"""
import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData

pytestmark = pytest.mark.gpu
TOL, COS = O.MAX_ABS_REL_TOL, O.COSINE_TOL


def run_mlp(dev, d, variant=M.MLP_FUSED):
    out = dev.alloc(d.T * d.H * 4)
    dev.mlp_forward(variant, d.T, d.H, d.I, d.x, d.weights, out)
    dt = np.float32 if variant == M.MLP_REFROW else np.float16
    got = dev.download(out, dt, (d.T, d.H))
    out.free()
    return got


def oracle_mlp(d, mode=O.MLP_F16):
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    return O.mlp_mxfp4(mode, x, qg, sg, qu, su, qd, sd, d.H, d.I, threads=16)


def check(got, ref, what, tol=TOL, cos_min=COS):
    rel, cos = O.mlp_error(got, ref)
    print(f"{what}: max_abs/rms={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(np.asarray(got, np.float64)).all(), what
    assert rel <= tol and cos >= cos_min, (what, rel, cos)


# T: one ragged tile (1, 17), 100 (ragged last tiles of both kernels), 128
# (C0's token count); I: the down GEMM's 256-K chunks per wave, 1 .. 4
# (the 3-slot ring refills from 4 on); H = 1024 takes the gate/up kernel.
@pytest.mark.parametrize("T", [1, 17, 100, 128])
@pytest.mark.parametrize("I", [1024, 2048, 3072, 4096])
def test_small_mlp_fused(dev, T, I):
    d = MlpData(dev, T, 1024, I, seed=500 + T + I)
    got = run_mlp(dev, d)
    check(got, oracle_mlp(d), f"small fused T={T} I={I}")
    assert np.array_equal(run_mlp(dev, d).view(np.uint16), got.view(np.uint16))
    d.free()


@pytest.mark.parametrize("T,H,I", [(128, 1024, 4096), (33, 2048, 1024), (64, 96, 1024)])
def test_small_down_shapes(dev, T, H, I):
    """Down GEMMs of other widths (H = 2048, the largest taken; H = 96, three
    32-row tiles) behind the tiled gate/up (H != 1024) or the small one."""
    d = MlpData(dev, T, H, I, seed=600 + H)
    check(run_mlp(dev, d), oracle_mlp(d), f"small down T={T} H={H} I={I}")
    d.free()


def test_small_refrow(dev):
    """The reference fused-row epilogue (swiglu_half, f32 out) on both
    kernels at C0's shape."""
    d = MlpData(dev, 128, 1024, 4096, seed=77)
    got = run_mlp(dev, d, M.MLP_REFROW)
    check(got, oracle_mlp(d, O.MLP_REFROW), "small refrow", tol=3e-3, cos_min=0.99999)
    d.free()


@pytest.mark.parametrize("m,n,k", [(1, 32, 1024), (77, 96, 2048), (128, 2048, 4096), (16, 1056, 3072)])
def test_small_matmul(dev, m, n, k):
    """mx_mxfp4_matmul (mxfp4_native_sp_h_f_n64's ABI) on the small plain
    GEMM: f32 out within 1e-3 of rms of the float64 oracle, f16 out within
    one f16 rounding."""
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = rng.integers(112, 128, (n, k // 32), dtype=np.uint8)  # sums stay inside f16's range
    da, dq, ds = dev.upload(a), dev.upload(q), dev.upload(s)
    ref = O.mxfp4_matmul(a, q, s, n)
    for c_dtype, npdt, tol in ((M.DT_F32, np.float32, 1e-3), (M.DT_F16, np.float16, 3e-3)):
        dc = dev.alloc(m * n * 4)
        dev.mxfp4_matmul(da, M.DT_F16, dq, dc, c_dtype, m, n, k, ds)
        check(dev.download(dc, npdt, (m, n)), ref, f"small matmul {m}x{n}x{k} c={c_dtype}", tol=tol,
              cos_min=0.99999)
        dc.free()
    for b in (da, dq, ds):
        b.free()


def _plant(dev, d, which, rows_255, row_0):
    q, s, n, k = d.mats[{"gate": 0, "up": 1, "down": 2}[which]]
    sc = dev.download(s, np.uint8, (n, k // 32))
    for r, b in rows_255:
        if b is None:
            sc[r, :] = 255
        else:
            sc[r, b] = 255
    sc[row_0, 0] = 0
    dev.upload(sc, s)


@pytest.mark.parametrize("which", ["gate", "up", "down"])
def test_small_e8m0_endpoints(dev, which):
    """E8M0 byte 255 (+inf to the reference, MXFP4Kernels.metal:26-29; NaN
    to the hardware's converts) takes the exact decode on both small
    kernels, byte 0 gives 0.0: NaN, +inf and -inf land where the oracle's
    do, every finite output within tolerance."""
    T, H, I = 40, 1024, 2048
    d = MlpData(dev, T, H, I, seed=141 + len(which))
    n_rows = I if which != "down" else H
    _plant(dev, d, which, [(3, 2), (n_rows - 1, None)], 100)
    got = run_mlp(dev, d).astype(np.float64)
    ref = oracle_mlp(d)
    assert np.isnan(ref).any() or np.isinf(ref).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref)), which
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)), which
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), which
    fin = np.isfinite(ref)
    if fin.any():  # a whole gate / up row at 255 reaches every output
        rel, cos = O.mlp_error(got[fin], ref[fin])
        assert rel <= TOL and cos >= COS, (which, rel, cos)
    d.free()
