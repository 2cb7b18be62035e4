"""GPU parity of the MXFP4 gate/up GEMM that splits K inside a workgroup
(mx_gemm_kq.hip).  launch_gemm_q takes it for f16 activations (fused and
reference-row variants) and for F8X2 ones (the scaled variant) x MXFP4
weights with a SwiGLU epilogue when the 64 x 64-channel tiles number 192 to
256 and K % 256 == 0, K >= 1024: BASELINE configs[2] (T=512, H=7168,
I=2048, also covered by test_config2_fused_and_dequant) and the shapes
below, which land there with 256 (512 x 2048), 224 (ragged 390-token last
tile) and 200 tiles.  Reference semantics: MXFP4Kernels.metal:42-173 with
the fused rows' SwiGLU (MPPMLPKernels.metal:186-220); E8M0 byte 255 is +inf
(MXFP4Kernels.metal:26-29).
"""
import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData

pytestmark = pytest.mark.gpu
TOL, COS = 5e-3, 0.99999  # mid is rounded to f16 between the GEMMs (2.5e-3 of rms measured)
SHAPES = [(512, 1024, 2048), (390, 1280, 2048), (500, 1536, 1600)]


def run(dev, d, variant):
    out = dev.alloc(d.T * d.H * 4)
    dev.mlp_forward(variant, d.T, d.H, d.I, d.x, d.weights, out)
    got = dev.download(out, np.float32 if variant == M.MLP_REFROW else np.float16, (d.T, d.H))
    out.free()
    return got


def oracle(d, variant):
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    mode = O.MLP_REFROW if variant == M.MLP_REFROW else O.MLP_F16
    return O.mlp_mxfp4(mode, x, qg, sg, qu, su, qd, sd, d.H, d.I, threads=16)


@pytest.mark.parametrize("variant", [M.MLP_FUSED, M.MLP_REFROW])
@pytest.mark.parametrize("T,H,I", SHAPES)
def test_kq_mlp(dev, variant, T, H, I):
    d = MlpData(dev, T, H, I, seed=300 + T + variant)
    got = run(dev, d, variant)
    rel, cos = O.mlp_error(got, oracle(d, variant))
    print(f"kq variant {variant} T={T} H={H} I={I}: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(got.astype(np.float32)).all()
    assert rel <= TOL and cos >= COS
    # deterministic: the K quarters are added in wave order
    assert np.array_equal(run(dev, d, variant), got)
    d.free()


@pytest.mark.parametrize("which", ["gate", "up"])
def test_kq_e8m0_255(dev, which):
    """Byte 255 in a gate or up scale: the loop's NaN sums are recomputed with
    the reference's dequantization, so NaN / +inf / -inf land where the
    oracle has them; byte 0 stays within tolerance."""
    T, H, I = 512, 1024, 2048
    d = MlpData(dev, T, H, I, seed=331)
    q, s, n, k = d.mats[0 if which == "gate" else 1]
    sc = dev.download(s, np.uint8, (n, k // 32))
    sc[3, 2] = 255          # one block of channel 3
    sc[I - 1, :] = 255      # every block of the last channel
    sc[70, 0] = 0
    dev.upload(sc, s)
    got = run(dev, d, M.MLP_FUSED).astype(np.float64)
    ref = oracle(d, M.MLP_FUSED)
    assert np.isnan(ref).any() or np.isinf(ref).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    if fin.any():
        rel, cos = O.mlp_error(got[fin], ref[fin])
        assert rel <= TOL and cos >= COS, (rel, cos)
    d.free()


def test_kq_nonfinite_x(dev):
    T, H, I = 390, 1280, 2048
    d = MlpData(dev, T, H, I, seed=341)
    x = dev.download(d.x, np.float16, (T, H))
    x[0, 5] = np.inf
    x[T - 1, H - 3] = np.nan
    x[200, 7] = -np.inf
    dev.upload(x, d.x)
    got = run(dev, d, M.MLP_FUSED).astype(np.float64)
    ref = oracle(d, M.MLP_FUSED)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    rel, cos = O.mlp_error(got[fin], ref[fin])
    assert rel <= TOL and cos >= COS, (rel, cos)
    d.free()


@pytest.mark.parametrize("T,H,I", SHAPES)
def test_kq_scaled(dev, T, H, I):
    """The scaled variant (F8X2 x x FP4 on the scaled MFMA): BASELINE
    tolerance against the oracle and 1e-2 of rms against the fused variant,
    as the scaled rows are held elsewhere; deterministic."""
    d = MlpData(dev, T, H, I, seed=350 + T)
    got = run(dev, d, M.MLP_SCALED)
    rel, cos = O.mlp_error(got, oracle(d, M.MLP_FUSED))
    print(f"kq scaled T={T} H={H} I={I}: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    rel2, cos2 = O.mlp_error(got, run(dev, d, M.MLP_FUSED).astype(np.float64))
    assert rel2 <= 1e-2 and cos2 >= 0.99999, (rel2, cos2)
    assert np.array_equal(run(dev, d, M.MLP_SCALED).view(np.uint16), got.view(np.uint16))
    d.free()


def test_kq_scaled_nonfinite_x(dev):
    """Non-finite x in the scaled variant: its F8X2 groups carry scale bytes
    255, and the mid values they reach are recomputed from the f16 x."""
    T, H, I = 390, 1280, 2048
    d = MlpData(dev, T, H, I, seed=361)
    x = dev.download(d.x, np.float16, (T, H))
    x[0, 5] = np.inf
    x[T - 1, H - 3] = np.nan
    x[200, 7] = -np.inf
    dev.upload(x, d.x)
    got = run(dev, d, M.MLP_SCALED).astype(np.float64)
    ref = oracle(d, M.MLP_FUSED)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    rel, cos = O.mlp_error(got[fin], ref[fin])
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL, (rel, cos)
    d.free()
