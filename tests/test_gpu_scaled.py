"""GPU parity of the scaled-MFMA MLP variant (MX_MLP_SCALED) vs the CPU oracle.

The variant computes the same MLP as the fused row (dequantize-then-FP32-
accumulate, MXFP4Kernels.metal:138-173, swiglu_float) with x and mid split
into two FP8 E4M3 terms per value and FP8 x FP4 scaled MFMAs, so it is held
to the north-star tolerance against the oracle's float64 MLP: max-abs error
<= 2e-2 * rms(ref) and cosine >= 0.9995.  The split's own error (<= 2^-8 of
each value) is far inside it; the small-shape tests also hold it to half
that bound against the fp16-MFMA fused variant.
"""
import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData, sample_rows

pytestmark = pytest.mark.gpu
TOL, COS = O.MAX_ABS_REL_TOL, O.COSINE_TOL


def run(dev, d, variant):
    out = dev.alloc(d.T * d.H * 2)
    dev.mlp_forward(variant, d.T, d.H, d.I, d.x, d.weights, out)
    got = dev.download(out, np.float16, (d.T, d.H))
    out.free()
    return got


def oracle(d, rows=None):
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    return O.mlp_mxfp4(O.MLP_F16, x, qg, sg, qu, su, qd, sd, d.H, d.I, rows=rows, threads=16)


def check(got, ref, what, tol=TOL, cos_min=COS):
    rel, cos = O.mlp_error(got, ref)
    print(f"{what}: max_abs/rms={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(np.asarray(got, np.float64)).all(), what
    assert rel <= tol and cos >= cos_min, (what, rel, cos)
    return rel


# T covers one ragged M tile (1, 17), one full tile (64 < 128 rows), two
# tiles with a partial one (130); I = 1024 / K = 512 give split-K GEMMs.
@pytest.mark.parametrize("T", [1, 17, 64, 130])
def test_mlp_scaled_small(dev, T):
    d = MlpData(dev, T, 512, 1024, seed=200 + T)
    got = run(dev, d, M.MLP_SCALED)
    check(got, oracle(d), f"scaled T={T}")
    # deterministic: the split-K partials are added in a fixed order
    assert np.array_equal(run(dev, d, M.MLP_SCALED).view(np.uint16), got.view(np.uint16))
    # and close to the fp16-MFMA fused row (measured ~5e-3 of rms, ~7e-7 off cosine 1)
    check(got, run(dev, d, M.MLP_FUSED).astype(np.float64), f"scaled vs fused T={T}", tol=1e-2, cos_min=0.99999)
    d.free()


def test_config0_scaled(dev):
    d = MlpData(dev, 128, 1024, 4096, seed=7)
    check(run(dev, d, M.MLP_SCALED), oracle(d), "C0 scaled")
    d.free()


def test_config2_scaled(dev):
    d = MlpData(dev, 512, 7168, 2048, seed=13)
    rows = sample_rows(512, 24)
    check(run(dev, d, M.MLP_SCALED)[rows], oracle(d, rows=rows), "C2 scaled")
    d.free()


def test_scaled_scales_from_global(dev):
    """Gate/up with 192 tiles and no K split over K = 8192 (128 stages): the
    workgroup's weight scales do not fit its LDS copy, so each stage loads
    them from global memory next to the F8X2 scale pairs."""
    d = MlpData(dev, 1536, 8192, 1024, seed=23)
    rows = sample_rows(1536, 16)
    check(run(dev, d, M.MLP_SCALED)[rows], oracle(d, rows=rows), "scaled, global scales")
    d.free()


def test_scaled_rejects_bad_shapes(dev):
    d = MlpData(dev, 4, 256, 512, seed=3)
    out = dev.alloc(4 * 256 * 2)
    with pytest.raises(M.MxError):
        dev.mlp_forward(M.MLP_SCALED, 4, 96, 512, d.x, d.weights, out)  # hidden % 64
    out.free()
    d.free()


def _plant(dev, d, which):
    """Cases the reference (bits << 23: byte 255 = +inf, 0 = 0.0) makes
    +-inf as well as NaN.  x row 0 is positive and row 1 negative; gate / up
    rows 96..127 and down row 7 are all code +1.0.
      gate / up: byte 255 on block 0 of row 96.  Token 0 gets g or u = +inf
        there, token 1 g = -inf (silu -> NaN) or u = -inf (mid = +inf); the
        other tokens' mixed signs give NaN.  A token with an infinite mid
        has +-inf outputs (NaN where a down code is zero).
      down: byte 255 at (3, 2), on all of row H-1, and at (7, 3), where
        tokens 0 and 1 meet equal-signed mid values: out[0][7] = +inf.
    Byte 0 rides along in each plane."""
    x = dev.download(d.x, np.float16, (d.T, d.H))
    x[0] = np.abs(x[0]) + np.float16(0.25)
    x[1] = -(np.abs(x[1]) + np.float16(0.25))
    dev.upload(x, d.x)
    for j in (0, 1):
        q, _, n, k = d.mats[j]
        codes = dev.download(q, np.uint8, (n, k // 2))
        codes[96:128, :] = 0x22
        dev.upload(codes, q)
    q, _, n, k = d.mats[2]
    codes = dev.download(q, np.uint8, (n, k // 2))
    codes[7, :] = 0x22
    dev.upload(codes, q)
    q, s_, n, k = d.mats[{"gate": 0, "up": 1, "down": 2}[which]]
    sc = dev.download(s_, np.uint8, (n, k // 32))
    if which == "down":
        sc[3, 2] = 255
        sc[n - 1, :] = 255
        sc[7, 3] = 255
        sc[11, 0] = 0
    else:
        sc[96, 0] = 255
        sc[100, 1] = 0
    dev.upload(sc, s_)


# (64, 512, 256): both GEMMs store from their own epilogue (no K split);
# C0 (128, 1024, 4096): both split K, so the reduce kernels store;
# (512, 1024, 2048): the gate/up GEMM splits K between the waves of one
# workgroup per tile (mx_gemm_kq.hip) and recomputes in its own epilogue.
@pytest.mark.parametrize("T,H,I", [(64, 512, 256), (128, 1024, 4096), (512, 1024, 2048)])
@pytest.mark.parametrize("which", ["gate", "up", "down"])
def test_scaled_e8m0_endpoints(dev, which, T, H, I):
    """E8M0 byte 255 is +inf to the reference (bits << 23,
    MXFP4Kernels.metal:26-29) and NaN to the scaled MFMA.  The outputs it
    turns NaN are recomputed with the reference's dequantization, so NaN,
    +inf and -inf land exactly where the oracle's do, and every finite
    output stays within tolerance."""
    d = MlpData(dev, T, H, I, seed=177 + T)
    _plant(dev, d, which)
    got = run(dev, d, M.MLP_SCALED).astype(np.float64)
    ref = oracle(d)
    if which == "down":
        assert np.isposinf(ref[0, 7]), ref[0, 7]
        assert np.isfinite(ref[:, 8:H - 1]).all()
    else:  # token 0's mid[96] = +inf: +-inf outputs, NaN at zero down codes
        assert np.isinf(ref[0]).sum() > H // 2, np.isinf(ref[0]).sum()
    if which == "up":  # u[1][96] = -inf times silu(g) < 0: mid = +inf
        assert np.isinf(ref[1]).sum() > H // 2, np.isinf(ref[1]).sum()
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (which, np.isnan(got).sum(), np.isnan(ref).sum())
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)), which
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), which
    # finite outputs within tolerance, the two planted tokens apart from the
    # rest: their all-+1 rows give mid values ~50x the others, so their
    # outputs would set the rms that the other tokens' errors are held to
    fin = np.isfinite(ref)
    for rows in (slice(0, 2), slice(2, T)):
        f = fin[rows]
        if f.any():
            rel, cos = O.mlp_error(got[rows][f], ref[rows][f])
            assert rel <= TOL and cos >= COS, (which, rows, rel, cos)
    d.free()
