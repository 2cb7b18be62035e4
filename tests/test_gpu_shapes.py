"""GPU parity over the reference's shape domain.

The reference runs its MXFP4 rows whenever hidden % 32 == 0 and
intermediate % 32 == 0 (main.swift:1043), and its matmul tiles guard
column < n (MXFP4Kernels.metal:98), so any n works there.  The library's
64-K-stage GEMM family needs multiples of 64; the other shapes go to the
K-step-32 kernel with a masked N tail.  Every shape here is checked
against the oracle (dequantize-then-accumulate, float64) within the
BASELINE tolerance.
"""
import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData, sample_rows

pytestmark = pytest.mark.gpu
TOL, COS = O.MAX_ABS_REL_TOL, O.COSINE_TOL


def check(got, ref, what, tol=TOL, cos_min=COS):
    rel, cos = O.mlp_error(got, ref)
    print(f"{what}: max_abs/rms={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(np.asarray(got, np.float64)).all(), what
    assert rel <= tol and cos >= cos_min, (what, rel, cos)


def run_mlp(dev, d, variant):
    out = dev.alloc(d.T * d.H * 4)
    dev.mlp_forward(variant, d.T, d.H, d.I, d.x, d.weights, out)
    dt = np.float32 if variant == M.MLP_REFROW else np.float16
    got = dev.download(out, dt, (d.T, d.H))
    out.free()
    return got


def oracle_mlp(d, variant, rows):
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    mode = O.MLP_REFROW if variant == M.MLP_REFROW else O.MLP_F16
    return O.mlp_mxfp4(mode, x, qg, sg, qu, su, qd, sd, d.H, d.I, rows=rows, threads=16)


# (5, 96, 160): neither size % 64, T below the MFMA tile; (40, 1056, 2080)
# and (130, 544, 1120): % 32 only, ragged M tiles; (8, 192, 320): % 64 but not
# % 128 with few tokens (64-K-stage family, not the decode GEMV); (3, 32, 64):
# the smallest MXFP4 block shape.
SHAPES = [(5, 96, 160), (40, 1056, 2080), (130, 544, 1120), (8, 192, 320), (3, 32, 64)]


@pytest.mark.parametrize("T,H,I", SHAPES)
@pytest.mark.parametrize("variant", [M.MLP_FUSED, M.MLP_DEQUANT, M.MLP_REFROW])
def test_mlp_shape_domain(dev, variant, T, H, I):
    d = MlpData(dev, T, H, I, seed=300 + T + H % 97)
    rows = sample_rows(T, 24)
    got = run_mlp(dev, d, variant)[rows]
    # the reference row's swiglu_half epilogue rounds mid to f16 like the
    # oracle's, and stores f32: it is held to 2e-3 of rms like the C0 row
    tol = 2e-3 if variant == M.MLP_REFROW else TOL
    check(got, oracle_mlp(d, variant, rows), f"variant {variant} T={T} H={H} I={I}", tol=tol)
    d.free()


def test_mlp_shape_domain_rejects(dev):
    """% 32 is the floor for every MXFP4 variant; the scaled variant needs
    % 64 and W4A4 % 128."""
    d = MlpData(dev, 4, 128, 256)
    out = dev.alloc(4 * 128 * 4)
    for v, (T, H, I) in ((M.MLP_FUSED, (4, 112, 256)), (M.MLP_DEQUANT, (4, 128, 240)),
                         (M.MLP_SCALED, (4, 96, 256)), (M.MLP_W4A4, (4, 192, 256))):
        with pytest.raises(M.MxError) as e:
            dev.mlp_forward(v, T, H, I, d.x, d.weights, out)
        assert e.value.code == M.MX_EINVAL
    out.free()
    d.free()


@pytest.mark.parametrize("m,n,k", [(7, 1056, 256), (64, 1000, 96), (3, 33, 64), (130, 96, 512)])
def test_mxfp4_matmul_any_n(dev, m, n, k):
    rng = np.random.default_rng(m * 3 + n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = rng.integers(118, 136, (n, k // 32), dtype=np.uint8)
    da, dq, ds = dev.upload(a), dev.upload(q), dev.upload(s)
    ref = O.mxfp4_matmul(a, q, s, n)
    for c_dtype, npdt in ((M.DT_F32, np.float32), (M.DT_F16, np.float16)):
        end = m * n * np.dtype(npdt).itemsize
        dc = dev.alloc(end + 64)
        # a canary past the last element: the N tail must not store there
        dev.upload(np.full(16, 0x7E7E7E7E, np.uint32), M.DevBuf(dev, dc.ptr + end, 64))
        dev.mxfp4_matmul(da, M.DT_F16, dq, dc, c_dtype, m, n, k, ds)
        got = dev.download(dc, npdt, (m, n))
        assert (dev.download(dc.offset(end), np.uint32, (16,)) == 0x7E7E7E7E).all()
        if c_dtype == M.DT_F32:
            check(got, ref, f"matmul {m}x{n}x{k} c=f32", tol=1e-3, cos_min=0.99999)
        else:
            # f16 C: one rounding of the f32 sum, so within one f16 step of
            # each element (2^-10 relative) plus the f32 accumulation error
            err = np.abs(got.astype(np.float64) - ref)
            rms = np.sqrt((ref ** 2).mean())
            assert (err <= 2.0 ** -10 * np.abs(ref) + 1e-4 * rms).all(), (m, n, k, (err / rms).max())
        dc.free()
    for b in (da, dq, ds):
        b.free()


@pytest.mark.parametrize("m,n,k", [(96, 1056, 512), (17, 100, 96)])
def test_gemm_f16_any_n(dev, m, n, k):
    rng = np.random.default_rng(n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    b = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    da, db, dc = dev.upload(a), dev.upload(b), dev.alloc(m * n * 4)
    dev.gemm_f16(da, M.DT_F16, db, dc, m, n, k)
    got = dev.download(dc, np.float32, (m, n))
    check(got, a.astype(np.float64) @ b.astype(np.float64).T, f"gemm_f16 {m}x{n}x{k}", tol=1e-4, cos_min=0.99999)
    for buf in (da, db, dc):
        buf.free()


@pytest.mark.parametrize("wfmt", [M.WFMT_FP8_E4M3, M.WFMT_FP8_E5M2, M.WFMT_INT8, M.WFMT_INT4])
def test_format_mlp_shape_domain(dev, wfmt):
    """The weight-format rows at % 32 shapes run on the K-step-32 kernel."""
    T, H, I = 5, 96, 160
    d = MlpData(dev, T, H, I, seed=400 + wfmt, wfmt=wfmt)
    out = dev.alloc(T * H * 2)
    dev.fmt_mlp_forward(wfmt, T, H, I, d.x, d.weights, out)
    got = dev.download(out, np.float16, (T, H))
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    ref = O.mlp_format(wfmt, x, qg, sg, qu, su, qd, sd, H, I)
    check(got, ref, f"format {wfmt} T={T} H={H} I={I}")
    out.free()
    d.free()
