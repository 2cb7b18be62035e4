"""GPU parity of the weight-format rows.

Reference rows: mpp_mlp_h_fp8e4m3_f / _h_fp8e5m2_f / _h_i8_f / _h_i4_f /
i8_i8_i32 (MPPMLPKernels.metal:50-125), unscaled in the reference; BASELINE
adds per-row (FP8, INT8) and per-32 f16 (INT4) scales.  Quantizers must be
bit-exact with the oracle; MLP outputs within the BASELINE tolerance.
"""
import types

import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData, sample_rows

pytestmark = pytest.mark.gpu
FMTS = [M.WFMT_FP8_E4M3, M.WFMT_FP8_E5M2, M.WFMT_INT8, M.WFMT_INT4]
MLP_FMTS = FMTS + [M.WFMT_W8A8]


@pytest.mark.parametrize("m,n,k", [(1, 64, 128), (77, 192, 1024), (128, 256, 4096), (260, 128, 256)])
def test_gemm_i8_bitexact(dev, m, n, k):
    """The W8A8 core (mpp_mlp_i8_i8_i32_n128, MPPMLPKernels.metal:61-70):
    exact int32 sums, including split K (128 x 256 x 4096) and ragged M."""
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.integers(-128, 128, (m, k), dtype=np.int8)
    b = rng.integers(-128, 128, (n, k), dtype=np.int8)
    a[0, :] = -128   # extreme row: |sum| up to k * 2^14
    b[0, :] = -128
    da, db, dc = dev.upload(a), dev.upload(b), dev.alloc(m * n * 4)
    dev.gemm_i8(da, db, dc, m, n, k)
    got = dev.download(dc, np.int32, (m, n))
    ref = a.astype(np.int64) @ b.astype(np.int64).T
    assert np.array_equal(got.astype(np.int64), ref)
    for buf in (da, db, dc):
        buf.free()


def test_gemm_i8_rejects_bad_shapes(dev):
    a, b, c = dev.alloc(64 * 256), dev.alloc(64 * 256), dev.alloc(64 * 64 * 4)
    for (m, n, k) in ((4, 64, 96), (4, 96, 128), (0, 64, 128)):
        with pytest.raises(M.MxError) as e:
            dev.gemm_i8(a, b, c, m, n, k)
        assert e.value.code == M.MX_EINVAL


@pytest.mark.parametrize("wfmt", FMTS)
def test_format_quantizer_bitexact(dev, wfmt):
    rng = np.random.default_rng(wfmt)
    rows, k = 96, 1024
    w = rng.normal(0, 0.02, (rows, k)).astype(np.float32)
    w[3] *= 1e4
    w[5, :64] = 0
    dw = dev.upload(w)
    if wfmt == M.WFMT_INT4:
        q, s = dev.alloc(rows * k // 2), dev.alloc(rows * k // 32 * 2)
        dev.fmt_quantize(wfmt, dw, rows, k, q, s)
        oq, os_ = O.quant_int4_g32(w)
        assert np.array_equal(dev.download(s, np.uint16, (rows, k // 32)), os_.view(np.uint16))
        assert np.array_equal(dev.download(q, np.uint8, (rows, k // 2)), oq)
    else:
        q, s = dev.alloc(rows * k), dev.alloc(rows * 4)
        dev.fmt_quantize(wfmt, dw, rows, k, q, s)
        oq, os_ = O.quant_rowwise(wfmt, w)
        assert np.array_equal(dev.download(s, np.float32, (rows,)), os_)
        assert np.array_equal(dev.download(q, np.uint8, (rows, k)), oq)


def run_fmt(dev, d, wfmt):
    out = dev.alloc(d.T * d.H * 2)
    dev.fmt_mlp_forward(wfmt, d.T, d.H, d.I, d.x, d.weights, out)
    got = dev.download(out, np.float16, (d.T, d.H))
    out.free()
    return got


def oracle_fmt(d, wfmt, rows=None):
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    return O.mlp_format(wfmt, x, qg, sg, qu, su, qd, sd, d.H, d.I, rows=rows, threads=16)


@pytest.mark.parametrize("wfmt", MLP_FMTS)
@pytest.mark.parametrize("T", [3, 128])
def test_format_mlp_small(dev, wfmt, T):
    d = MlpData(dev, T, 512, 1024, seed=wfmt * 10 + T, wfmt=wfmt)
    got = run_fmt(dev, d, wfmt)
    rel, cos = O.mlp_error(got, oracle_fmt(d, wfmt))
    print(f"fmt {wfmt} T={T}: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    d.free()


@pytest.mark.parametrize("wfmt", MLP_FMTS)
def test_format_mlp_deep_ragged(dev, wfmt):
    """Gate/up on the deep ring (K = 1024: 16 stages; 2 x 32 tiles), a
    ragged second token tile, and per-workgroup start stages that wrap
    (7 (w / 8) mod 16)."""
    d = MlpData(dev, 130, 1024, 2048, seed=53 + wfmt, wfmt=wfmt)
    got = run_fmt(dev, d, wfmt)
    rel, cos = O.mlp_error(got, oracle_fmt(d, wfmt))
    print(f"fmt {wfmt} T=130 H=1024 I=2048: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    d.free()


@pytest.mark.parametrize("wfmt", [M.WFMT_FP8_E4M3, M.WFMT_INT8])
def test_format_mlp_deep_kt12(dev, wfmt):
    """Gate/up on the deep ring with 12 stages (K = 768) over 192 tiles:
    start stages 7 (w / 8) mod 12 take every residue, so the wrap of the
    rotated K order is exercised away from a power of two."""
    d = MlpData(dev, 128, 768, 12288, seed=61 + wfmt, wfmt=wfmt)
    rows = sample_rows(128, 16)
    got = run_fmt(dev, d, wfmt)[rows]
    rel, cos = O.mlp_error(got, oracle_fmt(d, wfmt, rows=rows))
    print(f"fmt {wfmt} T=128 H=768 I=12288: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    d.free()


@pytest.mark.parametrize("wfmt", MLP_FMTS)
def test_config3_formats(dev, wfmt):
    d = MlpData(dev, 128, 4096, 14336, seed=31 + wfmt, wfmt=wfmt)
    rows = sample_rows(128, 16)
    got = run_fmt(dev, d, wfmt)[rows]
    rel, cos = O.mlp_error(got, oracle_fmt(d, wfmt, rows=rows))
    print(f"C3 fmt {wfmt}: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    d.free()


def test_int4_scale_planes_4_byte_aligned(dev):
    """INT4 scale planes at a 4-byte offset against 16-byte aligned ones,
    same output bits.  The gate/up GEMM (224 tiles, deep ring) copies its
    32 KB of f16 scales per workgroup to LDS by dword DMA either way; the
    down GEMM (2-slot ring, scales not in LDS) loads a B chunk's scales
    with one 16-byte load per lane from aligned planes and one scale per
    stage from shifted ones."""
    T, H, I = 32, 4096, 14336
    d = MlpData(dev, T, H, I, seed=41, wfmt=M.WFMT_INT4)
    ref = run_fmt(dev, d, M.WFMT_INT4)
    shifted, mats = [], []
    for q, s, n, k in d.mats:
        host = dev.download(s, np.uint8, (n * (k // 32) * 2,))
        buf = dev.upload(np.concatenate([np.zeros(4, np.uint8), host, np.zeros(12, np.uint8)]))
        shifted.append(buf)
        mats.append((q, types.SimpleNamespace(ptr=buf.ptr + 4)))
    out = dev.alloc(T * H * 2)
    dev.fmt_mlp_forward(M.WFMT_INT4, T, H, I, d.x, M.Device.weights(*mats), out)
    got = dev.download(out, np.float16, (T, H))
    assert np.isfinite(ref.astype(np.float64)).all()
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    out.free()
    for b in shifted:
        b.free()
    d.free()


# ---- FP8 rows on the FP8 matrix cores (MX_WFMT_FP8_*_F8X2) -------------------
# Same weights and reference semantics as MX_WFMT_FP8_E4M3 / _E5M2 (the
# oracle's modes 1 / 2); x and mid go in as two E4M3 terms per value (F8X2,
# relative error <= 2^-8 each), so the rows are held to the BASELINE
# tolerance against the oracle and to 1e-2 of rms against the widening row.
F8X2_FMTS = [(M.WFMT_FP8_E4M3_F8X2, M.WFMT_FP8_E4M3), (M.WFMT_FP8_E5M2_F8X2, M.WFMT_FP8_E5M2)]


# T: ragged single tiles (1, 17), a full tile's worth (64), two tiles with a
# partial one (130); H = 512 / I = 1024 split K in both GEMMs
@pytest.mark.parametrize("fmt,base", F8X2_FMTS)
@pytest.mark.parametrize("T", [1, 17, 64, 130])
def test_f8x2_format_mlp_small(dev, fmt, base, T):
    d = MlpData(dev, T, 512, 1024, seed=300 + T + fmt, wfmt=base)
    got = run_fmt(dev, d, fmt)
    rel, cos = O.mlp_error(got, oracle_fmt(d, base))
    print(f"fmt {fmt} T={T}: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(got.astype(np.float64)).all()
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    # deterministic (split-K partials summed in a fixed order)
    assert np.array_equal(run_fmt(dev, d, fmt).view(np.uint16), got.view(np.uint16))
    rel2, cos2 = O.mlp_error(got, run_fmt(dev, d, base).astype(np.float64))
    assert rel2 <= 1e-2 and cos2 >= 0.99999, (rel2, cos2)
    d.free()


@pytest.mark.parametrize("fmt,base", F8X2_FMTS)
def test_f8x2_config3(dev, fmt, base):
    """C3 shape: gate/up on the deep ring unsplit (224 tiles), down on the
    deep ring with 8 K splits and the reduce."""
    d = MlpData(dev, 128, 4096, 14336, seed=41 + fmt, wfmt=base)
    rows = sample_rows(128, 16)
    got = run_fmt(dev, d, fmt)[rows]
    rel, cos = O.mlp_error(got, oracle_fmt(d, base, rows=rows))
    print(f"C3 fmt {fmt}: rel={rel:.3e} cos={cos:.7f}", flush=True)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL
    d.free()


@pytest.mark.parametrize("fmt,base", F8X2_FMTS)
@pytest.mark.parametrize("T,H,I", [(64, 512, 256), (128, 1024, 4096)])
def test_f8x2_nonfinite_x(dev, fmt, base, T, H, I):
    """A non-finite activation cannot be an F8X2 term: its group is marked
    (E8M0 255, NaN in the MFMA) and the outputs it reaches are recomputed
    with the reference's arithmetic, so NaN, +inf and -inf land where the
    oracle's do.  Token 0 holds +inf, token 1 -inf, token 2 NaN; (64, 512,
    256) stores from the GEMM epilogues, (128, 1024, 4096) from the split-K
    reduces."""
    d = MlpData(dev, T, H, I, seed=61 + fmt, wfmt=base)
    x = dev.download(d.x, np.float16, (T, H))
    x[0, 5] = np.inf
    x[1, 70] = -np.inf
    x[2, 300] = np.nan
    dev.upload(x, d.x)
    got = run_fmt(dev, d, fmt).astype(np.float64)
    ref = oracle_fmt(d, base).astype(np.float64)
    assert not np.isfinite(ref[:3]).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref)), (np.isnan(got).sum(), np.isnan(ref).sum())
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    rel, cos = O.mlp_error(got[3:], ref[3:])
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL, (rel, cos)
    d.free()


def test_f8x2_format_rejects_bad_shapes(dev):
    d = MlpData(dev, 4, 256, 512, seed=3, wfmt=M.WFMT_FP8_E4M3)
    out = dev.alloc(4 * 256 * 2)
    with pytest.raises(M.MxError) as e:
        dev.fmt_mlp_forward(M.WFMT_FP8_E4M3_F8X2, 4, 96, 512, d.x, d.weights, out)  # hidden % 64
    assert e.value.code == M.MX_EINVAL
    out.free()
    d.free()
