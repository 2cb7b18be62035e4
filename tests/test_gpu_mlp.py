"""GPU parity of the MXFP4 matmul, SwiGLU and MLP variants vs the CPU oracle.

Tolerance: max-abs error <= 2e-2 * rms(ref) and
cosine >= 0.9995 against the dequantize-then-accumulate oracle (which
accumulates in float64).  Single matmuls are held to 1e-3 * rms.
"""
import json
import os
import types

import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData, sample_rows

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")
TOL, COS = O.MAX_ABS_REL_TOL, O.COSINE_TOL
VARIANT_MODE = {M.MLP_FUSED: O.MLP_F16, M.MLP_DEQUANT: O.MLP_F16, M.MLP_W4A4: O.MLP_W4A4}


def check(got, ref, tol=TOL, cos_min=COS, what=""):
    rel, cos = O.mlp_error(got, ref)
    print(f"{what}: max_abs/rms={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(np.asarray(got, np.float64)).all(), what
    assert rel <= tol and cos >= cos_min, (what, rel, cos)


# Shapes cover both tile widths (n % 128, n % 64), split K (few tiles, long
# K), ragged M and the K-step-32 fallback kernel (k % 64 != 0).
@pytest.mark.parametrize("m,n,k", [(1, 128, 256), (7, 192, 512), (64, 128, 1024), (100, 256, 512),
                                   (300, 64, 2048), (5, 64, 96)])
def test_mxfp4_matmul(dev, m, n, k):
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(np.float16)
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = rng.integers(118, 136, (n, k // 32), dtype=np.uint8)
    da, dq, ds = dev.upload(a), dev.upload(q), dev.upload(s)
    for c_dtype, npdt in ((M.DT_F32, np.float32), (M.DT_F16, np.float16)):
        dc = dev.alloc(m * n * 4)
        dev.mxfp4_matmul(da, M.DT_F16, dq, dc, c_dtype, m, n, k, ds)
        got = dev.download(dc, npdt, (m, n))
        ref = O.mxfp4_matmul(a, q, s, n)
        check(got, ref, tol=1e-3 if c_dtype == M.DT_F32 else 3e-3, cos_min=0.99999,
              what=f"matmul {m}x{n}x{k} c={c_dtype}")
        dc.free()


# (96, 128, 512): the tiled family; (40, 96, 160): k % 64 != 0, the
# K-step-32 kernel.  An f32 A goes in as two f16 terms (hi + lo), so both A
# types are held to f32 accumulation error (mpp_mlp_f_h_f_n128 multiplies
# f32 x half, MPPMLPKernels.metal:164-173); rounding A to f16 instead
# measured ~3e-3 of rms.
@pytest.mark.parametrize("a_f32", [False, True])
@pytest.mark.parametrize("m,n,k", [(96, 128, 512), (40, 96, 160)])
def test_gemm_f16(dev, a_f32, m, n, k):
    rng = np.random.default_rng(3 + k)
    a = rng.standard_normal((m, k)).astype(np.float32 if a_f32 else np.float16)
    b = (rng.standard_normal((n, k)) * 0.05).astype(np.float16)
    da, db, dc = dev.upload(a), dev.upload(b), dev.alloc(m * n * 4)
    dev.gemm_f16(da, M.DT_F32 if a_f32 else M.DT_F16, db, dc, m, n, k)
    got = dev.download(dc, np.float32, (m, n))
    ref = a.astype(np.float64) @ b.astype(np.float64).T
    check(got, ref, tol=1e-4, cos_min=0.9999999, what=f"gemm_f16 {m}x{n}x{k} a_f32={a_f32}")


@pytest.mark.parametrize("m,n,k", [(64, 128, 1024), (33, 96, 160)])
def test_mxfp4_matmul_f32_a(dev, m, n, k):
    """f32 activations against MXFP4 weights (two f16 terms per value, as in
    test_gemm_f16): within 1e-4 of rms of the float64 oracle."""
    rng = np.random.default_rng(m + k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    q = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    s = rng.integers(118, 130, (n, k // 32), dtype=np.uint8)
    da, dq, ds, dc = dev.upload(a), dev.upload(q), dev.upload(s), dev.alloc(m * n * 4)
    dev.mxfp4_matmul(da, M.DT_F32, dq, dc, M.DT_F32, m, n, k, ds)
    got = dev.download(dc, np.float32, (m, n))
    check(got, O.mxfp4_matmul(a, q, s, n), tol=1e-4, cos_min=0.9999999, what=f"matmul f32 A {m}x{n}x{k}")
    for buf in (da, dq, ds, dc):
        buf.free()


def test_swiglu_variants(dev):
    rng = np.random.default_rng(4)
    T, I = 8, 512
    g = (rng.standard_normal((T, I)) * 8).astype(np.float32)
    u = (rng.standard_normal((T, I)) * 8).astype(np.float32)
    dg, du = dev.upload(g), dev.upload(u)
    mid = dev.alloc(T * I * 4)
    dev.swiglu(0, dg, du, mid, T, I)
    np.testing.assert_allclose(dev.download(mid, np.float32, (T, I)), O.swiglu_float(g, u),
                               rtol=2e-6, atol=1e-6)
    dev.swiglu(1, dg, du, mid, T, I)
    got = dev.download(mid, np.float16, (T, I)).astype(np.float32)
    want = O.swiglu_half(g, u).astype(np.float32)
    np.testing.assert_allclose(got, want, rtol=1e-3, atol=1e-6)
    gh, uh = dev.upload(g.astype(np.float16)), dev.upload(u.astype(np.float16))
    dev.swiglu(2, gh, uh, mid, T, I)
    want2 = O.swiglu_half(g.astype(np.float16).astype(np.float32), u.astype(np.float16).astype(np.float32))
    np.testing.assert_allclose(dev.download(mid, np.float16, (T, I)).astype(np.float32),
                               want2.astype(np.float32), rtol=1e-3, atol=1e-6)


def test_swiglu_i8(dev):
    """Variant 3, mpp_mlp_swiglu_i8 (MPPMLPKernels.metal:240-257): int32 gate
    and up -> int8 mid, against the oracle.  Equal except where the two
    sides' exp differ in the last bit at an exact rounding midpoint (then
    by one); the closed-form cases (gate >= 20 * 4096) are exact."""
    rng = np.random.default_rng(8)
    T, I = 16, 1024
    g = rng.integers(-120000, 120000, (T, I)).astype(np.int32)
    u = rng.integers(-40000, 40000, (T, I)).astype(np.int32)
    g[0, :64] = 81920 + rng.integers(0, 1 << 20, 64)
    u[0, :64] = np.arange(-32, 32) * 16
    dg, du = dev.upload(g), dev.upload(u)
    mid = dev.alloc(T * I)
    dev.swiglu(3, dg, du, mid, T, I)
    got = dev.download(mid, np.int8, (T, I)).astype(np.int64)
    want = O.swiglu_i8(g, u).astype(np.int64)
    assert np.array_equal(got[0, :64], want[0, :64])
    assert np.abs(got - want).max() <= 1 and (got != want).mean() < 1e-3


def run_mlp(dev, d: MlpData, variant):
    out = dev.alloc(d.T * d.H * 4)
    dev.mlp_forward(variant, d.T, d.H, d.I, d.x, d.weights, out)
    dt = np.float32 if variant == M.MLP_REFROW else np.float16
    got = dev.download(out, dt, (d.T, d.H))
    out.free()
    return got


def oracle_mlp(d: MlpData, variant, rows=None):
    x, ((qg, sg), (qu, su), (qd, sd)) = d.host()
    mode = O.MLP_REFROW if variant == M.MLP_REFROW else VARIANT_MODE[variant]
    return O.mlp_mxfp4(mode, x, qg, sg, qu, su, qd, sd, d.H, d.I, rows=rows, threads=16)


@pytest.mark.parametrize("T", [1, 2, 3, 4, 8, 16, 17, 64, 128])
def test_mlp_fused_small(dev, T):
    d = MlpData(dev, T, 512, 1024, seed=T)
    got = run_mlp(dev, d, M.MLP_FUSED)
    check(got, oracle_mlp(d, M.MLP_FUSED), what=f"fused T={T}")
    # deterministic (split-K partials are added in a fixed order)
    assert np.array_equal(run_mlp(dev, d, M.MLP_FUSED).view(np.uint16), got.view(np.uint16))
    d.free()


@pytest.mark.parametrize("T", [5, 64, 130])
def test_mlp_dequant_small(dev, T):
    d = MlpData(dev, T, 512, 1024, seed=100 + T)
    check(run_mlp(dev, d, M.MLP_DEQUANT), oracle_mlp(d, M.MLP_DEQUANT), what=f"dequant T={T}")
    d.free()


# hidden % 256 == 0 runs the stage-major 256x256 kernels; (96, 640, 1152)
# takes the 256x128 kernels that read the reference scale layout directly.
# Split-K of the down GEMM (f32 partials + reduce launch) on the stage-major
# path: (64, 512, 1024) in 2 splits, (256, 1024, 2048) in 4, (130, 1024,
# 4096) in 8 with a ragged last tile row, (400, 512, 2048) in 4 over two
# row tiles (the second ragged).  Unsplit grids with H and I multiples of
# 512 run both GEMMs on the 128-K-stage kernel with stage-major x and mid:
# (300, 1024, 1536) with a ragged second row tile, (520, 1024, 1536) with
# three row tiles (36 gate/up tiles, not a multiple of the 8 XCDs).
@pytest.mark.parametrize("T,H,I", [(64, 512, 1024), (256, 1024, 2048), (300, 768, 1536), (96, 640, 1152),
                                   (130, 1024, 4096), (400, 512, 2048), (300, 1024, 1536), (520, 1024, 1536)])
def test_mlp_w4a4_small(dev, T, H, I):
    d = MlpData(dev, T, H, I, seed=200 + T)
    got = run_mlp(dev, d, M.MLP_W4A4)
    check(got, oracle_mlp(d, M.MLP_W4A4), what=f"w4a4 T={T}")
    # deterministic (split-K partials are added in a fixed order)
    assert np.array_equal(run_mlp(dev, d, M.MLP_W4A4).view(np.uint16), got.view(np.uint16))
    d.free()


def test_refrow_reference_checksum(dev):
    """The reference's fused-row semantics on its own LCG data reproduce the
    published checksum 403573 (README.md:292-294)."""
    kat = json.load(open(os.path.join(GOLD, "checksum_kat.json")))
    T, H, I = kat["tokens"], kat["hidden"], kat["intermediate"]
    pat = kat["e8m0"]["pattern"]
    x = M.lcg_half(kat["x"]["seed"], T * H, kat["x"]["scale"]).reshape(T, H)
    q = [M.lcg_bytes(kat["fp4"][n], I * H // 2) for n in ("gate", "up", "down")]
    s = [M.lcg_pattern(kat["e8m0"][n], I * H // 32, pat) for n in ("gate", "up", "down")]
    dx = dev.upload(x)
    dq = [dev.upload(a) for a in q]
    ds = [dev.upload(a) for a in s]
    w = M.Device.weights((dq[0], ds[0]), (dq[1], ds[1]), (dq[2], ds[2]))
    out = dev.alloc(T * H * 4)
    dev.mlp_forward(M.MLP_REFROW, T, H, I, dx, w, out)
    got = dev.download(out, np.float32, (T, H))
    ref = O.mlp_mxfp4(O.MLP_REFROW, x, q[0].reshape(I, -1), s[0].reshape(I, -1), q[1].reshape(I, -1),
                      s[1].reshape(I, -1), q[2].reshape(H, -1), s[2].reshape(H, -1), H, I, threads=16)
    check(got, ref, tol=2e-3, cos_min=0.99999, what="refrow C0")
    cs, n = M.checksum_f32(got)
    print(f"checksum: {cs:.6g} over {n} samples", flush=True)
    assert n == 32 and abs(cs - 403573) / 403573 < 2e-5


def test_mlp_invalid_arguments(dev):
    d = MlpData(dev, 4, 128, 256)
    out = dev.alloc(4 * 128 * 2)
    # zero tokens; hidden or intermediate not a multiple of 16 / of 32 (the
    # reference's MXFP4 rows need % 32, main.swift:1043)
    for (T, H, I) in ((0, 128, 256), (4, 120, 256), (4, 128, 240), (4, 112, 256)):
        with pytest.raises(M.MxError) as e:
            dev.mlp_forward(M.MLP_FUSED, T, H, I, d.x, d.weights, out)
        assert e.value.code == M.MX_EINVAL
    with pytest.raises(M.MxError):
        dev.mlp_forward(M.MLP_W4A4, 4, 192, 256, d.x, d.weights, out)   # W4A4 needs % 128
    with pytest.raises(M.MxError):
        dev.mlp_forward(9, 4, 128, 256, d.x, d.weights, out)
    d.free()


# ---- BASELINE configurations (full sizes, sampled token rows) --------------
def test_config0_all_variants(dev):
    d = MlpData(dev, 128, 1024, 4096, seed=7)
    for v in (M.MLP_FUSED, M.MLP_DEQUANT, M.MLP_W4A4):
        check(run_mlp(dev, d, v), oracle_mlp(d, v), what=f"C0 variant {v}")
    d.free()


@pytest.mark.parametrize("T", [1, 8])
def test_config1_decode(dev, T):
    d = MlpData(dev, T, 7168, 2048, seed=11 + T)
    check(run_mlp(dev, d, M.MLP_FUSED), oracle_mlp(d, M.MLP_FUSED), what=f"C1 T={T}")
    d.free()


def test_config2_fused_and_dequant(dev):
    d = MlpData(dev, 512, 7168, 2048, seed=13)
    rows = sample_rows(512, 24)
    ref = oracle_mlp(d, M.MLP_FUSED, rows=rows)
    for v in (M.MLP_FUSED, M.MLP_DEQUANT):
        check(run_mlp(dev, d, v)[rows], ref, what=f"C2 variant {v}")
    d.free()


def test_fused_gate_up_chunk_scales(dev):
    """Fused MLP whose gate/up GEMM has more workgroups than CUs (288 tiles,
    2-slot ring) and 28 KB of E8M0 scales per workgroup (K = 8192): the
    scales are loaded per 4-stage B chunk, one 8-byte load per lane."""
    T, H, I = 2304, 8192, 1024
    d = MlpData(dev, T, H, I, seed=29)
    rows = sample_rows(T, 12)
    check(run_mlp(dev, d, M.MLP_FUSED)[rows], oracle_mlp(d, M.MLP_FUSED, rows=rows), what="fused, chunk scales")
    d.free()


def test_w4a4_ragged_scale_tiles(dev):
    """W4A4 with more than 2^20 weight-scale dwords (the tiled stage-major
    conversion) and stage counts that leave partial 32-stage tiles (gate/up
    18 stages, down 157)."""
    T, H, I = 64, 2304, 20096
    d = MlpData(dev, T, H, I, seed=19)
    rows = sample_rows(T, 8)
    check(run_mlp(dev, d, M.MLP_W4A4)[rows], oracle_mlp(d, M.MLP_W4A4, rows=rows), what="W4A4 ragged tiles")
    d.free()


def test_config4_w4a4(dev):
    d = MlpData(dev, 4096, 8192, 28672, seed=17)
    rows = sample_rows(4096, 12)
    got = run_mlp(dev, d, M.MLP_W4A4)
    check(got[rows], oracle_mlp(d, M.MLP_W4A4, rows=rows), what="C4 W4A4")
    assert np.isfinite(got.astype(np.float32)).all()
    d.free()


def test_benchmark_entry_point(dev):
    d = MlpData(dev, 8, 1024, 2048, seed=3)
    out = dev.alloc(8 * 1024 * 2)
    secs, kern = dev.mlp_benchmark(M.MLP_FUSED, 8, 1024, 2048, d.x, [d.weights] * 2, out,
                                   warmup=1, iterations=5)
    # 8 tokens: the decode GEMVs
    assert secs > 0 and list(kern) == ["gemv_mxfp4_gate_up_swiglu", "gemv_mxfp4_down"], kern
    assert all(v > 0 for v in kern.values()), kern
    secs, kern = dev.mlp_benchmark(M.MLP_FUSED, 8, 1024, 2048, d.x, [d.weights] * 2, out,
                                   warmup=1, iterations=5, graph=False)
    assert secs > 0
    dev.sync()
    out.free()
    d.free()


# ---- decode GEMV path (tokens <= 16) -----------------------------------------
# Shapes: fewest workgroups (H = I = 128, down waves with no K step), several
# load batches per wave (K = 8192 and 16384), the largest token count, and
# gate/up K with an odd number of 128-K steps under the rolling whole-line
# issue (H = 4480 and 4224: a half last line column, tail columns clamped).
@pytest.mark.parametrize("T,H,I", [(3, 128, 128), (4, 256, 8192), (1, 16384, 128), (16, 1024, 512),
                                   (1, 4480, 384), (5, 4224, 640)])
def test_decode_gemv_shapes(dev, T, H, I):
    d = MlpData(dev, T, H, I, seed=T + H // 128)
    check(run_mlp(dev, d, M.MLP_FUSED), oracle_mlp(d, M.MLP_FUSED), what=f"decode T={T} H={H} I={I}")
    d.free()


@pytest.mark.parametrize("T,which", [(1, "down"), (5, "down"), (1, "gate"), (3, "up")])
def test_decode_e8m0_255(dev, T, which):
    """E8M0 byte 255 is +inf to the reference (bits << 23), NaN to the
    hardware's scaled convert: the GEMV decodes a workgroup holding one
    exactly, so NaN and +-inf land where the oracle's do and the finite
    outputs stay within tolerance.  A byte-0 block (2^-127) rides along."""
    H, I = 512, 1024
    d = MlpData(dev, T, H, I, seed=91 + T)
    q, s, n, k = d.mats[{"gate": 0, "up": 1, "down": 2}[which]]
    sc = dev.download(s, np.uint8, (n, k // 32))
    sc[3, 2] = 255
    sc[n - 1, :] = 255
    sc[100, 0] = 0
    dev.upload(sc, s)
    got = run_mlp(dev, d, M.MLP_FUSED).astype(np.float64)
    ref = oracle_mlp(d, M.MLP_FUSED)
    assert np.isnan(ref).any()
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    if which == "down":  # columns 3 and H-1 are non-finite, the rest are not
        assert fin.sum() == T * (H - 2)
        rel, cos = O.mlp_error(got[fin], ref[fin])
        assert rel <= TOL and cos >= COS, (rel, cos)
    d.free()


@pytest.mark.parametrize("T", [1, 5])
def test_decode_scale_planes_4_byte_aligned(dev, T):
    """The C ABI accepts scale planes that are only 4-byte aligned.  The
    decode GEMV stages 16-byte aligned planes in 16-byte pieces and others
    in dwords: copies of the same planes at a 4-byte offset must give the
    same output bits."""
    H, I = 1024, 2048
    d = MlpData(dev, T, H, I, seed=71 + T)
    ref = run_mlp(dev, d, M.MLP_FUSED)
    shifted, mats = [], []
    for q, s, n, k in d.mats:
        host = dev.download(s, np.uint8, (n * (k // 32),))
        buf = dev.upload(np.concatenate([np.zeros(4, np.uint8), host, np.zeros(12, np.uint8)]))
        shifted.append(buf)
        mats.append((q, types.SimpleNamespace(ptr=buf.ptr + 4)))
    w = M.Device.weights(*mats)
    out = dev.alloc(T * H * 2)
    dev.mlp_forward(M.MLP_FUSED, T, H, I, d.x, w, out)
    got = dev.download(out, np.float16, (T, H))
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    check(got, oracle_mlp(d, M.MLP_FUSED), what=f"decode T={T}, 4-byte aligned scale planes")
    out.free()
    for b in shifted:
        b.free()
    d.free()


def test_decode_back_to_back_distinct_inputs(dev):
    """Consecutive forwards with different inputs share the context's mid
    buffer; enqueued back to back, each must produce its own result."""
    T, H, I = 2, 1024, 2048
    a, b = MlpData(dev, T, H, I, seed=41), MlpData(dev, T, H, I, seed=43)
    refs = [run_mlp(dev, a, M.MLP_FUSED), run_mlp(dev, b, M.MLP_FUSED)]
    assert not np.array_equal(refs[0], refs[1])
    outs = [dev.alloc(T * H * 2) for _ in range(24)]
    for n, o in enumerate(outs):  # no host sync in between
        d = (a, b)[n % 2]
        dev.mlp_forward(M.MLP_FUSED, T, H, I, d.x, d.weights, o)
    dev.sync()
    for n, o in enumerate(outs):
        got = dev.download(o, np.float16, (T, H))
        assert np.array_equal(got.view(np.uint16), refs[n % 2].view(np.uint16)), n
        o.free()
    a.free()
    b.free()


def test_decode_many_launches(dev):
    """The decode MLP over rotated weight sets, 200 forwards from one captured
    graph (the benchmark's form) and 200 from the stream, then one forward
    per set checked against the oracle: the shared mid buffer and the graph
    replays leave every later forward correct."""
    T, H, I = 1, 1024, 2048
    sets = [MlpData(dev, T, H, I, seed=500 + s) for s in range(4)]
    out = dev.alloc(T * H * 2)
    dev.mlp_benchmark(M.MLP_FUSED, T, H, I, sets[0].x, [d.weights for d in sets], out, warmup=2,
                      iterations=200, per_kernel=False, graph=True)
    dev.mlp_benchmark(M.MLP_FUSED, T, H, I, sets[0].x, [d.weights for d in sets], out, warmup=0,
                      iterations=200, per_kernel=False, graph=False)
    for d in sets:
        check(run_mlp(dev, d, M.MLP_FUSED), oracle_mlp(d, M.MLP_FUSED), what="after many launches")
        d.free()
    out.free()


@pytest.mark.parametrize("T,H,I", [(1, 512, 1024), (3, 1024, 2048)])
def test_decode_nonfinite_activations(dev, T, H, I):
    """An inf or NaN activation propagates through the decode path as through
    the reference's dequantize-then-accumulate: the outputs are non-finite
    where the oracle's are and within tolerance elsewhere."""
    d = MlpData(dev, T, H, I, seed=71 + T)
    x = dev.download(d.x, np.float16, (T, H))
    x[0, 5] = np.inf
    x[T - 1, H - 3] = np.nan if T > 1 else x[T - 1, H - 3]
    dev.upload(x, d.x)
    got = run_mlp(dev, d, M.MLP_FUSED).astype(np.float64)
    ref = oracle_mlp(d, M.MLP_FUSED)
    assert np.array_equal(np.isnan(got), np.isnan(ref))
    assert np.array_equal(np.isposinf(got), np.isposinf(ref))
    assert np.array_equal(np.isneginf(got), np.isneginf(ref))
    fin = np.isfinite(ref)
    if fin.any():
        rel, cos = O.mlp_error(got[fin], ref[fin])
        assert rel <= TOL and cos >= COS, (rel, cos)
    d.free()


def _plant_e8m0(dev, d, which, rows_255, row_0):
    q, s, n, k = d.mats[{"gate": 0, "up": 1, "down": 2}[which]]
    sc = dev.download(s, np.uint8, (n, k // 32))
    for r, b in rows_255:
        if b is None:
            sc[r, :] = 255
        else:
            sc[r, b] = 255
    sc[row_0, 0] = 0
    dev.upload(sc, s)


def _check_nonfinite_pattern(got, ref, what):
    got = got.astype(np.float64)
    assert np.array_equal(np.isnan(got), np.isnan(ref)), what
    assert np.array_equal(np.isposinf(got), np.isposinf(ref)), what
    assert np.array_equal(np.isneginf(got), np.isneginf(ref)), what
    fin = np.isfinite(ref)
    if fin.any():
        rel, cos = O.mlp_error(got[fin], ref[fin])
        assert rel <= TOL and cos >= COS, (what, rel, cos)


@pytest.mark.parametrize("variant", [M.MLP_FUSED, M.MLP_DEQUANT])
@pytest.mark.parametrize("which", ["gate", "down"])
def test_e8m0_endpoints_tiled_paths(dev, variant, which):
    """E8M0 bytes 255 (+inf in the reference, MXFP4Kernels.metal:26-29) and
    0 (0.0) on the tiled small-M GEMM (fused, T > 16) and on the
    dequant-to-half path: non-finite outputs where the oracle has them,
    tolerance elsewhere."""
    T, H, I = 40, 512, 1024
    d = MlpData(dev, T, H, I, seed=131 + variant)
    _plant_e8m0(dev, d, which, [(3, 2), (I - 1 if which != "down" else H - 1, None)], 100)
    got = run_mlp(dev, d, variant)
    ref = oracle_mlp(d, variant)
    assert np.isnan(ref).any() or np.isinf(ref).any()
    _check_nonfinite_pattern(got, ref, f"variant {variant} {which}")
    d.free()


# (64, 512, 1024): stage-major planes, the down GEMM split over K (its reduce
# stores); (512, 2048, 512): the 128-K-stage kernel with stage-major x and
# mid (gate/up epilogue and down stores); (300, 768, 1536): the unsplit
# 256-K-stage down GEMM stores;
# (64, 512, 640): the 128-K-stage down GEMM (K % 512 != 0) stores; (96, 640,
# 1152): reference-layout planes with the separate byte-255 pass.
@pytest.mark.parametrize("T,H,I", [(64, 512, 1024), (512, 2048, 512), (300, 768, 1536), (64, 512, 640),
                                   (96, 640, 1152)])
@pytest.mark.parametrize("which", ["up", "down"])
def test_e8m0_endpoints_w4a4(dev, T, H, I, which):
    """W4A4 (both scale layouts): byte 255 in an up scale makes the channel's
    mid non-finite on both sides, so every output of those tokens is NaN;
    in a down scale the scaled MFMA's NaN is rewritten to the reference's
    +-inf where every product of the block is an infinity of one sign.  A
    down row whose codes are all non-zero and positive, met by a token whose
    mid codes there are too, must come out +inf.  Byte 0 (0.0 in the
    reference, 2^-127 in hardware) stays within tolerance."""
    d = MlpData(dev, T, H, I, seed=151 + T)
    if which == "up":
        _plant_e8m0(dev, d, "up", [(5, 1)], 17)
    else:
        # token 0 meets down row 7 with an infinite scale on block 3 (mid
        # channels 96..127) through all-positive, non-zero products: x row 0
        # positive, gate/up rows 96..127 and down row 7 all code +1.0, so
        # mid[0][96..127] are equal positive values -> +inf in the reference
        x = dev.download(d.x, np.float16, (T, H))
        x[0] = np.abs(x[0]) + np.float16(0.25)
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
        _plant_e8m0(dev, d, "down", [(7, 3), (H - 1, None), (11, 0)], 17)
    got = run_mlp(dev, d, M.MLP_W4A4)
    ref = oracle_mlp(d, M.MLP_W4A4)
    assert (~np.isfinite(ref)).any()
    if which == "down":
        assert np.isposinf(ref[0, 7]), ref[0, 7]
    _check_nonfinite_pattern(got, ref, f"w4a4 {which} T={T} H={H} I={I}")
    d.free()
