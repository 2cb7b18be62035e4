"""Accumulator precision / overflow probe (the reference's --accum-probe,
main.swift:1523-1713 over AccumProbeKernels.metal:41-127) through
mx_accum_gemm, and the parity of its FP4 x FP4 / FP8 x FP8 kernel.

What the reference measured and its README states (README.md:342-352) is
asserted here for this build's paths: accumulation is f32-wide (sums of
ones are exact to K = 131072 with a float destination), a half destination
is one RNE rounding of that sum (65448 -> 65440) and overflows to inf once
the value reaches the rounding boundary 65520 (FP8 16 x 16 at K = 256: half
inf, float 65536), with no saturation."""
import numpy as np
import pytest

import mxfp4hip as M
import oracle as O

pytestmark = pytest.mark.gpu

MM, NN, MAX_K = 64, 128, 131072
ONES_KS = [1024, 2048, 2080, 4096, 4160, 8192, 16384, 32768, 65504, 65536, 131072]


@pytest.fixture(scope="module")
def fills(dev):
    """Constant-filled operands at the largest K (main.swift:1545-1580)."""
    bufs = {}

    def half(rows, bits):
        return dev.upload(np.full(rows * MAX_K, bits, np.uint16))

    def byte(rows, per_elem, value):
        b = dev.alloc(int(rows * MAX_K * per_elem))
        dev.memset(b, value)
        return b

    bufs["h1"] = (half(MM, 0x3C00), half(NN, 0x3C00))
    bufs["h8"] = (half(MM, 0x4800), half(NN, 0x4800))
    bufs["q1"] = (byte(MM, 0.5, 0x22), byte(NN, 0.5, 0x22))
    bufs["q6"] = (byte(MM, 0.5, 0x77), byte(NN, 0.5, 0x77))
    bufs["e1"] = (byte(MM, 1, 0x38), byte(NN, 1, 0x38))
    bufs["e16"] = (byte(MM, 1, 0x58), byte(NN, 1, 0x58))
    yield bufs
    for a, b in bufs.values():
        a.free()
        b.free()


PATHS = {  # name: (a_fmt, b_fmt, fill, product, ks)
    "h_h_ones": (M.PROBE_F16, M.PROBE_F16, "h1", 1.0, ONES_KS),
    "h_fp4_ones": (M.PROBE_F16, M.PROBE_FP4, "h1q1", 1.0, ONES_KS),
    "fp4_fp4_ones": (M.PROBE_FP4, M.PROBE_FP4, "q1", 1.0, ONES_KS),
    "fp8_fp8_ones": (M.PROBE_FP8, M.PROBE_FP8, "e1", 1.0, ONES_KS),
    "h_h_64": (M.PROBE_F16, M.PROBE_F16, "h8", 64.0, [512, 1022, 1024, 2048]),
    "fp4_fp4_36": (M.PROBE_FP4, M.PROBE_FP4, "q6", 36.0, [1024, 1818, 1820, 2048, 4096]),
    "fp8_fp8_256": (M.PROBE_FP8, M.PROBE_FP8, "e16", 256.0, [128, 254, 256, 1024]),
}


def run_probe(dev, fills, path, k, half):
    a_fmt, b_fmt, fill, _, _ = PATHS[path]
    a, b = (fills["h1"][0], fills["q1"][1]) if fill == "h1q1" else fills[fill]
    c = dev.alloc(MM * NN * (2 if half else 4))
    dev.accum_gemm(a_fmt, a, b_fmt, b, c, M.DT_F16 if half else M.DT_F32, MM, NN, k)
    got = dev.download(c, np.float16 if half else np.float32, (MM, NN)).astype(np.float64)
    c.free()
    return got


@pytest.mark.parametrize("path", list(PATHS))
def test_accum_probe_sweep(dev, fills, path):
    _, _, _, product, ks = PATHS[path]
    for k in ks:
        exact = product * k
        f = run_probe(dev, fills, path, k, half=False)
        h = run_probe(dev, fills, path, k, half=True)
        assert (f == f[0, 0]).all() and (h == h[0, 0]).all(), (path, k)  # uniform tile
        # f32 accumulation: every exact sum here is an integer below 2^24
        assert f[0, 0] == exact, (path, k, f[0, 0])
        # one RNE rounding of that sum to half (IEEE conversion, overflow -> inf)
        with np.errstate(over="ignore"):
            assert h[0, 0] == float(np.float16(np.float32(exact))), (path, k, h[0, 0])
        print(f"{path} K={k}: exact {exact:.0f} half {h[0, 0]} float {f[0, 0]}", flush=True)


def test_accum_probe_reference_findings(dev, fills):
    """The reference's published results (README.md:342-352), literally."""
    assert run_probe(dev, fills, "fp4_fp4_ones", 131072, half=False)[0, 0] == 131072
    assert run_probe(dev, fills, "h_h_ones", 65504, half=True)[0, 0] == 65504
    assert run_probe(dev, fills, "fp4_fp4_36", 1818, half=True)[0, 0] == 65440   # exact 65448
    assert np.isposinf(run_probe(dev, fills, "fp4_fp4_36", 1820, half=True)[0, 0])  # 65520
    assert np.isposinf(run_probe(dev, fills, "fp8_fp8_256", 256, half=True)[0, 0])
    assert run_probe(dev, fills, "fp8_fp8_256", 256, half=False)[0, 0] == 65536
    # no saturation to 65504 and no wrap-around anywhere past the boundary
    assert np.isposinf(run_probe(dev, fills, "h_h_64", 2048, half=True)[0, 0])


@pytest.mark.parametrize("fmt,m,n,k", [(M.PROBE_FP4, 64, 128, 512), (M.PROBE_FP4, 96, 64, 1024),
                                       (M.PROBE_FP4, 64, 64, 544), (M.PROBE_FP4, 32, 64, 1818),
                                       (M.PROBE_FP8, 64, 128, 512), (M.PROBE_FP8, 32, 192, 256),
                                       (M.PROBE_FP8, 32, 64, 288), (M.PROBE_FP8, 64, 64, 254)])
def test_accum_gemm_random_parity(dev, fmt, m, n, k):
    """Random codes (FP8 NaN codes 0x7F / 0xFF excluded) against the oracle's
    decode and a float64 dot product; checks the MFMA operand layout and the
    zero padding of K to a multiple of 64 (k = 544, 1818, 288, 254)."""
    rng = np.random.default_rng(m + n + k + fmt)
    if fmt == M.PROBE_FP4:
        a_b = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
        b_b = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
        dec = lambda x, rows: O.unpack(M.FMT_FP4_E2M1, x.reshape(-1), rows * k).reshape(rows, k)
    else:
        a_b = rng.integers(0, 256, (m, k), dtype=np.uint8)
        b_b = rng.integers(0, 256, (n, k), dtype=np.uint8)
        a_b[(a_b & 0x7F) == 0x7F] = 0
        b_b[(b_b & 0x7F) == 0x7F] = 0
        dec = lambda x, rows: O.unpack(M.FMT_FP8_E4M3, x.reshape(-1), rows * k).reshape(rows, k)
    ref = dec(a_b, m).astype(np.float64) @ dec(b_b, n).astype(np.float64).T
    a, b = dev.upload(a_b), dev.upload(b_b)
    outs = {}
    for half in (False, True):
        c = dev.alloc(m * n * (2 if half else 4))
        dev.accum_gemm(fmt, a, fmt, b, c, M.DT_F16 if half else M.DT_F32, m, n, k)
        outs[half] = dev.download(c, np.float16 if half else np.float32, (m, n))
        c.free()
    # f32 accumulation against the exact (float64) dot products
    scale = np.abs(dec(a_b, m)).max() * np.abs(dec(b_b, n)).max() * k
    assert np.abs(outs[False].astype(np.float64) - ref).max() <= 1e-6 * scale, (fmt, m, n, k)
    # the half destination is one RNE rounding of the same f32 sum (the two
    # launches add in the same order), inf past 65520
    with np.errstate(over="ignore"):
        want = outs[False].astype(np.float16)
    assert np.array_equal(outs[True].view(np.uint16), want.view(np.uint16)), (fmt, m, n, k)
    a.free()
    b.free()


def test_accum_gemm_rejects_bad_arguments(dev):
    a, b, c = dev.alloc(64 * 512), dev.alloc(128 * 512), dev.alloc(64 * 128 * 4)
    with pytest.raises(M.MxError):   # FP4 x FP8 is not one of the probe pairs
        dev.accum_gemm(M.PROBE_FP4, a, M.PROBE_FP8, b, c, M.DT_F32, 64, 128, 512)
    with pytest.raises(M.MxError):   # m % 32 for the FP4 / FP8 kernel
        dev.accum_gemm(M.PROBE_FP8, a, M.PROBE_FP8, b, c, M.DT_F32, 48, 128, 512)
    with pytest.raises(M.MxError):   # packed FP4 rows need an even k
        dev.accum_gemm(M.PROBE_FP4, a, M.PROBE_FP4, b, c, M.DT_F32, 64, 128, 497)
    with pytest.raises(M.MxError):   # n % 64
        dev.accum_gemm(M.PROBE_F16, a, M.PROBE_F16, b, c, M.DT_F32, 64, 96, 128)
    with pytest.raises(M.MxError):   # C must be f16 or f32
        dev.accum_gemm(M.PROBE_F16, a, M.PROBE_F16, b, c, M.DT_I32, 64, 128, 512)
    for x in (a, b, c):
        x.free()


@pytest.mark.parametrize("k", [1022, 64, 100])
def test_accum_gemm_half_paths_random(dev, k):
    """f16 x f16 and f16 x unscaled FP4 at dot lengths that are not multiples
    of 32, against a float64 product of the same operands."""
    m, n = 48, 64
    rng = np.random.default_rng(k)
    a16 = rng.standard_normal((m, k)).astype(np.float16)
    b16 = rng.standard_normal((n, k)).astype(np.float16)
    q = rng.integers(0, 256, (n, (k + 1) // 2), dtype=np.uint8)
    if k % 2 == 0:
        cases = [(M.PROBE_F16, b16, b16.astype(np.float64)),
                 (M.PROBE_FP4, q, O.unpack(M.FMT_FP4_E2M1, q.reshape(-1), n * k).reshape(n, k).astype(np.float64))]
    else:
        cases = [(M.PROBE_F16, b16, b16.astype(np.float64))]
    a = dev.upload(a16)
    for b_fmt, b_host, b_val in cases:
        ref = a16.astype(np.float64) @ b_val.T
        b = dev.upload(b_host)
        c = dev.alloc(m * n * 4)
        dev.accum_gemm(M.PROBE_F16, a, b_fmt, b, c, M.DT_F32, m, n, k)
        got = dev.download(c, np.float32, (m, n)).astype(np.float64)
        scale = np.abs(a16.astype(np.float64)).max() * np.abs(b_val).max() * k
        assert np.abs(got - ref).max() <= 1e-6 * scale, (b_fmt, k)
        b.free()
        c.free()
    a.free()


def _int4(b):
    """Signed INT4 codes, low nibble = even k (PackedNumericKernels.metal:25-28)."""
    lo, hi = (b & 15).astype(np.int64), (b >> 4).astype(np.int64)
    out = np.empty(b.shape[:-1] + (b.shape[-1] * 2,), np.int64)
    out[..., 0::2], out[..., 1::2] = (lo ^ 8) - 8, (hi ^ 8) - 8
    return out


@pytest.mark.parametrize("m,n,k", [(64, 128, 256), (48, 64, 1022), (32, 192, 130)])
def test_int_pairs(dev, m, n, k):
    """half x INT4 and INT8 x half against float64; INT4 x INT4 exact i32."""
    rng = np.random.default_rng(m * n + k)
    a16 = (rng.standard_normal((m, k)) * 0.25).astype(np.float16)
    a8 = rng.integers(-128, 128, (m, k), dtype=np.int8)
    a4 = rng.integers(0, 256, (m, k // 2), dtype=np.uint8)
    b4 = rng.integers(0, 256, (n, k // 2), dtype=np.uint8)
    b16 = (rng.standard_normal((n, k)) * 0.03).astype(np.float16)
    bufs = {name: dev.upload(arr) for name, arr in
            (("a16", a16), ("a8", a8), ("a4", a4), ("b4", b4), ("b16", b16))}
    c = dev.alloc(m * n * 4)
    cases = [(M.PROBE_F16, "a16", M.PROBE_INT4, "b4", a16.astype(np.float64) @ _int4(b4).T.astype(np.float64)),
             (M.PROBE_I8, "a8", M.PROBE_F16, "b16", a8.astype(np.float64) @ b16.astype(np.float64).T)]
    for a_fmt, a_name, b_fmt, b_name, ref in cases:
        dev.accum_gemm(a_fmt, bufs[a_name], b_fmt, bufs[b_name], c, M.DT_F32, m, n, k)
        got = dev.download(c, np.float32, (m, n)).astype(np.float64)
        assert np.abs(got - ref).max() <= 1e-5 * (np.abs(ref).max() + 1), (a_fmt, b_fmt, m, n, k)
    dev.accum_gemm(M.PROBE_INT4, bufs["a4"], M.PROBE_INT4, bufs["b4"], c, M.DT_I32, m, n, k)
    got = dev.download(c, np.int32, (m, n)).astype(np.int64)
    assert np.array_equal(got, _int4(a4) @ _int4(b4).T)
    with pytest.raises(M.MxError):   # INT4 x INT4 writes i32 only
        dev.accum_gemm(M.PROBE_INT4, bufs["a4"], M.PROBE_INT4, bufs["b4"], c, M.DT_F32, m, n, k)
    c.free()
    for b in bufs.values():
        b.free()


def test_device_timer(dev):
    dev.timer_start()
    a, b, c = dev.alloc(64 * 1024 * 2), dev.alloc(128 * 1024 * 2), dev.alloc(64 * 128 * 4)
    for _ in range(3):
        dev.accum_gemm(M.PROBE_F16, a, M.PROBE_F16, b, c, M.DT_F32, 64, 128, 1024)
    assert dev.timer_stop() > 0
    for x in (a, b, c):
        x.free()
