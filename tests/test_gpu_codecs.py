"""GPU parity of the element codecs, quantizer and dequant (bit-exact).

Reference: pack/unpack roundtrip kernels PackedNumericKernels.metal:35-96 and
their KATs main.swift:108-132; dequant MXFP4Kernels.metal:509-564; the
MXFP4 quantizer defined by BASELINE.json.  Oracle: oracle/mx_oracle.c.
"""
import json
import os

import numpy as np
import pytest

import mxfp4hip as M
import oracle as O

pytestmark = pytest.mark.gpu
GOLD = os.path.join(os.path.dirname(__file__), "golden")


def structured_floats(extra_random=1 << 20, seed=0):
    """Every f32 exponent x every top-8 mantissa pattern x round/sticky low
    patterns, both signs, plus random bit patterns: covers every rounding
    decision of E2M1/E4M3/E5M2 conversion."""
    e = np.arange(0, 256, dtype=np.uint32)
    top = np.arange(0, 256, dtype=np.uint32) << 15
    low = np.array([0, 1, 0x3fff, 0x4000, 0x4001, 0x7fff], np.uint32)
    m = (top[:, None] | low[None, :]).reshape(-1)
    # also exact mid/round points of 1-3 mantissa-bit formats
    m2 = np.array([(1 << 21), (1 << 21) + 1, (1 << 21) - 1, (1 << 20), (1 << 20) + 1, (1 << 19),
                   (1 << 19) + 1, (3 << 20), (3 << 19)], np.uint32)
    m = np.concatenate([m, m2])
    bits = ((e[:, None] << 23) | m[None, :]).reshape(-1)
    rng = np.random.default_rng(seed)
    bits = np.concatenate([bits, bits | 0x80000000,
                           rng.integers(0, 1 << 32, extra_random, dtype=np.uint64).astype(np.uint32)])
    return bits.view(np.float32)


def dev_pack(dev, fmt, x):
    x = np.ascontiguousarray(x, np.float32)
    n = x.size
    src = dev.upload(x)
    nb = (n + 1) // 2 if fmt == M.FMT_FP4_E2M1 else n
    dst = dev.alloc(max(16, (nb + 15) // 16 * 16))
    dev.pack(fmt, src, n, dst)
    out = dev.download(dst, np.uint8, (nb,))
    src.free()
    dst.free()
    return out


def test_roundtrip_kats(dev):
    kats = json.load(open(os.path.join(GOLD, "kats.json")))
    fmts = {"FP4 E2M1": M.FMT_FP4_E2M1, "FP8 E4M3": M.FMT_FP8_E4M3, "FP8 E5M2": M.FMT_FP8_E5M2}
    for case in kats:
        packed, out = dev.roundtrip(fmts[case["name"]], case["inputs"])
        assert list(packed) == case["bytes"], (case["name"], packed)
        assert np.array_equal(out, np.array(case["expected"], np.float32)), case["name"]


@pytest.mark.parametrize("fmt", [M.FMT_FP4_E2M1, M.FMT_FP8_E4M3, M.FMT_FP8_E5M2])
def test_pack_bitexact_structured(dev, fmt):
    x = structured_floats(seed=fmt)
    nan = np.isnan(x)
    xs = x[~nan]
    if xs.size % 2:
        xs = xs[:-1]
    got = dev_pack(dev, fmt, xs)
    want = O.pack(fmt, xs)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(hex(int(xs[2 * i if fmt == 0 else i].view(np.uint32))), got[i], want[i])
                           for i in bad[:8]]


@pytest.mark.parametrize("fmt", [M.FMT_FP4_E2M1, M.FMT_FP8_E4M3, M.FMT_FP8_E5M2])
def test_pack_nan_inputs(dev, fmt):
    """NaN is not pinned by the reference; the oracle's choice must match the
    hardware path (sign | max-magnitude code for E2M1, the NaN code for FP8)."""
    x = np.array([np.nan, -np.nan, 1.0, np.nan], np.float32)
    x[1] = -np.float32(np.nan)
    got = dev_pack(dev, fmt, x)
    want = O.pack(fmt, x)
    if fmt == M.FMT_FP4_E2M1:
        assert np.array_equal(got, want), (got, want)
    else:
        dec = O.unpack(fmt, got, 4)
        assert np.isnan(dec[[0, 1, 3]]).all() and dec[2] == 1.0, got


@pytest.mark.parametrize("fmt", [M.FMT_FP4_E2M1, M.FMT_FP8_E4M3, M.FMT_FP8_E5M2])
def test_unpack_all_codes(dev, fmt):
    codes = np.arange(256, dtype=np.uint8)
    n = 512 if fmt == M.FMT_FP4_E2M1 else 256
    src = dev.upload(codes)
    dst = dev.alloc(n * 4)
    dev.unpack(fmt, src, n, dst)
    got = dev.download(dst, np.float32, (n,))
    want = O.unpack(fmt, codes, n)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all(), np.nonzero(~same)[0][:8]


def _quant_inputs():
    rng = np.random.default_rng(5)
    rows = []
    rows.append(rng.normal(0, 0.02, 4096))
    rows.append(rng.normal(0, 1, 4096))
    rows.append(rng.normal(0, 1e3, 4096))
    rows.append(rng.normal(0, 1e-30, 4096))          # subnormal-range blocks
    rows.append(rng.normal(0, 1, 4096) * np.exp(rng.uniform(-30, 30, 4096)))
    r = np.zeros(4096)
    r[40] = 3.0                                       # single value
    r[100:132] = 0.0                                  # zero block
    r[200] = 6.0 * 2 ** 20
    r[300:332] = np.linspace(-5, 5, 32)               # ties
    rows.append(r)
    return np.array(rows, np.float32)


def test_mxfp4_quantize_bitexact_f32(dev):
    x = _quant_inputs()
    rows, k = x.shape
    src = dev.upload(x)
    q, s = dev.alloc(rows * k // 2), dev.alloc(rows * k // 32)
    dev.mxfp4_quantize(src, M.DT_F32, rows, k, q, s)
    gq = dev.download(q, np.uint8, (rows, k // 2))
    gs = dev.download(s, np.uint8, (rows, k // 32))
    oq, os_ = O.mxfp4_quantize(x)
    assert np.array_equal(gs, os_)
    assert np.array_equal(gq, oq)


def test_mxfp4_quantize_bitexact_f16_and_specials(dev):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((64, 1024)).astype(np.float16)
    x[0, 0] = np.inf
    x[1, 33] = np.nan
    x[2, :32] = 0
    x[3, :32] = np.float16(6.1e-5)
    src = dev.upload(x)
    q, s = dev.alloc(64 * 512), dev.alloc(64 * 32)
    dev.mxfp4_quantize(src, M.DT_F16, 64, 1024, q, s)
    gq = dev.download(q, np.uint8, (64, 512))
    gs = dev.download(s, np.uint8, (64, 32))
    oq, os_ = O.mxfp4_quantize(x)
    assert gs[0, 0] == 255 and gs[1, 1] == 255 and gs[2, 0] == 127
    assert np.array_equal(gs, os_)
    assert np.array_equal(gq, oq)


def test_dequant_bitexact_every_code_and_scale(dev):
    q = np.tile(np.array([0x10, 0x32, 0x54, 0x76, 0x98, 0xba, 0xdc, 0xfe] * 2, np.uint8), (256, 1))
    s = np.arange(256, dtype=np.uint8).reshape(256, 1)
    rng = np.random.default_rng(7)
    q = np.concatenate([q, rng.integers(0, 256, (256, 16), dtype=np.uint8)])
    s = np.concatenate([s, rng.integers(100, 150, (256, 1), dtype=np.uint8)])
    dq, ds = dev.upload(q), dev.upload(s)
    out = dev.alloc(512 * 32 * 2)
    dev.mxfp4_dequant_f16(dq, ds, out, 512, 32)
    got = dev.download(out, np.uint16, (512, 32))
    want = O.mxfp4_dequant_f16(q, s, 512, 32).view(np.uint16)
    nan = ((got & 0x7c00) == 0x7c00) & ((got & 0x3ff) != 0) & ((want & 0x7c00) == 0x7c00) & ((want & 0x3ff) != 0)
    bad = np.nonzero((got != want) & ~nan)
    assert bad[0].size == 0, list(zip(bad[0][:8], bad[1][:8]))
