"""Pin the CPU oracle's element codecs (CPU only).

Each check is chosen so a plausible slip (wrong bias, wrong nibble order,
round-half-up instead of half-even, missing saturation) fails:
  * the reference's three known-answer cases (main.swift:108-132) and their
    packed bytes,
  * closed forms: all 256 E8M0 bytes, all 16 FP4 nibbles,
  * RNE tie tables derived from the decode tables alone (tests/golden),
  * brute force: nearest-representable search over the decode table,
  * a library routine: numpy's float16 cast and torch's float8 casts.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")


def _f(bits):
    return np.array(bits, np.uint32).view(np.float32)


def test_reference_kats_bytes_and_values():
    kats = json.load(open(os.path.join(GOLD, "kats.json")))
    fmts = {"FP4 E2M1": O.FMT_FP4, "FP8 E4M3": O.FMT_E4M3, "FP8 E5M2": O.FMT_E5M2}
    for case in kats:
        fmt = fmts[case["name"]]
        x = np.array(case["inputs"], np.float32)
        packed = O.pack(fmt, x)
        assert list(packed) == case["bytes"], case["name"]
        back = O.unpack(fmt, packed, x.size)
        assert np.array_equal(back, np.array(case["expected"], np.float32)), case["name"]


def test_e8m0_and_fp4_tables_closed_form():
    t = json.load(open(os.path.join(GOLD, "tables.json")))
    L = O.lib()
    for b in range(256):
        got = np.float32(L.orc_e8m0_to_float(b)).view(np.uint32)
        assert int(got) == t["e8m0_f32_bits"][b]
        if 1 <= b <= 254:
            assert L.orc_e8m0_to_float(b) == 2.0 ** (b - 127)
    assert L.orc_e8m0_to_float(0) == 0.0
    assert np.isinf(L.orc_e8m0_to_float(255))
    for n in range(16):
        v = L.orc_fp4_decode(n)
        assert v == t["fp4_e2m1"][n]
        assert np.signbit(np.float32(v)) == bool(n & 8)


@pytest.mark.parametrize("name,fmt,maxcode", [("e2m1", O.FMT_FP4, 7), ("e4m3", O.FMT_E4M3, 0x7e),
                                              ("e5m2", O.FMT_E5M2, 0x7b)])
def test_rne_tie_tables(name, fmt, maxcode):
    ties = json.load(open(os.path.join(GOLD, "ties.json")))[name]
    bits = np.array([r[0] for r in ties], np.uint32)
    want = np.array([r[1] for r in ties])
    x = bits.view(np.float32)
    if fmt == O.FMT_FP4:
        codes = O.pack(fmt, np.repeat(x, 2))[:]  # each byte holds the same code twice
        got = codes & 15
    else:
        got = O.pack(fmt, x)
    assert np.array_equal(got.astype(int), want), name
    # negative side: same magnitude code with the sign bit
    sign = 8 if fmt == O.FMT_FP4 else 0x80
    if fmt == O.FMT_FP4:
        gotn = O.pack(fmt, np.repeat(-x, 2)) & 15
    else:
        gotn = O.pack(fmt, -x)
    assert np.array_equal(gotn.astype(int), want | sign)


def _decode_table(fmt):
    if fmt == O.FMT_FP4:
        return np.array([O.lib().orc_fp4_decode(i) for i in range(8)], np.float64), 7
    dec = O.lib().orc_fp8_e4m3_decode if fmt == O.FMT_E4M3 else O.lib().orc_fp8_e5m2_decode
    mx = 0x7e if fmt == O.FMT_E4M3 else 0x7b
    return np.array([dec(i) for i in range(mx + 1)], np.float64), mx


@pytest.mark.parametrize("fmt", [O.FMT_FP4, O.FMT_E4M3, O.FMT_E5M2])
def test_encoder_brute_force_nearest(fmt):
    """Encoder == nearest representable magnitude, ties to the even code,
    saturating above the largest finite value."""
    table, mx = _decode_table(fmt)
    rng = np.random.default_rng(fmt + 7)
    top = table[-1]
    # log-uniform magnitudes across and beyond the format's range, plus grid
    mags = np.concatenate([
        np.exp(rng.uniform(np.log(table[1] / 8), np.log(top * 4), 200000)),
        np.linspace(0, top * 1.5, 50001),
    ]).astype(np.float32)
    x = np.concatenate([mags, -mags])
    got = O.pack(fmt, np.repeat(x, 2)) & 15 if fmt == O.FMT_FP4 else O.pack(fmt, x)
    a = np.abs(x.astype(np.float64))
    d = np.abs(a[:, None] - table[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    # ties: choose the even code
    idx = np.where(cand.sum(1) > 1, np.argmax(cand & (np.arange(mx + 1) % 2 == 0), axis=1),
                   np.argmax(cand, axis=1))
    want = idx + (8 if fmt == O.FMT_FP4 else 0x80) * np.signbit(x)
    assert np.array_equal(got.astype(int), want.astype(int))


def test_f32_to_f16_matches_numpy_structured():
    """RNE to binary16 incl. subnormals/overflow vs numpy's cast.  (A one-time
    run over all 2^32 inputs found no mismatch; this keeps a structured
    subset: every exponent, top-10 mantissa bits x round/sticky patterns.)"""
    e = np.arange(0, 256, dtype=np.uint32)
    top = np.arange(0, 1 << 10, dtype=np.uint32) << 13
    low = np.array([0, 1, 0xfff, 0x1000, 0x1001, 0x1fff], np.uint32)
    m = (top[:, None] | low[None, :]).reshape(-1)
    bits = ((e[:, None] << 23) | m[None, :]).reshape(-1)
    bits = np.concatenate([bits, bits | 0x80000000])
    x = bits.view(np.float32)
    finite = np.isfinite(x)
    with np.errstate(over="ignore"):
        want = x[finite].astype(np.float16).view(np.uint16)
    got = O.f32_to_f16_bits(x[finite])
    assert np.array_equal(got, want)
    nan = O.f32_to_f16_bits(np.array([np.nan], np.float32))[0]
    assert (nan & 0x7c00) == 0x7c00 and (nan & 0x3ff) != 0


def test_fp8_against_torch_casts():
    torch = pytest.importorskip("torch")
    # decode: all bytes
    for fmt, tdt in ((O.FMT_E4M3, torch.float8_e4m3fn), (O.FMT_E5M2, torch.float8_e5m2)):
        codes = np.arange(256, dtype=np.uint8)
        ours = O.unpack(fmt, codes, 256)
        theirs = torch.from_numpy(codes).view(tdt).float().numpy()
        both_nan = np.isnan(ours) & np.isnan(theirs)
        assert np.array_equal(ours[~both_nan], theirs[~both_nan])
        # encode: in-range values (torch does not saturate, so stay in range)
        lim = 448.0 if fmt == O.FMT_E4M3 else 57344.0
        rng = np.random.default_rng(3)
        x = np.concatenate([rng.uniform(-lim, lim, 100000),
                            np.exp(rng.uniform(-25, np.log(lim), 100000)) * rng.choice([-1, 1], 100000)])
        x = x[np.abs(x) <= lim].astype(np.float32)
        ours = O.pack(fmt, x)
        theirs = torch.from_numpy(x).to(tdt).view(torch.uint8).numpy()
        assert np.array_equal(ours, theirs)


def test_saturation_and_specials():
    L = O.lib()
    assert L.orc_fp4_encode(1e30) == 7 and L.orc_fp4_encode(-1e30) == 15
    assert L.orc_fp4_encode(float("inf")) == 7
    assert L.orc_fp8_e4m3_encode(1e30) == 0x7e and L.orc_fp8_e4m3_encode(-464.0) == 0xfe
    assert L.orc_fp8_e4m3_encode(float("nan")) & 0x7f == 0x7f
    assert L.orc_fp8_e5m2_encode(1e30) == 0x7b and L.orc_fp8_e5m2_encode(-float("inf")) == 0xfb
    assert L.orc_fp4_encode(-0.1) == 8  # rounds to -0, sign kept
