"""Pin the oracle's W4A4 composition and its swiglu_i8 (CPU only).

W4A4 has no reference code: x is quantized to
MXFP4 along H, mid = silu(gate) * up is quantized to MXFP4 along I, and all
products are FP4 x FP4 with FP32 accumulation.  The oracle's mode 1
(`orc_mlp_mxfp4`) is checked here against an independent numpy restatement
whose only shared part is nothing: its MXFP4 quantizer is written below from
the BASELINE definition (scale 2^(floor(log2 amax) - 2), round to nearest
even on the E2M1 grid, saturate at 6), its GEMMs are float64 matmuls of the
dequantized operands, and its SwiGLU is float32 arithmetic.  Plausible
mistakes - mid quantized along the token axis, a skipped re-quantization of
x or of mid - are planted in the restatement and must fail the comparison.

swiglu_i8 (mpp_mlp_swiglu_i8, MPPMLPKernels.metal:240-257) is pinned by
closed forms: gate >= 20 * 4096 makes silu(clamp(gate / 4096, +-20)) = 20
exactly in f32, so mid = rint(clamp(20 * up / 4096 * 32)) = rint(up * 0.15625)
(exact), which pins the 2^-12 input scale, the x32 output scale, the clamp
of g, the saturation at -128 / 127 and round-half-even; gate = 0 gives 0.
"""
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(__file__), "golden")
E2M1 = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def mxfp4_qdq(v):
    """BASELINE MXFP4 quantize-dequantize along the last axis (blocks of 32),
    float64, written from the definition (not from the oracle's code)."""
    v = np.asarray(v, np.float64)
    blocks = v.reshape(*v.shape[:-1], -1, 32)
    amax = np.abs(blocks).max(-1, keepdims=True)
    with np.errstate(divide="ignore"):
        e = np.where(amax > 0, np.floor(np.log2(np.where(amax > 0, amax, 1.0))) - 2, 0.0)
    e = np.maximum(e, -127)
    scale = 2.0 ** e
    a = np.abs(blocks) / scale
    # nearest E2M1 magnitude, ties to the even code (index)
    d = np.abs(a[..., None] - E2M1)
    best = np.argmin(d + 1e-9 * (np.arange(8) % 2), axis=-1)
    q = E2M1[best] * np.sign(blocks)
    q = np.where(a >= 6.0, 6.0 * np.sign(blocks), q)
    return (q * scale).reshape(v.shape)


def w4a4_numpy(x, wg, wu, wd, mid_axis="I", requant_x=True, requant_mid=True):
    """W4A4 MLP restated: weights already dequantized (float64)."""
    xa = x.astype(np.float64)
    if requant_x:
        xa = mxfp4_qdq(xa)
    g = (xa @ wg.T).astype(np.float32)
    u = (xa @ wu.T).astype(np.float32)
    mid = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32).astype(np.float64)
    if requant_mid:
        mid = mxfp4_qdq(mid) if mid_axis == "I" else mxfp4_qdq(mid.T).T
    return (mid @ wd.T).astype(np.float32).astype(np.float16)


def deq(q, s, k):
    codes = np.stack([q & 15, q >> 4], -1).reshape(q.shape[0], k)
    mag = E2M1[codes & 7] * np.where(codes & 8, -1.0, 1.0)
    return mag * np.repeat(2.0 ** (s.astype(np.float64) - 127), 32, axis=1)


def close(a, b):
    """f16 outputs equal up to one f16 rounding step on almost every element
    (a float32 vs float64 difference can move a value across a rounding
    boundary of the quantizer, moving one mid code by one step)."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    rms = np.sqrt((b ** 2).mean())
    err = np.abs(a - b)
    return err.max() / rms, (err <= 1e-3 * np.abs(b) + 1e-6 * rms).mean()


def test_mxfp4_qdq_restatement_matches_oracle_quantizer():
    rng = np.random.default_rng(5)
    w = rng.normal(0, 1, (64, 256)).astype(np.float32)
    q, s = O.mxfp4_quantize(w)
    np.testing.assert_array_equal(deq(q, s, 256), mxfp4_qdq(w))


@pytest.mark.parametrize("T,H,I,seed", [(2, 64, 128, None), (16, 256, 512, 11), (32, 128, 256, 12)])
def test_w4a4_oracle_vs_independent_numpy(T, H, I, seed):
    if seed is None:  # the committed tiny fixture
        z = np.load(os.path.join(GOLD, "tiny_mlp.npz"))
        x, qg, sg, qu, su, qd, sd = (z[k] for k in ("x", "qg", "sg", "qu", "su", "qd", "sd"))
    else:
        rng = np.random.default_rng(seed)
        x = rng.standard_normal((T, H)).astype(np.float16)
        (qg, sg), (qu, su), (qd, sd) = (O.mxfp4_quantize(rng.normal(0, 0.02, s).astype(np.float32))
                                        for s in ((I, H), (I, H), (H, I)))
    got = O.mlp_mxfp4(O.MLP_W4A4, x, qg, sg, qu, su, qd, sd, H, I)
    wg, wu, wd = deq(qg, sg, H), deq(qu, su, H), deq(qd, sd, I)
    ref = w4a4_numpy(x, wg, wu, wd)
    rel, frac = close(got, ref)
    assert rel <= 5e-3 and frac >= 0.99, (rel, frac)
    # planted mistakes in the restatement must not match the oracle
    for kw in (dict(mid_axis="T"), dict(requant_mid=False), dict(requant_x=False)):
        if kw.get("mid_axis") == "T" and T % 32:
            continue
        bad = w4a4_numpy(x, wg, wu, wd, **kw)
        rel_b, frac_b = close(got, bad)
        assert rel_b > 2e-2 and frac_b < 0.9, (kw, rel_b, frac_b)


def test_swiglu_i8_closed_forms():
    up = np.array([0, 16, 48, -16, -48, 4, 3, -4, 32, 64, 800, 812, 819, 820, -819, -820, 1 << 20, -(1 << 20)],
                  np.int32)
    for gate_v in (81920, 81921, 1 << 20, (1 << 31) - 1):
        gate = np.full_like(up, gate_v)
        got = O.swiglu_i8(gate, up).astype(np.int64)
        # g clamps to 20, silu(20) = 20 exactly in f32; v = 20 * up * 2^-12 * 32
        want = np.clip(np.round(up.astype(np.float64) * 0.15625), -128, 127)  # numpy round = half to even
        np.testing.assert_array_equal(got, want)
    # ties: 2.5 -> 2, 7.5 -> 8, -2.5 -> -2, -7.5 -> -8
    np.testing.assert_array_equal(O.swiglu_i8(np.full(4, 81920, np.int32), np.array([16, 48, -16, -48], np.int32)),
                                  [2, 8, -2, -8])
    # gate 0: silu(0) = 0 for any up
    assert not O.swiglu_i8(np.zeros(5, np.int32), np.array([1, -1, 1 << 30, -(1 << 30), 7], np.int32)).any()


def test_swiglu_i8_vs_float64():
    rng = np.random.default_rng(6)
    g = rng.integers(-120000, 120000, 4096).astype(np.int32)
    u = rng.integers(-30000, 30000, 4096).astype(np.int32)
    got = O.swiglu_i8(g, u).astype(np.int64)
    gf = np.clip(g / 4096.0, -20, 20)
    v = np.clip(gf / (1 + np.exp(-gf)) * (u / 4096.0) * 32, -128, 127)
    want = np.round(v)
    frac = v - np.floor(v)
    near_half = np.abs(frac - 0.5) < 1e-4  # f32 vs float64 may differ only at a rounding midpoint
    assert np.array_equal(got[~near_half], want[~near_half])
    assert np.all(np.abs(got - want) <= 1)
