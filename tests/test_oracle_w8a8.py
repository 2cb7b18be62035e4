"""Pin the oracle's W8A8 composition (CPU only).

W8A8 is BASELINE.json configs[3]'s "int8 activations with per-token scale,
int32 accumulate" row: the reference's int8 x int8 -> int32 matmul
(mpp_mlp_i8_i8_i32_n128, MPPMLPKernels.metal:61-70) with the scales the
reference leaves out.  The oracle's format mode 5 (`orc_mlp_format`) is
compared here with an independent numpy restatement written from that
definition:

  * x (f16 -> f32) is quantized per token: s = amax / 127 (1 for an all-zero
    row), q = clamp(rint(x / s), -127, 127), rint rounding half to even;
  * gate / up are exact int64 dot products of the int8 codes, scaled in f32
    as (sum * s_token) * s_row;
  * mid = silu(gate) * up in float32;
  * mid is quantized per token the same way, and the down projection runs
    like gate / up;
  * the output is rounded to f16.

The only shared inputs are the weight codes and row scales, whose quantizer
is pinned separately (`test_rowwise_format_quantizers`).  Plausible mistakes
planted in the restatement - x or mid quantized per column (along the token
axis) or per tensor, mid not re-quantized - each move most outputs, so each
must fail the comparison that the correct restatement passes.
"""
import numpy as np
import pytest

import oracle as O


def q8(v, axis):
    """int8 quantization of a [T][K] f32 matrix: one scale per token
    ("token"), per column ("column") or for the whole tensor ("tensor").
    Returns the int64 codes and the f32 scales, broadcastable to v."""
    v = np.asarray(v, np.float32)
    if axis == "token":
        amax = np.abs(v).max(1, keepdims=True)
    elif axis == "column":
        amax = np.abs(v).max(0, keepdims=True)
    else:
        amax = np.abs(v).max(keepdims=True)
    s = np.where(amax > 0, amax / np.float32(127), np.float32(1)).astype(np.float32)
    q = np.clip(np.rint(v / s), -127, 127)  # np.rint: half to even, like rintf
    return q.astype(np.int64), s


def gemm(qa, sa, qw, sw, axis):
    """[T][K] codes with scales sa times int8 weight rows [N][K] with f32 row
    scales sw.  Per-token scales factor out of the integer sum, so the sum is
    exact and scaled once in f32, (sum * s_token) * s_row; any other scale
    axis does not factor out and is applied per element before the sum."""
    if axis == "token":
        acc = qa @ qw.T  # int64, exact
        return (acc.astype(np.float32) * sa) * sw[None, :]
    a = qa.astype(np.float64) * sa.astype(np.float64)
    return (a @ qw.T.astype(np.float64) * sw[None, :].astype(np.float64)).astype(np.float32)


def w8a8_numpy(x, qg, sg, qu, su, qd, sd, x_axis="token", mid_axis="token", requant_mid=True):
    xa = x.astype(np.float32)
    qx, sx = q8(xa, x_axis)
    g = gemm(qx, sx, qg, sg, x_axis)
    u = gemm(qx, sx, qu, su, x_axis)
    e = np.exp(-g.astype(np.float64)).astype(np.float32)  # correctly rounded expf
    mid = (g / (np.float32(1) + e)) * u
    if requant_mid:
        qm, sm = q8(mid, mid_axis)
        o = gemm(qm, sm, qd, sd, mid_axis)
    else:
        o = (mid.astype(np.float64) @ (qd.T.astype(np.float64) * sd[None, :].astype(np.float64))).astype(np.float32)
    return o.astype(np.float16)


def compare(got, ref):
    """(max |got - ref| / rms(ref), fraction of bit-identical f16 outputs)."""
    a, b = got.astype(np.float64), ref.astype(np.float64)
    rms = np.sqrt((b ** 2).mean())
    return np.abs(a - b).max() / rms, (got.view(np.uint16) == ref.view(np.uint16)).mean()


def make(T, H, I, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float16)
    mats = []
    for n, k in ((I, H), (I, H), (H, I)):
        q, s = O.quant_rowwise(O.WF_INT8, rng.normal(0, 0.02, (n, k)).astype(np.float32))
        mats += [q.view(np.int8).astype(np.int64), s, q]
    return x, mats


@pytest.mark.parametrize("T,H,I,seed", [(16, 256, 512, 31), (32, 128, 256, 32), (3, 64, 96, 33)])
def test_w8a8_oracle_vs_independent_numpy(T, H, I, seed):
    x, m = make(T, H, I, seed)
    (cg, sg, qg), (cu, su, qu), (cd, sd, qd) = m[0:3], m[3:6], m[6:9]
    got = O.mlp_format(O.WF_W8A8, x, qg, sg, qu, su, qd, sd, H, I)
    ref = w8a8_numpy(x, cg, sg, cu, su, cd, sd)
    rel, same = compare(got, ref)
    # exact integer sums and the same f32 scale products: the outputs agree
    # bit for bit except where an expf ulp moves a mid code across a rint
    # midpoint (measured: all bits equal at these seeds)
    assert rel <= 2e-3 and same >= 0.99, (rel, same)
    # planted mistakes in the restatement must not match the oracle
    planted = [dict(x_axis="column"), dict(x_axis="tensor"), dict(mid_axis="column"),
               dict(mid_axis="tensor"), dict(requant_mid=False)]
    for kw in planted:
        bad = w8a8_numpy(x, cg, sg, cu, su, cd, sd, **kw)
        rel_b, same_b = compare(got, bad)
        assert rel_b > 5 * max(rel, 1e-3) and same_b < 0.9, (kw, rel_b, same_b)


def test_w8a8_all_zero_token_row():
    """An all-zero x row takes scale 1 and codes 0: its outputs are exactly 0
    on both sides, and the other rows are unaffected."""
    x, m = make(4, 64, 128, 34)
    x[2] = 0
    (cg, sg, qg), (cu, su, qu), (cd, sd, qd) = m[0:3], m[3:6], m[6:9]
    got = O.mlp_format(O.WF_W8A8, x, qg, sg, qu, su, qd, sd, 64, 128)
    assert not got[2].any()
    ref = w8a8_numpy(x, cg, sg, cu, su, cd, sd)
    assert compare(got, ref)[1] >= 0.99


def test_w8a8_int8_per_token_quantizer():
    """The oracle's per-token activation quantizer against the restatement's:
    codes and scales identical, including a saturating row and ties."""
    rng = np.random.default_rng(35)
    v = rng.standard_normal((8, 96)).astype(np.float32)
    v[3, :4] = [127.0, -127.0, 63.5, -0.5]  # amax 127: scale 1, ties 63.5 -> 64, -0.5 -> -0
    q, s = O.quant_int8_per_token(v)
    q2, s2 = q8(v, "token")
    np.testing.assert_array_equal(s, s2[:, 0])
    np.testing.assert_array_equal(q.astype(np.int64), q2)
    assert q[3, 2] == 64 and q[3, 3] == 0
