"""The allocation-free MLP forward (mx_mlp_forward_noalloc) against
mx_mlp_forward.

Both run the same kernels on the same inputs, so outputs must agree bit for
bit.  Each case makes two allocation-free calls in a row, the second with
fewer tokens (often on another kernel path), so the second call runs over the
first call's stale scratch contents; both are then checked against the
allocating entry point.
"""
import numpy as np
import pytest

import mxfp4hip as M
from mlp_data import MlpData

pytestmark = pytest.mark.gpu

# (variant, H, I, first tokens, second tokens)
CASES = [
    (M.MLP_FUSED, 7168, 2048, 8, 1),      # decode GEMV, both calls
    (M.MLP_FUSED, 1024, 4096, 128, 4),    # tiled GEMM (split K) -> GEMV
    (M.MLP_REFROW, 512, 1024, 64, 3),
    (M.MLP_DEQUANT, 512, 1024, 130, 5),
    (M.MLP_W4A4, 1024, 2048, 256, 64),    # stage-major kernels, split-K down GEMM
    (M.MLP_W4A4, 1024, 1536, 300, 44),    # 128-K-stage kernels, stage-major x and mid
    (M.MLP_W4A4, 640, 1152, 96, 17),      # reference scale layout
    (M.MLP_SCALED, 1024, 2048, 128, 9),   # split of x, F8X2 mid, split-K reduce
]


def _width(variant):
    """Bytes per output element: the fused-row variant writes f32, the others f16."""
    return 4 if variant == M.MLP_REFROW else 2


def _forward(dev, fn, variant, d, T):
    out = dev.alloc(T * d.H * _width(variant))
    fn(variant, T, d.H, d.I, d.x, d.weights, out)
    return out


def _bits(dev, buf, T, H, variant=M.MLP_FUSED):
    dev.sync()
    return dev.download(buf, np.uint32 if _width(variant) == 4 else np.uint16, (T, H))


@pytest.mark.parametrize("variant,H,I,T1,T2", CASES)
def test_noalloc_matches_forward(dev, variant, H, I, T1, T2):
    print(f"noalloc variant={variant} H={H} I={I} T={T1},{T2}", flush=True)
    d = MlpData(dev, T1, H, I, seed=300 + variant)
    o1 = _forward(dev, dev.mlp_forward_noalloc, variant, d, T1)
    o2 = _forward(dev, dev.mlp_forward_noalloc, variant, d, T2)
    got1, got2 = _bits(dev, o1, T1, H, variant), _bits(dev, o2, T2, H, variant)
    r1 = _forward(dev, dev.mlp_forward, variant, d, T1)
    r2 = _forward(dev, dev.mlp_forward, variant, d, T2)
    want1, want2 = _bits(dev, r1, T1, H, variant), _bits(dev, r2, T2, H, variant)
    assert np.isfinite(got1.view(np.float32 if _width(variant) == 4 else np.float16)).all()
    assert np.array_equal(got1, want1), f"first call differs ({variant}, T={T1})"
    assert np.array_equal(got2, want2), f"second call differs ({variant}, T={T2})"
    for b in (o1, o2, r1, r2):
        b.free()
    d.free()


def test_noalloc_second_context(dev):
    """A second context on the same device shares that device's array."""
    d = MlpData(dev, 16, 512, 1024, seed=11)
    other = M.Device(0)
    try:
        o = other.alloc(16 * 512 * 2)
        other.mlp_forward_noalloc(M.MLP_FUSED, 16, 512, 1024, d.x, d.weights, o)
        got = _bits(other, o, 16, 512)
        o.free()
    finally:
        other.close()
    r = _forward(dev, dev.mlp_forward, M.MLP_FUSED, d, 16)
    assert np.array_equal(got, _bits(dev, r, 16, 512))
    r.free()
    d.free()


def test_noalloc_rejects_oversized_scratch(dev):
    """The dequantize variant at the decode shape needs ~90 MB of scratch
    (three f16 weight copies), beyond the fixed array: a clear error, no
    launch."""
    d = MlpData(dev, 1, 7168, 2048, seed=12)
    out = dev.alloc(7168 * 2)
    with pytest.raises(M.MxError, match="allocation-free forward has"):
        dev.mlp_forward_noalloc(M.MLP_DEQUANT, 1, 7168, 2048, d.x, d.weights, out)
    dev.sync()
    out.free()
    d.free()
