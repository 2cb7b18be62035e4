"""mx_load_mxfp4: MXFP4 checkpoint tensors (blocks [..., n, k/32, 16] +
scales [..., n, k/32]) land on the device byte for byte (no repack), and an
MLP / MoE run on loaded weights matches the oracle on the same bytes."""
import numpy as np
import pytest

import mxfp4hip as M
import oracle as O

pytestmark = pytest.mark.gpu
st = pytest.importorskip("safetensors.numpy")


def quantized(rng, n, k):
    q, s = O.mxfp4_quantize(rng.normal(0, 0.02, (n, k)).astype(np.float32))
    return q.reshape(n, k // 2), s.reshape(n, k // 32)


def test_load_is_byte_exact_and_runs_the_mlp(dev, tmp_path):
    T, H, I = 3, 256, 512
    rng = np.random.default_rng(5)
    mats = {"gate": quantized(rng, I, H), "up": quantized(rng, I, H), "down": quantized(rng, H, I)}
    tensors = {}
    for name, (q, s) in mats.items():
        tensors[f"mlp.{name}.blocks"] = q.reshape(q.shape[0], -1, 16)   # [n, k/32, 16]
        tensors[f"mlp.{name}.scales"] = s
    path = tmp_path / "mlp.safetensors"
    st.save_file(tensors, str(path))
    loaded = {}
    for name, (q, s) in mats.items():
        data, scales, count, n, k = dev.load_mxfp4(path, f"mlp.{name}.blocks", f"mlp.{name}.scales")
        assert (count, n, k) == (1, q.shape[0], q.shape[1] * 2)
        assert np.array_equal(dev.download(data, np.uint8, q.shape), q)
        assert np.array_equal(dev.download(scales, np.uint8, s.shape), s)
        loaded[name] = (data, scales)
    x16 = rng.standard_normal((T, H)).astype(np.float16)
    x = dev.upload(x16)
    out = dev.alloc(T * H * 2)
    w = M.Device.weights(loaded["gate"], loaded["up"], loaded["down"])
    dev.mlp_forward(M.MLP_FUSED, T, H, I, x, w, out)
    got = dev.download(out, np.float16, (T, H))
    ref = O.mlp_mxfp4(O.MLP_F16, x16, *mats["gate"], *mats["up"], *mats["down"], H, I)
    rel, cos = O.mlp_error(got, ref)
    assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL, (rel, cos)
    for d, s in loaded.values():
        d.free()
        s.free()
    x.free()
    out.free()


def test_load_stacked_experts_for_moe(dev, tmp_path):
    E, H, I = 3, 128, 256
    counts = [2, 0, 3]
    rng = np.random.default_rng(7)
    shapes = {"gate": (I, H), "up": (I, H), "down": (H, I)}
    per = {name: [quantized(rng, *shapes[name]) for _ in range(E)] for name in shapes}
    tensors = {}
    for name, lst in per.items():
        tensors[f"experts.{name}.blocks"] = np.stack([q.reshape(q.shape[0], -1, 16) for q, _ in lst])
        tensors[f"experts.{name}.scales"] = np.stack([s for _, s in lst])
    path = tmp_path / "experts.safetensors"
    st.save_file(tensors, str(path))
    loaded = {}
    for name in per:
        data, scales, count, n, k = dev.load_mxfp4(path, f"experts.{name}.blocks", f"experts.{name}.scales")
        assert count == E
        loaded[name] = (data, scales)
    x16 = rng.standard_normal((sum(counts), H)).astype(np.float16)
    x = dev.upload(x16)
    out = dev.alloc(sum(counts) * H * 2)
    dev.moe_forward(H, I, counts, x, M.Device.weights(loaded["gate"], loaded["up"], loaded["down"]), out)
    got = dev.download(out, np.float16, (sum(counts), H))
    t0 = 0
    for e, c in enumerate(counts):
        if c:
            ref = O.mlp_mxfp4(O.MLP_F16, x16[t0:t0 + c], *per["gate"][e], *per["up"][e], *per["down"][e], H, I)
            rel, cos = O.mlp_error(got[t0:t0 + c], ref)
            assert rel <= O.MAX_ABS_REL_TOL and cos >= O.COSINE_TOL, (e, rel, cos)
        t0 += c
    for d, s in loaded.values():
        d.free()
        s.free()
    x.free()
    out.free()


def test_load_rejects_mismatched_tensors(dev, tmp_path):
    rng = np.random.default_rng(9)
    path = tmp_path / "bad.safetensors"
    st.save_file({"a.blocks": rng.integers(0, 256, (8, 2, 16), dtype=np.uint8),
                  "a.scales": rng.integers(0, 256, (8, 3), dtype=np.uint8),       # k/32 disagrees
                  "b.blocks": rng.standard_normal((8, 2, 16)).astype(np.float32),  # not U8
                  "b.scales": rng.integers(0, 256, (8, 2), dtype=np.uint8)}, str(path))
    for b, s in (("a.blocks", "a.scales"), ("b.blocks", "b.scales"), ("a.blocks", "missing")):
        with pytest.raises(M.MxError):
            dev.load_mxfp4(path, b, s)


def test_load_rejects_overflowing_shapes(dev, tmp_path):
    """Shapes whose element or byte counts overflow, or exceed the int
    outputs, are rejected with MX_EINVAL before anything is allocated."""
    import json
    import struct
    for s_shape, b_shape in (([1 << 62, 4, 1], [1 << 62, 4, 1, 16]),     # count * n * kb wraps
                             ([1 << 31, 1], [1 << 31, 1, 16]),           # n beyond INT_MAX
                             ([3, 1 << 40, 2], [3, 1 << 40, 2, 16])):
        hdr = {"b": {"dtype": "U8", "shape": b_shape, "data_offsets": [0, 16]},
               "s": {"dtype": "U8", "shape": s_shape, "data_offsets": [16, 17]}}
        text = json.dumps(hdr).encode()
        p = tmp_path / "o.safetensors"
        p.write_bytes(struct.pack("<Q", len(text)) + text + bytes(17))
        with pytest.raises(M.MxError) as e:
            dev.load_mxfp4(p, "b", "s")
        assert e.value.code == M.MX_EINVAL
