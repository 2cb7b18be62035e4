"""On-disk MXFP4 weights: the library's safetensors header reader
(mx_safetensors_find, host only, no device) against files written by the
safetensors package, including metadata, several tensors and other dtypes,
and its error paths."""
import json
import os
import struct

import numpy as np
import pytest

import mxfp4hip as M

pytestmark = pytest.mark.skipif(not os.path.exists(M.LIB_PATH), reason="library not built (run build())")
st = pytest.importorskip("safetensors.numpy")


def test_finds_every_tensor_and_its_bytes(tmp_path):
    rng = np.random.default_rng(0)
    tensors = {
        "model.layers.0.mlp.gate.blocks": rng.integers(0, 256, (64, 4, 16), dtype=np.uint8),
        "model.layers.0.mlp.gate.scales": rng.integers(118, 124, (64, 4), dtype=np.uint8),
        "experts.down.blocks": rng.integers(0, 256, (3, 32, 2, 16), dtype=np.uint8),
        "bias": rng.standard_normal(33).astype(np.float32),
        'odd "name" \\ with escapes': np.arange(5, dtype=np.int16),
    }
    path = tmp_path / "w.safetensors"
    st.save_file(tensors, str(path), metadata={"format": "mxfp4", "note": "{not: json}"})
    raw = path.read_bytes()
    for name, arr in tensors.items():
        dtype, shape, off, nbytes = M.safetensors_find(path, name)
        assert shape == list(arr.shape), name
        assert nbytes == arr.nbytes, name
        assert raw[off:off + nbytes] == arr.tobytes(), name
        assert dtype == {np.uint8: "U8", np.float32: "F32", np.int16: "I16"}[arr.dtype.type], name


def test_hand_written_header(tmp_path):
    """A header written by hand: whitespace, key order, nested metadata."""
    data = bytes(range(48))
    header = {"__metadata__": {"a": "b"},
              "t": {"data_offsets": [16, 48], "shape": [2, 16], "dtype": "U8"},
              "u": {"dtype": "U8", "shape": [16], "data_offsets": [0, 16]}}
    text = json.dumps(header, indent=2).encode()
    path = tmp_path / "h.safetensors"
    path.write_bytes(struct.pack("<Q", len(text)) + text + data)
    dtype, shape, off, nbytes = M.safetensors_find(path, "t")
    assert (dtype, shape, nbytes) == ("U8", [2, 16], 32)
    assert path.read_bytes()[off:off + nbytes] == data[16:48]
    assert M.safetensors_find(path, "u")[2] == 8 + len(text)


def test_errors(tmp_path):
    path = tmp_path / "w.safetensors"
    st.save_file({"x": np.zeros(4, np.uint8)}, str(path))
    with pytest.raises(M.MxError):
        M.safetensors_find(path, "missing")
    bad = tmp_path / "bad.safetensors"
    bad.write_bytes(b"\x05\x00\x00\x00\x00\x00\x00\x00{oops")
    with pytest.raises(M.MxError):
        M.safetensors_find(bad, "x")
    short = tmp_path / "short.safetensors"  # data range past the end of the file
    text = json.dumps({"x": {"dtype": "U8", "shape": [64], "data_offsets": [0, 64]}}).encode()
    short.write_bytes(struct.pack("<Q", len(text)) + text + bytes(10))
    with pytest.raises(M.MxError):
        M.safetensors_find(short, "x")
    with pytest.raises(M.MxError):
        M.safetensors_find(tmp_path / "nope.safetensors", "x")


@pytest.mark.parametrize("shape_txt", ["[99999999999999999999999]", "[-]", "[9223372036854775808]", "[1, -]"])
def test_oversized_or_malformed_integers_fail_cleanly(tmp_path, shape_txt):
    """The header is untrusted: an integer outside long long (or a bare minus
    sign) is a parse error reported as a status, not an exception across the
    C ABI."""
    text = ('{"x": {"dtype": "U8", "shape": %s, "data_offsets": [0, 4]}}' % shape_txt).encode()
    p = tmp_path / "big.safetensors"
    p.write_bytes(struct.pack("<Q", len(text)) + text + bytes(4))
    with pytest.raises(M.MxError):
        M.safetensors_find(p, "x")
