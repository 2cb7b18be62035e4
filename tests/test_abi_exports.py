"""The C ABI library loads and exports what include/mxfp4hip.h declares (CPU).

No GPU compute here: only symbol presence, the no-device error path, and the
host-side helpers (reference LCG generators and checksums), which must match
the oracle bit for bit.
"""
import ctypes
import os
import re

import numpy as np
import pytest

import mxfp4hip as M
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    src = open(os.path.join(ROOT, "include", "mxfp4hip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(mx_[a-z0-9_]+)\s*\(", src)))


def test_every_declared_symbol_is_exported():
    lib = M.load()
    names = header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert sorted(M.EXPORTS) == names


def test_status_strings_mirror_probe_errors():
    assert M.status_string(M.MX_OK) == "ok"
    assert "No HIP device" in M.status_string(M.MX_ENODEV)
    assert M.status_string(99) == "unknown status"


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present")
def test_no_device_is_reported():
    with pytest.raises(M.MxError) as e:
        M.Device(0)
    assert e.value.code == M.MX_ENODEV


def test_lcg_generators_match_oracle():
    for seed in (0x11112222, 0xabcd1357, 0x0badcafe):
        assert np.array_equal(M.lcg_bytes(seed, 5000), O.lcg_bytes(seed, 5000))
        assert np.array_equal(M.lcg_half(seed, 5000, 0.125).view(np.uint16),
                              O.lcg_half(seed, 5000, 0.125).view(np.uint16))
        assert np.array_equal(M.lcg_int8(seed, 5000), O.lcg_int8(seed, 5000))
        pat = [124, 125, 126, 127, 127, 128, 128, 129, 130]
        assert np.array_equal(M.lcg_pattern(seed, 5000, pat), O.lcg_pattern(seed, 5000, pat))


def test_checksums_match_oracle():
    rng = np.random.default_rng(0)
    a = rng.standard_normal(131072).astype(np.float32)
    assert M.checksum_f32(a) == O.checksum_f32(a)
    h = a.astype(np.float16)
    assert M.checksum_f16raw(h) == O.checksum_f16raw(h)
    assert M.checksum_f32(a[:10])[1] == 10       # step = max(1, count/32)


def test_kernel_names_follow_the_shape():
    """The per-kernel names report the kernel each shape runs (host logic of
    the library, no device): the decode GEMV for <= 16 tokens at % 128, the
    64-K-stage family at % 64, the K-step-32 kernel at % 32 only."""
    assert M.mlp_kernel_name(M.MLP_FUSED, 8, 256, 512, 0) == "gemv_mxfp4_gate_up_swiglu"
    assert M.mlp_kernel_name(M.MLP_FUSED, 8, 192, 320, 0) == "gemm_q_mxfp4_gate_up_swiglu"
    assert M.mlp_kernel_name(M.MLP_FUSED, 5, 96, 160, 0) == "gemm_h_mxfp4_gate_up_swiglu"
    assert M.mlp_kernel_name(M.MLP_FUSED, 40, 1056, 2080, 1) == "gemm_h_mxfp4_down"
    assert M.mlp_kernel_name(M.MLP_REFROW, 5, 96, 160, 1) == "gemm_h_mxfp4_down_f32"
    assert M.mlp_kernel_name(M.MLP_REFROW, 128, 1024, 4096, 0) == "gemm_q_mxfp4_gate_up_swiglu_half"
    assert M.mlp_kernel_name(M.MLP_FUSED, 5, 96, 160, 2) is None
