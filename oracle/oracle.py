"""ctypes + numpy front end of the CPU oracle (oracle/mx_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product (libmxfp4hip) never
loads it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_u8p = ctypes.POINTER(ctypes.c_uint8)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_int = ctypes.c_int

FMT_FP4, FMT_E4M3, FMT_E5M2 = 0, 1, 2
# weight-format ids of orc_mlp_format / orc_quant_rowwise
WF_E4M3, WF_E5M2, WF_INT8, WF_INT4, WF_W8A8 = 1, 2, 3, 4, 5

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "orc_f32_to_f16": (ctypes.c_uint16, [ctypes.c_float]),
            "orc_f16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
            "orc_f32_to_f16_bulk": (None, [_vp, _sz, _vp]),
            "orc_e8m0_to_float": (ctypes.c_float, [ctypes.c_uint8]),
            "orc_fp4_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "orc_fp4_encode": (ctypes.c_uint8, [ctypes.c_float]),
            "orc_fp8_e4m3_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "orc_fp8_e4m3_encode": (ctypes.c_uint8, [ctypes.c_float]),
            "orc_fp8_e5m2_decode": (ctypes.c_float, [ctypes.c_uint8]),
            "orc_fp8_e5m2_encode": (ctypes.c_uint8, [ctypes.c_float]),
            "orc_pack": (None, [_int, _vp, _sz, _vp]),
            "orc_unpack": (None, [_int, _vp, _sz, _vp]),
            "orc_mxfp4_scale_byte": (ctypes.c_uint8, [ctypes.c_float]),
            "orc_mxfp4_quantize_f32": (None, [_vp, _int, _int, _vp, _vp]),
            "orc_mxfp4_quantize_f16": (None, [_vp, _int, _int, _vp, _vp]),
            "orc_mxfp4_dequant_f16": (None, [_vp, _vp, _int, _int, _vp]),
            "orc_mxfp4_matmul": (None, [_vp, _int, _vp, _vp, _int, _int, _int, _vp]),
            "orc_silu": (ctypes.c_float, [ctypes.c_float]),
            "orc_swiglu_float": (None, [_vp, _vp, _sz, _vp]),
            "orc_swiglu_half": (None, [_vp, _vp, _sz, _vp]),
            "orc_swiglu_i8": (None, [_vp, _vp, _sz, _vp]),
            "orc_set_accum_f32": (None, [_int]),
            "orc_mlp_mxfp4": (None, [_int, _int, _int, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                     _vp, _int, _vp, _int]),
            "orc_quant_rowwise": (None, [_int, _vp, _int, _int, _vp, _vp]),
            "orc_quant_int4_g32": (None, [_vp, _int, _int, _vp, _vp]),
            "orc_quant_int8_per_token": (None, [_vp, _int, _int, _vp, _vp]),
            "orc_mlp_format": (None, [_int, _int, _int, _int, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                      _vp, _int, _vp, _int]),
            "orc_lcg_bytes": (None, [ctypes.c_uint32, _sz, _vp]),
            "orc_lcg_pattern": (None, [ctypes.c_uint32, _sz, _vp, _int, _vp]),
            "orc_lcg_half": (None, [ctypes.c_uint32, _sz, ctypes.c_float, _vp]),
            "orc_lcg_int8": (None, [ctypes.c_uint32, _sz, _vp]),
            "orc_checksum_f32": (ctypes.c_double, [_vp, _sz, ctypes.POINTER(_int)]),
            "orc_checksum_i32": (ctypes.c_int64, [_vp, _sz, ctypes.POINTER(_int)]),
            "orc_checksum_f16raw": (ctypes.c_uint64, [_vp, _sz, ctypes.POINTER(_int)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ---- codecs ---------------------------------------------------------------
def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_f16_bulk(_p(x), x.size, _p(out))
    return out


def pack(fmt: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    nbytes = (x.size + 1) // 2 if fmt == FMT_FP4 else x.size
    out = np.zeros(nbytes, np.uint8)
    lib().orc_pack(fmt, _p(x), x.size, _p(out))
    return out


def unpack(fmt: int, packed: np.ndarray, n: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.empty(n, np.float32)
    lib().orc_unpack(fmt, _p(packed), n, _p(out))
    return out


def mxfp4_quantize(x: np.ndarray):
    """[rows][k] f32 or f16 -> (packed [rows][k/2] u8, scales [rows][k/32] u8)."""
    rows, k = x.shape
    packed = np.empty((rows, k // 2), np.uint8)
    scales = np.empty((rows, k // 32), np.uint8)
    if x.dtype == np.float16:
        xb = np.ascontiguousarray(x).view(np.uint16)
        lib().orc_mxfp4_quantize_f16(_p(xb), rows, k, _p(packed), _p(scales))
    else:
        xf = np.ascontiguousarray(x, dtype=np.float32)
        lib().orc_mxfp4_quantize_f32(_p(xf), rows, k, _p(packed), _p(scales))
    return packed, scales


def mxfp4_dequant_f16(packed: np.ndarray, scales: np.ndarray, rows: int, depth: int) -> np.ndarray:
    out = np.empty((rows, depth), np.uint16)
    lib().orc_mxfp4_dequant_f16(_p(np.ascontiguousarray(packed)), _p(np.ascontiguousarray(scales)),
                                rows, depth, _p(out))
    return out.view(np.float16)


def mxfp4_matmul(a: np.ndarray, b: np.ndarray, s: np.ndarray, n: int) -> np.ndarray:
    m, k = a.shape
    c = np.empty((m, n), np.float32)
    if a.dtype == np.float16:
        lib().orc_mxfp4_matmul(_p(np.ascontiguousarray(a).view(np.uint16)), 0, _p(b), _p(s), m, n,
                               k, _p(c))
    else:
        lib().orc_mxfp4_matmul(_p(np.ascontiguousarray(a, dtype=np.float32)), 1, _p(b), _p(s), m,
                               n, k, _p(c))
    return c


def swiglu_float(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().orc_swiglu_float(_p(g), _p(u), g.size, _p(out))
    return out


def swiglu_half(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty(g.shape, np.uint16)
    lib().orc_swiglu_half(_p(g), _p(u), g.size, _p(out))
    return out.view(np.float16)


def swiglu_i8(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    """mpp_mlp_swiglu_i8 (MPPMLPKernels.metal:240-257): int32 gate/up -> int8 mid."""
    g = np.ascontiguousarray(g, np.int32)
    u = np.ascontiguousarray(u, np.int32)
    out = np.empty(g.shape, np.int8)
    lib().orc_swiglu_i8(_p(g), _p(u), g.size, _p(out))
    return out


MLP_F16, MLP_W4A4, MLP_REFROW = 0, 1, 2


def mlp_mxfp4(mode: int, x: np.ndarray, wg, sg, wu, su, wd, sd, hidden: int, inter: int,
              rows=None, threads: int = 1) -> np.ndarray:
    """MXFP4 MLP on the CPU.  x: [T][H] float16.  rows: token indices or None."""
    tokens = x.shape[0]
    xb = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    sel = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    n_sel = tokens if sel is None else sel.size
    if mode == MLP_REFROW:
        out = np.empty((n_sel, hidden), np.float32)
    else:
        out = np.empty((n_sel, hidden), np.uint16)
    lib().orc_mlp_mxfp4(mode, tokens, hidden, inter, _p(xb), _p(wg), _p(sg), _p(wu), _p(su),
                        _p(wd), _p(sd), _p(sel), n_sel, _p(out), threads)
    return out if mode == MLP_REFROW else out.view(np.float16)


def set_accum_f32(on: bool) -> None:
    """float32 (True) or float64 (False, the default) dot-product accumulation
    in mlp_mxfp4 / mlp_format; float32 only for timing the CPU baseline."""
    lib().orc_set_accum_f32(1 if on else 0)


def quant_rowwise(fmt: int, w: np.ndarray):
    rows, k = w.shape
    q = np.empty((rows, k), np.uint8)
    sc = np.empty(rows, np.float32)
    lib().orc_quant_rowwise(fmt, _p(np.ascontiguousarray(w, np.float32)), rows, k, _p(q), _p(sc))
    return q, sc


def quant_int4_g32(w: np.ndarray):
    rows, k = w.shape
    q = np.empty((rows, k // 2), np.uint8)
    sc = np.empty((rows, k // 32), np.uint16)
    lib().orc_quant_int4_g32(_p(np.ascontiguousarray(w, np.float32)), rows, k, _p(q), _p(sc))
    return q, sc.view(np.float16)


def quant_int8_per_token(x: np.ndarray):
    rows, k = x.shape
    q = np.empty((rows, k), np.int8)
    sc = np.empty(rows, np.float32)
    lib().orc_quant_int8_per_token(_p(np.ascontiguousarray(x, np.float32)), rows, k, _p(q),
                                   _p(sc))
    return q, sc


def mlp_format(fmt: int, x: np.ndarray, qg, sg, qu, su, qd, sd, hidden: int, inter: int,
               rows=None, threads: int = 1) -> np.ndarray:
    tokens = x.shape[0]
    xb = np.ascontiguousarray(x, dtype=np.float16).view(np.uint16)
    sel = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
    n_sel = tokens if sel is None else sel.size
    out = np.empty((n_sel, hidden), np.uint16)
    conv = lambda s: np.ascontiguousarray(s).view(np.uint16) if s.dtype == np.float16 else \
        np.ascontiguousarray(s)
    lib().orc_mlp_format(fmt, tokens, hidden, inter, _p(xb), _p(qg), _p(conv(sg)), _p(qu),
                         _p(conv(su)), _p(qd), _p(conv(sd)), _p(sel), n_sel, _p(out), threads)
    return out.view(np.float16)


# ---- reference generators and checksums (main.swift:2785-2884) ------------
def lcg_bytes(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint8)
    lib().orc_lcg_bytes(seed, count, _p(out))
    return out


def lcg_pattern(seed: int, count: int, pattern) -> np.ndarray:
    pat = np.asarray(pattern, np.uint8)
    out = np.empty(count, np.uint8)
    lib().orc_lcg_pattern(seed, count, _p(pat), pat.size, _p(out))
    return out


def lcg_half(seed: int, count: int, scale: float) -> np.ndarray:
    out = np.empty(count, np.uint16)
    lib().orc_lcg_half(seed, count, scale, _p(out))
    return out.view(np.float16)


def lcg_int8(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.int8)
    lib().orc_lcg_int8(seed, count, _p(out))
    return out


def checksum_f32(a: np.ndarray):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    n = _int(0)
    s = lib().orc_checksum_f32(_p(a), a.size, ctypes.byref(n))
    return s, n.value


def checksum_i32(a: np.ndarray):
    a = np.ascontiguousarray(a, np.int32).reshape(-1)
    n = _int(0)
    s = lib().orc_checksum_i32(_p(a), a.size, ctypes.byref(n))
    return s, n.value


def checksum_f16raw(a: np.ndarray):
    a = np.ascontiguousarray(a).view(np.uint16).reshape(-1)
    n = _int(0)
    s = lib().orc_checksum_f16raw(_p(a), a.size, ctypes.byref(n))
    return s, n.value


# ---- tolerance --------------------------------------
def mlp_error(got: np.ndarray, ref: np.ndarray):
    """(max_abs / rms(ref), cosine) of got vs ref."""
    g = np.asarray(got, np.float64).reshape(-1)
    r = np.asarray(ref, np.float64).reshape(-1)
    rms = float(np.sqrt(np.mean(r * r)))
    max_abs = float(np.max(np.abs(g - r)))
    cos = float(np.dot(g, r) / (np.linalg.norm(g) * np.linalg.norm(r)))
    return max_abs / rms, cos


MAX_ABS_REL_TOL = 2e-2     # max-abs error <= 2e-2 * rms(ref)
COSINE_TOL = 0.9995        # cosine >= 0.9995
