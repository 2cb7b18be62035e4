"""Python binding of libmxfp4hip (ctypes over the C ABI in include/mxfp4hip.h).

This is plumbing for tests and bench.py: every compute call goes through the
HIP library.  There is no CPU fallback; if the shared library is missing the
import fails with an error that says how to build it.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libmxfp4hip.so")

MX_OK, MX_EINVAL, MX_ENODEV, MX_ENOKERNEL, MX_ENOMEM, MX_EGPU = range(6)
DT_F32, DT_F16, DT_I8, DT_I32, DT_U8 = range(5)
FMT_FP4_E2M1, FMT_FP8_E4M3, FMT_FP8_E5M2 = range(3)
MLP_FUSED, MLP_DEQUANT, MLP_W4A4, MLP_REFROW, MLP_SCALED = range(5)
PROBE_F16, PROBE_FP4, PROBE_FP8, PROBE_INT4, PROBE_I8 = range(5)
WFMT_FP8_E4M3, WFMT_FP8_E5M2, WFMT_INT8, WFMT_INT4, WFMT_W8A8 = 1, 2, 3, 4, 5
WFMT_FP8_E4M3_F8X2, WFMT_FP8_E5M2_F8X2 = 6, 7  # FP8 weights on the scaled FP8 MFMA (F8X2 activations)

# Every symbol the header declares (checked by tests/test_abi_exports.py).
EXPORTS = [
    "mx_create", "mx_destroy", "mx_last_error", "mx_status_string", "mx_device_info",
    "mx_set_stream", "mx_get_stream", "mx_sync", "mx_timer_start", "mx_timer_stop", "mx_alloc", "mx_free", "mx_upload",
    "mx_download", "mx_memset", "mx_roundtrip", "mx_pack", "mx_unpack", "mx_mxfp4_quantize",
    "mx_mxfp4_dequant_f16", "mx_mxfp4_matmul", "mx_gemm_f16", "mx_gemm_i8", "mx_accum_gemm", "mx_swiglu", "mx_mlp_forward",
    "mx_mlp_benchmark", "mx_mlp_kernel_name", "mx_mlp_forward_noalloc", "mx_moe_forward", "mx_moe_benchmark",
    "mx_safetensors_find", "mx_load_mxfp4",
    "mx_fmt_quantize", "mx_fmt_mlp_forward",
    "mx_fmt_mlp_benchmark", "mx_fmt_mlp_kernel_name", "mx_fill_normal", "mx_lcg_bytes", "mx_lcg_pattern", "mx_lcg_half",
    "mx_lcg_int8", "mx_checksum_f32", "mx_checksum_i32", "mx_checksum_f16raw",
]


def safetensors_find(path, name):
    """(dtype, shape, file offset, byte size) of a tensor in a safetensors
    file, from the library's own header reader (no device needed)."""
    dt = ctypes.create_string_buffer(16)
    shape = (ctypes.c_longlong * 8)()
    nd = ctypes.c_int()
    off, nb = ctypes.c_ulonglong(), ctypes.c_ulonglong()
    rc = load().mx_safetensors_find(str(path).encode(), name.encode(), dt, 16, shape, 8, ctypes.byref(nd),
                                    ctypes.byref(off), ctypes.byref(nb))
    if rc:
        raise MxError(rc, f"tensor {name} not found or file unreadable")
    return dt.value.decode(), list(shape[:nd.value]), off.value, nb.value


class MxError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code
        self.message = message


class MlpConfig(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_uint32), ("hidden", ctypes.c_uint32),
                ("intermediate", ctypes.c_uint32)]


class QMatrix(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("scales", ctypes.c_void_p)]


class MlpWeights(ctypes.Structure):
    _fields_ = [("gate", QMatrix), ("up", QMatrix), ("down", QMatrix)]


_vp, _sz, _int, _u32, _u64, _f = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint32,
                                  ctypes.c_uint64, ctypes.c_float)
_lib = None


def load() -> ctypes.CDLL:
    """Load the built library (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: build it with "
                          "`python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER
    sig = {
        "mx_create": (_int, [_int, P(_vp)]),
        "mx_destroy": (None, [_vp]),
        "mx_last_error": (ctypes.c_char_p, [_vp]),
        "mx_status_string": (ctypes.c_char_p, [_int]),
        "mx_device_info": (_int, [_vp, ctypes.c_char_p, _sz, P(_int), P(_int)]),
        "mx_set_stream": (_int, [_vp, _vp]),
        "mx_get_stream": (_vp, [_vp]),
        "mx_sync": (_int, [_vp]),
        "mx_timer_start": (_int, [_vp]),
        "mx_timer_stop": (_int, [_vp, P(ctypes.c_double)]),
        "mx_alloc": (_int, [_vp, _sz, P(_vp)]),
        "mx_free": (_int, [_vp, _vp]),
        "mx_upload": (_int, [_vp, _vp, _vp, _sz]),
        "mx_download": (_int, [_vp, _vp, _vp, _sz]),
        "mx_memset": (_int, [_vp, _vp, _int, _sz]),
        "mx_roundtrip": (_int, [_vp, _int, _vp, _sz, _vp, _vp]),
        "mx_pack": (_int, [_vp, _int, _vp, _sz, _vp]),
        "mx_unpack": (_int, [_vp, _int, _vp, _sz, _vp]),
        "mx_mxfp4_quantize": (_int, [_vp, _vp, _int, _int, _int, _vp, _vp]),
        "mx_mxfp4_dequant_f16": (_int, [_vp, _vp, _vp, _vp, _int, _int]),
        "mx_mxfp4_matmul": (_int, [_vp, _vp, _int, _vp, _vp, _int, _int, _int, _int, _vp]),
        "mx_gemm_f16": (_int, [_vp, _vp, _int, _vp, _vp, _int, _int, _int]),
        "mx_gemm_i8": (_int, [_vp, _vp, _vp, _vp, _int, _int, _int]),
        "mx_accum_gemm": (_int, [_vp, _int, _vp, _int, _vp, _vp, _int, _int, _int, _int]),
        "mx_swiglu": (_int, [_vp, _vp, _vp, _vp, P(MlpConfig), _int]),
        "mx_mlp_forward": (_int, [_vp, _int, P(MlpConfig), _vp, P(MlpWeights), _vp]),
        "mx_mlp_forward_noalloc": (_int, [_vp, _int, P(MlpConfig), _vp, P(MlpWeights), _vp]),
        "mx_mlp_benchmark": (_int, [_vp, _int, P(MlpConfig), _vp, P(MlpWeights), _int, _vp, _int,
                                    _int, _int, P(ctypes.c_double), P(ctypes.c_double), P(_int)]),
        "mx_mlp_kernel_name": (ctypes.c_char_p, [_int, ctypes.c_void_p, _int]),
        "mx_moe_forward": (_int, [_vp, P(MlpConfig), _int, P(_int), _vp, P(MlpWeights), _vp]),
        "mx_safetensors_find": (_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, _sz,
                                       P(ctypes.c_longlong), _int, P(_int), P(ctypes.c_ulonglong),
                                       P(ctypes.c_ulonglong)]),
        "mx_load_mxfp4": (_int, [_vp, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, P(QMatrix),
                                 P(_int), P(_int), P(_int)]),
        "mx_moe_benchmark": (_int, [_vp, P(MlpConfig), _int, P(_int), _vp, P(MlpWeights), _int, _vp,
                                    _int, _int, _int, P(ctypes.c_double)]),
        "mx_fmt_quantize": (_int, [_vp, _int, _vp, _int, _int, _vp, _vp]),
        "mx_fmt_mlp_forward": (_int, [_vp, _int, P(MlpConfig), _vp, P(MlpWeights), _vp]),
        "mx_fmt_mlp_benchmark": (_int, [_vp, _int, P(MlpConfig), _vp, P(MlpWeights), _int, _vp,
                                        _int, _int, _int, P(ctypes.c_double), _vp, _vp]),
        "mx_fmt_mlp_kernel_name": (ctypes.c_char_p, [_int, ctypes.c_void_p, _int]),
        "mx_fill_normal": (_int, [_vp, _vp, _int, _sz, _u64, _f, _f]),
        "mx_lcg_bytes": (None, [_u32, _sz, _vp]),
        "mx_lcg_pattern": (None, [_u32, _sz, _vp, _int, _vp]),
        "mx_lcg_half": (None, [_u32, _sz, _f, _vp]),
        "mx_lcg_int8": (None, [_u32, _sz, _vp]),
        "mx_checksum_f32": (ctypes.c_double, [_vp, _sz, P(_int)]),
        "mx_checksum_i32": (ctypes.c_int64, [_vp, _sz, P(_int)]),
        "mx_checksum_f16raw": (ctypes.c_uint64, [_vp, _sz, P(_int)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _np_ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


class DevBuf:
    """A device allocation owned by a Device (freed with it or by free())."""

    def __init__(self, dev: "Device", ptr: int, nbytes: int):
        self.dev, self.ptr, self.nbytes = dev, ptr, nbytes

    @property
    def p(self):
        return ctypes.c_void_p(self.ptr)

    def offset(self, nbytes: int) -> ctypes.c_void_p:
        return ctypes.c_void_p(self.ptr + nbytes)

    def free(self):
        if self.ptr:
            self.dev._check(load().mx_free(self.dev.ctx, ctypes.c_void_p(self.ptr)))
            self.dev._bufs.discard(self)
            self.ptr = 0


class Device:
    """One libmxfp4hip context (device + stream)."""

    def __init__(self, device: int = 0):
        L = load()
        h = ctypes.c_void_p()
        rc = L.mx_create(device, ctypes.byref(h))
        if rc != MX_OK:
            raise MxError(rc, L.mx_status_string(rc).decode())
        self.ctx = h
        self._bufs: set[DevBuf] = set()

    def close(self):
        if self.ctx:
            for b in list(self._bufs):
                b.free()
            load().mx_destroy(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc: int):
        if rc != MX_OK:
            raise MxError(rc, load().mx_last_error(self.ctx).decode())

    def info(self):
        name = ctypes.create_string_buffer(256)
        cus, clk = ctypes.c_int(), ctypes.c_int()
        self._check(load().mx_device_info(self.ctx, name, 256, ctypes.byref(cus), ctypes.byref(clk)))
        return name.value.decode(), cus.value, clk.value

    # ---- memory ----
    def alloc(self, nbytes: int) -> DevBuf:
        p = ctypes.c_void_p()
        self._check(load().mx_alloc(self.ctx, max(int(nbytes), 1), ctypes.byref(p)))
        b = DevBuf(self, p.value, int(nbytes))
        self._bufs.add(b)
        return b

    def upload(self, a: np.ndarray, buf: DevBuf | None = None) -> DevBuf:
        a = np.ascontiguousarray(a)
        if buf is None:
            buf = self.alloc(a.nbytes)
        self._check(load().mx_upload(self.ctx, buf.p, _np_ptr(a), a.nbytes))
        return buf

    def download(self, buf, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        src = buf.p if isinstance(buf, DevBuf) else buf
        self._check(load().mx_download(self.ctx, _np_ptr(out), src, out.nbytes))
        return out

    def memset(self, buf: DevBuf, value: int = 0):
        self._check(load().mx_memset(self.ctx, buf.p, value, buf.nbytes))

    def sync(self):
        self._check(load().mx_sync(self.ctx))

    def timer_start(self):
        self._check(load().mx_timer_start(self.ctx))

    def timer_stop(self) -> float:
        secs = ctypes.c_double()
        self._check(load().mx_timer_stop(self.ctx, ctypes.byref(secs)))
        return secs.value

    # ---- codecs ----
    def roundtrip(self, fmt: int, values) -> tuple[np.ndarray, np.ndarray]:
        x = np.ascontiguousarray(values, np.float32)
        nb = (x.size + 1) // 2 if fmt == FMT_FP4_E2M1 else x.size
        packed = np.zeros(nb, np.uint8)
        out = np.zeros(x.size, np.float32)
        self._check(load().mx_roundtrip(self.ctx, fmt, _np_ptr(x), x.size, _np_ptr(packed),
                                        _np_ptr(out)))
        return packed, out

    def pack(self, fmt, src: DevBuf, n: int, dst: DevBuf):
        self._check(load().mx_pack(self.ctx, fmt, src.p, n, dst.p))

    def unpack(self, fmt, src: DevBuf, n: int, dst: DevBuf):
        self._check(load().mx_unpack(self.ctx, fmt, src.p, n, dst.p))

    def mxfp4_quantize(self, src: DevBuf, src_dtype: int, rows: int, k: int, packed: DevBuf,
                       scales: DevBuf):
        self._check(load().mx_mxfp4_quantize(self.ctx, src.p, src_dtype, rows, k, packed.p,
                                             scales.p))

    def mxfp4_dequant_f16(self, packed: DevBuf, scales: DevBuf, out: DevBuf, rows: int, depth: int):
        self._check(load().mx_mxfp4_dequant_f16(self.ctx, packed.p, scales.p, out.p, rows, depth))

    def mxfp4_matmul(self, a: DevBuf, a_dtype, b: DevBuf, c: DevBuf, c_dtype, m, n, k,
                     scales: DevBuf):
        self._check(load().mx_mxfp4_matmul(self.ctx, a.p, a_dtype, b.p, c.p, c_dtype, m, n, k,
                                           scales.p))

    def gemm_f16(self, a: DevBuf, a_dtype, b: DevBuf, c: DevBuf, m, n, k):
        self._check(load().mx_gemm_f16(self.ctx, a.p, a_dtype, b.p, c.p, m, n, k))

    def gemm_i8(self, a: DevBuf, b: DevBuf, c: DevBuf, m, n, k):
        self._check(load().mx_gemm_i8(self.ctx, a.p, b.p, c.p, m, n, k))

    def accum_gemm(self, a_fmt, a: DevBuf, b_fmt, b: DevBuf, c: DevBuf, c_dtype, m, n, k):
        """Accumulator-probe GEMM (AccumProbeKernels.metal:41-127)."""
        self._check(load().mx_accum_gemm(self.ctx, a_fmt, a.p, b_fmt, b.p, c.p, c_dtype, m, n, k))

    def swiglu(self, variant, gate: DevBuf, up: DevBuf, mid: DevBuf, tokens, inter):
        """mx_swiglu: gate, up, mid, MLPConfig, then the variant (0 float,
        1 half, 2 half from half, 3 i8)."""
        cfg = MlpConfig(tokens, 0, inter)
        self._check(load().mx_swiglu(self.ctx, gate.p, up.p, mid.p, ctypes.byref(cfg), variant))

    def fill_normal(self, buf: DevBuf, dtype: int, n: int, seed: int, mean=0.0, std=1.0):
        self._check(load().mx_fill_normal(self.ctx, buf.p, dtype, n, seed, mean, std))

    # ---- MLP ----
    @staticmethod
    def weights(gate, up, down) -> MlpWeights:
        """gate/up/down: (data DevBuf, scales DevBuf) pairs."""
        q = lambda m: QMatrix(m[0].ptr, m[1].ptr)
        return MlpWeights(q(gate), q(up), q(down))

    def mlp_forward(self, variant, tokens, hidden, inter, x: DevBuf, w: MlpWeights, out: DevBuf):
        cfg = MlpConfig(tokens, hidden, inter)
        self._check(load().mx_mlp_forward(self.ctx, variant, ctypes.byref(cfg), x.p,
                                          ctypes.byref(w), out.p))

    def mlp_forward_noalloc(self, variant, tokens, hidden, inter, x: DevBuf, w: MlpWeights, out: DevBuf):
        """mx_mlp_forward with the library's static scratch array (no device
        allocation)."""
        cfg = MlpConfig(tokens, hidden, inter)
        self._check(load().mx_mlp_forward_noalloc(self.ctx, variant, ctypes.byref(cfg), x.p,
                                                  ctypes.byref(w), out.p))

    def mlp_benchmark(self, variant, tokens, hidden, inter, x: DevBuf, sets, out: DevBuf,
                      warmup=1, iterations=20, per_kernel=True, graph=True):
        cfg = MlpConfig(tokens, hidden, inter)
        arr = (MlpWeights * len(sets))(*sets)
        secs = ctypes.c_double()
        kus = (ctypes.c_double * 8)()
        nk = ctypes.c_int(0)
        self._check(load().mx_mlp_benchmark(
            self.ctx, variant, ctypes.byref(cfg), x.p, arr, len(sets), out.p, warmup, iterations,
            1 if graph else 0, ctypes.byref(secs), kus if per_kernel else None,
            ctypes.byref(nk) if per_kernel else None))
        names = [load().mx_mlp_kernel_name(variant, ctypes.byref(cfg), i).decode() for i in range(nk.value)]
        return secs.value, dict(zip(names, list(kus)[:nk.value]))

    # ---- on-disk MXFP4 weights ----
    def load_mxfp4(self, path, blocks_name, scales_name):
        """(data DevBuf, scales DevBuf, experts, n, k) of a safetensors MXFP4 matrix."""
        q = QMatrix()
        cnt, n, k = _int(), _int(), _int()
        self._check(load().mx_load_mxfp4(self.ctx, str(path).encode(), blocks_name.encode(),
                                         scales_name.encode(), ctypes.byref(q), ctypes.byref(cnt),
                                         ctypes.byref(n), ctypes.byref(k)))
        data = DevBuf(self, q.data, cnt.value * n.value * k.value // 2)
        scales = DevBuf(self, q.scales, cnt.value * n.value * k.value // 32)
        self._bufs.update((data, scales))
        return data, scales, cnt.value, n.value, k.value

    # ---- MoE (experts stacked; x rows grouped by expert) ----
    def moe_forward(self, hidden, inter, counts, x: DevBuf, w: MlpWeights, out: DevBuf):
        cfg = MlpConfig(int(sum(counts)), hidden, inter)
        cnt = (_int * len(counts))(*counts)
        self._check(load().mx_moe_forward(self.ctx, ctypes.byref(cfg), len(counts), cnt, x.p,
                                          ctypes.byref(w), out.p))

    def moe_benchmark(self, hidden, inter, counts, x: DevBuf, sets, out: DevBuf, warmup=1,
                      iterations=20, graph=True):
        cfg = MlpConfig(int(sum(counts)), hidden, inter)
        cnt = (_int * len(counts))(*counts)
        arr = (MlpWeights * len(sets))(*sets)
        secs = ctypes.c_double()
        self._check(load().mx_moe_benchmark(self.ctx, ctypes.byref(cfg), len(counts), cnt, x.p, arr,
                                            len(sets), out.p, warmup, iterations, 1 if graph else 0,
                                            ctypes.byref(secs)))
        return secs.value

    def fmt_quantize(self, wfmt, w: DevBuf, rows, k, q: DevBuf, scales: DevBuf):
        self._check(load().mx_fmt_quantize(self.ctx, wfmt, w.p, rows, k, q.p, scales.p))

    def fmt_mlp_forward(self, wfmt, tokens, hidden, inter, x: DevBuf, w: MlpWeights,
                        out: DevBuf):
        cfg = MlpConfig(tokens, hidden, inter)
        self._check(load().mx_fmt_mlp_forward(self.ctx, wfmt, ctypes.byref(cfg), x.p,
                                              ctypes.byref(w), out.p))

    def fmt_mlp_benchmark(self, wfmt, tokens, hidden, inter, x: DevBuf, sets, out: DevBuf,
                          warmup=1, iterations=20, graph=True, per_kernel=False):
        """Seconds for `iterations` forwards; with per_kernel, also
        {kernel name: us per launch} (mx_fmt_mlp_benchmark)."""
        cfg = MlpConfig(tokens, hidden, inter)
        arr = (MlpWeights * len(sets))(*sets)
        secs = ctypes.c_double()
        kus = (ctypes.c_double * 8)()
        nk = ctypes.c_int(0)
        self._check(load().mx_fmt_mlp_benchmark(self.ctx, wfmt, ctypes.byref(cfg), x.p, arr,
                                                len(sets), out.p, warmup, iterations,
                                                1 if graph else 0, ctypes.byref(secs),
                                                kus if per_kernel else None,
                                                ctypes.byref(nk) if per_kernel else None))
        if not per_kernel:
            return secs.value
        names = [load().mx_fmt_mlp_kernel_name(wfmt, ctypes.byref(cfg), i).decode() for i in range(nk.value)]
        return secs.value, dict(zip(names, list(kus)[:nk.value]))


# ---- host helpers (no GPU needed) -------------------------------------------
def mlp_kernel_name(variant: int, tokens: int, hidden: int, inter: int, index: int):
    """Name of kernel `index` of the forward `variant` runs at this shape
    (mx_mlp_kernel_name; host logic, no device); None past the last one."""
    cfg = MlpConfig(tokens, hidden, inter)
    name = load().mx_mlp_kernel_name(variant, ctypes.byref(cfg), index)
    return None if name is None else name.decode()


def lcg_bytes(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.uint8)
    load().mx_lcg_bytes(seed, count, _np_ptr(out))
    return out


def lcg_pattern(seed: int, count: int, pattern) -> np.ndarray:
    pat = np.ascontiguousarray(pattern, np.uint8)
    out = np.empty(count, np.uint8)
    load().mx_lcg_pattern(seed, count, _np_ptr(pat), pat.size, _np_ptr(out))
    return out


def lcg_half(seed: int, count: int, scale: float) -> np.ndarray:
    out = np.empty(count, np.uint16)
    load().mx_lcg_half(seed, count, scale, _np_ptr(out))
    return out.view(np.float16)


def lcg_int8(seed: int, count: int) -> np.ndarray:
    out = np.empty(count, np.int8)
    load().mx_lcg_int8(seed, count, _np_ptr(out))
    return out


def checksum_f32(a: np.ndarray):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    n = ctypes.c_int()
    return load().mx_checksum_f32(_np_ptr(a), a.size, ctypes.byref(n)), n.value


def checksum_f16raw(a: np.ndarray):
    a = np.ascontiguousarray(a).view(np.uint16).reshape(-1)
    n = ctypes.c_int()
    return load().mx_checksum_f16raw(_np_ptr(a), a.size, ctypes.byref(n)), n.value


def status_string(code: int) -> str:
    return load().mx_status_string(code).decode()
