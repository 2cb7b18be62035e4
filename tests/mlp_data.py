"""Shared synthetic data for the GPU parity tests.

Inputs follow BASELINE.json: x ~ N(0,1) rounded to f16; weights ~ N(0,0.02)
in f32, quantized per 32 K-elements by the library's MXFP4 quantizer (whose
own parity with the oracle is tested separately).  Everything the oracle
consumes is downloaded from the device, so both sides see identical bits.
"""
import numpy as np

import mxfp4hip as M


class MlpData:
    def __init__(self, dev: M.Device, T: int, H: int, I: int, seed: int = 1, wfmt: int = 0):
        self.dev, self.T, self.H, self.I = dev, T, H, I
        self.x = dev.alloc(T * H * 2)
        dev.fill_normal(self.x, M.DT_F16, T * H, seed * 1000 + 1, 0.0, 1.0)
        self.mats = []
        for j, (n, k) in enumerate(((I, H), (I, H), (H, I))):
            w = dev.alloc(n * k * 4)
            dev.fill_normal(w, M.DT_F32, n * k, seed * 1000 + 2 + j, 0.0, 0.02)
            if wfmt == 0:
                q = dev.alloc(n * k // 2)
                s = dev.alloc(n * k // 32)
                dev.mxfp4_quantize(w, M.DT_F32, n, k, q, s)
            else:
                qbytes = n * k // 2 if wfmt == M.WFMT_INT4 else n * k
                sbytes = n * (k // 32) * 2 if wfmt == M.WFMT_INT4 else n * 4
                q = dev.alloc(qbytes)
                s = dev.alloc(sbytes)
                dev.fmt_quantize(wfmt, w, n, k, q, s)
            w.free()
            self.mats.append((q, s, n, k))
        self.weights = M.Device.weights(*[(q, s) for q, s, _, _ in self.mats])
        self.wfmt = wfmt

    def host(self):
        """(x f16, [(q, s) per matrix]) downloaded for the oracle."""
        x = self.dev.download(self.x, np.float16, (self.T, self.H))
        out = []
        for q, s, n, k in self.mats:
            if self.wfmt == 0:
                out.append((self.dev.download(q, np.uint8, (n, k // 2)),
                            self.dev.download(s, np.uint8, (n, k // 32))))
            elif self.wfmt == M.WFMT_INT4:
                out.append((self.dev.download(q, np.uint8, (n, k // 2)),
                            self.dev.download(s, np.float16, (n, k // 32))))
            else:
                out.append((self.dev.download(q, np.uint8, (n, k)),
                            self.dev.download(s, np.float32, (n,))))
        return x, out

    def free(self):
        self.x.free()
        for q, s, _, _ in self.mats:
            q.free()
            s.free()


def sample_rows(T: int, n: int, seed: int = 0):
    """Token rows to check: always the first and last, plus a random spread."""
    if T <= n:
        return np.arange(T, dtype=np.int32)
    rng = np.random.default_rng(seed)
    mid = rng.choice(np.arange(1, T - 1), n - 2, replace=False)
    return np.sort(np.concatenate([[0, T - 1], mid])).astype(np.int32)
