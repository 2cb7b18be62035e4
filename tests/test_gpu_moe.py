"""MoE grouped experts (mx_moe_forward): every expert's MXFP4 MLP over its own
rows of one token batch, in two grouped launches.  Each expert is checked
against the CPU oracle's MLP on that expert's rows and weights (BASELINE
tolerance), on both the decode-GEMV form (<= 16 tokens per expert) and the
small-M GEMM form, with empty experts in the mix."""
import types

import numpy as np
import pytest

import mxfp4hip as M
import oracle as O
from mlp_data import MlpData

pytestmark = pytest.mark.gpu
TOL, COS = O.MAX_ABS_REL_TOL, O.COSINE_TOL


class MoeData:
    """x [T][H] f16 ~ N(0,1); experts stacked: gate / up [E*I][H], down
    [E*H][I], each N(0, 0.02) quantized by the library's MXFP4 quantizer
    (rows are independent, so a stacked quantize is each expert's)."""

    def __init__(self, dev, counts, H, I, seed):
        self.dev, self.counts, self.H, self.I, self.E = dev, list(counts), H, I, len(counts)
        self.T = int(sum(counts))
        self.x = dev.alloc(self.T * H * 2)
        dev.fill_normal(self.x, M.DT_F16, self.T * H, seed * 1000 + 1, 0.0, 1.0)
        self.mats = []
        for j, (n, k) in enumerate(((self.E * I, H), (self.E * I, H), (self.E * H, I))):
            w = dev.alloc(n * k * 4)
            dev.fill_normal(w, M.DT_F32, n * k, seed * 1000 + 2 + j, 0.0, 0.02)
            q, s = dev.alloc(n * k // 2), dev.alloc(n * k // 32)
            dev.mxfp4_quantize(w, M.DT_F32, n, k, q, s)
            w.free()
            self.mats.append((q, s, n, k))
        self.weights = M.Device.weights(*[(q, s) for q, s, _, _ in self.mats])

    def oracle(self, rows=None):
        """Oracle MLP of every expert on its rows; `rows` (token indices)
        limits the work to those tokens (the others stay zero)."""
        x = self.dev.download(self.x, np.float16, (self.T, self.H))
        host = [(self.dev.download(q, np.uint8, (n, k // 2)), self.dev.download(s, np.uint8, (n, k // 32)))
                for q, s, n, k in self.mats]
        out = np.zeros((self.T, self.H), np.float64)
        t0 = 0
        H, I = self.H, self.I
        for e, cnt in enumerate(self.counts):
            sel = np.arange(t0, t0 + cnt) if rows is None else np.array([r for r in rows if t0 <= r < t0 + cnt], int)
            if len(sel):
                sl = lambda m, rows: (m[0][e * rows:(e + 1) * rows], m[1][e * rows:(e + 1) * rows])
                (qg, sg), (qu, su), (qd, sd) = sl(host[0], I), sl(host[1], I), sl(host[2], H)
                out[sel] = O.mlp_mxfp4(O.MLP_F16, x[sel], qg, sg, qu, su, qd, sd, H, I, threads=16)
            t0 += cnt
        return out

    def run(self):
        out = self.dev.alloc(self.T * self.H * 2)
        self.dev.moe_forward(self.H, self.I, self.counts, self.x, self.weights, out)
        got = self.dev.download(out, np.float16, (self.T, self.H))
        out.free()
        return got

    def free(self):
        self.x.free()
        for q, s, _, _ in self.mats:
            q.free()
            s.free()


def check(got, ref, what):
    rel, cos = O.mlp_error(got, ref)
    print(f"{what}: max_abs/rms={rel:.3e} cos={cos:.7f}", flush=True)
    assert np.isfinite(got.astype(np.float64)).all(), what
    assert rel <= TOL and cos >= COS, (what, rel, cos)


@pytest.mark.parametrize("counts,H,I", [
    ([1, 0, 3, 16, 2, 8], 512, 1024),      # decode GEMV form, one empty expert
    ([4] * 12, 256, 512),                   # many experts
    ([0, 0, 1], 128, 256),                  # only the last expert has work
    ([3, 0, 5, 1, 2, 4, 0, 1, 5, 3, 2, 1, 4, 0, 2, 3, 1, 5, 2, 1], 1024, 1024),  # >= 1024 workgroups:
                                                                              # two row groups each
    ([i % 5 for i in range(64)], 1024, 512),  # >= 4096 one-group workgroups in both launches: four each
    ([i % 4 for i in range(128)], 1024, 256),  # down >= 8192: eight each; gate/up four
    ([2, 0, 3, 1], 4480, 384),              # gate/up: rolling whole-line issue, odd step count
])
def test_moe_decode_experts(dev, counts, H, I):
    d = MoeData(dev, counts, H, I, seed=len(counts) + H)
    got = d.run()
    ref = d.oracle()
    t0 = 0
    for e, cnt in enumerate(counts):  # every expert on its own rows
        if cnt:
            check(got[t0:t0 + cnt], ref[t0:t0 + cnt], f"expert {e} ({cnt} tokens)")
        t0 += cnt
    d.free()


def test_moe_decode_scale_planes_4_byte_aligned(dev):
    """The grouped decode GEMV stages 16-byte aligned scale planes in 16-byte
    pieces and 4-byte aligned ones in dwords: copies of the same planes at a
    4-byte offset give the same output bits."""
    d = MoeData(dev, [3, 0, 5, 1, 16, 2], 512, 1024, seed=77)
    ref = d.run()
    shifted, mats = [], []
    for q, s, n, k in d.mats:
        host = dev.download(s, np.uint8, (n * (k // 32),))
        buf = dev.upload(np.concatenate([np.zeros(4, np.uint8), host, np.zeros(12, np.uint8)]))
        shifted.append(buf)
        mats.append((q, types.SimpleNamespace(ptr=buf.ptr + 4)))
    out = dev.alloc(d.T * d.H * 2)
    dev.moe_forward(d.H, d.I, d.counts, d.x, M.Device.weights(*mats), out)
    got = dev.download(out, np.float16, (d.T, d.H))
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    out.free()
    for b in shifted:
        b.free()
    d.free()


# (320, 576): channel counts that are multiples of 64 but not 128, so the
# down GEMM takes its 64-row weight tiles.
@pytest.mark.parametrize("counts,H,I", [([40, 0, 200], 512, 1024), ([17, 130, 5, 64], 256, 640),
                                        ([20, 33, 0, 150], 320, 576)])
def test_moe_gemm_experts(dev, counts, H, I):
    d = MoeData(dev, counts, H, I, seed=len(counts) + I)
    got = d.run()
    ref = d.oracle()
    t0 = 0
    for e, cnt in enumerate(counts):
        if cnt:
            check(got[t0:t0 + cnt], ref[t0:t0 + cnt], f"expert {e} ({cnt} tokens)")
        t0 += cnt
    d.free()


def test_moe_gemm_large_groups(dev):
    """Grouped GEMMs at a larger shape: 8 experts of up to 256 tokens
    (two 128-row tiles, the second ragged for most experts), H=4096,
    I=2048, 512 gate/up and 512 down workgroups.  Six sampled tokens per
    expert are checked, the first and last among them."""
    counts, H, I = [256, 200, 256, 130, 256, 256, 64, 256], 4096, 2048
    d = MoeData(dev, counts, H, I, seed=91)
    got = d.run()
    rng = np.random.default_rng(5)
    rows, t0 = [], 0
    for cnt in counts:
        rows += sorted(set([t0, t0 + cnt - 1] + list(t0 + rng.integers(0, cnt, 4))))
        t0 += cnt
    ref = d.oracle(rows=rows)
    t0 = 0
    for e, cnt in enumerate(counts):
        sel = [r for r in rows if t0 <= r < t0 + cnt]
        check(got[sel], ref[sel], f"expert {e} ({cnt} tokens, {len(sel)} sampled)")
        t0 += cnt
    d.free()


def test_moe_gemm_long_k_chunk_scales(dev):
    """Grouped gate/up GEMM at H=7168: its E8M0 scales (28 KB per workgroup)
    do not fit the LDS copy, so each lane loads a B chunk's scales with one
    8-byte load.  Sampled tokens against the oracle; the same planes copied
    to a 4-byte offset take the per-stage byte loads and give the same bits."""
    counts, H, I = [40, 0, 150, 17], 7168, 256
    d = MoeData(dev, counts, H, I, seed=93)
    got = d.run()
    rows, t0 = [], 0
    for cnt in counts:
        if cnt:
            rows += [t0, t0 + cnt // 2, t0 + cnt - 1]
        t0 += cnt
    ref = d.oracle(rows=rows)
    check(got[rows], ref[rows], f"H={H} sampled tokens")
    shifted, mats = [], []
    for q, s, n, k in d.mats:
        host = dev.download(s, np.uint8, (n * (k // 32),))
        buf = dev.upload(np.concatenate([np.zeros(4, np.uint8), host, np.zeros(12, np.uint8)]))
        shifted.append(buf)
        mats.append((q, types.SimpleNamespace(ptr=buf.ptr + 4)))
    out = dev.alloc(d.T * d.H * 2)
    dev.moe_forward(d.H, d.I, d.counts, d.x, M.Device.weights(*mats), out)
    moved = dev.download(out, np.float16, (d.T, d.H))
    assert np.array_equal(moved.view(np.uint16), got.view(np.uint16))
    out.free()
    for b in shifted:
        b.free()
    d.free()


def test_moe_one_expert_is_the_decode_mlp(dev):
    """One expert through the grouped GEMV runs the same arithmetic as the
    ungrouped decode GEMV: bit-identical to mx_mlp_forward.  T = 3 keeps
    both launchers on the same K split (the ungrouped down GEMV pairs row
    groups from 4 tokens on, the grouped one from 1024 workgroups on)."""
    T, H, I = 3, 512, 1024
    d = MlpData(dev, T, H, I, seed=61)
    out = dev.alloc(T * H * 2)
    dev.moe_forward(H, I, [T], d.x, d.weights, out)
    got = dev.download(out, np.float16, (T, H))
    dev.mlp_forward(M.MLP_FUSED, T, H, I, d.x, d.weights, out)
    want = dev.download(out, np.float16, (T, H))
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    out.free()
    d.free()


def test_moe_benchmark_runs(dev):
    d = MoeData(dev, [2, 3, 0, 1], 256, 512, seed=71)
    out = dev.alloc(d.T * d.H * 2)
    for graph in (True, False):
        secs = dev.moe_benchmark(d.H, d.I, d.counts, d.x, [d.weights], out, warmup=1, iterations=5, graph=graph)
        assert secs > 0
    out.free()
    d.free()


def test_moe_rejects_bad_arguments(dev):
    d = MoeData(dev, [2, 2], 128, 256, seed=81)
    out = dev.alloc(d.T * d.H * 2)
    lib = M.load()
    w = d.weights

    def call(counts, tokens):
        cfg = M.MlpConfig(tokens, d.H, d.I)
        import ctypes
        cnt = (ctypes.c_int * max(len(counts), 1))(*counts)
        return lib.mx_moe_forward(dev.ctx, ctypes.byref(cfg), len(counts), cnt, d.x.p, ctypes.byref(w), out.p)

    assert call([2, 2], 4) == 0
    assert call([2, 2], 5) != 0           # counts do not add up to tokens
    assert call([3, -1], 2) != 0          # negative count
    assert call([], 4) != 0               # no experts
    assert call([0] * 256 + [4], 4) != 0  # more than 256 experts
    out.free()
    d.free()
