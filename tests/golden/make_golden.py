"""Write the golden fixtures under tests/golden/.

Sources, per file:
  kats.json        the reference's three pack/unpack known-answer cases,
                   copied as data from main.swift:108-132 (inputs/expected);
                   the packed bytes are derived from the E2M1/E4M3/E5M2 bit
                   layouts (low nibble = even index, MXFP4Kernels.metal:345).
  tables.json      E8M0 (all 256 bytes, bits<<23, MXFP4Kernels.metal:26-29)
                   and FP4 E2M1 (16 nibbles, MXFP4Kernels.metal:33-36) decodes,
                   computed here from their closed forms.
  ties.json        round-to-nearest-even tie tables for E2M1, E4M3, E5M2,
                   derived from the decode tables alone: the midpoint of two
                   adjacent codes must encode to the even code, and one ulp
                   either side must encode to the nearer code.
  tiny_mlp.npz     a T=2, H=64, I=128 MXFP4 MLP: inputs, plus outputs of the
                   CPU oracle (modes f16 / W4A4 / reference-row) and an
                   independent float64 numpy evaluation of the f16 mode.
  checksum_kat.json the reference's published checksum of the native
                   scale-plane rows at T=128, H=1024, I=4096 (README.md:292-294)
                   and the data recipe (main.swift:611-638).

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def f32_bits(x):
    return int(np.float32(x).view(np.uint32))


def fp4_value(n):
    mag = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0][n & 7]
    return -mag if n & 8 else mag


def e4m3_value(b):
    s, e, m = b >> 7, (b >> 3) & 15, b & 7
    if e == 15 and m == 7:
        return float("nan")
    v = m * 2.0 ** -9 if e == 0 else (8 + m) * 2.0 ** (e - 10)
    return -v if s else v


def e5m2_value(b):
    s, e, m = b >> 7, (b >> 2) & 31, b & 3
    if e == 31:
        return float("nan") if m else float("inf")
    v = m * 2.0 ** -16 if e == 0 else (4 + m) * 2.0 ** (e - 17)
    return -v if s else v


def pack_codes(codes, bits):
    if bits == 4:
        return [int(codes[i] | (codes[i + 1] << 4)) for i in range(0, len(codes), 2)]
    return [int(c) for c in codes]


def kats():
    cases = [
        ("FP4 E2M1", [-8.0, -6.0, -4.0, -3.0, -2.0, -1.5, -1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 8.0],
         [-6.0, -6.0, -4.0, -3.0, -2.0, -1.5, -1.0, -0.5, 0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]),
        ("FP8 E4M3", [-512.0, -448.0, -16.0, -0.5, 0.0, 0.125, 16.0, 512.0],
         [-448.0, -448.0, -16.0, -0.5, 0.0, 0.125, 16.0, 448.0]),
        ("FP8 E5M2", [-57344.0, -1024.0, -2.0, -0.5, 0.0, 0.25, 1024.0, 57344.0],
         [-57344.0, -1024.0, -2.0, -0.5, 0.0, 0.25, 1024.0, 57344.0]),
    ]
    out = []
    for name, inp, exp in cases:
        if name.startswith("FP4"):
            codes = [next(n for n in range(16) if fp4_value(n) == v and (v != 0 or n == 0)) for v in exp]
            packed = pack_codes(codes, 4)
        elif name.endswith("E4M3"):
            codes = [next(b for b in range(256) if e4m3_value(b) == v and (v != 0 or b == 0)) for v in exp]
            packed = codes
        else:
            codes = [next(b for b in range(256) if e5m2_value(b) == v and (v != 0 or b == 0)) for v in exp]
            packed = codes
        out.append({"name": name, "inputs": inp, "expected": exp, "bytes": packed})
    return out


def tie_table(values, max_code):
    """values[c] for c in 0..max_code (magnitudes, increasing)."""
    rows = []
    for c in range(max_code):
        lo, hi = np.float32(values[c]), np.float32(values[c + 1])
        mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        even = c if c % 2 == 0 else c + 1
        rows.append([f32_bits(mid), even])
        below = np.nextafter(mid, np.float32(0))
        above = np.nextafter(mid, np.float32(np.inf))
        rows.append([f32_bits(below), c])
        rows.append([f32_bits(above), c + 1])
    return rows


def main():
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(kats(), f, indent=1)

    e8m0 = [f32_bits(np.uint32(b << 23).view(np.float32)) for b in range(256)]
    fp4 = [fp4_value(n) for n in range(16)]
    with open(os.path.join(HERE, "tables.json"), "w") as f:
        json.dump({"e8m0_f32_bits": e8m0, "fp4_e2m1": fp4}, f)

    ties = {
        "e2m1": tie_table([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], 7),
        "e4m3": tie_table([e4m3_value(b) for b in range(0x7f)], 0x7e),
        "e5m2": tie_table([e5m2_value(b) for b in range(0x7c)], 0x7b),
    }
    with open(os.path.join(HERE, "ties.json"), "w") as f:
        json.dump(ties, f)

    rng = np.random.default_rng(20261201)
    T, H, I = 2, 64, 128
    x = rng.standard_normal((T, H)).astype(np.float16)
    wg = rng.normal(0, 0.02, (I, H)).astype(np.float32)
    wu = rng.normal(0, 0.02, (I, H)).astype(np.float32)
    wd = rng.normal(0, 0.02, (H, I)).astype(np.float32)
    qg, sg = O.mxfp4_quantize(wg)
    qu, su = O.mxfp4_quantize(wu)
    qd, sd = O.mxfp4_quantize(wd)
    out_f16 = O.mlp_mxfp4(O.MLP_F16, x, qg, sg, qu, su, qd, sd, H, I)
    out_w4a4 = O.mlp_mxfp4(O.MLP_W4A4, x, qg, sg, qu, su, qd, sd, H, I)
    out_ref = O.mlp_mxfp4(O.MLP_REFROW, x, qg, sg, qu, su, qd, sd, H, I)

    # independent float64 evaluation (table decode + numpy matmul)
    def deq(q, s, k):
        lo, hi = q & 15, q >> 4
        codes = np.stack([lo, hi], -1).reshape(q.shape[0], k)
        vals = np.array(fp4, np.float64)[codes]
        sc = 2.0 ** (s.astype(np.float64) - 127)
        return vals * np.repeat(sc, 32, axis=1)

    xf = x.astype(np.float64)
    g = xf @ deq(qg, sg, H).T
    u = xf @ deq(qu, su, H).T
    mid = g / (1 + np.exp(-g)) * u
    out64 = mid @ deq(qd, sd, I).T
    np.savez(os.path.join(HERE, "tiny_mlp.npz"), x=x, qg=qg, sg=sg, qu=qu, su=su, qd=qd, sd=sd,
             out_f16=out_f16, out_w4a4=out_w4a4, out_ref=out_ref, out_f64=out64)

    with open(os.path.join(HERE, "checksum_kat.json"), "w") as f:
        json.dump({
            "source": "README.md:292-294 (native scale-plane n64/n128, host handle, coop-input rows)",
            "checksum": "403573", "samples": 32,
            "tokens": 128, "hidden": 1024, "intermediate": 4096,
            "x": {"seed": 0x11112222, "scale": 0.125},
            "fp4": {"gate": 0xabcd1357, "up": 0x2468bdf0, "down": 0x0badcafe},
            "e8m0": {"gate": 0x7777dddd, "up": 0x8888eeee, "down": 0x9999ffff,
                     "pattern": [124, 125, 126, 127, 127, 128, 128, 129, 130]},
        }, f, indent=1)
    print("golden fixtures written to", HERE)


if __name__ == "__main__":
    main()
