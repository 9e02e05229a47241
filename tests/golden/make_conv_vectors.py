"""Golden vectors for the conv oracle, computed with an independent library routine.

Each case holds seeded f16 inputs (NHWC views, OIHW weights, bias, slope, residual) and the expected f16 output,
computed with torch.nn.functional.conv2d in float64 on the CPU (not the oracle), followed by the reference's
epilogue: + bias, PReLU / LeakyReLU, f16 round, then the residual add rounded again
(shaders/conv_tiled.wgsl:57-67, shaders/binary.wgsl:15-16). Written to conv_vectors.npz beside this script.

Run in the build container:  python tests/golden/make_conv_vectors.py
"""
import os

import numpy as np
import torch

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "conv_vectors.npz")

# name: n, h, w, cin, cout, k, stride, act, residual, (x_cstride, x_c0), (y_cstride, y_c0), (r_cstride, r_c0)
CASES = {
    "s1_5to7_prelu": (1, 9, 11, 5, 7, 3, 1, 1, 0, None, None, None),
    "s2_3to6_odd": (1, 10, 13, 3, 6, 3, 2, 1, 0, None, None, None),
    "s2_3to6_even": (1, 12, 16, 3, 6, 3, 2, 1, 0, None, None, None),
    "s1_8to8_res_batch2": (2, 6, 7, 8, 8, 3, 1, 1, 1, None, None, None),
    "k1_12to5_none": (1, 4, 6, 12, 5, 1, 1, 0, 0, None, None, None),
    "s1_16to16_leaky": (1, 8, 8, 16, 16, 3, 1, 2, 0, None, None, None),
    "s2_14to24_res": (1, 7, 9, 14, 24, 3, 2, 1, 1, None, None, None),
    "s1_views": (1, 5, 6, 4, 3, 3, 1, 1, 1, (10, 3), (9, 2), (7, 4)),
    "s1_40to12_none": (1, 5, 5, 40, 12, 3, 1, 0, 0, None, None, None),
    "s1_1x1img": (1, 1, 1, 9, 4, 3, 1, 1, 0, None, None, None),
    "s2_1col": (1, 7, 1, 6, 5, 3, 2, 1, 0, None, None, None),
}
LEAKY = 0.1


def f16(a):
    return np.asarray(a, dtype=np.float64).astype(np.float16)


def make(name, spec, rng):
    n, h, w, cin, cout, k, s, act, residual, xv, yv, rv = spec
    pad = 1 if k == 3 else 0
    hout, wout = (h + 2 * pad - k) // s + 1, (w + 2 * pad - k) // s + 1
    xcs, xc0 = xv or (cin, 0)
    ycs, yc0 = yv or (cout, 0)
    rcs, rc0 = rv or (cout, 0)
    xbuf = f16(rng.uniform(-1, 1, size=(n, h, w, xcs)))
    wt = f16(rng.normal(0, np.sqrt(2.0 / (k * k * cin)), size=(cout, cin, k, k)))
    bias = f16(rng.normal(0, 0.1, size=cout))
    slope = f16(rng.uniform(0.05, 0.3, size=cout))
    rbuf = f16(rng.uniform(-1, 1, size=(n, hout, wout, rcs)))
    ybuf0 = f16(rng.uniform(-1, 1, size=(n, hout, wout, ycs)))  # prior contents: the untouched channels keep them

    x = torch.from_numpy(xbuf[..., xc0:xc0 + cin].astype(np.float64)).permute(0, 3, 1, 2)
    acc = torch.nn.functional.conv2d(x, torch.from_numpy(wt.astype(np.float64)), stride=s, padding=pad)
    v = acc.permute(0, 2, 3, 1).numpy() + bias.astype(np.float64)
    if act == 1:
        v = np.where(v > 0, v, slope.astype(np.float64) * v)
    elif act == 2:
        v = np.where(v > 0, v, np.float64(np.float32(LEAKY)) * v)
    o = f16(v)
    if residual:
        o = f16(o.astype(np.float64) + rbuf[..., rc0:rc0 + cout].astype(np.float64))
    ybuf = ybuf0.copy()
    ybuf[..., yc0:yc0 + cout] = o
    meta = np.array([n, h, w, cin, cout, k, s, pad, act, residual, xcs, xc0, ycs, yc0, rcs, rc0], dtype=np.int64)
    return {f"{name}.meta": meta, f"{name}.x": xbuf.view(np.uint16), f"{name}.w": wt.view(np.uint16),
            f"{name}.bias": bias.view(np.uint16), f"{name}.slope": slope.view(np.uint16),
            f"{name}.res": rbuf.view(np.uint16), f"{name}.y0": ybuf0.view(np.uint16),
            f"{name}.y": ybuf.view(np.uint16), f"{name}.alpha": np.array([LEAKY], dtype=np.float32)}


def main():
    out = {}
    for i, (name, spec) in enumerate(CASES.items()):
        out.update(make(name, spec, np.random.default_rng(1000 + i)))
    np.savez_compressed(OUT, **out)
    print(f"{len(CASES)} cases -> {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
