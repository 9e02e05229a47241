"""Shared helpers of the test suite: case generation, the oracle and GPU runners, and the parity measures.

The oracle (oracle/) is used here only as the checker.
"""
from __future__ import annotations

import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "oracle"), os.path.join(ROOT, "flyhigh-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

import oracle  # noqa: E402
import fhconv  # noqa: E402

# north-star parity bar: per-element |diff| <= 1e-2 * max|ref| for f16 results with f32 accumulation
REL_TOL = 1e-2


def f16_ord(u):
    """Monotonic integer image of f16 bit patterns (for ulp distances)."""
    u = np.asarray(u, dtype=np.uint16).astype(np.int32)
    return np.where(u & 0x8000, 0x8000 - (u & 0x7FFF), 0x8000 + u)


def ulp_dist(a, b):
    return np.abs(f16_ord(a) - f16_ord(b))


def as_f64(u):
    return np.asarray(u, dtype=np.uint16).view(np.float16).astype(np.float64)


def f16_bits(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float64).astype(np.float16).view(np.uint16))


class Case:
    """One conv with seeded inputs, as NHWC buffers of f16 bit patterns (uint16)."""

    def __init__(self, n, h, w, cin, cout, k=3, stride=1, act=1, alpha=0.1, residual=False, seed=0,
                 xv=None, yv=None, rv=None, poison=False, wscale=None):
        rng = np.random.default_rng(seed)
        self.n, self.h, self.w, self.cin, self.cout, self.k, self.stride = n, h, w, cin, cout, k, stride
        self.pad = 1 if k == 3 else 0
        self.act, self.alpha, self.residual = act, alpha, bool(residual)
        self.hout = (h + 2 * self.pad - k) // stride + 1
        self.wout = (w + 2 * self.pad - k) // stride + 1
        self.xcs, self.xc0 = xv or (cin, 0)
        self.ycs, self.yc0 = yv or (cout, 0)
        self.rcs, self.rc0 = rv or (cout, 0)
        x = rng.uniform(-1, 1, size=(n, h, w, self.xcs))
        if poison and self.xcs > cin:  # channels outside the view hold NaN: they must never be read
            x[..., :self.xc0] = np.nan
            x[..., self.xc0 + cin:] = np.nan
        self.x = f16_bits(x)
        std = wscale if wscale is not None else np.sqrt(2.0 / (k * k * cin))
        self.wt = f16_bits(rng.normal(0, std, size=(cout, cin, k, k)))
        self.bias = f16_bits(rng.normal(0, 0.01, size=cout))
        self.slope = f16_bits(rng.uniform(0.05, 0.3, size=cout))
        r = rng.uniform(-1, 1, size=(n, self.hout, self.wout, self.rcs))
        self.res = f16_bits(r)
        y0 = np.full((n, self.hout, self.wout, self.ycs), np.nan if poison else 0.0)
        self.y0 = f16_bits(y0)

    def oracle_desc(self):
        return oracle.make_desc(self.n, self.h, self.w, self.cin, self.cout, k=self.k, stride=self.stride,
                                pad=self.pad, act=self.act, alpha=self.alpha, residual=self.residual,
                                x_cstride=self.xcs, x_c0=self.xc0, y_cstride=self.ycs, y_c0=self.yc0,
                                r_cstride=self.rcs, r_c0=self.rc0)

    def fhc_desc(self, variant=0, ksplit=0, ref_cand=0xFF):
        return fhconv.make_desc(self.n, self.h, self.w, self.cin, self.cout, k=self.k, stride=self.stride,
                                pad=self.pad, act=self.act, alpha=self.alpha, residual=self.residual,
                                x_cstride=self.xcs, x_c0=self.xc0, y_cstride=self.ycs, y_c0=self.yc0,
                                r_cstride=self.rcs, r_c0=self.rc0, variant=variant, ksplit=ksplit,
                                ref_cand=ref_cand)

    def run_oracle(self, order=oracle.ORDER_TILED, ksplit=1, threads=0):
        y = self.y0.copy().ravel()
        oracle.conv(self.oracle_desc(), self.x, self.wt, self.bias, self.slope if self.act == 1 else None,
                    self.res if self.residual else None, y=y, order=order, ksplit=ksplit, threads=threads)
        return y.reshape(self.y0.shape)

    def run_gpu(self, variant=0, ksplit=0, ref_cand=0xFF, plan=None, return_plan=False):
        import torch
        dev = torch.device("cuda", 0)
        if plan is None:
            plan = fhconv.ConvPlan(self.fhc_desc(variant, ksplit, ref_cand), self.wt, self.bias,
                                   self.slope if self.act == 1 else None)
        host = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16))  # noqa: E731
        x = host(self.x).to(dev)
        y = host(self.y0).to(dev)
        r = host(self.res).to(dev) if self.residual else None
        ws = torch.empty(plan.workspace_bytes // 2 + 8, dtype=torch.int16, device=dev) \
            if plan.workspace_bytes else None
        plan.run(x, y, r, ws)
        torch.cuda.synchronize()
        out = y.cpu().numpy().view(np.uint16)
        return (out, plan) if return_plan else out


def parity(got, ref, tol=REL_TOL, view=None):
    """(ok, max|diff|, max|ref|) with the north-star bar |diff| <= tol * max|ref| over the written view."""
    g, r = as_f64(got), as_f64(ref)
    if view is not None:
        g, r = g[..., view], r[..., view]
    if np.isnan(r).any() or np.isnan(g).any():
        return False, float("nan"), float("nan")
    mref = float(np.abs(r).max()) if r.size else 0.0
    md = float(np.abs(g - r).max()) if r.size else 0.0
    return md <= tol * max(mref, 1e-30), md, mref


def oracle_rows(case, r0, r1, img=0, threads=0):
    """Oracle output rows [r0, r1) of image `img`, computed on the crop of input rows they read (for layers too
    large to run through the oracle whole). The crop starts on a multiple of the stride one output row early, so
    no row in [r0, r1) sees the crop's own zero padding unless it is the image's."""
    import copy
    s = case.stride
    a = (r0 - 1) * s if r0 > 0 else 0
    first = a // s
    b = min(case.h, (r1 - 1) * s + 2) if case.k == 3 else min(case.h, (r1 - 1) * s + 1)
    c = copy.copy(case)
    c.n, c.h = 1, b - a
    c.hout = (c.h + 2 * case.pad - case.k) // s + 1
    c.x = case.x[img:img + 1, a:b]
    c.res = case.res[img:img + 1, first:first + c.hout]
    c.y0 = case.y0[img:img + 1, first:first + c.hout]
    y = c.run_oracle(threads=threads)
    return y[0, r0 - first:r1 - first]
