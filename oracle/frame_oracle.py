"""The CPU oracle as a backend of flyhighfg_net's program: TEST INFRASTRUCTURE ONLY (the checker of the end-to-end
frame in tests/, and the CPU baseline of bench.py). Every conv runs through the oracle's tiled-order conv
(multithreaded over rows), every other op through fh_ops_oracle.c, on numpy NHWC buffers with the same views and
slices as the GPU backend; the fused op chains run as their ops one after another (ComposedChains)."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
for _p in (HERE, os.path.join(HERE, "..", "flyhigh-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import oracle  # noqa: E402
from flyhighfg_net import CONVS, ComposedChains, cpu_threads  # noqa: E402


class CpuBackend(ComposedChains):
    def __init__(self, W):
        self.W, self.threads, self.gs, self.g_slot = W, cpu_threads(), {}, 0
        self.convs = dict(CONVS)  # conv layer -> (cin, cout, stride, act); a replayed plan adds its own

    def zeros(self, n, h, w, cs):
        return np.zeros((n, h, w, cs), np.uint16)

    def frames(self, n, h, w):
        return np.zeros((n, h, w), np.uint32)

    def upload_frames(self, buf, rgba):
        buf[...] = rgba

    def host_frames(self, buf):
        return buf

    def image(self, buf, i):
        return buf[i:i + 1]

    def upload(self, a):
        return np.ascontiguousarray(a, np.uint16).copy()

    def host(self, buf):
        return buf

    def set_g(self, g_bits, slot=0):
        self.gs[slot] = np.asarray(g_bits, np.uint16).reshape(-1, 96)  # one FiLM vector per image

    def use_g(self, slot):
        self.g_slot = slot

    @property
    def g(self):
        return self.gs[self.g_slot]

    @staticmethod
    def _put(out, c, y):
        out.buf[..., out.c0:out.c0 + c] = y.reshape(out.buf.shape[:3] + (c,))

    def conv(self, name, x, y, res=None):
        cin, cout, stride, act = self.convs[name]
        n, h, w, xcs = x.buf.shape
        d = oracle.make_desc(n, h, w, cin, cout, stride=stride, act=act, residual=res is not None, x_cstride=xcs,
                             x_c0=x.c0, y_cstride=y.buf.shape[3], y_c0=y.c0,
                             r_cstride=res.buf.shape[3] if res is not None else None,
                             r_c0=res.c0 if res is not None else 0)
        wt, b, s = self.W[name]
        oracle.conv(d, x.buf, wt, b, s, None if res is None else res.buf, y=y.buf, threads=self.threads)

    def pair(self, a, b, x, mid, y, res_mid):
        self.conv(a, x, mid)
        self.conv(b, mid, y, mid if res_mid else None)

    def interp(self, x, c, out, oh, ow, aa):
        self._put(out, c, oracle.interp(x.buf, c, oh, ow, aa=aa, c0=x.c0, scale=x.scale))

    def avgpool(self, x, c, out, k):
        assert x.scale == 1.0
        self._put(out, c, oracle.avgpool(x.buf, c, k, c0=x.c0))

    def luma(self, x, out, grad=False):
        self._put(out, 1, oracle.luma(x.buf, grad=grad, c0=x.c0, scale=x.scale))

    def sad(self, la, lb, out, r):
        self._put(out, (2 * r + 1) ** 2, oracle.sad(la.buf, lb.buf, r, la_c0=la.c0, lb_c0=lb.c0))

    def warp(self, img, c, flow, out):
        self._put(out, c, oracle.warp(img.buf, flow.buf, c, img_c0=img.c0, img_scale=img.scale, flow_c0=flow.c0,
                                      flow_scale=flow.scale))

    def chcopy(self, x, c, out):
        self._put(out, c, oracle.chcopy(x.buf, c, c0=x.c0, scale=x.scale))

    def binary(self, a, b, c, out, op=0):
        self._put(out, c, oracle.binary(a.buf, b.buf, c, op=op, a_c0=a.c0, a_scale=a.scale, b_c0=b.c0,
                                        b_scale=b.scale, cb=c))

    def unary(self, x, c, out, op, a=0.0):
        self._put(out, c, oracle.unary(x.buf, c, op, a=a, c0=x.c0, scale=x.scale))

    def film(self, hv, c, out):
        self._put(out, c, oracle.film(hv.buf, self.g, c, c0=hv.c0))

    def convex(self, wt, x, c, out):
        self._put(out, c, oracle.convex(wt.buf, x.buf, c, wt_c0=wt.c0, x_c0=x.c0))

    def blendmix(self, wa, wb, vis, out):
        self._put(out, 3, oracle.blendmix(wa.buf, wb.buf, vis.buf, vis_c0=vis.c0, vis_scale=vis.scale,
                                          wa_c0=wa.c0, wb_c0=wb.c0))

    def render(self, a, b, flow, vis, rt, out, cubic, flags, fsx=None, fsy=None):
        _, hq, wq, _ = flow.buf.shape
        self._put(out, 3, oracle.render(a.buf, b.buf, flow.buf, vis.buf, rt.buf, hq, wq, cubic=cubic, flags=flags,
                                        a_c0=a.c0, b_c0=b.c0, flow_c0=flow.c0,
                                        fsx=flow.scale if fsx is None else fsx,
                                        fsy=flow.scale if fsy is None else fsy,
                                        vis_c0=vis.c0, vis_scale=vis.scale, rt_c0=rt.c0, threads=self.threads))

    def gmhs(self, a, b, flow, full_w, level):
        out, _, _ = oracle.gmhs(a.buf, b.buf, flow.buf, full_w, level, a_c0=a.c0, b_c0=b.c0, flow_c0=flow.c0)
        flow.buf[...] = out

    def rgba_in(self, frames, out, hp, wp):
        self._put(out, 3, oracle.rgba_in(frames, hp, wp))

    def rgba_out(self, x, out_frames):
        _, h, w = out_frames.shape
        out_frames[...] = oracle.rgba_out(x.buf, h, w, c0=x.c0)
