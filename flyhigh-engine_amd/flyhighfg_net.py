"""One FlyHighFG pair() and mid() end to end: every op of models/graph.json from the network-size inputs A, B to the
network's outputs (the rendered in-between picture, R_t, flow_tq, vis_tq, the streaming state), as the reference's
planner walks it
(crates/flyhigh-engine/src/net/build.rs:186-450), over a backend.

The program is written once (``FlyHighFG.pair`` / ``mid``) against a small backend interface: ``GpuBackend`` runs it
through libfhconv.so (conv plans and fused pairs of fhc_conv.h, the ops of fhc_ops.h) on a HIP stream, so it can be
captured in a HIP graph; a checker can run the same program over the CPU oracle with the same weights. Tensors are
NHWC f16 buffers (n, h, w, cstride) with the channel stride padded to 8 where a conv or an 8-byte path reads them;
the graph's slices and scales are views (``V``) and its concats are buffers the producers write into by slice, so
only a scaled input of a concat costs a copy (as the reference's chcopy does). The A and B branches share weights
and run as a batch of 2 where their consumers read one tensor (resize, the first encoder pair, the first pool). Given a
frame size, the program starts from the host's two RGBA8 frames and ends with the generated RGBA8 frame, as the
reference's Session does (net/session.rs:26-66): rgba_in, the antialiased downscale to the network size, the network,
the render at the frame size and rgba_out (the downscale and the render each one launch on the GPU, reading the 8-bit
frames directly).

Differences of launch structure from the reference (same arithmetic): the encoders' outputs are copied into their
slices of the 279-channel concat (and f16b into the streaming state) by one copy launch; consecutive convs whose
intermediate has no other reader run as fused pairs on the GPU when asked; flow and vis share one buffer, so the fine
loop's two adds are one, and that add is fine.out's residual (the planner's residual peephole, net/build.rs:222-237);
the periodic-structure repair (gmhs.rs, level 1 by default as in the engine) ends pair() in 8 launches where the
reference records 14. The program is one chain of launches: independent stretches (the pair's cost volume beside the
encoders, the repair beside up.w and the FiLM branch) on side streams, joined by events, made the captured 1080p frame
slower, by 16 to 43 us per fork (the graph's cross-stream dependencies cost more than the overlap returns at these
kernel sizes).
"""
from __future__ import annotations

import os
from typing import Dict, Optional

import numpy as np

# The graph's convs (models/flyhighfg.json shapes): name -> (cin, cout, stride, act). act 1: the graph's "conv"
# (PReLU with its own slope); 0: "conv2d" and the convex-upsample conv up.w (no activation, net/build.rs:210-220, :381)
CONVS = {
    "enc.e1": (3, 36, 2, 1), "enc.e2": (36, 36, 1, 1), "enc.e3": (36, 72, 2, 1), "enc.e4": (72, 72, 1, 1),
    "coarse.c1": (279, 96, 1, 1), "coarse.c2": (96, 96, 1, 1), "coarse.c3": (96, 96, 1, 1),
    "coarse.c4": (96, 96, 1, 1), "coarse.head": (96, 12, 1, 0),
    "fine.r1": (155, 48, 1, 1), "fine.r2": (48, 48, 1, 1), "fine.r3": (48, 48, 1, 1), "fine.out": (48, 7, 1, 0),
    "film.h1": (48, 48, 1, 1), "film.h2": (48, 48, 1, 1), "film.out": (48, 5, 1, 0), "up.w": (48, 36, 1, 0),
    "refine.q1": (14, 24, 1, 1), "refine.q2": (24, 24, 1, 1), "refine.q3": (24, 24, 1, 1), "refine.q4": (24, 3, 1, 0),
}
FILM_HIDDEN, FILM_OUT = 64, 96  # film.film.0: [64, 1]; film.film.2: [96, 64] (models/flyhighfg.json:385-414)


def f16_bits(a):
    return np.ascontiguousarray(np.asarray(a, np.float64).astype(np.float16).view(np.uint16))


def make_weights(seed: int = 0) -> dict:
    """Random weights of the graph's architecture (the trained ones, models/flyhighfg.bin, are licensed CC BY-NC
    and stay out of this repository; model/blob.rs reads them where a host provides them): He-normal
    convs, small biases, PReLU slopes in [0.05, 0.3], an f16-representable FiLM MLP. Returns name -> (w OIHW, bias,
    slope or None) as f16 bits, and "film" -> (w1, b1, w2, b2) as f32 (the reference decodes its f16 weights to
    f32 for the MLP, model/blob.rs:32-41)."""
    rng = np.random.default_rng(seed)
    W = {}
    for name, (cin, cout, _, act) in CONVS.items():
        w = f16_bits(rng.normal(0, np.sqrt(2.0 / (9 * cin)), (cout, cin, 3, 3)))
        b = f16_bits(rng.normal(0, 0.01, cout))
        s = f16_bits(rng.uniform(0.05, 0.3, cout)) if act == 1 else None
        W[name] = (w, b, s)
    q = lambda a: np.asarray(a, np.float64).astype(np.float16).astype(np.float32)  # noqa: E731
    W["film"] = (q(rng.normal(0, 1, FILM_HIDDEN)), q(rng.normal(0, 0.1, FILM_HIDDEN)),
                 q(rng.normal(0, 0.1, (FILM_OUT, FILM_HIDDEN))), q(rng.normal(0, 0.01, FILM_OUT)))
    return W


def film_mlp(W: dict, t: float) -> np.ndarray:
    """The FiLM vector g(t) on the host, f16 bits [96]: g[o] = b2[o] + sum_i w2[o][i] relu(w1[i] t + b1[i]), f32,
    the sum in index order (net/build.rs:331-340); stored as f16 (:345-355)."""
    w1, b1, w2, b2 = W["film"]
    t = np.float32(t)
    hv = np.maximum(w1 * t + b1, np.float32(0))
    g = np.empty(FILM_OUT, np.float32)
    for o in range(FILM_OUT):
        acc = np.float32(0)
        for i in range(FILM_HIDDEN):
            acc = np.float32(acc + w2[o, i] * hv[i])
        g[o] = np.float32(b2[o] + acc)
    return f16_bits(g)


class V:
    """A view: channels c0.. of a backend buffer (n, h, w, cstride), read times `scale`."""
    __slots__ = ("buf", "c0", "scale")

    def __init__(self, buf, c0: int = 0, scale: float = 1.0):
        self.buf, self.c0, self.scale = buf, c0, scale


def pad8(c):
    return (c + 7) // 8 * 8


class ComposedChains:
    """The graph's fused op chains as their ops run one after another (the reference's launches): the CPU oracle
    backend always runs them this way, the GPU backend when asked to (a check of the fused kernels)."""

    def pair_input(self, ab: V, q: V, i8: V, i16: V, l16: V, oh: int, ow: int):
        """The resize of every picture, then each pair's pyramid (pair k: images 2k, 2k + 1 of ab, q and i8, image
        k of i16 and l16)."""
        self.interp(ab, 3, q, oh, ow, True)
        for k in range(q.buf.shape[0] // 2):
            one = lambda x, i=k: V(sl(x.buf, i), x.c0, x.scale)  # noqa: E731
            two = lambda x, i=k: V(sl(x.buf, 2 * i, 2), x.c0, x.scale)  # noqa: E731
            self.pair_pyramid(two(q), two(i8), one(i16), one(l16))

    def coarse_up(self, o: V, out: V, state: Optional[V], oh: int, ow: int, flow_scale: float):
        if state is not None:
            self.chcopy(V(o.buf, o.c0, flow_scale), 4, state)
        self.interp(V(o.buf, o.c0, flow_scale), 4, V(out.buf, out.c0), oh, ow, False)
        self.interp(V(o.buf, o.c0 + 4), 3, V(out.buf, out.c0 + 4), oh, ow, False)

    def fold_pair(self, x: V, c: int, out: V, also: Optional[V]):
        for i in range(2):
            self.chcopy(V(self.image(x.buf, i), x.c0), c, V(out.buf, out.c0 + c * i))
        if also is not None:
            self.chcopy(V(self.image(x.buf, 1), x.c0), c, also)

    def fold_pair_sad(self, x: V, c: int, out: V, also: Optional[V], la: V, lb: V, sad_out: V, r: int):
        """fold_pair of every pair of x (pair k: images 2k, 2k + 1 into image k of out and also) and a sad that
        neither reads what the other writes (one launch on the GPU)."""
        for k in range(x.buf.shape[0] // 2):
            self.fold_pair(V(sl(x.buf, 2 * k, 2), x.c0), c, V(sl(out.buf, k), out.c0),
                           None if also is None else V(sl(also.buf, k), also.c0))
        self.sad(la, lb, sad_out, r)

    def pair_affine_out(self, a, b, x: V, mid: V, y: V, out: V, c: int):
        """The pair a, b (no residual) into y, then affine_out of y's c channels into out (on the GPU one launch,
        which writes out and neither mid nor y)."""
        self.pair(a, b, x, mid, y, False)
        self.unary(y, c, out, 2)

    def film_pair(self, a, b, h: V, c: int, hm: V, mid: V, y: V):
        """film_modulate of h's c channels into hm, then the pair a, b (no residual) on hm into y (on the GPU one
        launch, which writes y and neither hm nor mid)."""
        self.film(h, c, hm)
        self.pair(a, b, hm, mid, y, False)

    def conv_siblings(self, a, b, x: V, ya: V, res_a: Optional[V], yb: V):
        """The convs a (with its residual, if any) and b of the same input x (on the GPU one launch)."""
        self.conv(a, x, ya, res_a)
        self.conv(b, x, yb)

    def gmhs_n(self, ab: V, flow: V, full_w: int, level: int):
        """gmhs of every pair: pair k's pictures are images 2k, 2k + 1 of ab, its flow image k of flow."""
        for k in range(flow.buf.shape[0]):
            self.gmhs(V(sl(ab.buf, 2 * k), ab.c0), V(sl(ab.buf, 2 * k + 1), ab.c0), V(sl(flow.buf, k), flow.c0),
                      full_w, level)

    def gmhs_film(self, a: V, b: V, flow: V, full_w: int, level: int, fa, fb, h: V, c: int, hm: V, mid: V, y: V,
                  fo, yo: V):
        """The repair, the FiLM pair of film_pair(fa, fb, h, c, hm, mid, y) and the conv fo of y into yo, which touch
        none of the repair's data (on the GPU the pair's workgroups run inside the repair's first launch, the
        conv's inside the second)."""
        self.gmhs(a, b, flow, full_w, level)
        self.film_pair(fa, fb, h, c, hm, mid, y)
        self.conv(fo, y, yo)

    def pair_pyramid(self, q: V, i8: V, i16: V, l16: V):
        self.avgpool(q, 3, i8, 2)
        for i in range(2):
            self.avgpool(V(self.image(i8.buf, i), i8.c0), 3, V(i16.buf, i16.c0 + 3 * i), 2)
        for i in range(2):
            self.luma(V(i16.buf, i16.c0 + 3 * i), V(l16.buf, l16.c0 + i))

    def fine_input(self, f8: V, i8: V, flow: V, fx: V, l8: V, c: int):
        for i in range(2):
            fl = V(flow.buf, flow.c0 + 2 * i, flow.scale)
            self.warp(V(self.image(f8.buf, i), f8.c0), c, fl, V(fx.buf, fx.c0 + c * i))
            self.warp(V(self.image(i8.buf, i), i8.c0), 3, fl, V(fx.buf, fx.c0 + 2 * c + 3 * i))
            self.luma(V(fx.buf, fx.c0 + 2 * c + 3 * i), V(l8.buf, l8.c0 + i))
        self.chcopy(flow, 4, V(fx.buf, fx.c0 + 2 * c + 6))

    def coarse_fine_input(self, o: V, fv: V, state: Optional[V], flow_scale: float, f8: V, i8: V,
                          fine_scale: float, fx: V, l8: V, c: int):
        """coarse_up then fine_input for every pair: pair k's image k of o, fv, state, fx and l8, its maps and
        pictures images 2k, 2k + 1 of f8 and i8."""
        _, h, w, _ = f8.buf.shape
        for k in range(o.buf.shape[0]):
            one = lambda x, i=k: V(sl(x.buf, i), x.c0, x.scale)  # noqa: E731
            two = lambda x, i=k: V(sl(x.buf, 2 * i, 2), x.c0, x.scale)  # noqa: E731
            self.coarse_up(one(o), one(fv), None if state is None else one(state), h, w, flow_scale)
            self.fine_input(two(f8), two(i8), V(sl(fv.buf, k), fv.c0, fine_scale), one(fx), one(l8), c)

    def coarse_fine_input_sad(self, o: V, fv: V, state: Optional[V], flow_scale: float, f8: V, i8: V,
                              fine_scale: float, fx: V, l8: V, c: int, sad_out: V, r: int):
        """coarse_fine_input, then the sad of its two lumas (l8's channels 0 and 1) into sad_out (on the GPU one
        launch, whose cost volume computes the lumas it reads)."""
        self.coarse_fine_input(o, fv, state, flow_scale, f8, i8, fine_scale, fx, l8, c)
        self.sad(V(l8.buf, l8.c0), V(l8.buf, l8.c0 + 1), sad_out, r)

    def flow_vis_t_convex(self, wt: V, fv: V, dfilm: V, t: float, out: V, ftvt: V, lin: V, dvis: V):
        """ftvt, lin, dvis: where the op-by-op chain keeps its intermediates (the fused launch stores none)."""
        self.flow_vis_t(fv, dfilm, ftvt, t, lin, dvis)
        self.convex(wt, ftvt, 7, out)

    def flow_vis_t_convex_n(self, wt: V, fv: V, dfilm: V, ts, out: V, ftvt: V, lin: V, dvis: V):
        """flow_vis_t_convex for each phase j of ts over fv's P pairs: dfilm, out and the intermediates hold phase j
        of pair p at image j * P + p."""
        P = fv.buf.shape[0]
        for j, t in enumerate(ts):
            m = lambda x, i=j: V(sl(x.buf, i * P, P), x.c0, x.scale)  # noqa: E731
            self.flow_vis_t_convex(wt, fv, m(dfilm), t, m(out), m(ftvt), m(lin), m(dvis))

    def flow_vis_t(self, fv: V, dfilm: V, out: V, t: float, lin: V, dvis: V):
        self.unary(V(fv.buf, fv.c0), 2, V(lin.buf, lin.c0), 0, 2.0 * t)
        self.unary(V(fv.buf, fv.c0 + 2), 2, V(lin.buf, lin.c0 + 2), 0, 2.0 * (1.0 - t))
        self.binary(lin, V(dfilm.buf, dfilm.c0), 4, V(out.buf, out.c0))
        self.chcopy(V(dfilm.buf, dfilm.c0 + 4), 1, V(dvis.buf, dvis.c0))
        self.chcopy(V(dfilm.buf, dfilm.c0 + 4, -1.0), 1, V(dvis.buf, dvis.c0 + 1))
        self.binary(V(fv.buf, fv.c0 + 4), dvis, 3, V(out.buf, out.c0 + 4))

    def frame_input(self, frames, full, ab: V, hp: int, wp: int, oh: int, ow: int):
        """The two RGBA8 frames -> the network's inputs A, B at oh x ow: rgba_in to the padded frame size, then the
        antialiased resize (net/session.rs:56-60, net/build.rs:615-620)."""
        self.rgba_in(frames, V(full), hp, wp)
        self.interp(V(full), 3, ab, oh, ow, True)

    def frame_render(self, frames, full, pic, flow: V, vis: V, rt: V, out_frames, hp: int, wp: int, fsx: float,
                     fsy: float, cubic: bool, flags: int):
        """The frame-size render of the internal-size mode (net/build.rs:717-736) and rgba_out (net/session.rs:63):
        render_pix of the padded frames A, B (rgba_in) at hp x wp with the flow scaled per axis, then the crop to
        the frame's RGBA8."""
        self.rgba_in(frames, V(full), hp, wp)
        self.render(V(self.image(full, 0)), V(self.image(full, 1)), flow, vis, rt, V(pic), cubic, flags, fsx, fsy)
        self.rgba_out(V(pic), out_frames)

    def frame_render_n(self, frames, full, pic, flow: V, vis: V, rt: V, out_frames, hp: int, wp: int, fsx: float,
                       fsy: float, cubic: bool, flags: int, phases: int):
        """frame_render of every generated frame, pair by pair (a pair's phases read the same two frames): phase j of
        pair p (frames 2p, 2p + 1) from maps image j * P + p into frame j * P + p of out_frames (on the GPU one
        launch, in the same order)."""
        P = frames.shape[0] // 2
        for i in (j * P + p for p in range(P) for j in range(phases)):
            p = i % P
            one = lambda x, k=i: V(sl(x.buf, k), x.c0, x.scale)  # noqa: E731
            self.frame_render(sl(frames, 2 * p, 2), None if full is None else sl(full, 2 * p, 2), pic, one(flow),
                              one(vis), one(rt), sl(out_frames, i), hp, wp, fsx, fsy, cubic, flags)

    def refine_input_n(self, q: V, flow: V, vis: V, rx: V, flow_out_scale: float, blend: V, qmod: int):
        """refine_input for every image k of flow (and vis, rx, blend), its pictures pair k % qmod of q"""
        for k in range(flow.buf.shape[0]):
            v = lambda x, i=k: V(sl(x.buf, i), x.c0, x.scale)  # noqa: E731
            self.refine_input(V(sl(q.buf, 2 * (k % qmod), 2), q.c0, q.scale), v(flow), v(vis), v(rx), flow_out_scale,
                              v(blend))

    def mid_input_n(self, wt: V, fv: V, dfilm: V, ts, up: V, ftvt: V, lin: V, dvis: V, q: V, rx: V,
                    flow_scale: float, flow_out_scale: float, blend: V):
        """flow_vis_t_convex_n into up, then refine_input_n on up (its flow read at flow_scale, its visibility
        unscaled) into rx, image j * P + p taking pair p's pictures from q (on the GPU one launch, which stores
        neither the convex upsample's input nor the blend)."""
        self.flow_vis_t_convex_n(wt, fv, dfilm, ts, up, ftvt, lin, dvis)
        self.refine_input_n(q, V(up.buf, up.c0, flow_scale), V(up.buf, up.c0 + 4), rx, flow_out_scale, blend,
                            fv.buf.shape[0])

    def refine_input(self, q: V, flow: V, vis: V, rx: V, flow_out_scale: float, blend: V):
        for i in range(2):
            self.warp(V(self.image(q.buf, i), q.c0), 3, V(flow.buf, flow.c0 + 2 * i, flow.scale),
                      V(rx.buf, rx.c0 + 3 * i))
        self.chcopy(vis, 3, V(rx.buf, rx.c0 + 6))
        self.chcopy(V(flow.buf, flow.c0, flow_out_scale), 4, V(rx.buf, rx.c0 + 9))
        self.blendmix(V(rx.buf, rx.c0), V(rx.buf, rx.c0 + 3), vis, blend)
        self.luma(blend, V(rx.buf, rx.c0 + 13), grad=True)


class GpuBackend(ComposedChains):
    """The program's ops on the GPU through libfhconv.so, on one stream. Plans are made on first use (the first
    run of the program; a captured replay then finds them all). With ``record`` a list, every launch is also
    appended to it as a dict (label, kind, fn: a callable that issues the same launch again, bytes and flops: its
    algorithmic work, f16 tensors read and written once), for per-launch measurement. The frame-size render fuses
    each product into the sum it feeds (bytes within 1 of the reference's order); exact_render takes the
    reference's f32 order instead (bit-identical to its ops one by one)."""

    def __init__(self, W, stream=None, fuse: bool = True, device: str = "cuda", chains: bool = True,
                 exact_render: bool = False):
        import torch
        import fhconv
        import fhops
        self.torch, self.fhconv, self.fh = torch, fhconv, fhops
        self.W, self.fuse, self.dev, self.chains, self.exact_render = W, fuse, device, chains, exact_render
        self.convs = dict(CONVS)  # conv layer -> (cin, cout, stride, act); a replayed plan adds its own
        self.stream = stream if stream is not None else torch.cuda.current_stream()
        self.plans: Dict[tuple, object] = {}
        self.gs: Dict[int, object] = {}  # FiLM vector slots (one per phase of a batched program)
        self.g_slot = 0
        self.record = None

    def _go(self, label, fn, nbytes, flops=0, kind="op", kernels=1):
        fn()
        if self.record is not None:
            self.record.append(dict(label=label, kind=kind, fn=fn, bytes=int(nbytes), flops=int(flops),
                                    kernels=kernels))

    def zeros(self, n, h, w, cs):
        return self.torch.zeros((n, h, w, cs), dtype=self.torch.int16, device=self.dev)

    def frames(self, n, h, w):
        return self.torch.zeros((n, h, w), dtype=self.torch.int32, device=self.dev)

    def upload_frames(self, buf, rgba):
        buf.copy_(self.torch.from_numpy(np.ascontiguousarray(rgba, np.uint32).view(np.int32)))

    def host_frames(self, buf):
        self.torch.cuda.synchronize()
        return buf.cpu().numpy().view(np.uint32)

    def image(self, buf, i):
        return buf[i:i + 1]

    def upload(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(self.dev)

    def host(self, buf):
        self.torch.cuda.synchronize()
        return buf.cpu().numpy().view(np.uint16)

    def set_g(self, g_bits, slot: int = 0):
        """The FiLM vector of slot `slot` (f16 bits [96]); a slot keeps its device buffer, so a captured program
        reads whatever was last written to it."""
        if slot not in self.gs:
            self.gs[slot] = self.upload(g_bits)
        else:
            self.gs[slot].copy_(self.torch.from_numpy(np.ascontiguousarray(g_bits).view(np.int16)))

    def use_g(self, slot: int):
        self.g_slot = slot

    @property
    def g(self):
        return self.gs[self.g_slot]

    def _v(self, v: V):
        return self.fh.View(v.buf, v.c0, v.scale)

    @staticmethod
    def _px(v: V) -> int:
        """pixels (all images) of a view's buffer"""
        n, h, w, _ = v.buf.shape
        return n * h * w

    def _desc(self, name, x: V, y: V, res: Optional[V], mid_res=False):
        cin, cout, stride, act = self.convs[name]
        n, h, w, xcs = x.buf.shape
        ycs = y.buf.shape[3]
        return self.fhconv.make_desc(n, h, w, cin, cout, stride=stride, act=act, residual=res is not None or mid_res,
                                     x_cstride=xcs, x_c0=x.c0, y_cstride=ycs, y_c0=y.c0,
                                     r_cstride=res.buf.shape[3] if res is not None else (ycs if mid_res else 0),
                                     r_c0=res.c0 if res is not None else 0)

    def _conv_plan(self, name, x: V, y: V, res: Optional[V] = None):
        key = ("conv", name, x.buf.shape[0], x.buf.data_ptr(), x.c0, y.buf.data_ptr(), y.c0,
               None if res is None else res.buf.data_ptr())
        p = self.plans.get(key)
        if p is None:
            w, b, s = self.W[name]
            p = self.plans[key] = self.fhconv.ConvPlan(self._desc(name, x, y, res), w, b, s)
            if p.workspace_bytes:
                raise RuntimeError(f"{name}: a split-K plan needs a workspace; give the frame convs a table entry")
            p._work = p.describe()
        return p

    def conv(self, name, x: V, y: V, res: Optional[V] = None):
        p = self._conv_plan(name, x, y, res)
        xb, yb, rb, st = x.buf, y.buf, None if res is None else res.buf, self.stream
        self._go(name, lambda: p.run(xb, yb, rb, stream=st), p._work["bytes"], p._work["flops"], "conv")

    def pair(self, a, b, x: V, mid: V, y: V, res_mid: bool):
        if not self.fuse:
            self.conv(a, x, mid)
            self.conv(b, mid, y, mid if res_mid else None)
            return
        key = ("pair", a, b, x.buf.shape[0], x.buf.data_ptr(), x.c0, y.buf.data_ptr(), y.c0)
        p = self.plans.get(key)
        if p is None:
            da = self._desc(a, x, mid, None)
            db = self._desc(b, mid, y, None, mid_res=res_mid)
            (wa, ba, sa), (wb, bb, sb) = self.W[a], self.W[b]
            try:
                p = self.fhconv.ConvPairPlan(da, wa, ba, sa, db, wb, bb, sb, res_mid=res_mid)
                p._work = p.describe()
            except self.fhconv.FhcError:
                p = False  # no fused kernel for these channels: two launches
            self.plans[key] = p
        if p is False:
            self.conv(a, x, mid)
            self.conv(b, mid, y, mid if res_mid else None)
        else:
            xb, yb, st = x.buf, y.buf, self.stream
            self._go(f"{a}+{b}", lambda: p.run(xb, yb, None, stream=st), p._work["bytes"], p._work["flops"], "conv")

    def pair_affine_out(self, a, b, x: V, mid: V, y: V, out: V, c: int):
        if not (self.chains and self.fuse) or CONVS[b][1] != c:
            return super().pair_affine_out(a, b, x, mid, y, out, c)
        key = ("pair_affine_out", a, b, x.buf.shape[0], x.buf.data_ptr(), x.c0, out.buf.data_ptr(), out.c0)
        p = self.plans.get(key)
        if p is None:
            da = self._desc(a, x, mid, None)
            db = self._desc(b, mid, out, None)
            (wa, ba, sa), (wb, bb, sb) = self.W[a], self.W[b]
            try:
                p = self.fhconv.ConvPairPlan(da, wa, ba, sa, db, wb, bb, sb, affine_out=True)
                p._work = p.describe()
            except self.fhconv.FhcError:
                p = False  # no fused kernel for these channels
            self.plans[key] = p
        if p is False:
            return super().pair_affine_out(a, b, x, mid, y, out, c)
        xb, ob, st = x.buf, out.buf, self.stream
        self._go(f"{a}+{b}+affine_out", lambda: p.run(xb, ob, None, stream=st), p._work["bytes"], p._work["flops"],
                 "conv")

    def _film_plan(self, a, b, h: V, c: int, mid: V, y: V):
        """The FiLM pair's plan (film_modulate in a, b's staging), or False where there is none."""
        if not (self.chains and self.fuse) or CONVS[a][0] != c or h.scale != 1.0:
            return False
        key = ("film_pair", a, b, h.buf.shape[0], h.buf.data_ptr(), h.c0, y.buf.data_ptr(), y.c0)
        p = self.plans.get(key)
        if p is None:
            da = self._desc(a, h, mid, None)
            db = self._desc(b, mid, y, None)
            (wa, ba, sa), (wb, bb, sb) = self.W[a], self.W[b]
            try:
                p = self.fhconv.ConvPairPlan(da, wa, ba, sa, db, wb, bb, sb, film_in=True)
                p._work = p.describe()
            except self.fhconv.FhcError:
                p = False  # no fused kernel for these channels
            self.plans[key] = p
        return p

    def gmhs_film(self, a: V, b: V, flow: V, full_w: int, level: int, fa, fb, h: V, c: int, hm: V, mid: V, y: V,
                  fo, yo: V):
        p = self._film_plan(fa, fb, h, c, mid, y)
        if p is False or level == 0:
            return super().gmhs_film(a, b, flow, full_w, level, fa, fb, h, c, hm, mid, y, fo, yo)
        q = self._conv_plan(fo, y, yo)
        va, vb, vf = self._v(a), self._v(b), self._v(flow)
        _, hh, ww, _ = va.shape
        _, h8, w8, _ = vf.shape
        key = ("gmhs", hh, ww, full_w, level)
        if key not in self.plans:
            self.plans[key] = self.fh.gmhs_workspace(hh, ww, full_w, level, self.dev)
        ws = self.plans[key]
        gp = self.fh.gmhs_params(hh, ww, full_w, level)
        cells = gp["hc"] * gp["wc"]
        nbytes = 5 * 4 * 2 * h8 * w8 + 2 * 3 * 2 * hh * ww + 4 * cells * (5 + 5 + 5 + 3) + 4 * 2 * h8 * w8
        hb, yb, ob, g, st = h.buf, y.buf, yo.buf, self.g, self.stream
        self._go(f"gmhs + film_modulate+{fa}+{fb} + {fo} (in the first two fit launches)",
                 lambda: self.fh.gmhs_film(va, vb, vf, full_w, level, ws, p, hb, g, yb, q, yb, ob, stream=st),
                 nbytes + p._work["bytes"] + 2 * 2 * c + q._work["bytes"], p._work["flops"] + q._work["flops"], "op",
                 kernels=8)

    def film_pair(self, a, b, h: V, c: int, hm: V, mid: V, y: V):
        p = self._film_plan(a, b, h, c, mid, y)
        if p is False:
            return super().film_pair(a, b, h, c, hm, mid, y)
        hb, yb, g, st = h.buf, y.buf, self.g, self.stream
        self._go(f"film_modulate+{a}+{b}", lambda: p.run_film(hb, g, yb, stream=st),
                 p._work["bytes"] + 2 * 2 * c, p._work["flops"], "conv")

    def conv_siblings(self, a, b, x: V, ya: V, res_a: Optional[V], yb: V):
        if not (self.chains and self.fuse):
            return super().conv_siblings(a, b, x, ya, res_a, yb)
        key = ("siblings", a, b, x.buf.shape[0], x.buf.data_ptr(), x.c0, ya.buf.data_ptr(), ya.c0, yb.buf.data_ptr(),
               yb.c0)
        p = self.plans.get(key)
        if p is None:
            da, db = self._desc(a, x, ya, res_a), self._desc(b, x, yb, None)
            (wa, ba, sa), (wb, bb, sb) = self.W[a], self.W[b]
            try:
                p = self.fhconv.ConvSiblingPlan(da, wa, ba, sa, db, wb, bb, sb)
                w = p.describe()
                p._work = dict(flops=w["flops"], bytes=w["bytes"])
            except self.fhconv.FhcError:
                p = False  # no sibling kernel for these channels
            self.plans[key] = p
        if p is False:
            return super().conv_siblings(a, b, x, ya, res_a, yb)
        xb, yab, rb, ybb, st = x.buf, ya.buf, None if res_a is None else res_a.buf, yb.buf, self.stream
        self._go(f"{a}+{b} (siblings)", lambda: p.run(xb, yab, rb, ybb, stream=st), p._work["bytes"],
                 p._work["flops"], "conv")

    def interp(self, x: V, c, out: V, oh, ow, aa):
        n = x.buf.shape[0]
        fx, fo = self._v(x), self._v(out)
        self._go("interp", lambda: self.fh.interp(fx, oh, ow, aa, c, out=fo, stream=self.stream),
                 2 * c * (self._px(x) + n * oh * ow))

    def avgpool(self, x: V, c, out: V, k):
        fx, fo = self._v(x), self._v(out)
        self._go("avgpool", lambda: self.fh.avgpool(fx, k, c, out=fo, stream=self.stream),
                 2 * c * (self._px(x) + self._px(out)))

    def luma(self, x: V, out: V, grad=False):
        fx, fo = self._v(x), self._v(out)
        self._go("luma_grad" if grad else "luma", lambda: self.fh.luma(fx, grad, out=fo, stream=self.stream),
                 2 * 4 * self._px(x))

    def sad(self, la: V, lb: V, out: V, r):
        fa, fb, fo = self._v(la), self._v(lb), self._v(out)
        self._go("sad_volume", lambda: self.fh.sad(fa, fb, r, out=fo, stream=self.stream),
                 2 * (2 + (2 * r + 1) ** 2) * self._px(la))

    def warp(self, img: V, c, flow: V, out: V):
        fi, ff, fo = self._v(img), self._v(flow), self._v(out)
        self._go("warp", lambda: self.fh.warp(fi, ff, c, out=fo, stream=self.stream), 2 * (2 * c + 2) * self._px(img))

    def chcopy(self, x: V, c, out: V):
        fx, fo = self._v(x), self._v(out)
        self._go("chcopy", lambda: self.fh.chcopy(fx, c, out=fo, stream=self.stream), 2 * 2 * c * self._px(x))

    def binary(self, a: V, b: V, c, out: V, op=0):
        fa, fb, fo = self._v(a), self._v(b), self._v(out)
        self._go("binary", lambda: self.fh.binary(fa, fb, op, c, out=fo, stream=self.stream), 2 * 3 * c * self._px(a))

    def unary(self, x: V, c, out: V, op, a=0.0):
        fx, fo = self._v(x), self._v(out)
        self._go("unary", lambda: self.fh.unary(fx, op, a, 0.0, c, out=fo, stream=self.stream),
                 2 * 2 * c * self._px(x))

    def film(self, hv: V, c, out: V):
        fh_, fo, g = self._v(hv), self._v(out), self.g
        self._go("film_modulate", lambda: self.fh.film(fh_, g, c, out=fo, stream=self.stream),
                 2 * (2 * c * self._px(hv) + 2 * c))

    def convex(self, wt: V, x: V, c, out: V):
        fw, fx, fo = self._v(wt), self._v(x), self._v(out)
        self._go("convex_upsample", lambda: self.fh.convex(fw, fx, c, out=fo, stream=self.stream),
                 2 * (36 + c + 4 * c) * self._px(x))

    def blendmix(self, wa: V, wb: V, vis: V, out: V):
        fa, fb, fv, fo = self._v(wa), self._v(wb), self._v(vis), self._v(out)
        self._go("blendmix", lambda: self.fh.blendmix(fa, fb, fv, out=fo, stream=self.stream),
                 2 * 12 * self._px(wa))

    def render(self, a: V, b: V, flow: V, vis: V, rt: V, out: V, cubic: bool, flags: int, fsx=None, fsy=None):
        fsx = flow.scale if fsx is None else fsx
        fsy = flow.scale if fsy is None else fsy
        # the flow's scale is carried by fsx, fsy (render_pix multiplies the raw flow by them)
        va, vb, vf, vv, vr, vo = (self._v(t) for t in (a, b, V(flow.buf, flow.c0), vis, rt, out))
        self._go("render_pix", lambda: self.fh.render(va, vb, vf, vv, vr, cubic, flags, fsx, fsy, out=vo,
                                                      stream=self.stream),
                 2 * (3 * 3 * self._px(out) + 10 * self._px(flow)))

    def rgba_in(self, frames, out: V, hp: int, wp: int):
        fo = self._v(out)
        self._go("rgba_in", lambda: self.fh.rgba_in(frames, hp, wp, out=fo, stream=self.stream),
                 4 * frames.numel() + 2 * 3 * self._px(out))

    def rgba_out(self, x: V, out_frames):
        _, h, w = out_frames.shape
        fx = self._v(x)
        self._go("rgba_out", lambda: self.fh.rgba_out(fx, h, w, out=out_frames, stream=self.stream),
                 (2 * 3 + 4) * out_frames.numel())

    def frame_input(self, frames, full, ab: V, hp: int, wp: int, oh: int, ow: int):
        if not self.chains:
            return super().frame_input(frames, full, ab, hp, wp, oh, ow)
        fo = self._v(ab)
        self._go("frame_input (rgba_in + resize)",
                 lambda: self.fh.rgba_resize(frames, hp, wp, oh, ow, out=fo, stream=self.stream),
                 4 * frames.numel() + 2 * 3 * self._px(ab))

    def frame_render(self, frames, full, pic, flow: V, vis: V, rt: V, out_frames, hp: int, wp: int, fsx: float,
                     fsy: float, cubic: bool, flags: int):
        if not self.chains:
            return super().frame_render(frames, full, pic, flow, vis, rt, out_frames, hp, wp, fsx, fsy, cubic, flags)
        vf, vv, vr = self._v(flow), self._v(vis), self._v(rt)
        fa, fb = frames[0:1], frames[1:2]
        fl = flags | (4 if self.exact_render else 0)  # bit 2: the reference's f32 order
        self._go("frame_render (render_pix + rgba_out)",
                 lambda: self.fh.render_rgba(fa, fb, vf, vv, vr, hp, wp, cubic, fl, fsx, fsy, out=out_frames,
                                             stream=self.stream),
                 4 * (frames.numel() + out_frames.numel()) + 2 * 10 * self._px(flow))

    def frame_render_n(self, frames, full, pic, flow: V, vis: V, rt: V, out_frames, hp: int, wp: int, fsx: float,
                       fsy: float, cubic: bool, flags: int, phases: int):
        if not self.chains or frames.shape[0] * phases == 2:
            return super().frame_render_n(frames, full, pic, flow, vis, rt, out_frames, hp, wp, fsx, fsy, cubic,
                                          flags, phases)
        vf, vv, vr = self._v(flow), self._v(vis), self._v(rt)
        fl = flags | (4 if self.exact_render else 0)  # bit 2: the reference's f32 order
        self._go("frame_render (render_pix + rgba_out, every generated frame)",
                 lambda: self.fh.render_rgba_n(frames, vf, vv, vr, hp, wp, phases, cubic, fl, fsx, fsy,
                                               out=out_frames, stream=self.stream),
                 4 * (frames.numel() * phases + out_frames.numel()) + 2 * 10 * self._px(flow))

    def gmhs(self, a: V, b: V, flow: V, full_w: int, level: int):
        va, vb, vf = self._v(a), self._v(b), self._v(flow)
        _, h, w, _ = va.shape
        _, h8, w8, _ = vf.shape
        key = ("gmhs", h, w, full_w, level)
        if key not in self.plans:
            self.plans[key] = self.fh.gmhs_workspace(h, w, full_w, level, self.dev)
        ws = self.plans[key]
        p = self.fh.gmhs_params(h, w, full_w, level)
        cells = p["hc"] * p["wc"]
        # algorithmic bytes: the flow read by 4 fit rounds and the cost maps, the two pictures' BGR, the 5 maps
        # written, read and written by the texture window, maps 0-2 read by the decision window, the flow written
        nbytes = 5 * 4 * 2 * h8 * w8 + 2 * 3 * 2 * h * w + 4 * cells * (5 + 5 + 5 + 3) + 4 * 2 * h8 * w8
        self._go("gmhs (fit x4, cost, texture window, decision window x2)",
                 lambda: self.fh.gmhs(va, vb, vf, full_w, level, ws=ws, stream=self.stream), nbytes, kernels=8)

    def gmhs_n(self, ab: V, flow: V, full_w: int, level: int):
        vab, vf = self._v(ab), self._v(flow)
        _, h, w, _ = vab.shape
        n, h8, w8, _ = vf.shape
        key = ("gmhs", h, w, full_w, level, n)
        if key not in self.plans:
            self.plans[key] = self.fh.gmhs_workspace(h, w, full_w, level, self.dev, n)
        ws = self.plans[key]
        p = self.fh.gmhs_params(h, w, full_w, level)
        nbytes = n * (5 * 4 * 2 * h8 * w8 + 2 * 3 * 2 * h * w + 4 * p["hc"] * p["wc"] * (5 + 5 + 5 + 3) + 4 * 2 * h8 * w8)
        self._go("gmhs (fit x4, cost, texture window, decision window x2)",
                 lambda: self.fh.gmhs_n(vab, vf, full_w, level, ws=ws, stream=self.stream), nbytes, kernels=8)

    # the fused chains (one launch each) unless asked for the ops one by one
    def coarse_up(self, o: V, out: V, state: Optional[V], oh: int, ow: int, flow_scale: float):
        if not self.chains:
            return super().coarse_up(o, out, state, oh, ow, flow_scale)
        vo, vout, vs = self._v(o), self._v(out), None if state is None else self._v(state)
        self._go("coarse_up", lambda: self.fh.coarse_up(vo, vout, vs, oh, ow, flow_scale, stream=self.stream),
                 2 * (7 + (0 if state is None else 4)) * self._px(o) + 2 * 7 * oh * ow)

    def fold_pair(self, x: V, c: int, out: V, also: Optional[V]):
        if not self.chains:
            return super().fold_pair(x, c, out, also)
        vx, vo, va = self._v(x), self._v(out), None if also is None else self._v(also)
        self._go("fold_pair", lambda: self.fh.fold_pair(vx, vo, va, stream=self.stream, c=c),
                 2 * c * (2 * self._px(x) + (self._px(x) // 2 if also is not None else 0)))

    def fold_pair_sad(self, x: V, c: int, out: V, also: Optional[V], la: V, lb: V, sad_out: V, r: int):
        if not self.chains:
            return super().fold_pair_sad(x, c, out, also, la, lb, sad_out, r)
        vx, vo, va = self._v(x), self._v(out), None if also is None else self._v(also)
        fa, fb, fs = self._v(la), self._v(lb), self._v(sad_out)
        self._go("fold_pair_sad (fold_pair + sad_volume)",
                 lambda: self.fh.fold_pair_sad(vx, vo, va, fa, fb, fs, r, stream=self.stream, c=c),
                 2 * c * (2 * self._px(x) + (self._px(x) // 2 if also is not None else 0))
                 + 2 * (2 + (2 * r + 1) ** 2) * self._px(la))

    def pair_input(self, ab: V, q: V, i8: V, i16: V, l16: V, oh: int, ow: int):
        if not self.chains:
            return super().pair_input(ab, q, i8, i16, l16, oh, ow)
        vs = [self._v(t) for t in (ab, q, i8, i16, l16)]
        self._go("pair_input (resize + pyramid)",
                 lambda: self.fh.pair_input(*vs, oh, ow, stream=self.stream),
                 2 * (3 * self._px(ab) + 3 * self._px(q) + 3 * self._px(i8) + 6 * self._px(i16) + 2 * self._px(l16)))

    def pair_pyramid(self, q: V, i8: V, i16: V, l16: V):
        if not self.chains:
            return super().pair_pyramid(q, i8, i16, l16)
        vs = [self._v(t) for t in (q, i8, i16, l16)]
        self._go("pair_pyramid", lambda: self.fh.pair_pyramid(*vs, stream=self.stream),
                 2 * (3 * self._px(q) + 3 * self._px(i8) + 6 * self._px(i16) + 2 * self._px(l16)))

    def fine_input(self, f8: V, i8: V, flow: V, fx: V, l8: V, c: int):
        if not self.chains:
            return super().fine_input(f8, i8, flow, fx, l8, c)
        vs = [self._v(t) for t in (f8, i8, flow, fx, l8)]
        p1 = self._px(flow)
        self._go("fine_input", lambda: self.fh.fine_input(*vs, c, stream=self.stream),
                 2 * p1 * (2 * c + 6 + 4 + (2 * c + 6 + 4) + 2))

    def flow_vis_t(self, fv: V, dfilm: V, out: V, t: float, lin: V, dvis: V):
        if not self.chains:
            return super().flow_vis_t(fv, dfilm, out, t, lin, dvis)
        vs = [self._v(x) for x in (fv, dfilm, out)]
        self._go("flow_vis_t", lambda: self.fh.flow_vis_t(*vs, t, stream=self.stream), 2 * (7 + 5 + 7) * self._px(fv))

    def coarse_fine_input(self, o: V, fv: V, state: Optional[V], flow_scale: float, f8: V, i8: V,
                          fine_scale: float, fx: V, l8: V, c: int):
        if not self.chains:
            return super().coarse_fine_input(o, fv, state, flow_scale, f8, i8, fine_scale, fx, l8, c)
        vo, vfv, vs = self._v(o), self._v(fv), None if state is None else self._v(state)
        vf8, vi8, vfx, vl8 = (self._v(x) for x in (f8, i8, fx, l8))
        p1, po = self._px(f8) // 2, self._px(o)
        # o read (7 channels, +4 for the state), fv (7) and the state (4) written, then fine_input's traffic
        self._go("coarse_fine_input (coarse_up + fine_input)",
                 lambda: self.fh.coarse_fine_input(vo, vfv, vs, flow_scale, vf8, vi8, fine_scale, vfx, vl8, c,
                                                   stream=self.stream),
                 2 * (7 + (0 if state is None else 8)) * po + 2 * 7 * p1 + 2 * p1 * (2 * c + 6 + (2 * c + 6 + 4) + 2))

    def coarse_fine_input_sad(self, o: V, fv: V, state: Optional[V], flow_scale: float, f8: V, i8: V,
                              fine_scale: float, fx: V, l8: V, c: int, sad_out: V, r: int):
        if not self.chains:
            return super().coarse_fine_input_sad(o, fv, state, flow_scale, f8, i8, fine_scale, fx, l8, c, sad_out, r)
        vo, vfv, vs = self._v(o), self._v(fv), None if state is None else self._v(state)
        vf8, vi8, vfx, vl8, vsd = (self._v(x) for x in (f8, i8, fx, l8, sad_out))
        p1, po = self._px(f8) // 2, self._px(o)
        span2 = (2 * r + 1) ** 2
        # coarse_fine_input's traffic, then the cost volume written (its lumas are recomputed, not read)
        self._go("coarse_fine_input_sad (coarse_up + fine_input + sad_volume)",
                 lambda: self.fh.coarse_fine_input_sad(vo, vfv, vs, flow_scale, vf8, vi8, fine_scale, vfx, vl8, c,
                                                       vsd, r, stream=self.stream),
                 2 * (7 + (0 if state is None else 8)) * po + 2 * 7 * p1 + 2 * p1 * (2 * c + 6 + (2 * c + 6 + 4) + 2)
                 + 2 * p1 * span2)

    def flow_vis_t_convex(self, wt: V, fv: V, dfilm: V, t: float, out: V, ftvt: V, lin: V, dvis: V):
        if not self.chains:
            return super().flow_vis_t_convex(wt, fv, dfilm, t, out, ftvt, lin, dvis)
        vw, vfv, vd, vo = (self._v(x) for x in (wt, fv, dfilm, out))
        px = self._px(fv)
        self._go("flow_vis_t_convex (flow_vis_t + convex_upsample)",
                 lambda: self.fh.flow_vis_t_convex(vw, vfv, vd, t, vo, stream=self.stream),
                 2 * (36 + 7 + 5 + 4 * 7) * px)

    def flow_vis_t_convex_n(self, wt: V, fv: V, dfilm: V, ts, out: V, ftvt: V, lin: V, dvis: V):
        if not self.chains:
            return super().flow_vis_t_convex_n(wt, fv, dfilm, ts, out, ftvt, lin, dvis)
        vw, vfv, vd, vo = (self._v(x) for x in (wt, fv, dfilm, out))
        ts = tuple(float(t) for t in ts)
        self._go("flow_vis_t_convex (flow_vis_t + convex_upsample)",
                 lambda: self.fh.flow_vis_t_convex(vw, vfv, vd, ts, vo, stream=self.stream),
                 2 * (36 + 7 + 5 + 4 * 7) * self._px(fv) * len(ts))

    def mid_input_n(self, wt: V, fv: V, dfilm: V, ts, up: V, ftvt: V, lin: V, dvis: V, q: V, rx: V,
                    flow_scale: float, flow_out_scale: float, blend: V):
        if not self.chains:
            return super().mid_input_n(wt, fv, dfilm, ts, up, ftvt, lin, dvis, q, rx, flow_scale, flow_out_scale,
                                       blend)
        vw, vfv, vd, vu, vq, vr = (self._v(x) for x in (wt, fv, dfilm, up, q, rx))
        ts = tuple(float(t) for t in ts)
        # the convex upsample's reads (wt, fv at the input grid, dfilm every phase) and up written; the refine
        # input's two warps of the pictures and rx written
        self._go("mid_input (flow_vis_t + convex_upsample + refine_input)",
                 lambda: self.fh.mid_input(vw, vfv, vd, ts, vu, vq, vr, flow_scale, flow_out_scale,
                                           stream=self.stream),
                 2 * (36 + 7) * self._px(fv) + 2 * 5 * self._px(dfilm) + 2 * self._px(up) * (7 + 6 + 14))

    def refine_input(self, q: V, flow: V, vis: V, rx: V, flow_out_scale: float, blend: V):
        if not self.chains:
            return super().refine_input(q, flow, vis, rx, flow_out_scale, blend)
        vs = [self._v(x) for x in (q, flow, vis, rx)]
        self._go("refine_input", lambda: self.fh.refine_input(*vs, flow_out_scale, stream=self.stream),
                 2 * self._px(flow) * (6 + 4 + 3 + 14))

    def refine_input_n(self, q: V, flow: V, vis: V, rx: V, flow_out_scale: float, blend: V, qmod: int):
        if not self.chains:
            return super().refine_input_n(q, flow, vis, rx, flow_out_scale, blend, qmod)
        vs = [self._v(x) for x in (q, flow, vis, rx)]
        self._go("refine_input", lambda: self.fh.refine_input(*vs, flow_out_scale, qmod=qmod, stream=self.stream),
                 2 * self._px(flow) * (6 + 4 + 3 + 14))


def sl(buf, i: int, n: int = 1):
    """Images i .. i + n - 1 of a buffer (a view of the same memory on either backend)."""
    return buf[i:i + n]


class FlyHighFG:
    """The buffers of frame pairs at network size net_w x net_h and the program of pair() and mid(t) over them.
    Outputs after mid(): ``out`` (render_pix, the in-between picture), ``up7`` (flow_tq channels 0-3, vis_tq 4-6,
    quarter size), ``Rt`` (R_t, 3 channels), ``state_out`` (f16b then flow16, 1/16 size); ``o`` holds the coarse head
    (conf, gate, sal in channels 7-11). cubic / render_flags: render_pix's sampler (the model's manifest asks for
    bicubic, models/flyhighfg.json:67) and mode word (0: neither the decisive blend nor the still test, the
    engine's defaults, options.rs:306-327).

    pairs P independent frame pairs and mids M phases per pair run as one batch: the reference's sessions of one
    pair each, side by side. The pictures of pair p are images 2p (A) and 2p + 1 (B) of the A/B buffers, so each
    pair's A and B are one contiguous batch of 2, as every op chain of one pair takes them; the pair stage's one-image
    tensors hold pair p at image p, and the mid stage's hold phase j of pair p at image j * P + p (each phase's P
    images contiguous). Every conv and every op chain runs once over the whole batch (2P, P or M * P images), but
    the FiLM pair once per phase (over its P images) and the frame-size render once per generated frame. P = M = 1 is the reference's single session."""

    def __init__(self, be, net_w: int = 864, net_h: int = 480, cubic: bool = True, render_flags: int = 0,
                 frame: Optional[tuple] = None, repair: int = 1, pairs: int = 1, mids: int = 1):
        self.be = be
        self.P, self.M = P, M = int(pairs), int(mids)
        if P < 1 or M < 1:
            raise ValueError("pairs and mids must be at least 1")
        # repair: the periodic-structure repair's level (gmhs.rs; 0 off, 1 the engine's default, options.rs:305,
        # 2 aggressive), run on the E8 flow at the end of pair() (net/build.rs:640-660)
        self.repair = repair
        # frame (w, h): the program starts from the host's two RGBA8 frames (``frames``, uploaded by the caller) and
        # ends with the generated RGBA8 frame (``rgba``), as the reference's Session does (net/session.rs:26-66).
        # The frames are padded to a multiple of 32; when that differs from the network size the network runs on
        # the antialiased downscale and the render runs at the padded frame size (the internal-size mode,
        # net/build.rs:549-551, :615-620, :717-736). Without a frame the caller fills AB at network size.
        self.frame = frame
        if frame is not None:
            fw, fh = frame
            self.hp, self.wp = (fh + 31) // 32 * 32, (fw + 31) // 32 * 32
            self.internal = (self.wp, self.hp) != (net_w, net_h)
            self.frames = be.frames(2 * P, fh, fw)  # A, B of each pair: RGBA8 words
            self.rgba = be.frames(M * P, fh, fw)     # the generated frames, phase-major
            # the composed chains' full-size intermediates (rgba_in's pictures, the render's f16 picture); the fused
            # GPU chains never touch them
            composed = not getattr(be, "chains", False)
            self.full = be.zeros(2 * P, self.hp, self.wp, 4) if composed else None
            self.pic = be.zeros(1, self.hp, self.wp, 4) if composed and self.internal else None
            # the flow's scale per axis at the frame size: ftq.scale * wp / iwp (net/build.rs:720), in f32
            self.fsx = float(np.float32(self.wp) / np.float32(net_w))
            self.fsy = float(np.float32(self.hp) / np.float32(net_h))
        qh, qw = net_h // 4, net_w // 4
        e8h, e8w = (qh - 1) // 2 + 1, (qw - 1) // 2 + 1
        e16h, e16w = (e8h - 1) // 2 + 1, (e8w - 1) // 2 + 1
        self.shape = dict(net=(net_h, net_w), q=(qh, qw), e8=(e8h, e8w), e16=(e16h, e16w))
        Z, AB, PP, MP = be.zeros, 2 * P, P, M * P
        # the A/B stage: image 2p is pair p's A, 2p + 1 its B
        self.AB = Z(AB, net_h, net_w, 4)        # the inputs A, B at network size (BGR in [0, 1]), 8-byte pixels
        self.aq = Z(AB, qh, qw, 8)              # aq, bq
        self.e1 = Z(AB, e8h, e8w, 40)           # a_e1, b_e1
        self.f8 = Z(AB, e8h, e8w, 40)           # f8a, f8b
        self.e3 = Z(AB, e16h, e16w, 72)         # a_e3, b_e3
        self.f16 = Z(AB, e16h, e16w, 72)        # f16a, f16b (then folded into the concat)
        self.i8 = Z(AB, e8h, e8w, 8)            # i8a, i8b
        # the pair stage: image p is pair p
        self.cin = Z(PP, e16h, e16w, 280)       # f16a 0 | f16b 72 | img16 144 | side 150 | state 154 | cv 230
        self.l16 = Z(PP, e16h, e16w, 2)         # la | lb
        self.ch1, self.ch2, self.ch3r, self.hc = (Z(PP, e16h, e16w, 96) for _ in range(4))
        self.o = Z(PP, e16h, e16w, 16)          # coarse head: flow 0-3, vis 4-6, conf, gate, sal
        self.fv = Z(PP, e8h, e8w, 8)            # flow 0-3 | vis 4-6 (the fine loop updates both in one add)
        self.state_out = Z(PP, e16h, e16w, 80)  # f16b 0 | flow16 72
        self.fx = Z(PP, e8h, e8w, 160)          # wa 0 | wb 36 | ia 72 | ib 75 | flow8 78 | h 82 | fcv 130
        self.l8 = Z(PP, e8h, e8w, 2)            # fla | flb
        self.fr1, self.fr2, self.h = (Z(PP, e8h, e8w, 48) for _ in range(3))
        self.wt36 = Z(PP, e8h, e8w, 40)
        # the mid stage: image j * P + p is phase j of pair p
        self.lin = Z(MP, e8h, e8w, 8)           # linf | linb
        self.hm, self.fh1, self.fh2 = (Z(MP, e8h, e8w, 48) for _ in range(3))
        self.dfilm = Z(MP, e8h, e8w, 8)         # d_flow 0-3, d_mask 4
        self.dvis = Z(MP, e8h, e8w, 8)          # d_mask | -d_mask | 0
        self.ftvt = Z(MP, e8h, e8w, 8)          # flow_t 0-3 | vis_t 4-6
        self.up7 = Z(MP, qh, qw, 8)             # flow_tq 0-3 | vis_tq 4-6
        self.blend = Z(MP, qh, qw, 8)
        self.rx = Z(MP, qh, qw, 16)             # rwa 0 | rwb 3 | vis_tq 6 | flow_tq20 9 | lg 13
        self.rq1, self.rq2, self.rq3 = (Z(MP, qh, qw, 24) for _ in range(3))
        self.rr, self.Rt = Z(MP, qh, qw, 8), Z(MP, qh, qw, 8)
        self.out = Z(MP, net_h, net_w, 4)        # render_pix: the in-between picture at network size
        self.cubic, self.render_flags = cubic, render_flags
        # the padded frame width the repair's windows scale with (the network's own without a frame)
        self.full_w = self.wp if frame is not None else net_w

    def pair(self, cofilm: bool = False) -> bool:
        """pair(): models/graph.json ops 0-43 (the fine loop once, K = 1), and op 62 (up.w, which reads only h), for
        every pair. cofilm: also the next mid(t)'s FiLM head (ops 50-53: it reads only h and the FiLM vector of t,
        which must be in place), inside the repair's first two launches (one pair, one phase); returns whether it ran
        (mid(t, film_done=True) then skips it)."""
        be, S, P = self.be, self.shape, self.P
        (qh, qw), (e8h, e8w) = S["q"], S["e8"]
        if self.frame is not None:  # the frames -> A, B (rgba_in; in the internal-size mode, the downscale)
            nh, nw = S["net"]
            if self.internal:
                be.frame_input(self.frames, self.full, V(self.AB), self.hp, self.wp, nh, nw)
            else:
                be.rgba_in(self.frames, V(self.AB), nh, nw)
        be.pair_input(V(self.AB), V(self.aq), V(self.i8), V(self.cin, 144), V(self.l16), qh, qw)  # 0-1, 14-24
        be.pair("enc.e1", "enc.e2", V(self.aq), V(self.e1), V(self.f8), True)                 # 2-4, 8-10
        be.pair("enc.e3", "enc.e4", V(self.f8), V(self.e3), V(self.f16), True)                # 5-7, 11-13
        # 26, 43: f16a f16b into the concat and the state, beside the 1/16 lumas' cost volume (25, 26; 19-20 zeros),
        # which reads and writes nothing the encoders touch
        be.fold_pair_sad(V(self.f16), 72, V(self.cin, 0), V(self.state_out, 0), V(self.l16, 0), V(self.l16, 1),
                         V(self.cin, 230), 3)
        be.conv("coarse.c1", V(self.cin), V(self.ch1))                                        # 27
        be.conv("coarse.c2", V(self.ch1), V(self.ch2))                                        # 28
        be.conv("coarse.c3", V(self.ch2), V(self.ch3r), V(self.ch1))                          # 29, 30
        be.conv("coarse.c4", V(self.ch3r), V(self.hc))                                        # 31
        be.conv("coarse.head", V(self.hc), V(self.o))                                         # 32
        # 33-40 (43: flow16), then the fine loop's input, K = 1 (op 42: wa .. flow8); h enters as zeros (op 41: the
        # fx slice is never written)
        # and the fine block's cost volume (fcv) of the warped pictures' lumas into its slice of fx
        be.coarse_fine_input_sad(V(self.o), V(self.fv), V(self.state_out, 72), 16.0, V(self.f8), V(self.i8), 0.125,
                                 V(self.fx), V(self.l8), 36, V(self.fx, 130), 2)
        be.conv("fine.r1", V(self.fx), V(self.fr1))
        be.pair("fine.r2", "fine.r3", V(self.fr1), V(self.fr2), V(self.h), False)             # h = fr3
        # flow, vis += d: the add of fine.out's output as the conv's residual, written in place (the planner's
        # residual peephole, net/build.rs:222-237; f16(f32(d) + f32(fv)) either way)
        # up.w (graph op 62, mid's first conv) reads only h, so it runs here beside fine.out, which reads h too: one
        # launch, and a pair() followed by several mid(t) computes it once
        be.conv_siblings("fine.out", "up.w", V(self.h), V(self.fv), V(self.fv), V(self.wt36))
        if self.repair and cofilm and P == 1 and self.M == 1:  # the repair, with mid's FiLM pair in its first launch
            be.gmhs_film(V(be.image(self.AB, 0)), V(be.image(self.AB, 1)), V(self.fv), self.full_w, self.repair,
                         "film.h1", "film.h2", V(self.h), 48, V(self.hm), V(self.fh1), V(self.fh2), "film.out",
                         V(self.dfilm))
            return True
        if self.repair:  # the periodic-structure repair of each pair's flow, in place (gmhs.rs:149-206)
            be.gmhs_n(V(self.AB), V(self.fv), self.full_w, self.repair)
        return False

    def pair_mid(self, t: float, W: Optional[dict] = None):
        """pair() then mid(t), the FiLM head of t run inside the repair's first two launches (two launches fewer).
        With W None the FiLM vector of t must already be in place, as for mid()."""
        if W is not None:
            self.be.set_g(self.film_vectors(W, t))
        self.mid(t, None, film_done=self.pair(cofilm=True))

    def film_vectors(self, W: dict, t: float) -> np.ndarray:
        """The FiLM vector of t once per pair (f16 bits [P * 96]): the FiLM ops take one vector per image."""
        return np.tile(film_mlp(W, t), self.P)

    def mid(self, t: float, W: Optional[dict], film_done: bool = False):
        """mid(t): models/graph.json ops 44-82 but 62 (up.w, run by pair()), render_pix included, for every pair (one
        phase). With W None the FiLM vectors of t must already be in place (be.set_g(self.film_vectors(W, t))): a
        program captured in a HIP graph takes them that way, as the reference rewrites its t-dependent buffers before
        a replay (net/build.rs:16-22). film_done: the FiLM head (ops 50-53) already ran with this t's vector
        (pair(cofilm=True))."""
        if self.M != 1:
            raise ValueError("mid(t) runs one phase: a program of several phases runs them with mids()")
        if W is not None:
            self.be.set_g(self.film_vectors(W, t))                                            # 49
        self._mid_phase(0, t, film_done)
        self._mid_tail()

    def mids(self, ts, W: Optional[dict] = None):
        """mid(t) for each of the M phases ts of every pair: each phase's FiLM pair with that phase's FiLM vectors
        (slot j of the backend's vectors: be.set_g(self.film_vectors(W, t), j), set here when W is given), then
        film.out, flow_t / vis_t with the convex upsample (each phase its t), the refine input and the refine head
        over all M * P images at once, then the renders."""
        ts = tuple(ts)
        if len(ts) != self.M:
            raise ValueError(f"{len(ts)} phases for a program of {self.M}")
        be, P = self.be, self.P
        if W is not None:
            for j, t in enumerate(ts):
                be.set_g(self.film_vectors(W, t), j)
        for j in range(self.M):                                                               # 50-52
            m = lambda b: sl(b, j * P, P)  # noqa: E731  phase j's images
            be.use_g(j)
            be.film_pair("film.h1", "film.h2", V(self.h), 48, V(m(self.hm)), V(m(self.fh1)), V(m(self.fh2)))
        be.conv("film.out", V(self.fh2), V(self.dfilm))                                       # 53
        be.mid_input_n(V(self.wt36), V(self.fv), V(self.dfilm), ts, V(self.up7), V(self.ftvt), V(self.lin),
                       V(self.dvis), V(self.aq), V(self.rx), 0.25, 0.05, V(self.blend))       # 44-48, 54-76
        self._mid_tail()

    def run(self, ts, W: Optional[dict] = None):
        """pair() and mids(ts): the whole batched step (P pairs, M phases each)."""
        if self.P == 1 and self.M == 1:
            return self.pair_mid(ts[0], W)
        if W is not None:
            for j, t in enumerate(ts):
                self.be.set_g(self.film_vectors(W, t), j)
        self.pair()
        self.mids(ts)

    def _mid_phase(self, j: int, t: float, film_done: bool):
        """ops 44-61, 63-76 of phase j (FiLM vector slot j) for every pair."""
        be, P = self.be, self.P
        m = lambda b: sl(b, j * P, P)  # noqa: E731  phase j's images
        be.use_g(j)
        if not film_done:
            be.film_pair("film.h1", "film.h2", V(self.h), 48, V(m(self.hm)), V(m(self.fh1)), V(m(self.fh2)))  # 50-52
            be.conv("film.out", V(m(self.fh2)), V(m(self.dfilm)))                             # 53
        be.mid_input_n(V(self.wt36), V(self.fv), V(m(self.dfilm)), (t,), V(m(self.up7)), V(m(self.ftvt)),
                       V(m(self.lin)), V(m(self.dvis)), V(self.aq), V(m(self.rx)), 0.25, 0.05,
                       V(m(self.blend)))                                                      # 44-48, 54-76

    def _mid_tail(self):
        """ops 77-82 for all M * P images: the refine head at once, then each image's render, pair by pair (a pair's
        M renders read the same two frames, which the last-level cache then still holds for all but the first)."""
        be, P = self.be, self.P
        be.pair("refine.q1", "refine.q2", V(self.rx), V(self.rq1), V(self.rq2), False)        # 77, 78
        be.pair_affine_out("refine.q3", "refine.q4", V(self.rq2), V(self.rq3), V(self.rr), V(self.Rt), 3)  # 79-81
        if self.frame is not None and self.internal:  # the render at the frame size, to the RGBA8 frames
            be.frame_render_n(self.frames, self.full, self.pic, V(self.up7, 0), V(self.up7, 4), V(self.Rt), self.rgba,
                              self.hp, self.wp, self.fsx, self.fsy, self.cubic, self.render_flags, self.M)
            return
        for i in (j * P + p for p in range(P) for j in range(self.M)):
            p = i % P
            up7, rt = sl(self.up7, i), sl(self.Rt, i)
            out = sl(self.out, i)
            be.render(V(sl(self.AB, 2 * p)), V(sl(self.AB, 2 * p + 1)), V(up7, 0), V(up7, 4), V(rt), V(out),
                      self.cubic, self.render_flags)                                          # 82: render_pix
            if self.frame is not None:
                be.rgba_out(V(out), sl(self.rgba, i))


def cpu_threads():
    return max(1, min(16, len(os.sched_getaffinity(0))))


def procedural_frame(w: int, h: int, dx: int = 0, dy: int = 0, seed: int = 0) -> np.ndarray:
    """A synthetic RGBA8 frame (h, w) of uint32 words, the kind the reference's bench generates
    (crates/flyhigh-cli/src/cli/bench.rs:33-51): smooth sine patterns per channel plus 0.1 of hashed noise, the
    whole picture shifted by (dx, dy) pixels, alpha 255. seed 0 is that picture; another seed shifts the patterns'
    phases and salts the noise hash, a texture of its own. Test and benchmark data only."""
    if seed:
        rng = np.random.default_rng(seed)
        ph = rng.uniform(0.0, 2.0 * np.pi, 3).astype(np.float32)
        salt = np.uint32(rng.integers(1, 1 << 32))
    else:
        ph, salt = np.zeros(3, np.float32), np.uint32(0)
    # a row of columns and a column of rows, broadcast: every pixel's value comes from the same f32 operations as
    # over full grids
    sx = np.arange(w, dtype=np.int64)[None, :] + dx
    sy = np.arange(h, dtype=np.int64)[:, None] + dy
    # the hash in wrapping 32-bit arithmetic (equal to the 64-bit products masked to 32 bits)
    ux, uy = (sx & 0xFFFFFFFF).astype(np.uint32), (sy & 0xFFFFFFFF).astype(np.uint32)
    with np.errstate(over="ignore"):
        hsh = (ux * np.uint32(73856093)) ^ (uy * np.uint32(19349663)) ^ salt
        n = ((hsh * np.uint32(2654435761)) >> np.uint32(24)).astype(np.float32) / np.float32(255.0)
    fx, fy = sx.astype(np.float32), sy.astype(np.float32)
    r = 0.5 + 0.35 * np.sin(fx * 0.013 + ph[0]) * np.cos(fy * 0.017) + 0.1 * n
    g = 0.5 + 0.35 * np.cos(fx * 0.009 + 1.0 + ph[1]) * np.sin(fy * 0.021) + 0.1 * n
    b = 0.5 + 0.35 * np.sin((fx + fy) * 0.011 + ph[2]) + 0.1 * n
    byte = lambda v: (np.clip(v, 0.0, 1.0) * 255.0).astype(np.uint32)  # noqa: E731
    return (byte(r) | (byte(g) << 8) | (byte(b) << 16) | np.uint32(0xFF000000)).astype(np.uint32)


def pair_frames(w: int, h: int, seed: int, shift: int = 32) -> np.ndarray:
    """Frame pair `seed` of the batched workload, (2, h, w) RGBA8 words: a seeded texture (procedural_frame with
    seed + 1) and the same moved by a translation drawn uniformly from [-shift, shift] pixels per axis."""
    dx, dy = (int(v) for v in np.random.default_rng(1000 + seed).integers(-shift, shift + 1, 2))
    return np.stack([procedural_frame(w, h, 0, 0, seed + 1), procedural_frame(w, h, dx, dy, seed + 1)])


def conv_layer(weight_name: str) -> str:
    """The conv layer a weight tensor belongs to: "enc.e1.0.weight" -> "enc.e1", "coarse.head.weight" -> "coarse.head"."""
    for sfx in (".0.weight", ".weight"):
        if weight_name.endswith(sfx):
            return weight_name[:-len(sfx)]
    raise ValueError(f"not a conv weight: {weight_name}")


def weights_from_model(model, plan: Optional[dict] = None) -> dict:
    """The model's weights (fhmodel.Model, the manifest's f16 tensors) in make_weights' form: conv layer -> (w OIHW,
    bias, slope or None) as f16 bits, "film" -> (w1, b1, w2, b2) as f32 (model/blob.rs:32-41 decodes to f32). The
    layers are FlyHighFG's, or with a plan those of its conv steps (and the FiLM MLP where the model has one)."""
    W = {}
    if plan is None:
        layers = [(name, act, f"{name}.0.weight" if act else f"{name}.weight",
                   f"{name}.0.bias" if act else f"{name}.bias", f"{name}.1.weight" if act else None)
                  for name, (_, _, _, act) in CONVS.items()]
    else:
        layers = [(conv_layer(s["weight"]), s["act"], s["weight"], s["bias"], s["slope"])
                  for s in plan["steps"] if s["op"] == "conv"]
    for name, act, wn, bn, sn in layers:
        W[name] = (model.weight(wn), model.weight(bn), model.weight(sn) if act else None)
    f32 = lambda n: model.weight(n).view(np.float16).astype(np.float32)  # noqa: E731
    if plan is None or any(s["op"] == "film_mlp" for s in plan["steps"]):
        W["film"] = (f32("film.film.0.weight").reshape(-1), f32("film.film.0.bias"), f32("film.film.2.weight"),
                     f32("film.film.2.bias"))
    return W


class GraphProgram:
    """One pair() + mid(t) replayed from the static plan of fhc_model_plan (fhmodel.Model.plan): the graph walk of
    the reference's planner (net/build.rs:149-484) with its views, materialisations and peepholes, one backend call
    per plan step, on the backend interface FlyHighFG uses. Buffers are NHWC (1, h, w, c rounded up to 8). The
    frames are ``frames`` (2, h, w) RGBA8 words; the result is ``rgba`` (1, h, w). It runs the graph as the
    reference records it, without this library's fused chains and pairs, and so serves as the check of the
    hand-written frame program's wiring."""

    def __init__(self, be, plan: dict, cubic: bool = True, render_flags: int = 0):
        self.be, self.plan, self.cubic, self.render_flags = be, plan, cubic, render_flags
        # the plan's convs join the backend's table (a model other than FlyHighFG brings its own layers)
        for s in plan["steps"]:
            if s["op"] == "conv":
                name, shape = conv_layer(s["weight"]), (s["cin"], s["cout"], s["stride"], s["act"])
                if be.convs.setdefault(name, shape) != shape:
                    raise ValueError(f"{name}: the graph's conv {shape} differs from the program's "
                                     f"{be.convs[name]}")
        fw, fh = plan["frame"]
        self.frames, self.rgba = be.frames(2, fh, fw), be.frames(1, fh, fw)
        self.bufs = [be.zeros(1, b["h"], b["w"], pad8(b["c"])) for b in plan["buffers"]]
        self.named = {}
        for b, info in zip(self.bufs, plan["buffers"]):
            if info["name"]:
                self.named[info["name"]] = b  # the last buffer of a name (the graph rebinds carried names)

    def _v(self, v: dict) -> V:
        return V(self.bufs[v["buf"]], v["c0"], v["scale"])

    def run(self, t: float, W: dict, steps=None):
        """The plan's steps (or those of the index range `steps`) over the backend at phase t."""
        be, P = self.be, self.plan
        if "film" in W:
            be.set_g(film_mlp(W, t))
        for s in (P["steps"] if steps is None else [P["steps"][i] for i in steps]):
            op, ins, out = s["op"], [self._v(v) for v in s["in"]], self._v(s["out"])
            c = s["out"]["c"]
            ob = P["buffers"][s["out"]["buf"]]
            if op == "rgba_in":
                be.rgba_in(be.image(self.frames, s["frame"]), out, ob["h"], ob["w"])
            elif op == "rgba_out":
                be.rgba_out(ins[0], self.rgba)
            elif op == "interp":
                be.interp(ins[0], c, out, ob["h"], ob["w"], s["antialias"])
            elif op == "conv":
                name = conv_layer(s["weight"])
                res = None if s["residual"] is None else self._v(s["residual"])
                be.conv(name, ins[0], out, res)
            elif op == "mat":
                be.chcopy(ins[0], c, out)
            elif op == "concat":
                off = 0
                for v, iv in zip(ins, s["in"]):
                    be.chcopy(v, iv["c"], V(out.buf, out.c0 + off))
                    off += iv["c"]
            elif op == "avgpool":
                be.avgpool(ins[0], c, out, s["k"])
            elif op == "warp":
                be.warp(ins[0], c, ins[1], out)
            elif op == "binary":
                be.binary(ins[0], ins[1], c, out, s["fn"])
            elif op == "unary":
                if s["fn"] == 0:
                    be.unary(ins[0], c, out, 0, 2.0 * t if s["mode"] == "fwd" else 2.0 * (1.0 - t))
                elif s["fn"] == 2:
                    be.unary(ins[0], c, out, 2)
                else:
                    raise ValueError("the graph's clamp is not in this program")
            elif op == "luma":
                be.luma(ins[0], out)
            elif op == "luma_grad":
                be.luma(ins[0], out, grad=True)
            elif op == "sad":
                be.sad(ins[0], ins[1], out, s["radius"])
            elif op == "film_mlp":
                pass  # the FiLM vector: set on the backend above (the host computes it, net/build.rs:331-357)
            elif op == "film":
                be.film(ins[0], c, out)
            elif op == "convex":
                be.convex(ins[0], ins[1], c, out)
            elif op == "blendmix":
                be.blendmix(ins[0], ins[1], ins[2], out)
            elif op == "render":
                be.render(ins[0], ins[1], ins[2], ins[3], ins[4], out, self.cubic, self.render_flags, s["fsx"],
                          s["fsy"])
            elif op == "gmhs":
                be.gmhs(ins[0], ins[1], out, s["full_w"], s["level"])
            else:
                raise ValueError(f"plan step {op} has no backend call")
