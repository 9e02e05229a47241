"""Python host driver of the network ops between the convs (ctypes over include/fhc_ops.h in libfhconv.so).

One function per Gpu method of the reference (crates/flyhigh-engine/src/ops/network.rs, interp.rs, render.rs):
``warp``, ``luma``, ``sad`` (sad_volume), ``convex`` (convex_upsample after its conv), ``film``, ``blend``,
``blendmix``, ``avgpool``, ``interp``, and the elementwise ``binary`` (add / mul), ``unary`` (mul_t, affine_out,
clamp, neg) and ``chcopy`` (a scaled view into a concat slice). Inputs are torch NHWC f16 tensors on the GPU, or
``View`` objects that add the reference Tensor's channel offset and read scale (ops/tensor.rs); each function returns
a new dense output unless an ``out`` view is given (a concat slice is written in place). The module only passes
device pointers: when the library is missing, loading it raises, and nothing is computed on the host.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import fhconv
from fhconv import FhcError, _stream_handle


class FhcTensor(ctypes.Structure):
    _fields_ = [("p", ctypes.c_void_p), ("cstride", ctypes.c_uint32), ("c0", ctypes.c_uint32),
                ("scale", ctypes.c_float)]


class View:
    """Channels c0.. of an NHWC device tensor t of shape (n, h, w, cstride), read times `scale`."""

    def __init__(self, t, c0: int = 0, scale: float = 1.0):
        if t.dim() != 4 or not t.is_contiguous() or t.element_size() != 2:
            raise FhcError("a view needs a contiguous 4-d 16-bit NHWC tensor")
        self.t, self.c0, self.scale = t, c0, scale

    @property
    def shape(self):
        return tuple(self.t.shape)

    @property
    def channels(self):
        return self.t.shape[3] - self.c0

    def c_struct(self):
        return FhcTensor(self.t.data_ptr(), self.t.shape[3], self.c0, self.scale)


class GmhsPar(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("hc", "wc", "r_blk", "r_dwin")] + [
        (n, ctypes.c_float) for n in ("s", "dmin", "delta", "eps", "tex")] + [
        ("ws_bytes", ctypes.c_uint64), ("maps_offset", ctypes.c_uint64), ("dec_offset", ctypes.c_uint64)]


def _v(x) -> View:
    return x if isinstance(x, View) else View(x)


_typed = False


def _lib():
    global _typed
    L = fhconv.load()
    if not _typed:
        T, U, I, P = ctypes.POINTER(FhcTensor), ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p
        sig = {
            "fhc_warp": [T, T, T, U, U, U, U, P],
            "fhc_luma": [T, T, U, U, U, I, P],
            "fhc_sad_volume": [T, T, T, U, U, U, U, P],
            "fhc_convex_upsample": [T, T, T, U, U, U, U, P],
            "fhc_film_modulate": [T, P, T, U, U, U, U, P],
            "fhc_blend_weights": [T, T, U, U, U, P],
            "fhc_blendmix": [T, T, T, T, U, U, U, P],
            "fhc_avgpool": [T, T, U, U, U, U, U, P],
            "fhc_interpolate": [T, T, U, U, U, U, U, U, I, P],
            "fhc_binary": [T, T, T, U, U, U, U, U, I, P],
            "fhc_unary": [T, T, U, U, U, U, I, ctypes.c_float, ctypes.c_float, P],
            "fhc_chcopy": [T, T, U, U, U, U, P],
            "fhc_pair_pyramid": [T, T, T, T, U, U, P],
            "fhc_pair_input": [T, T, T, T, T, U, U, U, U, P],
            "fhc_pair_input_n": [T, T, T, T, T, U, U, U, U, U, P],
            "fhc_render": [T, T, T, T, T, T, U, U, U, U, ctypes.c_float, ctypes.c_float, I, U, P],
            "fhc_fold_pair": [T, T, T, U, U, U, P],
            "fhc_fold_pair_sad": [T, T, T, U, U, U, T, T, T, U, U, U, U, P],
            "fhc_fold_pair_sad_n": [T, T, T, U, U, U, U, T, T, T, U, U, U, U, P],
            "fhc_coarse_up": [T, T, T, U, U, U, U, ctypes.c_float, P],
            "fhc_fine_input": [T, T, T, T, T, U, U, U, P],
            "fhc_flow_vis_t": [T, T, T, U, U, U, ctypes.c_float, P],
            "fhc_coarse_fine_input": [T, T, T, U, U, ctypes.c_float, T, T, ctypes.c_float, T, T, U, U, U, P],
            "fhc_coarse_fine_input_n": [T, T, T, U, U, ctypes.c_float, T, T, ctypes.c_float, T, T, U, U, U, U, P],
            "fhc_coarse_fine_input_sad_n": [T, T, T, U, U, ctypes.c_float, T, T, ctypes.c_float, T, T, U, U, U, U, T,
                                            U, P],
            "fhc_flow_vis_t_convex": [T, T, T, ctypes.c_float, T, U, U, U, P],
            "fhc_refine_input": [T, T, T, T, U, U, ctypes.c_float, P],
            "fhc_refine_input_n": [T, T, T, T, U, U, ctypes.c_float, U, U, P],
            "fhc_rgba_in": [P, U, U, U, U, ctypes.c_uint64, T, U, U, P],
            "fhc_rgba_out": [T, U, U, U, P, U, U, U, ctypes.c_uint64, P],
            "fhc_rgba_resize": [P, U, U, U, U, ctypes.c_uint64, U, U, T, U, U, P],
            "fhc_render_rgba": [P, P, U, U, U, U, U, T, T, T, U, U, ctypes.c_float, ctypes.c_float, I, U, P, U,
                                P],
            "fhc_render_rgba_n": [P, U, U, U, U, U, ctypes.c_uint64, U, U, T, T, T, U, U, ctypes.c_float,
                                  ctypes.c_float, I, U, P, U, ctypes.c_uint64, P],
            "fhc_gmhs_params": [U, U, U, U, ctypes.POINTER(GmhsPar)],
            "fhc_flow_vis_t_convex_n": [T, T, T, P, U, T, U, U, U, P],
            "fhc_mid_input_n": [T, T, T, P, U, T, T, T, U, U, U, ctypes.c_float, ctypes.c_float, P],
            "fhc_gmhs": [T, T, U, U, T, U, U, U, U, P, ctypes.c_size_t, P],
            "fhc_gmhs_n": [T, T, U, U, T, U, U, U, U, U, P, ctypes.c_size_t, P],
            "fhc_gmhs_film": [T, T, U, U, T, U, U, U, U, P, ctypes.c_size_t, P, P, P, P, P, P, P, P],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = ctypes.c_int
        _typed = True
    return L


def _out(out, like: View, n, h, w, c) -> View:
    if out is not None:
        return _v(out)
    import torch
    return View(torch.empty((n, h, w, c), dtype=like.t.dtype, device=like.t.device))


def _run(name, rc):
    if rc < 0:
        raise FhcError(f"{name}: {fhconv.last_error()}")


def _ref(v: View):
    return ctypes.byref(v.c_struct())


def warp(img, flow, c: Optional[int] = None, out=None, stream=None):
    """out[p] = img[p + flow[p]] (bilinear, border clamp); flow channels c0, c0 + 1 are x, y in pixels."""
    img, flow = _v(img), _v(flow)
    n, h, w, _ = img.shape
    c = img.channels if c is None else c
    o = _out(out, img, n, h, w, c)
    _run("warp", _lib().fhc_warp(_ref(img), _ref(flow), _ref(o), n, h, w, c, _stream_handle(stream)))
    return o.t


def luma(x, grad: bool = False, out=None, stream=None):
    x = _v(x)
    n, h, w, _ = x.shape
    o = _out(out, x, n, h, w, 1)
    _run("luma", _lib().fhc_luma(_ref(x), _ref(o), n, h, w, int(grad), _stream_handle(stream)))
    return o.t


def sad(la, lb, radius: int, out=None, stream=None):
    la, lb = _v(la), _v(lb)
    n, h, w, _ = la.shape
    o = _out(out, la, n, h, w, (2 * radius + 1) ** 2)
    _run("sad_volume", _lib().fhc_sad_volume(_ref(la), _ref(lb), _ref(o), n, h, w, radius, _stream_handle(stream)))
    return o.t


def convex(wt, x, c: Optional[int] = None, out=None, stream=None):
    wt, x = _v(wt), _v(x)
    n, h, w, _ = x.shape
    c = x.channels if c is None else c
    o = _out(out, x, n, 2 * h, 2 * w, c)
    _run("convex_upsample",
         _lib().fhc_convex_upsample(_ref(wt), _ref(x), _ref(o), n, h, w, c, _stream_handle(stream)))
    return o.t


def film(hv, g, c: Optional[int] = None, out=None, stream=None):
    """g: a contiguous device tensor of n * 2c f16 values (one FiLM vector per image)."""
    hv = _v(hv)
    n, h, w, _ = hv.shape
    c = hv.channels if c is None else c
    if not g.is_contiguous() or g.numel() != n * 2 * c or g.element_size() != 2:
        raise FhcError(f"film: g needs {n * 2 * c} contiguous f16 values")
    o = _out(out, hv, n, h, w, c)
    _run("film_modulate",
         _lib().fhc_film_modulate(_ref(hv), g.data_ptr(), _ref(o), n, h, w, c, _stream_handle(stream)))
    return o.t


def blend(vis, out=None, stream=None):
    vis = _v(vis)
    n, h, w, _ = vis.shape
    o = _out(out, vis, n, h, w, 2)
    _run("blend_weights", _lib().fhc_blend_weights(_ref(vis), _ref(o), n, h, w, _stream_handle(stream)))
    return o.t


def blendmix(wa, wb, vis, out=None, stream=None):
    wa, wb, vis = _v(wa), _v(wb), _v(vis)
    n, h, w, _ = vis.shape
    o = _out(out, vis, n, h, w, 3)
    _run("blendmix", _lib().fhc_blendmix(_ref(wa), _ref(wb), _ref(vis), _ref(o), n, h, w, _stream_handle(stream)))
    return o.t


def avgpool(x, k: int, c: Optional[int] = None, out=None, stream=None):
    x = _v(x)
    n, h, w, _ = x.shape
    c = x.channels if c is None else c
    o = _out(out, x, n, h // max(k, 1), w // max(k, 1), c)
    _run("avgpool", _lib().fhc_avgpool(_ref(x), _ref(o), n, h, w, c, k, _stream_handle(stream)))
    return o.t


def interp(x, oh: int, ow: int, antialias: bool = False, c: Optional[int] = None, out=None, stream=None):
    x = _v(x)
    n, ih, iw, _ = x.shape
    c = x.channels if c is None else c
    o = _out(out, x, n, oh, ow, c)
    _run("interpolate",
         _lib().fhc_interpolate(_ref(x), _ref(o), n, c, ih, iw, oh, ow, int(antialias), _stream_handle(stream)))
    return o.t


def binary(a, b, op: int = 0, c: Optional[int] = None, out=None, stream=None):
    """op 0: a * sa + b * sb; op 1: (a * sa) * (b * sb); b with one channel broadcasts."""
    a, b = _v(a), _v(b)
    n, h, w, _ = a.shape
    c = a.channels if c is None else c
    cb = 1 if b.channels == 1 else c
    o = _out(out, a, n, h, w, c)
    _run("binary", _lib().fhc_binary(_ref(a), _ref(b), _ref(o), n, h, w, c, cb, op, _stream_handle(stream)))
    return o.t


def unary(x, op: int, a: float = 0.0, b: float = 0.0, c: Optional[int] = None, out=None, stream=None):
    x = _v(x)
    n, h, w, _ = x.shape
    c = x.channels if c is None else c
    o = _out(out, x, n, h, w, c)
    _run("unary", _lib().fhc_unary(_ref(x), _ref(o), n, h, w, c, op, a, b, _stream_handle(stream)))
    return o.t


def chcopy(x, c: Optional[int] = None, out=None, stream=None):
    x = _v(x)
    n, h, w, _ = x.shape
    c = x.channels if c is None else c
    o = _out(out, x, n, h, w, c)
    _run("chcopy", _lib().fhc_chcopy(_ref(x), _ref(o), n, h, w, c, _stream_handle(stream)))
    return o.t


# ---- the graph's op chains, fused (include/fhc_ops.h); outputs are views into the caller's buffers ----------------

def pair_pyramid(q, i8, i16, l16, stream=None):
    q = _v(q)
    _, h, w, _ = q.shape
    _run("pair_pyramid", _lib().fhc_pair_pyramid(_ref(q), _ref(_v(i8)), _ref(_v(i16)), _ref(_v(l16)), h, w,
                                                 _stream_handle(stream)))


def fine_input(f8, i8, flow, fx, l8, c, stream=None):
    f8 = _v(f8)
    _, h, w, _ = f8.shape
    _run("fine_input", _lib().fhc_fine_input(_ref(f8), _ref(_v(i8)), _ref(_v(flow)), _ref(_v(fx)), _ref(_v(l8)),
                                             h, w, c, _stream_handle(stream)))


def flow_vis_t(fv, dfilm, out, t, stream=None):
    fv = _v(fv)
    n, h, w, _ = fv.shape
    _run("flow_vis_t", _lib().fhc_flow_vis_t(_ref(fv), _ref(_v(dfilm)), _ref(_v(out)), n, h, w, t,
                                             _stream_handle(stream)))


def coarse_fine_input(o, fv, state, flow_scale, f8, i8, fine_scale, fx, l8, c, stream=None):
    """coarse_up(o, fv, state, ...) to f8's grid, then fine_input(f8, i8, (fv, fine_scale), fx, l8, c): one launch
    for every pair (pair k: image k of o, fv, state, fx, l8; images 2k, 2k + 1 of f8 and i8)."""
    o, f8 = _v(o), _v(f8)
    pairs, hi, wi, _ = o.shape
    n2, h, w, _ = f8.shape
    if n2 != 2 * pairs:
        raise FhcError(f"coarse_fine_input: {n2} feature maps for {pairs} pairs")
    _run("coarse_fine_input",
         _lib().fhc_coarse_fine_input_n(_ref(o), _ref(_v(fv)), None if state is None else _ref(_v(state)), hi, wi,
                                        flow_scale, _ref(f8), _ref(_v(i8)), fine_scale, _ref(_v(fx)), _ref(_v(l8)),
                                        h, w, c, pairs, _stream_handle(stream)))


def coarse_fine_input_sad(o, fv, state, flow_scale, f8, i8, fine_scale, fx, l8, c, sad_out, radius, stream=None):
    """coarse_fine_input(...), then sad_volume(l8 channel 0, l8 channel 1, sad_out, radius) for every pair, in one
    launch (pair k's volume: image k of sad_out)."""
    o, f8 = _v(o), _v(f8)
    pairs, hi, wi, _ = o.shape
    n2, h, w, _ = f8.shape
    if n2 != 2 * pairs:
        raise FhcError(f"coarse_fine_input_sad: {n2} feature maps for {pairs} pairs")
    _run("coarse_fine_input_sad",
         _lib().fhc_coarse_fine_input_sad_n(_ref(o), _ref(_v(fv)), None if state is None else _ref(_v(state)), hi, wi,
                                            flow_scale, _ref(f8), _ref(_v(i8)), fine_scale, _ref(_v(fx)),
                                            _ref(_v(l8)), h, w, c, pairs, _ref(_v(sad_out)), radius,
                                            _stream_handle(stream)))


def flow_vis_t_convex(wt, fv, dfilm, t, out, stream=None):
    """flow_vis_t(fv, dfilm, ., t) then convex(wt, ., 7, out), the intermediate never stored: one launch. t: one
    phase, or a sequence of phases (dfilm and out then hold phase j of pair p at image j * n + p, n = fv's images)."""
    fv = _v(fv)
    n, h, w, _ = fv.shape
    ts = [float(t)] if isinstance(t, (int, float)) else [float(x) for x in t]
    arr = (ctypes.c_float * len(ts))(*ts)
    _run("flow_vis_t_convex", _lib().fhc_flow_vis_t_convex_n(_ref(_v(wt)), _ref(fv), _ref(_v(dfilm)), arr, len(ts),
                                                             _ref(_v(out)), n, h, w, _stream_handle(stream)))


def mid_input(wt, fv, dfilm, t, up, q, rx, flow_scale, flow_out_scale, stream=None):
    """flow_vis_t_convex(wt, fv, dfilm, t, up) then refine_input(q, (up, flow_scale), (up + 4), rx, flow_out_scale,
    qmod=n) in one launch (n = fv's images; t one phase or a sequence, up and rx holding phase j of pair p at image
    j * n + p)."""
    fv = _v(fv)
    n, h, w, _ = fv.shape
    ts = [float(t)] if isinstance(t, (int, float)) else [float(x) for x in t]
    arr = (ctypes.c_float * len(ts))(*ts)
    _run("mid_input", _lib().fhc_mid_input_n(_ref(_v(wt)), _ref(fv), _ref(_v(dfilm)), arr, len(ts), _ref(_v(up)),
                                             _ref(_v(q)), _ref(_v(rx)), n, h, w, flow_scale, flow_out_scale,
                                             _stream_handle(stream)))


def refine_input(q, flow, vis, rx, flow_out_scale, qmod=None, stream=None):
    """refine_input over every image of flow (n of them): image i's pictures are pair i % qmod of q (default: q's
    pairs, 2 images each)."""
    flow, q = _v(flow), _v(q)
    n, h, w, _ = flow.shape
    qmod = q.shape[0] // 2 if qmod is None else qmod
    _run("refine_input", _lib().fhc_refine_input_n(_ref(q), _ref(flow), _ref(_v(vis)), _ref(_v(rx)), h, w,
                                                   flow_out_scale, n, qmod, _stream_handle(stream)))


def pair_input(ab, q, i8, i16, l16, oh, ow, stream=None):
    """The pictures' resize and pyramid for every pair of ab (pair k: images 2k, 2k + 1 of ab, q and i8, image k of
    i16 and l16)."""
    ab = _v(ab)
    n2, ih, iw, _ = ab.shape
    if n2 % 2:
        raise FhcError(f"pair_input: {n2} pictures are no whole pairs")
    _run("pair_input", _lib().fhc_pair_input_n(_ref(ab), _ref(_v(q)), _ref(_v(i8)), _ref(_v(i16)), _ref(_v(l16)),
                                               ih, iw, oh, ow, n2 // 2, _stream_handle(stream)))


def render(a, b, flow, vis, rt, cubic=True, flags=0, fsx=1.0, fsy=1.0, out=None, stream=None):
    """render_pix: a, b at full size; flow (4), vis (3), rt (3) at quarter size; returns / writes 3 channels."""
    a, b, flow, vis, rt = _v(a), _v(b), _v(flow), _v(vis), _v(rt)
    _, h, w, _ = a.shape
    _, hq, wq, _ = flow.shape
    o = _out(out, a, 1, h, w, 3)
    _run("render", _lib().fhc_render(_ref(a), _ref(b), _ref(flow), _ref(vis), _ref(rt), _ref(o), h, w, hq, wq, fsx,
                                     fsy, int(cubic), flags, _stream_handle(stream)))
    return o.t


def fold_pair(x, out, also=None, stream=None, c=None):
    """Images 0 and 1 of x (2, h, w, c) side by side into out's channels (out.c0, out.c0 + c); image 1 also into
    `also` when given. c defaults to the channels of x's view."""
    x = _v(x)
    _, h, w, _ = x.shape
    c = x.channels if c is None else c
    _run("fold_pair", _lib().fhc_fold_pair(_ref(x), _ref(_v(out)), None if also is None else _ref(_v(also)), h, w, c,
                                           _stream_handle(stream)))


def fold_pair_sad(x, out, also, la, lb, sad_out, radius, stream=None, c=None):
    """fold_pair(x, out, also, c=c) of every pair of x (pair k: images 2k, 2k + 1, folded into image k of out and
    also) and sad(la, lb, radius, out=sad_out), which touch none of each other's tensors, in one launch."""
    x, la = _v(x), _v(la)
    n2, h, w, _ = x.shape
    n, sh, sw, _ = la.shape
    c = x.channels if c is None else c
    if n2 % 2:
        raise FhcError(f"fold_pair_sad: {n2} maps are no whole pairs")
    _run("fold_pair_sad",
         _lib().fhc_fold_pair_sad_n(_ref(x), _ref(_v(out)), None if also is None else _ref(_v(also)), h, w, c,
                                    n2 // 2, _ref(la), _ref(_v(lb)), _ref(_v(sad_out)), n, sh, sw, radius,
                                    _stream_handle(stream)))


def coarse_up(o, out, state, oh, ow, flow_scale, stream=None):
    o = _v(o)
    _, hi, wi, _ = o.shape
    _run("coarse_up", _lib().fhc_coarse_up(_ref(o), _ref(_v(out)), None if state is None else _ref(_v(state)), hi,
                                           wi, oh, ow, flow_scale, _stream_handle(stream)))


# ---- the host's 8-bit frames (rgba_in.wgsl, rgba_out.wgsl; the Session's first and last steps, net/session.rs:56-63)
# A batch of frames is a contiguous (n, h, w) int32 / uint32 device tensor of RGBA8 words (R | G << 8 | B << 16 |
# A << 24); the padded size (hp, wp) is the frame's rounded up to 32 (the reference's working size).

def _frames(f):
    if f.dim() != 3 or not f.is_contiguous() or f.element_size() != 4:
        raise FhcError("frames must be a contiguous (n, h, w) tensor of 32-bit RGBA8 words")
    return f.shape


def rgba_in(frames, hp: int, wp: int, out=None, stream=None):
    """frames (n, h, w) -> BGR f16 (n, hp, wp, 4) (or into `out`: channels c0..c0+2; channel 3 of a 4-channel
    pixel view written 0)."""
    n, h, w = _frames(frames)
    o = View(_pixels_like(frames, n, hp, wp)) if out is None else _v(out)
    _run("rgba_in", _lib().fhc_rgba_in(frames.data_ptr(), n, w, h, w, h * w, _ref(o), hp, wp, _stream_handle(stream)))
    return o.t


def _pixels_like(t, n, h, w):
    import torch
    return torch.empty((n, h, w, 4), dtype=torch.int16, device=t.device)


def rgba_out(x, h: int, w: int, out=None, stream=None):
    """x: (n, hp, wp, cs) BGR f16 (view channels c0..c0+2) -> (n, h, w) int32 RGBA8 words, cropped, alpha 255."""
    import torch
    x = _v(x)
    n, hp, wp, _ = x.shape
    o = torch.empty((n, h, w), dtype=torch.int32, device=x.t.device) if out is None else out
    _frames(o)
    _run("rgba_out", _lib().fhc_rgba_out(_ref(x), n, hp, wp, o.data_ptr(), w, h, w, h * w, _stream_handle(stream)))
    return o


def rgba_resize(frames, hp: int, wp: int, oh: int, ow: int, out=None, stream=None):
    """rgba_in of the frames at the padded size hp x wp, then the antialiased resize to oh x ow, in one launch:
    (n, oh, ow, 4) BGR f16 with channel 3 zero."""
    n, h, w = _frames(frames)
    o = View(_pixels_like(frames, n, oh, ow)) if out is None else _v(out)
    _run("rgba_resize", _lib().fhc_rgba_resize(frames.data_ptr(), n, w, h, w, h * w, hp, wp, _ref(o), oh, ow,
                                               _stream_handle(stream)))
    return o.t


def render_rgba(fa, fb, flow, vis, rt, hp: int, wp: int, cubic=True, flags=0, fsx=1.0, fsy=1.0, out=None,
                stream=None):
    """render_pix of the padded frames (hp x wp) sampled from the RGBA8 frames fa, fb ((1, h, w) each) with the
    quarter maps flow (4), vis (3), rt (3), written as RGBA8 (1, h, w): rgba_in, render, rgba_out in one launch."""
    import torch
    _, h, w = _frames(fa)
    _frames(fb)
    flow, vis, rt = _v(flow), _v(vis), _v(rt)
    _, hq, wq, _ = flow.shape
    o = torch.empty((1, h, w), dtype=torch.int32, device=fa.device) if out is None else out
    _run("render_rgba", _lib().fhc_render_rgba(fa.data_ptr(), fb.data_ptr(), w, h, w, hp, wp, _ref(flow), _ref(vis),
                                               _ref(rt), hq, wq, fsx, fsy, int(cubic), flags, o.data_ptr(), w,
                                               _stream_handle(stream)))
    return o


def render_rgba_n(frames, flow, vis, rt, hp: int, wp: int, phases: int, cubic=True, flags=0, fsx=1.0, fsy=1.0,
                  out=None, stream=None):
    """render_rgba of every pair of frames ((2P, h, w): A, B of pair p at 2p, 2p + 1) at `phases` phases, pair-major,
    in one launch: phase j of pair p from maps image j * P + p, into frame j * P + p of out ((phases * P, h, w))."""
    import torch
    n2, h, w = _frames(frames)
    if n2 % 2:
        raise FhcError(f"render_rgba_n: {n2} frames are no whole pairs")
    flow, vis, rt = _v(flow), _v(vis), _v(rt)
    _, hq, wq, _ = flow.shape
    P = n2 // 2
    o = torch.empty((phases * P, h, w), dtype=torch.int32, device=frames.device) if out is None else out
    _run("render_rgba", _lib().fhc_render_rgba_n(frames.data_ptr(), P, phases, w, h, w, h * w, hp, wp, _ref(flow),
                                                 _ref(vis), _ref(rt), hq, wq, fsx, fsy, int(cubic), flags,
                                                 o.data_ptr(), w, h * w, _stream_handle(stream)))
    return o


def gmhs_params(h: int, w: int, full_w: int, level: int = 1) -> dict:
    """The periodic-structure repair's grid, radii, thresholds and workspace for an h x w network of frames padded
    to full_w columns (fhc_gmhs_params)."""
    p = GmhsPar()
    _run("gmhs_params", _lib().fhc_gmhs_params(h, w, full_w, level, ctypes.byref(p)))
    return {n: getattr(p, n) for n, _ in GmhsPar._fields_}


def gmhs_workspace(h: int, w: int, full_w: int, level: int = 1, device="cuda", pairs: int = 1):
    """A workspace for fhc_gmhs (uint8, 256-byte aligned as torch's allocator aligns), or for fhc_gmhs_n over
    `pairs` pairs (pair k's at k * gmhs_ws_stride(...) bytes)."""
    import torch
    nb = gmhs_params(h, w, full_w, level)["ws_bytes"]
    return torch.empty((pairs - 1) * ((nb + 255) // 256 * 256) + nb, dtype=torch.uint8, device=device)


def gmhs_ws_stride(h: int, w: int, full_w: int, level: int = 1) -> int:
    """The bytes between two pairs' workspaces in fhc_gmhs_n's."""
    return (gmhs_params(h, w, full_w, level)["ws_bytes"] + 255) // 256 * 256


def gmhs(a, b, flow, full_w: int, level: int = 1, ws=None, stream=None):
    """The repair of flow channels c0 .. c0 + 3 (the E8 flow) in place, from the network pictures a, b (BGR). Returns
    the workspace: the coefficients and decision maps are gmhs_results(ws, ...)."""
    a, b, flow = _v(a), _v(b), _v(flow)
    _, h, w, _ = a.shape
    _, h8, w8, _ = flow.shape
    if ws is None:
        ws = gmhs_workspace(h, w, full_w, max(level, 1), a.t.device)
    _run("gmhs", _lib().fhc_gmhs(_ref(a), _ref(b), h, w, _ref(flow), h8, w8, full_w, level, ws.data_ptr(),
                                 ws.numel() * ws.element_size(), _stream_handle(stream)))
    return ws


def gmhs_n(ab, flow, full_w: int, level: int = 1, ws=None, stream=None):
    """The repair of every pair at once (fhc_gmhs_n): pair k's pictures are images 2k, 2k + 1 of ab (BGR), its E8
    flow image k of flow (channels c0 .. c0 + 3, repaired in place). Returns the workspace (pair k's at k *
    gmhs_ws_stride(...) bytes)."""
    ab, flow = _v(ab), _v(flow)
    n2, h, w, _ = ab.shape
    n, h8, w8, _ = flow.shape
    if n2 != 2 * n:
        raise FhcError(f"gmhs_n: {n2} pictures for {n} flows")
    if ws is None:
        ws = gmhs_workspace(h, w, full_w, max(level, 1), ab.t.device, n)
    a, b = View(ab.t[0:1], ab.c0, ab.scale), View(ab.t[1:2], ab.c0, ab.scale)
    _run("gmhs_n", _lib().fhc_gmhs_n(_ref(a), _ref(b), h, w, _ref(flow), h8, w8, full_w, level, n, ws.data_ptr(),
                                     ws.numel() * ws.element_size(), _stream_handle(stream)))
    return ws


def gmhs_film(a, b, flow, full_w: int, level, ws, pair, pair_x, pair_film, pair_y, conv=None, conv_x=None,
              conv_y=None, stream=None):
    """gmhs(a, b, flow, ...), pair.run_film(pair_x, pair_film, pair_y) (a fhconv.ConvPairPlan made with film_in) and
    conv.run(conv_x, conv_y) (a fhconv.ConvPlan, optional): the pair's workgroups inside the repair's first launch,
    the conv's inside the second (fhc_gmhs_film)."""
    a, b, flow = _v(a), _v(b), _v(flow)
    _, h, w, _ = a.shape
    _, h8, w8, _ = flow.shape
    d = pair.desc
    if not pair_film.is_contiguous() or pair_film.numel() != d.n * 2 * d.cin or pair_film.element_size() != 2:
        raise FhcError(f"gmhs_film: the FiLM vectors need {d.n * 2 * d.cin} contiguous f16 values")
    _run("gmhs_film",
         _lib().fhc_gmhs_film(_ref(a), _ref(b), h, w, _ref(flow), h8, w8, full_w, level, ws.data_ptr(),
                              ws.numel() * ws.element_size(), pair._h, pair_x.data_ptr(), pair_film.data_ptr(),
                              pair_y.data_ptr(), None if conv is None else conv._h,
                              None if conv_x is None else conv_x.data_ptr(),
                              None if conv_y is None else conv_y.data_ptr(), _stream_handle(stream)))
    return ws


def gmhs_results(ws, h: int, w: int, full_w: int, level: int = 1, h8: int = None, w8: int = None):
    """(coefficients (4, 4), the cost maps after the texture window (5, hc, wc), the values each E8 cell decided on
    (5, h8, w8)) as float32 device views of a workspace after gmhs of an h8 x w8 flow (default: h // 8, w // 8)."""
    p = gmhs_params(h, w, full_w, level)
    h8 = h // 8 if h8 is None else h8
    w8 = w // 8 if w8 is None else w8
    import torch
    f = ws.view(torch.float32)
    off, doff = p["maps_offset"] // 4, p["dec_offset"] // 4
    return (f[:16].view(4, 4), f[off:off + 5 * p["hc"] * p["wc"]].view(5, p["hc"], p["wc"]),
            f[doff:doff + 5 * h8 * w8].view(5, h8, w8))
