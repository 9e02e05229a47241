"""ctypes front end of the CPU oracle (fh_oracle.c): TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import this module, as the checker.
The product never imports it.

Arrays are numpy uint16 holding f16 bit patterns. Tensors are NHWC with a pixel stride (``*_cstride``) and a
channel offset (``*_c0``); weights are the reference's OIHW ``[cout][cin][kh][kw]``
(crates/flyhigh-engine/src/model/blob.rs:32-41).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfhoracle.so")

ORDER_TILED, ORDER_NAIVE, ORDER_SPLITK = 0, 1, 2


class FhoConv(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "n", "h", "w", "cin", "cout", "kh", "kw", "stride", "pad",
        "x_cstride", "x_c0", "y_cstride", "y_c0", "r_cstride", "r_c0", "act")] + [
        ("alpha", ctypes.c_float), ("residual", ctypes.c_uint32)]


_lib = None


def build():
    subprocess.run(["make", "-s", "-B", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        L.fho_conv_run.argtypes = [ctypes.POINTER(FhoConv), P, P, P, P, P, P, ctypes.c_int, ctypes.c_uint32]
        L.fho_conv_run.restype = ctypes.c_int
        L.fho_conv_run_mt.argtypes = [ctypes.POINTER(FhoConv), P, P, P, P, P, P, ctypes.c_int]
        L.fho_conv_run_mt.restype = ctypes.c_int
        L.fho_f32_to_f16.argtypes = [ctypes.c_float]
        L.fho_f32_to_f16.restype = ctypes.c_uint16
        L.fho_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.fho_f16_to_f32.restype = ctypes.c_float
        L.fho_f32_to_f16_n.argtypes = [P, P, ctypes.c_size_t]
        L.fho_f32_to_f16_n.restype = None
        L.fho_f16_to_f32_n.argtypes = [P, P, ctypes.c_size_t]
        L.fho_f16_to_f32_n.restype = None
        L.fho_out_size.argtypes = [ctypes.c_uint32] * 4
        L.fho_out_size.restype = ctypes.c_uint32
        _lib = L
    return _lib


def out_size(n, k, s, p):
    return (n + 2 * p - k) // s + 1


def make_desc(n, h, w, cin, cout, k=3, stride=1, pad=None, act=1, alpha=0.0, residual=False,
              x_cstride=None, x_c0=0, y_cstride=None, y_c0=0, r_cstride=None, r_c0=0):
    if pad is None:
        pad = 1 if k == 3 else 0
    return dict(n=n, h=h, w=w, cin=cin, cout=cout, kh=k, kw=k, stride=stride, pad=pad,
                x_cstride=x_cstride or cin, x_c0=x_c0, y_cstride=y_cstride or cout, y_c0=y_c0,
                r_cstride=r_cstride or cout, r_c0=r_c0, act=act, alpha=alpha, residual=int(bool(residual)))


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _struct(d):
    s = FhoConv()
    for k, v in d.items():
        setattr(s, k, v)
    return s


def conv(d, x, w, bias, slope=None, res=None, y=None, order=ORDER_TILED, ksplit=1, threads=0):
    """Runs the oracle conv; returns y (uint16 f16 bits, NHWC with y_cstride)."""
    if d["stride"] < 1 or d["kh"] < 1 or d["kw"] < 1:
        raise ValueError("oracle rejected the conv descriptor")
    hout = out_size(d["h"], d["kh"], d["stride"], d["pad"])
    wout = out_size(d["w"], d["kw"], d["stride"], d["pad"])
    arrs = [np.ascontiguousarray(a, dtype=np.uint16) if a is not None else None for a in (x, w, bias, slope, res)]
    if y is None:
        y = np.zeros(d["n"] * hout * wout * d["y_cstride"], dtype=np.uint16)
    s = _struct(d)
    if threads:
        rc = lib().fho_conv_run_mt(ctypes.byref(s), *[_ptr(a) for a in arrs], _ptr(y), threads)
    else:
        rc = lib().fho_conv_run(ctypes.byref(s), *[_ptr(a) for a in arrs], _ptr(y), order, ksplit)
    if rc != 0:
        raise ValueError("oracle rejected the conv descriptor")
    return y


def f32_to_f16(a):
    """float32 array -> uint16 f16 bits (round to nearest even)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().fho_f32_to_f16_n(_ptr(a), _ptr(out), a.size)
    return out


def f16_to_f32(a):
    """uint16 f16 bits -> float32 array (exact)."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().fho_f16_to_f32_n(_ptr(a), _ptr(out), a.size)
    return out


# ---- the network ops around the convs (fh_ops_oracle.c) --------------------------------------------------------
# Inputs are uint16 arrays (n, h, w, cs) of f16 bits read through a view (channel offset c0, read scale); outputs
# are new dense (n, oh, ow, c) arrays.

class FhoView(ctypes.Structure):
    _fields_ = [("p", ctypes.c_void_p), ("cs", ctypes.c_uint32), ("c0", ctypes.c_uint32), ("scale", ctypes.c_float)]


class FhoGmPar(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("hc", "wc", "r_blk", "r_dwin")] + [
        (n, ctypes.c_float) for n in ("s", "dmin", "delta", "eps", "tex")]


def _view(a, c0=0, scale=1.0):
    assert a.dtype == np.uint16 and a.ndim == 4 and a.flags.c_contiguous
    return ctypes.byref(FhoView(a.ctypes.data, a.shape[3], c0, scale))


def _ops_lib():
    L = lib()
    if not getattr(L, "_ops_typed", False):
        V, U, I = ctypes.POINTER(FhoView), ctypes.c_uint32, ctypes.c_int
        sig = {
            "fho_warp": [V, V, V, U, U, U, U],
            "fho_luma": [V, V, U, U, U, I],
            "fho_sad": [V, V, V, U, U, U, U],
            "fho_convex": [V, V, V, U, U, U, U],
            "fho_film": [V, ctypes.c_void_p, V, U, U, U, U],
            "fho_blend": [V, V, U, U, U],
            "fho_blendmix": [V, V, V, V, U, U, U],
            "fho_avgpool": [V, V, U, U, U, U, U],
            "fho_interp": [V, V, U, U, U, U, U, U, I],
            "fho_binary": [V, V, V, U, U, U, U, U, I],
            "fho_unary": [V, V, U, U, U, U, I, ctypes.c_float, ctypes.c_float],
            "fho_chcopy": [V, V, U, U, U, U],
            "fho_render": [V, V, V, V, V, V, U, U, U, U, ctypes.c_float, ctypes.c_float, I, U],
            "fho_render_rows": [V, V, V, V, V, V, U, U, U, U, ctypes.c_float, ctypes.c_float, I, U, U, U],
            "fho_rgba_in": [ctypes.c_void_p, U, U, U, U, ctypes.c_uint64, V, U, U],
            "fho_rgba_out": [V, U, U, U, ctypes.c_void_p, U, U, U, ctypes.c_uint64],
            "fho_gm_params": [U, U, U, U, ctypes.POINTER(FhoGmPar)],
            "fho_gm_fit": [V, U, U, ctypes.c_float, U, ctypes.c_void_p],
            "fho_gm_cost": [V, V, U, U, V, U, U, ctypes.c_void_p, U, U, ctypes.c_void_p],
            "fho_gm_box": [ctypes.c_void_p, ctypes.c_void_p, U, U, U, U, I],
            "fho_gm_select": [ctypes.c_void_p, ctypes.c_void_p, V, U, U, U, U, ctypes.c_float, ctypes.c_float,
                              ctypes.c_float],
            "fho_gmhs": [V, V, U, U, V, U, U, U, U, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
        }
        for name, args in sig.items():
            f = getattr(L, name)
            f.argtypes = args
            f.restype = None
        L._ops_typed = True
    return L


def _out(n, h, w, c):
    return np.zeros((n, h, w, c), np.uint16)


def warp(img, flow, c, img_c0=0, img_scale=1.0, flow_c0=0, flow_scale=1.0):
    n, h, w, _ = img.shape
    y = _out(n, h, w, c)
    _ops_lib().fho_warp(_view(img, img_c0, img_scale), _view(flow, flow_c0, flow_scale), _view(y), n, h, w, c)
    return y


def luma(x, grad=False, c0=0, scale=1.0):
    n, h, w, _ = x.shape
    y = _out(n, h, w, 1)
    _ops_lib().fho_luma(_view(x, c0, scale), _view(y), n, h, w, int(grad))
    return y


def sad(la, lb, r, la_c0=0, lb_c0=0):
    n, h, w, _ = la.shape
    y = _out(n, h, w, (2 * r + 1) ** 2)
    _ops_lib().fho_sad(_view(la, la_c0), _view(lb, lb_c0), _view(y), n, h, w, r)
    return y


def convex(wt, x, c, wt_c0=0, x_c0=0):
    n, h, w, _ = x.shape
    y = _out(n, 2 * h, 2 * w, c)
    _ops_lib().fho_convex(_view(wt, wt_c0), _view(x, x_c0), _view(y), n, h, w, c)
    return y


def film(hv, g, c, c0=0):
    """g: uint16 (n, 2c) f16 bits."""
    n, h, w, _ = hv.shape
    g = np.ascontiguousarray(g, np.uint16)
    assert g.shape == (n, 2 * c)
    y = _out(n, h, w, c)
    _ops_lib().fho_film(_view(hv, c0), g.ctypes.data_as(ctypes.c_void_p), _view(y), n, h, w, c)
    return y


def blend(vis, c0=0, scale=1.0):
    n, h, w, _ = vis.shape
    y = _out(n, h, w, 2)
    _ops_lib().fho_blend(_view(vis, c0, scale), _view(y), n, h, w)
    return y


def blendmix(wa, wb, vis, vis_c0=0, vis_scale=1.0, wa_c0=0, wb_c0=0):
    n, h, w, _ = vis.shape
    y = _out(n, h, w, 3)
    _ops_lib().fho_blendmix(_view(wa, wa_c0), _view(wb, wb_c0), _view(vis, vis_c0, vis_scale), _view(y), n, h, w)
    return y


def avgpool(x, c, k, c0=0):
    n, h, w, _ = x.shape
    y = _out(n, h // k, w // k, c)
    _ops_lib().fho_avgpool(_view(x, c0), _view(y), n, h, w, c, k)
    return y


def interp(x, c, oh, ow, aa=False, c0=0, scale=1.0):
    n, ih, iw, _ = x.shape
    y = _out(n, oh, ow, c)
    _ops_lib().fho_interp(_view(x, c0, scale), _view(y), n, c, ih, iw, oh, ow, int(aa))
    return y


def binary(a, b, c, op=0, a_c0=0, a_scale=1.0, b_c0=0, b_scale=1.0, cb=None):
    """cb: b's channel count (1 broadcasts)."""
    n, h, w, _ = a.shape
    y = _out(n, h, w, c)
    _ops_lib().fho_binary(_view(a, a_c0, a_scale), _view(b, b_c0, b_scale), _view(y), n, h, w, c,
                          c if cb is None else cb, op)
    return y


def unary(x, c, op, a=0.0, b=0.0, c0=0, scale=1.0):
    n, h, w, _ = x.shape
    y = _out(n, h, w, c)
    _ops_lib().fho_unary(_view(x, c0, scale), _view(y), n, h, w, c, op, a, b)
    return y


def chcopy(x, c, c0=0, scale=1.0):
    n, h, w, _ = x.shape
    y = _out(n, h, w, c)
    _ops_lib().fho_chcopy(_view(x, c0, scale), _view(y), n, h, w, c)
    return y


def render(a, b, flow, vis, rt, hq, wq, cubic=True, flags=0, a_c0=0, b_c0=0, flow_c0=0, fsx=1.0, fsy=1.0, vis_c0=0,
           vis_scale=1.0, rt_c0=0, threads=0):
    """a, b: (1, h, w, cs) pictures; flow, vis, rt: (1, hq, wq, cs) quarter-size maps; returns (1, h, w, 3).
    threads > 1: bands of rows on that many threads (the same result)."""
    _, h, w, _ = a.shape
    y = _out(1, h, w, 3)
    args = (_view(a, a_c0), _view(b, b_c0), _view(flow, flow_c0), _view(vis, vis_c0, vis_scale), _view(rt, rt_c0),
            _view(y), h, w, hq, wq, fsx, fsy, int(cubic), flags)
    nt = min(threads or 1, max(1, h // 16))
    if nt <= 1:
        _ops_lib().fho_render(*args)
        return y
    # bands of rows on threads (the foreign call releases the GIL); each output pixel is computed alone
    from concurrent.futures import ThreadPoolExecutor
    step = (h + nt - 1) // nt
    with ThreadPoolExecutor(nt) as ex:
        list(ex.map(lambda y0: _ops_lib().fho_render_rows(*args, y0, min(h, y0 + step)), range(0, h, step)))
    return y


def rgba_in(frames, hp, wp, cs=3):
    """frames: (n, h, w) uint32 RGBA8 words; returns (n, hp, wp, cs) f16 bits, channels 0-2 BGR (the rest 0)."""
    frames = np.ascontiguousarray(frames, np.uint32)
    n, h, w = frames.shape
    y = _out(n, hp, wp, cs)
    _ops_lib().fho_rgba_in(frames.ctypes.data, n, w, h, w, h * w, _view(y), hp, wp)
    return y


def rgba_out(x, h, w, c0=0):
    """x: (n, hp, wp, cs) f16 bits (channels c0.. BGR); returns (n, h, w) uint32 RGBA8 words, alpha 255."""
    n, hp, wp, _ = x.shape
    out = np.zeros((n, h, w), np.uint32)
    _ops_lib().fho_rgba_out(_view(x, c0), n, hp, wp, out.ctypes.data, w, h, w, h * w)
    return out


# ---- GMHS (fh_ops_oracle.c, gmhs.rs): maps are float32 (5, hc, wc), coef float32 (4, 4) ----------------------------

def gm_params(h, w, full_w, level=1):
    """The GMHS grid and windows (gmhs.rs:149-160) as a dict."""
    p = FhoGmPar()
    _ops_lib().fho_gm_params(h, w, full_w, level, ctypes.byref(p))
    return {n: getattr(p, n) for n, _ in FhoGmPar._fields_}


def gm_fit(flow, delta, iters=4, c0=0):
    """The robust affine fit of flow channels c0 .. c0 + 3 of a (1, h8, w8, cs) E8 flow; (4, 4) coefficients."""
    _, h8, w8, _ = flow.shape
    coef = np.zeros((4, 4), np.float32)
    _ops_lib().fho_gm_fit(_view(flow, c0), h8, w8, float(delta), iters, coef.ctypes.data)
    return coef


def gm_cost(a, b, flow, coef, hc, wc, a_c0=0, b_c0=0, flow_c0=0):
    """The 5 cost maps (5, hc, wc) of network pictures a, b (1, h, w, cs) under the E8 flow and the affine fit."""
    _, h, w, _ = a.shape
    _, h8, w8, _ = flow.shape
    maps = np.zeros((5, hc, wc), np.float32)
    coef = np.ascontiguousarray(coef, np.float32)
    _ops_lib().fho_gm_cost(_view(a, a_c0), _view(b, b_c0), h, w, _view(flow, flow_c0), h8, w8, coef.ctypes.data,
                           hc, wc, maps.ctypes.data)
    return maps


def gm_box(src, r, vert):
    """gm_box.wgsl over the planes of src (c, h, w) float32."""
    src = np.ascontiguousarray(src, np.float32)
    c, h, w = src.shape
    dst = np.zeros_like(src)
    _ops_lib().fho_gm_box(src.ctypes.data, dst.ctypes.data, c, h, w, r, int(vert))
    return dst


def gm_select(maps, coef, flow, eps, dmin, tex, c0=0):
    """gm_select.wgsl: a copy of flow (1, h8, w8, cs) with the selected cells rewritten."""
    out = np.ascontiguousarray(flow, np.uint16).copy()
    _, h8, w8, _ = out.shape
    maps = np.ascontiguousarray(maps, np.float32)
    coef = np.ascontiguousarray(coef, np.float32)
    _ops_lib().fho_gm_select(maps.ctypes.data, coef.ctypes.data, _view(out, c0), h8, w8, maps.shape[1],
                             maps.shape[2], eps, dmin, tex)
    return out


def gm_select_cells(n8, nc):
    """The cost-grid index the select reads for each of n8 E8 rows (or columns) of an nc-cell grid
    (gm_select.wgsl:17-18), in float32 as there."""
    i = np.arange(n8, dtype=np.float32)
    v = np.floor((i + np.float32(0.5)) * np.float32(nc) / np.float32(n8)).astype(np.int64)
    return np.clip(v, 0, nc - 1)


def gmhs_stages(a, b, flow, full_w, level=1, a_c0=0, b_c0=0, flow_c0=0):
    """The repair step by step (gmhs.rs:149-206): (repaired flow copy, coef (4, 4), the cost maps after the texture
    window (5, hc, wc), the five values each E8 cell decides on (5, h8, w8): maps 0-2 after the decision window and
    maps 3-4, at the cost cell the select reads)."""
    _, h, w, _ = a.shape
    _, h8, w8, _ = flow.shape
    p = gm_params(h, w, full_w, level)
    coef = gm_fit(flow, p["delta"], 4, flow_c0)
    raw = gm_cost(a, b, flow, coef, p["hc"], p["wc"], a_c0, b_c0, flow_c0)
    tex = gm_box(gm_box(raw, p["r_blk"], 0), p["r_blk"], 1)
    final = np.concatenate([gm_box(gm_box(tex[:3], p["r_dwin"], 0), p["r_dwin"], 1), tex[3:]])
    ys, xs = gm_select_cells(h8, p["hc"]), gm_select_cells(w8, p["wc"])
    dec = final[:, ys[:, None], xs[None, :]]
    out = gm_select(final, coef, flow, p["eps"], p["dmin"], p["tex"], flow_c0)
    return out, coef, tex, dec


def gmhs(a, b, flow, full_w, level=1, a_c0=0, b_c0=0, flow_c0=0):
    """The whole repair (gmhs.rs:149-206): (repaired flow copy, coef (4, 4), decision maps (5, hc, wc))."""
    _, h, w, _ = a.shape
    out = np.ascontiguousarray(flow, np.uint16).copy()
    _, h8, w8, _ = out.shape
    p = gm_params(h, w, full_w, level)
    coef = np.zeros((4, 4), np.float32)
    maps = np.zeros((5, p["hc"], p["wc"]), np.float32)
    tmp = np.zeros_like(maps)
    _ops_lib().fho_gmhs(_view(a, a_c0), _view(b, b_c0), h, w, _view(out, flow_c0), h8, w8, full_w, level,
                        coef.ctypes.data, maps.ctypes.data, tmp.ctypes.data)
    return out, coef, maps
