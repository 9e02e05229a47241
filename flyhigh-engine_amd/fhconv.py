"""Python host driver of libfhconv.so, the FlyHigh conv hot path on MI355X (ctypes over include/fhc_conv.h).

It mirrors the reference's conv-op interface at plan and run time (crates/flyhigh-engine/src/ops/conv/):

- ``ConvOp`` / ``conv_pick`` / ``conv`` : BuildCtx::conv_pick + the recorded Steps (autotune.rs:100-109, :159-235);
  here a plan is created once and run on a HIP stream;
- ``cand_list`` / ``cand_name`` / ``ref_conv_steps``: the reference planner restated (candidates.rs:17-85,
  kernels.rs:99-279), for planner parity;
- ``parse_tune`` / ``format_tune``: the choice table text (tune_cache.rs:71-94);
- errors raise ``FhcError`` with the library's ``fhc_last_error`` message (the reference's C ABI returns -1 and sets
  fh_last_error, crates/flyhigh-capi/src/lib.rs:27-48).

Tensors are torch f16 (or int16/uint16 bit patterns) on the GPU in NHWC layout; the module only passes their device
pointers and never computes a conv itself: when the library is missing, loading it raises.
"""
from __future__ import annotations

import ctypes
import json
import os
from dataclasses import dataclass
from typing import Optional, Sequence

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfhconv.so")

ACT_NONE, ACT_PRELU, ACT_LEAKY = 0, 1, 2

# reference candidate codes (ops/conv/candidates.rs:5-14)
CAND_DIRECT, CAND_TC, CAND_TILED, CAND_TILED8, CAND_DIRECT64 = 0, 1, 2, 3, 4
CAND_TILED16, CAND_TILEDN8, CAND_TILED88, CAND_TILEDM32, CAND_TILED8P = 5, 6, 7, 8, 9


class FhcError(RuntimeError):
    pass


class ConvDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "n", "h", "w", "cin", "cout", "kh", "kw", "stride", "pad",
        "x_cstride", "x_c0", "y_cstride", "y_c0", "r_cstride", "r_c0", "act")] + [
        ("alpha", ctypes.c_float)] + [(n, ctypes.c_uint32) for n in ("residual", "variant", "ksplit", "ref_cand")]


class RefConv(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in (
        "cin", "cout", "h", "w", "stride", "residual", "coop", "cand", "ksplit_env", "f32_mode")]


_lib = None


def load():
    """The library handle; raises if libfhconv.so has not been built (no fallback exists)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FhcError(f"{LIB_PATH} is missing: build it first (__graft_entry__.build() or make -C {HERE})")
    # torch (the driver's device memory and streams) loads its own HIP runtime; it must be in the process before the
    # library pulls in a HIP runtime by soname, or torch finds no GPU afterwards. One runtime then serves both.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    L = ctypes.CDLL(LIB_PATH)
    P, U32, SZ = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_size_t
    sig = {
        "fhc_last_error": ([], ctypes.c_char_p),
        "fhc_conv_plan_create": ([ctypes.POINTER(ConvDesc), P, P, P, ctypes.POINTER(P)], ctypes.c_int),
        "fhc_conv_workspace_bytes": ([P], SZ),
        "fhc_conv_out_shape": ([P, ctypes.POINTER(U32), ctypes.POINTER(U32)], ctypes.c_int),
        "fhc_conv_run": ([P, P, P, P, P, P], ctypes.c_int),
        "fhc_conv_pair_run_film": ([P, P, P, P, P], ctypes.c_int),
        "fhc_conv_sibling_plan_create": ([P, P, P, P, P, P, P, P, P], ctypes.c_int),
        "fhc_conv_sibling_run": ([P, P, P, P, P, P], ctypes.c_int),
        "fhc_conv_run_noalloc": ([P, P, P, P, P], ctypes.c_int),
        "fhc_conv_describe": ([P, ctypes.c_char_p, SZ], ctypes.c_int),
        "fhc_conv_plan_destroy": ([P], None),
        "fhc_conv_pair_plan_create": ([ctypes.POINTER(ConvDesc), P, P, P, ctypes.POINTER(ConvDesc), P, P, P, U32,
                                       ctypes.POINTER(P)], ctypes.c_int),
        "fhc_conv_plan_dry": ([ctypes.POINTER(ConvDesc), ctypes.c_char_p, SZ], ctypes.c_int),
        "fhc_tune_parse": ([ctypes.c_char_p], ctypes.c_int),
        "fhc_tune_format": ([ctypes.c_char_p, SZ], ctypes.c_int),
        "fhc_tune_clear": ([], ctypes.c_int),
        "fhc_tune_get": ([U32] * 5, ctypes.c_int),
        "fhc_tune_get_ex": ([U32] * 7, ctypes.c_int),
        "fhc_variant_name": ([U32, ctypes.c_char_p, SZ], ctypes.c_int),
        "fhc_variant_list": ([ctypes.POINTER(ConvDesc), ctypes.POINTER(U32), SZ], ctypes.c_int),
        "fhc_ref_cand_list": ([ctypes.c_int, U32, U32, U32, ctypes.c_int, ctypes.c_int,
                               ctypes.POINTER(ctypes.c_uint8), SZ], ctypes.c_int),
        "fhc_ref_cand_name": ([ctypes.c_uint8, ctypes.c_char_p, SZ], ctypes.c_int),
        "fhc_ref_conv_steps": ([ctypes.POINTER(RefConv), ctypes.c_char_p, SZ], ctypes.c_int),
        "fhc_probe_mfma_rate": ([U32, U32, P, P], ctypes.c_int),
        "fhc_probe_mfma_layout": ([P, P, P, P], ctypes.c_int),
        "fhc_conv_autotune": ([ctypes.POINTER(ConvDesc), P, P, P, P, P, P, ctypes.c_int,
                               ctypes.POINTER(ctypes.c_float)], ctypes.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L, name)
        f.argtypes = args
        f.restype = res
    _lib = L
    return L


def last_error() -> str:
    return load().fhc_last_error().decode()


def _check(rc, what):
    if rc < 0:
        raise FhcError(f"{what}: {last_error()}")
    return rc


def _ptr(t):
    """Device pointer of a torch tensor (or an int), None for None. The ABI reads dense NHWC buffers whose layout
    the descriptor states, so a torch tensor must be contiguous."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if not t.is_contiguous():
        raise FhcError("tensors passed to the conv must be contiguous (NHWC with the descriptor's strides)")
    return t.data_ptr()


def _stream_handle(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def make_desc(n, h, w, cin, cout, k=3, stride=1, pad=None, act=ACT_PRELU, alpha=0.0, residual=False,
              x_cstride=0, x_c0=0, y_cstride=0, y_c0=0, r_cstride=0, r_c0=0, variant=0, ksplit=0,
              ref_cand=0xFF) -> ConvDesc:
    if pad is None:
        pad = 1 if k == 3 else 0
    d = ConvDesc()
    for name, v in dict(n=n, h=h, w=w, cin=cin, cout=cout, kh=k, kw=k, stride=stride, pad=pad,
                        x_cstride=x_cstride, x_c0=x_c0, y_cstride=y_cstride, y_c0=y_c0, r_cstride=r_cstride,
                        r_c0=r_c0, act=act, alpha=alpha, residual=int(bool(residual)), variant=variant,
                        ksplit=ksplit, ref_cand=ref_cand).items():
        setattr(d, name, v)
    return d


def _host_u16(a):
    """A host buffer of f16 bit patterns (numpy uint16/float16 or a CPU torch tensor) and its pointer."""
    import numpy as np
    if a is None:
        return None, None
    if hasattr(a, "detach"):  # torch tensor
        a = a.detach().cpu().contiguous().view(-1)
        import torch
        if a.dtype == torch.float16:
            a = a.view(torch.int16)
        a = a.numpy()
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        a = a.view(np.uint16)
    if a.dtype not in (np.uint16, np.int16):
        raise FhcError(f"weights must be f16 bit patterns, got {a.dtype}")
    return a, a.ctypes.data_as(ctypes.c_void_p)


class ConvPlan:
    """A planned conv: fhc_conv_plan_create (conv_pick + buildb/buildb_tap), then run() per frame."""

    def __init__(self, desc: ConvDesc, w_oihw, bias, slope=None):
        L = load()
        self.desc = desc
        wa, wp = _host_u16(w_oihw)
        ba, bp = _host_u16(bias)
        sa, sp = _host_u16(slope)
        if wa is None or wa.size != desc.cout * desc.cin * desc.kh * desc.kw:
            raise FhcError("weights must hold cout*cin*kh*kw f16 values (OIHW)")
        if ba is None or ba.size != desc.cout or (sa is not None and sa.size != desc.cout):
            raise FhcError("bias and slope must hold cout f16 values")
        h = ctypes.c_void_p()
        _check(L.fhc_conv_plan_create(ctypes.byref(desc), wp, bp, sp, ctypes.byref(h)), "fhc_conv_plan_create")
        self._h = h
        ho, wo = ctypes.c_uint32(), ctypes.c_uint32()
        _check(L.fhc_conv_out_shape(h, ctypes.byref(ho), ctypes.byref(wo)), "fhc_conv_out_shape")
        self.hout, self.wout = ho.value, wo.value
        self.workspace_bytes = L.fhc_conv_workspace_bytes(h)

    @property
    def handle(self):
        return self._h.value

    def describe(self) -> dict:
        buf = ctypes.create_string_buffer(2048)
        _check(load().fhc_conv_describe(self._h, buf, len(buf)), "fhc_conv_describe")
        return json.loads(buf.value.decode())

    def run(self, x, y, res=None, workspace=None, stream=None):
        _check(load().fhc_conv_run(self._h, _ptr(x), _ptr(y), _ptr(res), _ptr(workspace),
                                   _stream_handle(stream)), "fhc_conv_run")

    def run_noalloc(self, x, y, res=None, stream=None):
        """fhc_conv_run_noalloc: the plan's scratch from the library's static device array (no workspace, nothing
        allocated)."""
        _check(load().fhc_conv_run_noalloc(self._h, _ptr(x), _ptr(y), _ptr(res), _stream_handle(stream)),
               "fhc_conv_run_noalloc")

    def out_elems(self):
        d = self.desc
        return d.n * self.hout * self.wout * (d.y_cstride or d.cout)

    def close(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            load().fhc_conv_plan_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


PAIR_RES_MID = 1
PAIR_AFFINE_OUT = 2
PAIR_FILM_IN = 4
PAIR_TAP32 = 0x400000


class ConvPairPlan(ConvPlan):
    """Two convs fused into one launch (fhc_conv_pair_plan_create): A (3x3, stride 1 or 2) then B (3x3 stride 1) on
    A's output, which stays on chip. run(x, y, res) takes A's input, B's output and B's external residual; with
    res_mid B's residual is A's output. tile_rows / wave_rows / loop 0 let the library choose (1, 2 or 4 rows; 1
    wave row; loop 1 one workgroup per tile, 2 a resident grid looping over tiles, 3 a resident grid with A and B
    on separate waves). affine_out: B's f16 output goes through the graph's affine_out op (2 / (1 + exp(-v)) - 1,
    rounded again) before it is stored; film_in: A's input goes through film_modulate as it is staged, with the FiLM
    vectors given to run_film (which runs such a plan; run refuses it); both one workgroup per tile. tap32: one tap
    per K-step of A even where its few input channels could share K-steps (8 or 16 channels per tap)."""

    def __init__(self, desc_a: ConvDesc, w_a, bias_a, slope_a, desc_b: ConvDesc, w_b, bias_b, slope_b,
                 res_mid=False, tile_rows=0, wave_rows=0, loop=0, affine_out=False, film_in=False, tap32=False):
        L = load()
        self.desc, self.desc_b = desc_a, desc_b
        arrays = []
        for d, w, b, sl in ((desc_a, w_a, bias_a, slope_a), (desc_b, w_b, bias_b, slope_b)):
            wa, wp = _host_u16(w)
            ba, bp = _host_u16(b)
            sa, sp = _host_u16(sl)
            if wa is None or wa.size != d.cout * d.cin * d.kh * d.kw:
                raise FhcError("weights must hold cout*cin*kh*kw f16 values (OIHW)")
            if ba is None or ba.size != d.cout or (sa is not None and sa.size != d.cout):
                raise FhcError("bias and slope must hold cout f16 values")
            arrays.append((wa, wp, ba, bp, sa, sp))
        (_, wpa, _, bpa, _, spa), (_, wpb, _, bpb, _, spb) = arrays
        flags = ((PAIR_RES_MID if res_mid else 0) | (PAIR_AFFINE_OUT if affine_out else 0) |
                 (PAIR_FILM_IN if film_in else 0) | (PAIR_TAP32 if tap32 else 0) | (int(tile_rows) << 8) |
                 (int(wave_rows) << 16) | (int(loop) << 20))
        h = ctypes.c_void_p()
        _check(L.fhc_conv_pair_plan_create(ctypes.byref(desc_a), wpa, bpa, spa, ctypes.byref(desc_b), wpb, bpb,
                                           spb, flags, ctypes.byref(h)), "fhc_conv_pair_plan_create")
        self._h = h
        ho, wo = ctypes.c_uint32(), ctypes.c_uint32()
        _check(L.fhc_conv_out_shape(h, ctypes.byref(ho), ctypes.byref(wo)), "fhc_conv_out_shape")
        self.hout, self.wout = ho.value, wo.value
        self.workspace_bytes = 0

    def out_elems(self):
        d = self.desc_b
        return d.n * self.hout * self.wout * (d.y_cstride or d.cout)

    def run_film(self, x, film, y, stream=None):
        """A film_in plan on device tensors: x A's input before the modulation, film the FiLM vectors (n x 2 x
        A.cin f16, contiguous), y B's output."""
        if not film.is_contiguous() or film.numel() != self.desc.n * 2 * self.desc.cin or film.element_size() != 2:
            raise FhcError(f"run_film: film needs {self.desc.n * 2 * self.desc.cin} contiguous f16 values")
        _check(load().fhc_conv_pair_run_film(self._h, _ptr(x), _ptr(film), _ptr(y), _stream_handle(stream)),
               "fhc_conv_pair_run_film")


class ConvSiblingPlan(ConvPlan):
    """Two convs A and B of one input view in one launch (fhc_conv_sibling_plan_create): A's output channels, then
    B's, each computed as its own plan computes it. run(x, y_a, res_a, y_b) takes the shared input, A's output and
    residual and B's output."""

    def __init__(self, desc_a: ConvDesc, w_a, bias_a, slope_a, desc_b: ConvDesc, w_b, bias_b, slope_b):
        L = load()
        self.desc, self.desc_b = desc_a, desc_b
        ptrs = []
        for d, w, b, sl in ((desc_a, w_a, bias_a, slope_a), (desc_b, w_b, bias_b, slope_b)):
            wa, wp = _host_u16(w)
            ba, bp = _host_u16(b)
            sa, sp = _host_u16(sl)
            if wa is None or wa.size != d.cout * d.cin * d.kh * d.kw:
                raise FhcError("weights must hold cout*cin*kh*kw f16 values (OIHW)")
            if ba is None or ba.size != d.cout or (sa is not None and sa.size != d.cout):
                raise FhcError("bias and slope must hold cout f16 values")
            ptrs.append((wa, wp, ba, bp, sa, sp))
        (_, wpa, _, bpa, _, spa), (_, wpb, _, bpb, _, spb) = ptrs
        h = ctypes.c_void_p()
        _check(L.fhc_conv_sibling_plan_create(ctypes.byref(desc_a), wpa, bpa, spa, ctypes.byref(desc_b), wpb, bpb,
                                              spb, ctypes.byref(h)), "fhc_conv_sibling_plan_create")
        self._h = h
        ho, wo = ctypes.c_uint32(), ctypes.c_uint32()
        _check(L.fhc_conv_out_shape(h, ctypes.byref(ho), ctypes.byref(wo)), "fhc_conv_out_shape")
        self.hout, self.wout = ho.value, wo.value
        self.workspace_bytes = 0

    def run(self, x, y_a, res_a=None, y_b=None, stream=None):
        _check(load().fhc_conv_sibling_run(self._h, _ptr(x), _ptr(y_a), _ptr(res_a), _ptr(y_b),
                                           _stream_handle(stream)), "fhc_conv_sibling_run")


@dataclass
class ConvOp:
    """One conv of the graph as the planner sees it (ConvOp, ops/conv/autotune.rs:100-109), NHWC."""
    weight: object          # OIHW f16 [cout][cin][k][k]
    bias: object            # f16 [cout]
    slope: object = None    # f16 [cout] (PReLU) or None (identity: the reference's `ones`)
    cin: int = 0
    cout: int = 0
    stride: int = 1
    k: int = 3


def conv_pick(op: ConvOp, n: int, h: int, w: int, residual: bool = False, **kw) -> ConvPlan:
    """Plan a conv of `op` over an NHWC input of n x h x w (BuildCtx::conv_pick, autotune.rs:159-235)."""
    act = ACT_PRELU if op.slope is not None else ACT_NONE
    d = make_desc(n, h, w, op.cin, op.cout, k=op.k, stride=op.stride, act=act, residual=residual, **kw)
    return ConvPlan(d, op.weight, op.bias, op.slope)


def conv(plan: ConvPlan, x, res=None, stream=None):
    """Run `plan` on NHWC f16 input x (torch, on the GPU); returns a new NHWC f16 output."""
    import torch
    d = plan.desc
    y = torch.empty((d.n, plan.hout, plan.wout, d.y_cstride or d.cout), dtype=torch.float16, device=x.device)
    ws = None
    if plan.workspace_bytes:
        ws = torch.empty(plan.workspace_bytes // 4 + 4, dtype=torch.float32, device=x.device)
    plan.run(x, y, res, ws, stream)
    return y


def plan_dry(desc: ConvDesc) -> dict:
    """The planner's choice for `desc` without a device (fhc_conv_plan_dry)."""
    buf = ctypes.create_string_buffer(2048)
    _check(load().fhc_conv_plan_dry(ctypes.byref(desc), buf, len(buf)), "fhc_conv_plan_dry")
    return json.loads(buf.value.decode())


def autotune(desc: ConvDesc, w_oihw, bias, slope, x, y, res=None, reps: int = 20):
    """Time every variant for `desc` on these device buffers, record the fastest in the choice table; returns
    (code, microseconds per launch). The per-shape autotune of conv_pick (ops/conv/autotune.rs:199-230)."""
    _, wp = _host_u16(w_oihw)
    _, bp = _host_u16(bias)
    _, sp = _host_u16(slope)
    us = ctypes.c_float()
    code = _check(load().fhc_conv_autotune(ctypes.byref(desc), wp, bp, sp, _ptr(x), _ptr(y), _ptr(res), reps,
                                           ctypes.byref(us)), "fhc_conv_autotune")
    return code, us.value


# ---- the reference planner restated, and the choice table ----------------------------------------------------

def cand_list(coop: bool, cout: int, hout: int, wout: int, direct_ok: bool, try_all: bool = False):
    buf = (ctypes.c_uint8 * 64)()
    n = _check(load().fhc_ref_cand_list(int(coop), cout, hout, wout, int(direct_ok), int(try_all), buf, 64),
               "fhc_ref_cand_list")
    return list(buf[:n])


def cand_name(code: int) -> str:
    buf = ctypes.create_string_buffer(64)
    _check(load().fhc_ref_cand_name(code, buf, 64), "fhc_ref_cand_name")
    return buf.value.decode()


def ref_conv_steps(cin, cout, h, w, stride, residual=False, coop=True, cand=0xFF, ksplit_env=0, f32_mode=False):
    """The reference's dispatches for one conv: list of (pipeline, (gx,gy,gz), weight_bytes, [param words])."""
    c = RefConv(cin=cin, cout=cout, h=h, w=w, stride=stride, residual=int(residual), coop=int(coop), cand=cand,
                ksplit_env=ksplit_env, f32_mode=int(f32_mode))
    buf = ctypes.create_string_buffer(4096)
    _check(load().fhc_ref_conv_steps(ctypes.byref(c), buf, len(buf)), "fhc_ref_conv_steps")
    out = []
    for line in buf.value.decode().splitlines():
        name, grid, wb, params = line.split(" ", 3)
        g = tuple(int(v) for v in grid.strip("()").split(","))
        words = [int(v, 16) for v in params[1:].split()]
        out.append((name, g, int(wb[1:]), words))
    return out


def parse_tune(text: str) -> int:
    return _check(load().fhc_tune_parse(text.encode()), "fhc_tune_parse")


def format_tune() -> str:
    buf = ctypes.create_string_buffer(1 << 16)
    _check(load().fhc_tune_format(buf, len(buf)), "fhc_tune_format")
    return buf.value.decode()


def tune_clear():
    load().fhc_tune_clear()


def tune_get(cin, cout, h, w, stride, n=1, k=3) -> Optional[int]:
    """The table's code for a conv of batch n and kernel size k (None without an entry)."""
    v = load().fhc_tune_get(cin, cout, h, w, stride) if (n, k) == (1, 3) else \
        load().fhc_tune_get_ex(cin, cout, h, w, stride, n, k)
    return None if v < 0 else v


def variant_name(code: int) -> str:
    buf = ctypes.create_string_buffer(128)
    _check(load().fhc_variant_name(code, buf, len(buf)), "fhc_variant_name")
    return buf.value.decode()


def variant_list(desc: ConvDesc) -> Sequence[int]:
    arr = (ctypes.c_uint32 * 256)()
    n = _check(load().fhc_variant_list(ctypes.byref(desc), arr, 256), "fhc_variant_list")
    return list(arr[:n])


def probe_mfma_layout(a, b, d, stream=None):
    _check(load().fhc_probe_mfma_layout(_ptr(a), _ptr(b), _ptr(d), _stream_handle(stream)), "fhc_probe_mfma_layout")


def probe_mfma_rate(blocks, iters, out, stream=None):
    """Launch the sustained-MFMA-rate probe: blocks * 4 * 16 * iters * 16384 FLOPs (out: blocks * 1024 floats)."""
    _check(load().fhc_probe_mfma_rate(blocks, iters, _ptr(out), _stream_handle(stream)), "fhc_probe_mfma_rate")
    return blocks * 4 * 16 * iters * 16384
