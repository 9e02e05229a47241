"""The C-ABI boundary without a GPU: the library loads, exports every function the header declares, and turns
bad input into an error status with a message (never an abort), as the reference's C ABI does
(crates/flyhigh-capi/src/lib.rs:27-48)."""
import ctypes
import os
import re
import threading

import numpy as np
import pytest

from fhtest import ROOT, fhconv


def declared_functions():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if fn.endswith(".h"):
            text = open(os.path.join(inc, fn)).read()
            text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
            names.update(re.findall(r"\b(fhc_\w+)\s*\(", text))
    return names


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("fhc_conv_plan_create", "fhc_conv_run", "fhc_conv_workspace_bytes", "fhc_conv_describe",
                     "fhc_conv_plan_destroy", "fhc_last_error", "fhc_ref_conv_steps", "fhc_tune_parse"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(fhconv.LIB_PATH)
    missing = [n for n in sorted(declared_functions()) if not hasattr(lib, n)]
    assert not missing, missing


BAD = [
    dict(stride=3), dict(cin=0), dict(cout=0), dict(n=0), dict(k=5), dict(pad=0), dict(k=1, pad=1),
    dict(k=1, stride=2), dict(x_cstride=16, x_c0=8), dict(y_cstride=30), dict(residual=True, r_cstride=10),
    dict(act=7), dict(ksplit=3), dict(cin=5000), dict(variant=31), dict(variant=4000),
]


@pytest.mark.parametrize("bad", BAD)
def test_bad_descriptor_is_an_error_status(bad):
    kw = dict(n=1, h=16, w=16, cin=16, cout=32)
    for k in ("n", "cin", "cout"):
        if k in bad:
            kw[k] = bad.pop(k)
    d = fhconv.make_desc(kw["n"], 16, 16, kw["cin"], kw["cout"], **bad)
    with pytest.raises(fhconv.FhcError) as e:
        fhconv.plan_dry(d)
    assert "fhc_conv_plan_dry" in str(e.value)
    # plan creation validates before touching the device: the same descriptor fails the same way
    h = ctypes.c_void_p(123)
    w = (ctypes.c_uint16 * (max(kw["cout"], 1) * max(kw["cin"], 1) * 25))()
    b = (ctypes.c_uint16 * max(kw["cout"], 1))()
    rc = fhconv.load().fhc_conv_plan_create(ctypes.byref(d), w, b, b, ctypes.byref(h))
    assert rc == -1 and h.value is None
    assert fhconv.last_error()


def test_null_arguments_are_errors():
    L = fhconv.load()
    d = fhconv.make_desc(1, 8, 8, 8, 8)
    h = ctypes.c_void_p()
    assert L.fhc_conv_plan_create(None, None, None, None, ctypes.byref(h)) == -1
    assert "NULL descriptor" in fhconv.last_error()
    assert L.fhc_conv_plan_create(ctypes.byref(d), None, None, None, ctypes.byref(h)) == -1
    assert "NULL weights" in fhconv.last_error()
    assert L.fhc_conv_plan_create(ctypes.byref(d), None, None, None, None) == -1
    assert L.fhc_conv_run(None, None, None, None, None, None) == -1
    assert "NULL plan" in fhconv.last_error()
    assert L.fhc_conv_pair_run_film(None, None, None, None, None) == -1
    assert "NULL plan" in fhconv.last_error()
    assert L.fhc_conv_sibling_run(None, None, None, None, None, None) == -1
    assert "NULL plan" in fhconv.last_error()
    assert L.fhc_conv_describe(None, None, 0) == -1
    assert L.fhc_conv_workspace_bytes(None) == 0
    L.fhc_conv_plan_destroy(None)


def test_prelu_without_slope_is_an_error():
    L = fhconv.load()
    d = fhconv.make_desc(1, 8, 8, 8, 8, act=fhconv.ACT_PRELU)
    w = (ctypes.c_uint16 * (8 * 8 * 9))()
    b = (ctypes.c_uint16 * 8)()
    h = ctypes.c_void_p()
    assert L.fhc_conv_plan_create(ctypes.byref(d), w, b, None, ctypes.byref(h)) == -1
    assert "slope" in fhconv.last_error()


def test_small_buffers_are_errors_not_overflows():
    L = fhconv.load()
    buf = ctypes.create_string_buffer(4)
    assert L.fhc_ref_cand_name(2, buf, 4) == -1  # "tiled" needs 6 bytes
    assert "too small" in fhconv.last_error()
    out = (ctypes.c_uint8 * 2)()
    assert L.fhc_ref_cand_list(1, 64, 60, 108, 0, 1, out, 2) == -1
    d = fhconv.make_desc(1, 136, 240, 32, 32)
    assert L.fhc_conv_plan_dry(ctypes.byref(d), ctypes.create_string_buffer(16), 16) == -1


def test_last_error_is_thread_local():
    L = fhconv.load()
    d = fhconv.make_desc(1, 8, 8, 8, 8, stride=3)
    assert L.fhc_conv_plan_dry(ctypes.byref(d), None, 0) == -1
    mine = fhconv.last_error()
    seen = []

    def other():
        seen.append(fhconv.last_error())

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert mine and seen == [""]


def test_pair_plan_rejects_what_it_cannot_fuse():
    # shape checks happen before any device call: a mismatched second conv, an unsupported channel combination and
    # a residual from the first conv without the residual flag are error statuses
    wa = np.zeros(36 * 3 * 9, np.uint16)
    ba = np.zeros(36, np.uint16)
    wb = np.zeros(36 * 36 * 9, np.uint16)
    bb = np.zeros(36, np.uint16)
    a = fhconv.make_desc(1, 40, 60, 3, 36, stride=2, act=0)
    for b, flags in [(fhconv.make_desc(1, 21, 30, 36, 36, act=0), 0),        # B's height is not A's output height
                     (fhconv.make_desc(1, 20, 30, 35, 36, act=0), 0),        # B's cin is not A's cout
                     (fhconv.make_desc(1, 20, 30, 36, 36, act=0), 1),        # residual from A without B's flag
                     (fhconv.make_desc(1, 20, 30, 36, 36, act=0, stride=2), 0)]:  # B must be stride 1
        with pytest.raises(fhconv.FhcError):
            fhconv.ConvPairPlan(a, wa, ba, None, b, wb if b.cin == 36 else np.zeros(36 * b.cin * 9, np.uint16), bb, None,
                                res_mid=bool(flags))
    big = fhconv.make_desc(1, 20, 30, 36, 96, act=0)  # 96 output channels: no pair instantiated
    with pytest.raises(fhconv.FhcError):
        fhconv.ConvPairPlan(a, wa, ba, None, big, np.zeros(96 * 36 * 9, np.uint16), np.zeros(96, np.uint16), None)
    # affine_out after the second conv runs in the one-workgroup-per-tile loop only
    b = fhconv.make_desc(1, 20, 30, 36, 36, act=0)
    for loop in (2, 3):
        with pytest.raises(fhconv.FhcError, match="one-workgroup-per-tile"):
            fhconv.ConvPairPlan(a, wa, ba, None, b, wb, bb, None, loop=loop, affine_out=True)
    # ... on a second conv of at most 4 output channels
    with pytest.raises(fhconv.FhcError, match="at most 4 output channels"):
        fhconv.ConvPairPlan(a, wa, ba, None, b, wb, bb, None, affine_out=True)
    # FiLM on the first conv's input: the one-workgroup-per-tile loop, no external residual for the second
    for loop in (2, 3):
        with pytest.raises(fhconv.FhcError, match="one-workgroup-per-tile"):
            fhconv.ConvPairPlan(a, wa, ba, None, b, wb, bb, None, loop=loop, film_in=True)
    br = fhconv.make_desc(1, 20, 30, 36, 36, act=0, residual=True)
    with pytest.raises(fhconv.FhcError, match="external residual"):
        fhconv.ConvPairPlan(a, wa, ba, None, br, wb, bb, None, film_in=True)


def test_sibling_plan_rejects_what_it_cannot_fuse():
    # checked before any device call: another input geometry, a residual on the second conv, LeakyReLU, input
    # channels or output channels no sibling kernel serves
    z = lambda co, ci: (np.zeros(co * ci * 9, np.uint16), np.zeros(co, np.uint16))  # noqa: E731
    a = fhconv.make_desc(1, 20, 30, 48, 7, act=0, residual=True)
    cases = [(fhconv.make_desc(1, 20, 31, 48, 36, act=0), "same input view"),
             (fhconv.make_desc(1, 20, 30, 48, 36, act=0, residual=True), "cannot take a residual"),
             (fhconv.make_desc(1, 20, 30, 48, 36, act=fhconv.ACT_LEAKY, alpha=0.1), "identity or PReLU"),
             (fhconv.make_desc(1, 20, 30, 48, 44, act=0), "no sibling kernel")]
    for b, msg in cases:
        with pytest.raises(fhconv.FhcError, match=msg):
            fhconv.ConvSiblingPlan(a, *z(7, 48), None, b, *z(b.cout, 48), None)
    small = fhconv.make_desc(1, 20, 30, 24, 7, act=0)
    with pytest.raises(fhconv.FhcError, match="no sibling kernel"):
        fhconv.ConvSiblingPlan(small, *z(7, 24), None, fhconv.make_desc(1, 20, 30, 24, 36, act=0), *z(36, 24), None)


def _ops():
    import fhops
    return fhops, fhops._lib()


def _tv(p=0x1000, cs=4, c0=0, scale=1.0):
    import fhops
    return ctypes.byref(fhops.FhcTensor(p, cs, c0, scale))


def test_network_ops_reject_bad_views_before_any_launch():
    """Validation happens on the host before any HIP call (no GPU needed): views too narrow for the channels an op
    reads or writes, scales on inputs an op reads unscaled, null views, out-of-range parameters."""
    fh, L = _ops()
    cases = [
        ("fhc_warp", (_tv(cs=3), _tv(cs=2), _tv(cs=4), 1, 4, 4, 4, None), "does not hold"),
        ("fhc_warp", (_tv(), _tv(cs=1), _tv(), 1, 4, 4, 4, None), "warp flow"),
        ("fhc_luma", (_tv(cs=2), _tv(), 1, 4, 4, 0, None), "luma x"),
        ("fhc_sad_volume", (_tv(), _tv(), _tv(cs=24), 1, 4, 4, 2, None), "sad_volume out"),
        ("fhc_sad_volume", (_tv(scale=0.5), _tv(), _tv(cs=64), 1, 4, 4, 2, None), "unscaled"),
        ("fhc_sad_volume", (_tv(), _tv(), _tv(cs=300), 1, 4, 4, 8, None), "radius"),
        ("fhc_convex_upsample", (_tv(cs=35), _tv(), _tv(), 1, 4, 4, 4, None), "convex_upsample wt"),
        ("fhc_film_modulate", (_tv(), None, _tv(), 1, 4, 4, 4, None), "null g"),
        ("fhc_blend_weights", (_tv(cs=3, c0=1), _tv(), 1, 4, 4, None), "blend_weights vis"),
        ("fhc_blendmix", (_tv(), _tv(cs=2), _tv(), _tv(), 1, 4, 4, None), "blendmix wb"),
        ("fhc_avgpool", (_tv(), _tv(), 1, 4, 4, 4, 0, None), "k is 0"),
        ("fhc_interpolate", (_tv(), _tv(p=0), 1, 4, 4, 4, 2, 2, 0, None), "null pointer"),
        ("fhc_interpolate", (_tv(scale=float("nan")), _tv(), 1, 4, 4, 4, 2, 2, 0, None), "not finite"),
        ("fhc_interpolate", (_tv(), _tv(), 1, 4, 0, 4, 2, 2, 1, None), "empty input"),
        ("fhc_warp", (None, _tv(), _tv(), 1, 4, 4, 4, None), "null view"),
        ("fhc_coarse_fine_input", (_tv(cs=8), _tv(cs=8), None, 2, 2, 16.0, _tv(cs=8), _tv(), 0.125, _tv(cs=16),
                                   _tv(), 4, 4, 4, None), "coarse_fine_input fx"),
        ("fhc_coarse_fine_input", (_tv(cs=8), _tv(cs=8), _tv(), 8, 8, 16.0, _tv(cs=8), _tv(), 0.125, _tv(cs=24),
                                   _tv(), 4, 4, 4, None), "state is larger"),
        ("fhc_flow_vis_t_convex", (_tv(cs=40), _tv(cs=8), _tv(cs=4), ctypes.c_float(0.5), _tv(cs=8), 1, 4, 4, None),
         "flow_vis_t_convex dfilm"),
        ("fhc_fold_pair_sad", (_tv(cs=8), _tv(cs=16), None, 4, 4, 8, _tv(), _tv(), _tv(cs=24), 1, 4, 4, 2, None),
         "fold_pair_sad sad out"),
        ("fhc_fold_pair_sad", (_tv(cs=8), _tv(cs=12), None, 4, 4, 8, _tv(), _tv(), _tv(cs=32), 1, 4, 4, 2, None),
         "fold_pair_sad out"),
        # the frame input: at most 10 taps (2160p to 432 x 240 takes 19) and an 84-pixel window; frames present
        ("fhc_rgba_resize", (0x1000, 1, 3840, 2160, 3840, 0, 2176, 3840, _tv(), 240, 432, None), "needs 19 taps"),
        ("fhc_rgba_resize", (None, 1, 3840, 2160, 3840, 0, 2176, 3840, _tv(), 480, 864, None), "null frame"),
        ("fhc_rgba_resize", (0x1000, 1, 3840, 2160, 3840, 0, 2176, 3840, _tv(cs=8), 480, 864, None), "8-byte"),
        # the frame render: every map view is checked before any of it is read
        ("fhc_render_rgba", (0x1000, 0x2000, 64, 32, 64, 32, 64, _tv(cs=8), _tv(cs=8, c0=4), None, 8, 16,
                             ctypes.c_float(1.0), ctypes.c_float(1.0), 1, 0, 0x3000, 64, None), "render_rgba rt"),
        ("fhc_render_rgba", (0x1000, 0x2000, 64, 32, 64, 32, 64, None, _tv(cs=8, c0=4), _tv(), 8, 16,
                             ctypes.c_float(1.0), ctypes.c_float(1.0), 1, 0, 0x3000, 64, None), "render_rgba flow"),
        ("fhc_render_rgba", (0x1000, None, 64, 32, 64, 32, 64, _tv(cs=8), _tv(cs=8, c0=4), _tv(), 8, 16,
                             ctypes.c_float(1.0), ctypes.c_float(1.0), 1, 0, 0x3000, 64, None), "null frame"),
        # the batched forms: their pair counts and the repair's workspace for all pairs
        ("fhc_refine_input_n", (_tv(cs=8), _tv(cs=8), _tv(cs=8), _tv(cs=16), 8, 8, ctypes.c_float(0.05), 4, 0, None),
         "picture pairs"),
        ("fhc_refine_input_n", (_tv(cs=8), _tv(cs=8), _tv(cs=8), _tv(cs=16), 8, 8, ctypes.c_float(0.05), 4, 5, None),
         "picture pairs"),
        ("fhc_refine_input_n", (_tv(cs=8), _tv(cs=8), _tv(cs=8), _tv(cs=16), 8, 8, ctypes.c_float(0.05), 70000, 1,
                                None), "launch limit"),
        ("fhc_gmhs_n", (_tv(), _tv(), 480, 864, _tv(), 60, 108, 1920, 1, 2, 0x1000,
                        fh.gmhs_params(480, 864, 1920, 1)["ws_bytes"], None), "workspace of"),
        ("fhc_gmhs_n", (_tv(), _tv(), 480, 864, _tv(), 60, 108, 1920, 1, 70000, 0x1000, 1 << 40, None),
         "launch limit"),
        ("fhc_fold_pair_sad_n", (_tv(cs=8), _tv(cs=16), None, 4, 4, 8, 70000, _tv(), _tv(), _tv(cs=32), 1, 4, 4, 2,
                                 None), "launch limit"),
        ("fhc_coarse_fine_input_n", (_tv(cs=8), _tv(cs=8), None, 2, 2, ctypes.c_float(16.0), _tv(cs=8), _tv(),
                                     ctypes.c_float(0.125), _tv(cs=24), _tv(), 4, 4, 4, 70000, None), "launch limit"),
        ("fhc_pair_input_n", (_tv(), _tv(), _tv(), _tv(cs=8), _tv(), 64, 64, 16, 16, 5_000_000, None),
         "too many tiles"),
        ("fhc_flow_vis_t_convex_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), (ctypes.c_float * 9)(*[0.5] * 9), 9,
                                     _tv(cs=8), 1, 4, 4, None), "phases"),
        ("fhc_flow_vis_t_convex_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), None, 2, _tv(cs=8), 1, 4, 4, None),
         "null phases"),
        # the fine input with its cost volume: the radius its tiles hold, the volume's channels, the pair count
        ("fhc_coarse_fine_input_sad_n", (_tv(cs=8), _tv(cs=8), None, 2, 2, ctypes.c_float(16.0), _tv(cs=8), _tv(),
                                         ctypes.c_float(0.125), _tv(cs=24), _tv(), 4, 4, 4, 1, _tv(cs=64), 4, None),
         "radius 4 above 3"),
        ("fhc_coarse_fine_input_sad_n", (_tv(cs=8), _tv(cs=8), None, 2, 2, ctypes.c_float(16.0), _tv(cs=8), _tv(),
                                         ctypes.c_float(0.125), _tv(cs=24), _tv(), 4, 4, 4, 1, _tv(cs=24), 2, None),
         "sad out"),
        ("fhc_coarse_fine_input_sad_n", (_tv(cs=8), _tv(cs=8), None, 2, 2, ctypes.c_float(16.0), _tv(cs=8), _tv(),
                                         ctypes.c_float(0.125), _tv(cs=24), _tv(), 4, 4, 4, 70000, _tv(cs=32), 2,
                                         None), "launch limit"),
        # the batched frame render: its frame count and strides before any launch
        ("fhc_render_rgba_n", (0x1000, 300, 300, 64, 32, 64, 64 * 32, 32, 64, _tv(cs=8), _tv(cs=8, c0=4), _tv(), 8, 16,
                               ctypes.c_float(1.0), ctypes.c_float(1.0), 1, 0, 0x3000, 64, 64 * 32, None),
         "launch limit"),
        ("fhc_render_rgba_n", (0x1000, 2, 3, 64, 32, 64, 100, 32, 64, _tv(cs=8), _tv(cs=8, c0=4), _tv(), 8, 16,
                               ctypes.c_float(1.0), ctypes.c_float(1.0), 1, 0, 0x3000, 64, 64 * 32, None),
         "frame stride"),
        ("fhc_render_rgba_n", (0x1000, 2, 3, 64, 32, 64, 64 * 32, 32, 64, _tv(cs=8), _tv(cs=8, c0=4), _tv(), 8, 16,
                               ctypes.c_float(1.0), ctypes.c_float(1.0), 1, 0, 0x3000, 64, 100, None),
         "frame stride"),
        # the convex upsample with the refine input: its phases, image count and every view before any launch
        ("fhc_mid_input_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), (ctypes.c_float * 9)(*[0.5] * 9), 9, _tv(cs=8),
                             _tv(cs=8), _tv(cs=16), 1, 4, 4, ctypes.c_float(0.25), ctypes.c_float(0.05), None),
         "phases"),
        ("fhc_mid_input_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), None, 2, _tv(cs=8), _tv(cs=8), _tv(cs=16), 1, 4, 4,
                             ctypes.c_float(0.25), ctypes.c_float(0.05), None), "null phases"),
        ("fhc_mid_input_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), (ctypes.c_float * 8)(*[0.5] * 8), 8, _tv(cs=8),
                             _tv(cs=8), _tv(cs=16), 9000, 4, 4, ctypes.c_float(0.25), ctypes.c_float(0.05), None),
         "launch limit"),
        ("fhc_mid_input_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), (ctypes.c_float * 1)(0.5), 1, _tv(cs=8), _tv(cs=8),
                             _tv(cs=12), 1, 4, 4, ctypes.c_float(0.25), ctypes.c_float(0.05), None), "mid_input rx"),
        ("fhc_mid_input_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), (ctypes.c_float * 1)(0.5), 1, _tv(cs=8), None,
                             _tv(cs=16), 1, 4, 4, ctypes.c_float(0.25), ctypes.c_float(0.05), None), "mid_input q"),
        ("fhc_mid_input_n", (_tv(cs=40), _tv(cs=8), _tv(cs=8), (ctypes.c_float * 1)(0.5), 1, _tv(cs=8), _tv(cs=8),
                             _tv(cs=16), 1, 4, 4, ctypes.c_float(float("inf")), ctypes.c_float(0.05), None),
         "not finite"),
    ]
    for name, args, msg in cases:
        rc = getattr(L, name)(*args)
        assert rc == -1, (name, msg, rc)
        assert msg in fhconv.last_error(), (name, fhconv.last_error())


def test_network_ops_on_empty_tensors_are_no_ops():
    fh, L = _ops()
    assert L.fhc_warp(None, None, None, 0, 4, 4, 4, None) == 0
    assert L.fhc_sad_volume(None, None, None, 1, 0, 4, 3, None) == 0
    assert L.fhc_avgpool(None, None, 1, 1, 1, 4, 2, None) == 0  # a 1x1 input pools to 0x0
    assert L.fhc_interpolate(None, None, 1, 3, 4, 4, 0, 8, 1, None) == 0
