"""Parity of the HIP network ops (through the C ABI, include/fhc_ops.h) with the CPU oracle, on the GPU.

Bar: bit-exact f16 results for the ops without a transcendental (warp, luma, luma_grad, sad_volume, film_modulate,
avgpool, interpolate: the same f32 operations in the same order, one RTNE rounding); where a softmax's expf is
involved (the GPU's expf and the host's may differ in the last f32 bit) at most 1 f16 ulp for blend_weights and
blendmix, and for convex_upsample, whose 9 signed terms can cancel, and affine_out (2 / (1 + exp(-v)) - 1, which
cancels near 0), 1 ulp or 2^-16 of the input's largest magnitude (of the result's range for affine_out). Views (channel offsets, wider pixel strides, read scales), batches, ragged sizes, flows reaching
far outside the image and outputs written into a concat slice are covered; channels outside an output view must
stay untouched. Sizes include the FlyHighFG shapes at 1080p (network 864x480: 216x120, 108x60, 54x30).
"""
import numpy as np
import pytest

from fhtest import f16_bits, oracle, ulp_dist

pytestmark = pytest.mark.gpu

SENTINEL = 0x7BFF  # f16 65504: what untouched channels of an output buffer hold


def say(*a):
    print(*a, flush=True)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint16)


def fhops():
    import fhops as m  # noqa: E402  (flyhigh-engine_amd is on sys.path through fhtest)
    return m


def rand(rng, shape, lo=-1.0, hi=1.0):
    return f16_bits(rng.uniform(lo, hi, shape))


def exact(got, want, what):
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{what}: {len(bad)} elements differ, first at {bad[0].tolist()}"


def within_ulp(got, want, what, ulps=1):
    d = ulp_dist(got, want)
    assert d.max() <= ulps, f"{what}: max {d.max()} ulps at {np.unravel_index(d.argmax(), d.shape)}"


def softmax_close(got, want, xmax, what):
    """1 f16 ulp, or 2^-16 * max|x| where the weighted sum cancels: a weight from a different last f32 bit of expf
    moves a sum of 9 terms by at most a few 2^-24 * max|x|."""
    g, w = got.view(np.float16).astype(np.float64), want.view(np.float16).astype(np.float64)
    unit = np.spacing(np.abs(w).astype(np.float16)).astype(np.float64)
    bad = np.abs(g - w) > np.maximum(unit, 2.0 ** -16 * xmax)
    assert not bad.any(), f"{what}: {bad.sum()} elements off, first at {np.argwhere(bad)[0].tolist()}"


def sliced_out(n, h, w, cs, c0):
    """An output buffer of cstride cs filled with the sentinel; the op writes channels c0.."""
    return np.full((n, h, w, cs), SENTINEL, np.uint16)


def check_slice(buf, got_dev, c0, c, want, what, ulps=0):
    got = host(got_dev)
    assert np.all(got[..., :c0] == SENTINEL) and np.all(got[..., c0 + c:] == SENTINEL), f"{what}: wrote outside view"
    (exact if ulps == 0 else within_ulp)(got[..., c0:c0 + c], want, what)


WARP_CASES = [  # n, h, w, c, img cstride, img c0, flow cstride, flow c0, flow range, flow scale, img scale
    (2, 60, 108, 36, 36, 0, 4, 0, 6.0, 0.125, 1.0),     # features at 1/8 (vector path)
    (1, 120, 216, 3, 3, 0, 4, 2, 40.0, 0.25, 1.0),      # the refine warp of a 3-channel image by a view of flow_tq
    (2, 17, 23, 5, 9, 3, 5, 1, 30.0, 1.0, 0.5),         # ragged, strided views, far outside the image
    (1, 30, 54, 8, 16, 8, 2, 0, 3.0, 2.0, 2.0),         # vector path through an offset view
]


@pytest.mark.parametrize("case", WARP_CASES)
def test_warp_matches_oracle(case):
    n, h, w, c, ics, ic0, fcs, fc0, fr, fs, isc = case
    say("warp", case)
    fh = fhops()
    rng = np.random.default_rng(hash(case) % 2**32)
    img, flow = rand(rng, (n, h, w, ics), -2, 2), rand(rng, (n, h, w, fcs), -fr, fr)
    want = oracle.warp(img, flow, c, img_c0=ic0, img_scale=isc, flow_c0=fc0, flow_scale=fs)
    buf = sliced_out(n, h, w, c + 6, 2)
    out = dev(buf)
    fh.warp(fh.View(dev(img), ic0, isc), fh.View(dev(flow), fc0, fs), c, out=fh.View(out, 2))
    check_slice(buf, out, 2, c, want, f"warp {case}")


@pytest.mark.parametrize("grad", [False, True])
@pytest.mark.parametrize("n,h,w,cs,c0,scale", [(2, 30, 54, 3, 0, 1.0), (1, 120, 216, 7, 4, 1.0),
                                                (1, 13, 9, 5, 1, 0.5)])
def test_luma_matches_oracle(grad, n, h, w, cs, c0, scale):
    say("luma", grad, n, h, w, cs, c0, scale)
    fh = fhops()
    rng = np.random.default_rng(n * h * w + cs + grad)
    x = rand(rng, (n, h, w, cs), 0, 1)
    want = oracle.luma(x, grad=grad, c0=c0, scale=scale)
    got = host(fh.luma(fh.View(dev(x), c0, scale), grad=grad))
    exact(got, want, f"luma grad={grad}")


@pytest.mark.parametrize("n,h,w,r", [(2, 30, 54, 3), (3, 60, 108, 2), (1, 5, 4, 3), (1, 1, 1, 2), (2, 9, 31, 0)])
def test_sad_volume_matches_oracle(n, h, w, r):
    say("sad", n, h, w, r)
    fh = fhops()
    rng = np.random.default_rng(n * h * w + r)
    la, lb = rand(rng, (n, h, w, 2), 0, 1), rand(rng, (n, h, w, 1), 0, 1)
    want = oracle.sad(la, lb, r, la_c0=1)
    s2 = (2 * r + 1) ** 2
    buf = sliced_out(n, h, w, s2 + 3, 3)
    out = dev(buf)
    fh.sad(fh.View(dev(la), 1), dev(lb), r, out=fh.View(out, 3))
    check_slice(buf, out, 3, s2, want, f"sad r={r}")


@pytest.mark.parametrize("n,h,w,c,logit", [(1, 60, 108, 7, 3.0), (2, 11, 6, 3, 20.0), (1, 30, 54, 16, 1.0)])
def test_convex_upsample_matches_oracle(n, h, w, c, logit):
    say("convex", n, h, w, c, logit)
    fh = fhops()
    rng = np.random.default_rng(n * h * w + c)
    wt = f16_bits(rng.normal(0, logit, (n, h, w, 40)))
    x = rand(rng, (n, h, w, c + 1), -4, 4)
    want = oracle.convex(wt, x, c, wt_c0=4, x_c0=1)
    got = host(fh.convex(fh.View(dev(wt), 4), fh.View(dev(x), 1), c))
    softmax_close(got, want, np.abs(x.view(np.float16)).max(), "convex")


@pytest.mark.parametrize("n,h,w,c,cs,c0", [(2, 60, 108, 48, 48, 0), (3, 7, 5, 6, 9, 2), (1, 30, 54, 12, 16, 4)])
def test_film_modulate_matches_oracle(n, h, w, c, cs, c0):
    say("film", n, h, w, c, cs, c0)
    fh = fhops()
    rng = np.random.default_rng(n * h * w + c)
    hv, g = rand(rng, (n, h, w, cs), -3, 3), rand(rng, (n, 2 * c), -1, 1)
    want = oracle.film(hv, g, c, c0=c0)
    got = host(fh.film(fh.View(dev(hv), c0), dev(g), c))
    exact(got, want, "film")


@pytest.mark.parametrize("n,h,w,cs,c0,scale", [(1, 120, 216, 3, 0, 1.0), (2, 13, 17, 7, 4, 2.0),
                                                (1, 60, 108, 5, 2, 0.5)])
def test_blend_weights_and_blendmix_match_oracle(n, h, w, cs, c0, scale):
    say("blend", n, h, w, cs, c0, scale)
    fh = fhops()
    rng = np.random.default_rng(n * h * w + cs)
    vis = f16_bits(rng.normal(0, 4, (n, h, w, cs)))
    wa, wb = rand(rng, (n, h, w, 3), 0, 1), rand(rng, (n, h, w, 3), 0, 1)
    vv = fh.View(dev(vis), c0, scale)
    within_ulp(host(fh.blend(vv)), oracle.blend(vis, c0=c0, scale=scale), "blend_weights")
    within_ulp(host(fh.blendmix(dev(wa), dev(wb), vv)), oracle.blendmix(wa, wb, vis, vis_c0=c0, vis_scale=scale),
               "blendmix")


@pytest.mark.parametrize("n,h,w,c,cs,c0,k", [(2, 120, 216, 3, 3, 0, 2), (2, 60, 108, 3, 3, 0, 2),
                                              (1, 61, 109, 8, 12, 4, 2), (1, 25, 14, 5, 5, 0, 3), (1, 8, 8, 4, 4, 0, 1)])
def test_avgpool_matches_oracle(n, h, w, c, cs, c0, k):
    say("avgpool", n, h, w, c, cs, c0, k)
    fh = fhops()
    rng = np.random.default_rng(n * h * w + c + k)
    x = rand(rng, (n, h, w, cs), 0, 1)
    want = oracle.avgpool(x, c, k, c0=c0)
    got = host(fh.avgpool(fh.View(dev(x), c0), k, c))
    exact(got, want, "avgpool")


INTERP_CASES = [  # n, ih, iw, oh, ow, c, cs, c0, aa, scale
    (1, 480, 864, 120, 216, 3, 3, 0, True, 1.0),   # the graph's A -> aq (antialiased quarter)
    (2, 480, 864, 120, 216, 3, 4, 0, True, 1.0),   # the same from 8-byte pixels (one load a pixel into LDS)
    (2, 30, 54, 60, 108, 4, 16, 0, False, 1.0),     # flow16 -> flow (vector path)
    (2, 30, 54, 60, 108, 3, 16, 4, False, 16.0),    # vis16 of an offset view, scaled
    (1, 23, 41, 7, 9, 5, 6, 1, True, 0.5),          # ragged antialias
    (1, 7, 9, 20, 31, 2, 2, 0, True, 1.0),          # antialias flag on an upsample (support 1)
    (1, 240, 432, 30, 54, 8, 8, 0, True, 1.0),      # a tile beyond the LDS budget: the per-output kernel
]


@pytest.mark.parametrize("case", INTERP_CASES)
def test_interpolate_matches_oracle(case):
    n, ih, iw, oh, ow, c, cs, c0, aa, scale = case
    say("interp", case)
    fh = fhops()
    rng = np.random.default_rng(ih * iw + oh + c)
    x = rand(rng, (n, ih, iw, cs), 0, 1)
    want = oracle.interp(x, c, oh, ow, aa=aa, c0=c0, scale=scale)
    got = host(fh.interp(fh.View(dev(x), c0, scale), oh, ow, antialias=aa, c=c))
    exact(got, want, f"interp {case}")


@pytest.mark.parametrize("c,cs_a,a0,cb,op,sa,sb", [(4, 4, 0, 4, 0, 1.0, 1.0), (3, 7, 4, 3, 0, 0.125, -1.0),
                                                   (3, 3, 0, 1, 1, 1.0, 2.0), (8, 12, 4, 1, 0, 2.0, 0.5)])
def test_binary_matches_oracle(c, cs_a, a0, cb, op, sa, sb):
    say("binary", c, cs_a, a0, cb, op, sa, sb)
    fh = fhops()
    rng = np.random.default_rng(c * 10 + cb + op)
    n, h, w = 2, 60, 108
    a, b = rand(rng, (n, h, w, cs_a), -3, 3), rand(rng, (n, h, w, cb + 1), -3, 3)
    want = oracle.binary(a, b, c, op=op, a_c0=a0, a_scale=sa, b_c0=1, b_scale=sb, cb=cb)
    got = host(fh.binary(fh.View(dev(a), a0, sa), fh.View(dev(b), 1, sb) if cb == 1 else
                         fh.View(dev(b)[..., :cb + 1].contiguous(), 1, sb), op, c))
    exact(got, want, "binary")


@pytest.mark.parametrize("op,a,b", [(0, 1.0, 0.0), (1, -0.5, 0.75), (2, 0.0, 0.0), (3, 0.0, 0.0)])
def test_unary_matches_oracle(op, a, b):
    say("unary", op, a, b)
    fh = fhops()
    rng = np.random.default_rng(op)
    x = rand(rng, (1, 120, 216, 5), -5, 5)
    want = oracle.unary(x, 3, op, a=a, b=b, c0=2, scale=0.5)
    got = host(fh.unary(fh.View(dev(x), 2, 0.5), op, a, b, 3))
    if op == 2:  # 2 / (1 + exp(-v)) - 1 cancels near v = 0: 1 ulp, or 2^-16 of its range (|result| <= 1)
        softmax_close(got, want, 1.0, "unary 2")
    else:
        exact(got, want, f"unary {op}")


@pytest.mark.parametrize("c,c0,scale", [(4, 0, 0.125), (3, 4, 1.0), (72, 0, 1.0)])
def test_chcopy_into_a_concat_slice_matches_oracle(c, c0, scale):
    say("chcopy", c, c0, scale)
    fh = fhops()
    rng = np.random.default_rng(c)
    n, h, w = 1, 30, 54
    x = rand(rng, (n, h, w, c0 + c + 1), -8, 8)
    want = oracle.chcopy(x, c, c0=c0, scale=scale)
    buf = sliced_out(n, h, w, c + 10, 5)
    out = dev(buf)
    fh.chcopy(fh.View(dev(x), c0, scale), c, out=fh.View(out, 5))
    check_slice(buf, out, 5, c, want, "chcopy")


# amp is the range of the quarter-resolution flow (4x that at full resolution): amp 0.4 keeps every tap near its
# pixel, amp 6 scatters them and clamps many at the picture's edges; 118x203 is a size no block shape divides.
@pytest.mark.parametrize("cubic,flags,cs,amp,hw", [(True, 0, 4, 6, (120, 216)), (False, 0, 4, 6, (120, 216)),
                                                   (True, 0, 3, 6, (120, 216)), (True, 1, 4, 6, (120, 216)),
                                                   (False, 2, 4, 6, (120, 216)), (True, 3, 3, 6, (120, 216)),
                                                   (True, 0, 4, 0.4, (120, 216)), (True, 2, 4, 0.4, (118, 203)),
                                                   (True, 1, 4, 2, (120, 216)), (True, 3, 4, 6, (118, 203))])
def test_render_matches_oracle(cubic, flags, cs, amp, hw):
    """Bit-exact except where expf's last bit moves the visibility weights (an f16 ulp or two of the output) or,
    with the decisive blend, flips which picture is trusted where the two weights are equal to the last bit."""
    say("render", cubic, flags, cs, amp, hw)
    fh = fhops()
    rng = np.random.default_rng(7 + flags + 10 * cubic + cs + int(10 * amp) + hw[1])
    (h, w), hq, wq = hw, 30, 54
    ab = rand(rng, (2, h, w, cs), 0, 1)
    up = np.zeros((1, hq, wq, 8), np.float32)
    up[..., :4] = rng.uniform(-amp, amp, (hq, wq, 4))
    up[..., 4:7] = rng.normal(0, 2, (hq, wq, 3))
    up = f16_bits(up)
    rt = rand(rng, (1, hq, wq, 4), -0.1, 0.1)
    want = oracle.render(ab[:1].copy(), ab[1:].copy(), up, up, rt, hq, wq, cubic=cubic, flags=flags, vis_c0=4)
    dab, dup = dev(ab), dev(up)
    got = host(fh.render(dab[0:1], dab[1:2], dup, fh.View(dup, 4), dev(rt), cubic=cubic, flags=flags))
    d = np.abs(got.view(np.float16).astype(np.float32) - want.view(np.float16).astype(np.float32))
    assert np.mean(d == 0) > 0.99, f"only {np.mean(d == 0):.4f} bit-equal"
    assert d.max() <= (0.5 if flags & 1 else 2e-3), d.max()


def test_empty_inputs_are_no_ops_and_bad_views_are_errors():
    import torch
    fh = fhops()
    x = dev(np.zeros((1, 4, 4, 3), np.uint16))
    assert fh.luma(x[:, :0]).shape == (1, 0, 4, 1)
    with pytest.raises(fh.FhcError, match="does not hold"):
        fh.warp(x, x, 5)  # 5 channels from a 3-channel view
    with pytest.raises(fh.FhcError, match="unscaled"):
        fh.sad(fh.View(x, 0, 2.0), x, 1)
    with pytest.raises(fh.FhcError, match="radius"):
        fh.sad(x, x, 8)
    torch.cuda.synchronize()


# ---- the host's 8-bit frames (rgba_in.wgsl, rgba_out.wgsl) and the fused frame-size kernels -------------------------

def _frames(rng, n, h, w):
    return rng.integers(0, 2 ** 32, (n, h, w), dtype=np.uint64).astype(np.uint32)


def dev32(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to("cuda")


def host32(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("n,h,w,hp,wp,cs,c0", [(2, 1080, 1920, 1088, 1920, 4, 0), (1, 37, 53, 64, 64, 4, 0),
                                               (2, 37, 53, 64, 64, 7, 2)])
def test_rgba_in_and_out_match_oracle(n, h, w, hp, wp, cs, c0):
    """Bit-exact: rgba_in's f16 values (BGR, /255, replicate padding) through a 4-channel pixel view (channel 3
    written 0) or a wider view (its other channels untouched), and rgba_out's bytes of the crop."""
    import torch
    say("rgba in/out", n, h, w, hp, wp, cs, c0)
    fh = fhops()
    rng = np.random.default_rng(h + cs)
    fr = _frames(rng, n, h, w)
    want = oracle.rgba_in(fr, hp, wp)
    buf = dev(np.full((n, hp, wp, cs), SENTINEL, np.uint16))
    fh.rgba_in(dev32(fr), hp, wp, out=fh.View(buf, c0))
    got = host(buf)
    exact(got[..., c0:c0 + 3], want, "rgba_in")
    if cs == 4:
        exact(got[..., 3], np.zeros_like(got[..., 3]), "rgba_in channel 3")
    else:
        assert np.all(got[..., :c0] == SENTINEL) and np.all(got[..., c0 + 3:] == SENTINEL)
    # rgba_out of random f16 pictures in [-0.2, 1.2] (clamped) and of rgba_in's own output (the round trip)
    pic = rand(rng, (n, hp, wp, cs), -0.2, 1.2)
    exact(host32(fh.rgba_out(fh.View(dev(pic), c0), h, w)), oracle.rgba_out(pic, h, w, c0=c0), "rgba_out")
    exact(host32(fh.rgba_out(fh.View(buf, c0), h, w)), fr | np.uint32(0xFF000000), "rgba_out(rgba_in)")
    torch.cuda.synchronize()


# the shapes reach each kernel instantiation (taps, window): (5, 40) at 1080p, (5, 48), (8, 80), (8, 48), (6, 48),
# (6, 80), (10, 78) at 2160p (10 taps, a 78-pixel window), (10, 84) at 4096 x 2160 (an 81-pixel window); the 80-,
# 78- and 84-pixel windows hold split 6-byte cells, the others 8-byte cells
@pytest.mark.parametrize("h,w,oh,ow", [(1080, 1920, 480, 864), (150, 300, 64, 128), (61, 97, 30, 40),
                                       (60, 30, 40, 8), (60, 30, 40, 11), (60, 90, 40, 32), (2160, 3840, 480, 864),
                                       (2160, 4096, 480, 864)])
def test_rgba_resize_equals_rgba_in_then_the_antialiased_resize(h, w, oh, ow):
    """The fused frame input against the oracle's rgba_in at the padded size then its antialiased interpolate:
    bit-exact (the same f16 inputs, f32 operations in the same order, one rounding)."""
    say("rgba_resize", h, w, oh, ow)
    fh = fhops()
    rng = np.random.default_rng(w)
    hp, wp = (h + 31) // 32 * 32, (w + 31) // 32 * 32
    fr = _frames(rng, 2, h, w)
    full = oracle.rgba_in(fr, hp, wp)
    want = oracle.interp(full, 3, oh, ow, aa=True)
    got = host(fh.rgba_resize(dev32(fr), hp, wp, oh, ow))
    exact(got[..., :3], want, "rgba_resize")
    exact(got[..., 3], np.zeros_like(got[..., 3]), "rgba_resize channel 3")


def _vis_ties(up, hq, wq, hp, wp, h, w, eps=1e-3):
    """Frame pixels (h, w) whose upsampled visibility logits for A and B lie within eps of each other (f64, the
    render's bilinear map sampling): there the decisive blend's choice of the trusted picture (wa >= wb) can fall
    either way between the host's and the device's expf."""
    vis = up.view(np.float16)[0, ..., 4:6].astype(np.float64)
    sy, sx = np.float32(hq) / np.float32(hp), np.float32(wq) / np.float32(wp)
    iy, ix = (np.arange(h) + 0.5) * sy - 0.5, (np.arange(w) + 0.5) * sx - 0.5
    y0, x0 = np.floor(iy).astype(int), np.floor(ix).astype(int)
    fy, fx = (iy - y0)[:, None, None], (ix - x0)[None, :, None]
    cy0, cy1 = np.clip(y0, 0, hq - 1), np.clip(y0 + 1, 0, hq - 1)
    cx0, cx1 = np.clip(x0, 0, wq - 1), np.clip(x0 + 1, 0, wq - 1)
    v = ((vis[cy0][:, cx0] * (1 - fx) + vis[cy0][:, cx1] * fx) * (1 - fy)
         + (vis[cy1][:, cx0] * (1 - fx) + vis[cy1][:, cx1] * fx) * fy)
    return np.abs(v[..., 0] - v[..., 1]) < eps


def _bytes_diff(a, b):
    diff = np.zeros(a.shape, np.int32)
    for sh in (0, 8, 16, 24):
        diff = np.maximum(diff, np.abs(((a >> sh) & 0xFF).astype(np.int32) - ((b >> sh) & 0xFF).astype(np.int32)))
    return diff


@pytest.mark.parametrize("P,M,flags,size", [(3, 2, 0, (97, 130)), (2, 3, 4, (150, 300)), (1, 2, 3, (64, 80))])
def test_render_rgba_n_equals_one_call_per_frame(P, M, flags, size):
    """The batched frame render (pair p's frames 2p, 2p + 1; phase j's maps and output image j * P + p) against
    one fhc_render_rgba call per generated frame: bit-identical, in the fused and the exact order."""
    import torch
    say("render_rgba_n", P, M, flags, size)
    fh = fhops()
    rng = np.random.default_rng(P * 10 + M)
    h, w = size
    hp, wp = (h + 31) // 32 * 32, (w + 31) // 32 * 32
    hq, wq = hp // 8, wp // 8
    fsx, fsy = float(np.float32(wp) / np.float32(4 * wq)), float(np.float32(hp) / np.float32(4 * hq))
    dfr = dev32(_frames(rng, 2 * P, h, w))
    up = np.zeros((M * P, hq, wq, 8), np.float32)
    up[..., :4] = rng.uniform(-6, 6, (M * P, hq, wq, 4))
    up[..., 4:7] = rng.normal(0, 2, (M * P, hq, wq, 3))
    dup, drt = dev(f16_bits(up)), dev(rand(rng, (M * P, hq, wq, 4), -0.1, 0.1))
    got = host32(fh.render_rgba_n(dfr, dup, fh.View(dup, 4), drt, hp, wp, M, flags=flags, fsx=fsx, fsy=fsy))
    for p in range(P):
        for j in range(M):
            i = j * P + p
            one = host32(fh.render_rgba(dfr[2 * p:2 * p + 1], dfr[2 * p + 1:2 * p + 2], dup[i:i + 1],
                                        fh.View(dup[i:i + 1], 4), drt[i:i + 1], hp, wp, flags=flags, fsx=fsx, fsy=fsy))
            exact(got[i:i + 1], one, f"render_rgba_n frame {i} (pair {p}, phase {j})")
    torch.cuda.synchronize()


@pytest.mark.parametrize("cubic,flags,amp,size,qdiv", [(True, 0, 6, (1080, 1920), 9), (False, 0, 6, (1080, 1920), 9),
                                                       (True, 2, 3, (150, 300), 9), (True, 3, 6, (150, 300), 9),
                                                       (False, 3, 2, (97, 130), 9), (True, 0, 40, (97, 130), 9),
                                                       (True, 0, 6, (97, 130), 1.5), (True, 3, 3, (150, 300), 1.5),
                                                       (True, 1, 6, (150, 300), 9)])
def test_render_rgba_matches_rgba_in_render_rgba_out(cubic, flags, amp, size, qdiv):
    """The fused frame-size render from the RGBA8 frames to the RGBA8 frame, against the oracle's rgba_in (padded),
    render at the padded size with the flow scaled per axis (the internal-size mode, maps at a non-integer ratio),
    and rgba_out. In the exact f32 order (flag bit 2): bit-identical to the GPU's own unfused composition (the same
    device expf) and bytes within 1 of the oracle (expf's last bit can move an f16 result next to a byte boundary),
    almost all identical. In the frame path's fused multiply-adds (bit 2 clear): bytes within 1 of the oracle, almost
    all identical. With the decisive blend the pixels whose visibility weights for A and B tie are left out of the
    1-byte bound (its choice of the trusted picture can fall either way there), and they must be few. amp: the range
    of the map-size flow; 40 sends taps far outside the frame (clamped). qdiv: frame rows per quarter-map row (9 as
    in the frame, 1.5 a mild upscale; with odd frame heights)."""
    import torch
    say("render_rgba", cubic, flags, amp, size, qdiv)
    fh = fhops()
    rng = np.random.default_rng(int(amp) + flags + 10 * cubic + size[1])
    h, w = size
    hp, wp = (h + 31) // 32 * 32, (w + 31) // 32 * 32
    hq, wq = max(2, int(hp // qdiv)), max(2, int(wp // qdiv))
    fsx, fsy = float(np.float32(wp) / np.float32(4 * wq)), float(np.float32(hp) / np.float32(4 * hq))
    fr = _frames(rng, 2, h, w)
    if flags & 2:  # make B mostly equal to A so the still test fires somewhere
        fr[1] = np.where(rng.uniform(size=(h, w)) < 0.7, fr[0], fr[1])
    up = np.zeros((1, hq, wq, 8), np.float32)
    up[..., :4] = rng.uniform(-amp, amp, (hq, wq, 4))
    up[..., 4:7] = rng.normal(0, 2, (hq, wq, 3))
    up = f16_bits(up)
    rt = rand(rng, (1, hq, wq, 4), -0.1, 0.1)
    full = oracle.rgba_in(fr, hp, wp, cs=4)
    pic = oracle.render(full[:1].copy(), full[1:].copy(), up, up, rt, hq, wq, cubic=cubic, flags=flags, vis_c0=4,
                        fsx=fsx, fsy=fsy)
    want = oracle.rgba_out(pic, h, w)
    ties = (_vis_ties(up, hq, wq, hp, wp, h, w) if flags & 1 else np.zeros((h, w), bool))[None]
    assert ties.mean() < 0.01
    dfr, dup, drt = dev32(fr), dev(up), dev(rt)
    for mode, bits, same in (("exact order", 4, 0.999), ("fused multiply-adds", 0, 0.995)):
        got = host32(fh.render_rgba(dfr[0:1], dfr[1:2], dup, fh.View(dup, 4), drt, hp, wp, cubic=cubic,
                                    flags=flags | bits, fsx=fsx, fsy=fsy))
        diff = _bytes_diff(got, want)
        say(f"  {mode}: max byte diff {diff.max()} ({diff[~ties].max()} off the {int(ties.sum())} ties), "
            f"{np.mean(diff == 0):.6f} identical")
        assert diff[~ties].max() <= 1 and np.mean(diff == 0) > same, mode
        if bits:
            exact_got = got
    # the GPU's unfused path: rgba_in, render, rgba_out
    dfull = fh.rgba_in(dfr, hp, wp)
    dpic = fh.render(dfull[0:1], dfull[1:2], dup, fh.View(dup, 4), drt, cubic=cubic, flags=flags, fsx=fsx, fsy=fsy)
    exact(exact_got, host32(fh.rgba_out(dpic, h, w)), "render_rgba (exact order) against the unfused GPU composition")
    torch.cuda.synchronize()
