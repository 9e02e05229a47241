"""Pins the CPU oracle of the network ops around the convs (oracle/fh_ops_oracle.c) without the reference running.

The reference's tests hold no vectors for these ops (its warp tests cover the camera warp, a different feature), so
each op is checked against what its mathematics fixes: identities, exact shifted copies, closed forms on ramps and
constants, softmax invariants, and torch's CPU interpolate, which shaders/interp.wgsl:1-3 says it matches. Each check
is chosen so that a plausible slip (swapped flow channels, a wrong clamp, mirrored weights, a wrong softmax channel
order, a batch index ignored) fails it.
"""
import os
import sys

import numpy as np
import pytest

sys.path.insert(0, os.path.join(os.path.dirname(__file__), "..", "oracle"))
import oracle  # noqa: E402


def f16(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16)).view(np.uint16)


def val(a):
    return a.view(np.float16).astype(np.float32)


def ulp_close(got, want, ulps=1):
    """|got - want| within `ulps` f16 units of the larger magnitude (denormal floor 2^-24)."""
    g, w = val(got), np.asarray(want, np.float32)
    unit = np.maximum(np.spacing(np.maximum(np.abs(g), np.abs(w)).astype(np.float16)).astype(np.float32), 2.0 ** -24)
    return np.all(np.abs(g - w) <= ulps * unit + 1e-30)


rng = np.random.default_rng(7)


# ---- warp (shaders/warp.wgsl) ---------------------------------------------------------------------------------

def test_warp_zero_flow_is_identity_and_views_are_honoured():
    img = f16(rng.uniform(-2, 2, (2, 9, 13, 6)))
    flow = np.zeros((2, 9, 13, 5), np.uint16)
    out = oracle.warp(img, flow, 4, img_c0=2, flow_c0=3)
    assert np.array_equal(out, img[..., 2:6])


def test_warp_integer_flow_is_a_clamped_shift():
    n, h, w, c = 2, 10, 12, 3
    img = f16(rng.uniform(-1, 1, (n, h, w, c)))
    flow = np.zeros((n, h, w, 2), np.float32)
    flow[0, ..., 0], flow[0, ..., 1] = 2.0, -1.0  # image 0: x + 2, y - 1
    flow[1, ..., 0], flow[1, ..., 1] = -3.0, 4.0  # image 1: x - 3, y + 4
    out = oracle.warp(img, f16(flow), c)
    for b, (dx, dy) in enumerate(((2, -1), (-3, 4))):
        ys = np.clip(np.arange(h) + dy, 0, h - 1)
        xs = np.clip(np.arange(w) + dx, 0, w - 1)
        assert np.array_equal(out[b], img[b][ys][:, xs])


def test_warp_fractional_flow_on_a_ramp_and_the_scales():
    h, w = 5, 40
    ramp = np.broadcast_to((np.arange(w, dtype=np.float32) / 64)[None, :, None], (h, w, 1))
    img = f16(ramp[None])
    flow = np.zeros((1, h, w, 2), np.float32)
    flow[..., 0] = 0.125  # read scale 2: a quarter pixel to the right
    out = oracle.warp(img, f16(flow), 1, flow_scale=2.0, img_scale=0.5)
    want = np.minimum(np.arange(w) + 0.25, w - 1) / 64 * 0.5  # the last column clamps onto itself
    assert np.array_equal(val(out)[0, :, :, 0], np.broadcast_to(want.astype(np.float32), (h, w)))
    flow[..., 0], flow[..., 1] = 0.0, 0.5  # vertical: a vertical ramp
    vimg = f16(np.broadcast_to((np.arange(h, dtype=np.float32) / 8)[:, None, None], (h, w, 1))[None])
    outv = oracle.warp(vimg, f16(flow), 1)
    wantv = np.minimum(np.arange(h) + 0.5, h - 1) / 8
    assert np.array_equal(val(outv)[0, :, 0, 0], wantv.astype(np.float32))


# ---- luma and luma_grad (shaders/luma.wgsl) ---------------------------------------------------------------------

def test_luma_weights_follow_bgr_order_and_scale():
    x = np.zeros((1, 1, 3, 5), np.float32)
    for ch in range(3):
        x[0, 0, ch, 1 + ch] = 1.0  # view channel ch of pixel ch (view c0 = 1)
    out = val(oracle.luma(f16(x), c0=1, scale=2.0))[0, 0, :, 0]
    want = np.array([0.114, 0.587, 0.299], np.float32) * 2  # channel 0 is B, 2 is R
    assert ulp_close(f16(out), want)
    assert not ulp_close(f16(out), want[::-1])


def test_luma_grad_of_constant_is_zero_and_of_a_ramp_is_its_slope():
    const = f16(np.full((1, 6, 7, 3), 0.75, np.float32))
    assert np.all(val(oracle.luma(const, grad=True)) == 0)
    ramp = np.broadcast_to((np.arange(8, dtype=np.float32) / 32)[None, :, None], (5, 8, 3))[None]
    g = val(oracle.luma(f16(ramp), grad=True))[0, :, :, 0]
    assert np.allclose(g[:, :-1], 1 / 32, atol=2e-4)  # the sum of the three weights is 1 up to f32 rounding
    assert np.all(g[:, -1] == 0)  # no right neighbour, and no change downwards


# ---- sad_volume (shaders/sad.wgsl) -------------------------------------------------------------------------------

def test_sad_of_a_shifted_copy_is_zero_in_its_displacement_channel():
    r, h, w = 3, 16, 20
    big = f16(rng.uniform(0, 1, (h + 8, w + 8)))
    dy0, dx0 = 2, -1
    la = big[4:4 + h, 4:4 + w][None, :, :, None].copy()
    lb = big[4 - dy0:4 - dy0 + h, 4 - dx0:4 - dx0 + w][None, :, :, None].copy()  # lb(y + dy0, x + dx0) = la(y, x)
    out = val(oracle.sad(la, lb, r))[0]
    ch = (dy0 + r) * (2 * r + 1) + dx0 + r
    inner = out[1 + max(0, -dy0) + 1:h - 1 - max(0, dy0) - 1, 1 + max(0, -dx0) + 1:w - 1 - max(0, dx0) - 1, ch]
    assert inner.size and np.all(inner == 0)
    assert np.all(out[1:-1, 1:-1, ch ^ 1] > 0)  # a neighbouring displacement is not zero
    same = val(oracle.sad(la, la, r))[0, :, :, r * (2 * r + 1) + r]
    assert np.all(same == 0)


def test_sad_of_constants_counts_the_window_inside_the_image():
    h, w, r = 6, 7, 2
    la = f16(np.full((2, h, w, 1), 0.75, np.float32))
    lb = f16(np.full((2, h, w, 1), 0.25, np.float32))
    out = val(oracle.sad(la, lb, r))
    cy = np.array([2] + [3] * (h - 2) + [2])
    cx = np.array([2] + [3] * (w - 2) + [2])
    count = (cy[:, None] * cx[None, :]).astype(np.float32)
    want = np.float16(np.float32(0.5) * count / np.float32(9))  # 0.5 summed `count` times is exact in f32
    assert np.all(out == want.astype(np.float32)[None, :, :, None])


# ---- convex upsample (shaders/convex.wgsl) -----------------------------------------------------------------------

def test_convex_with_equal_weights_is_a_zero_padded_box_average():
    n, h, w, c = 2, 5, 6, 3
    x = f16(rng.uniform(-1, 1, (n, h, w, c)))
    wt = np.zeros((n, h, w, 36), np.uint16)
    out = val(oracle.convex(wt, x, c))
    xp = np.pad(val(x), ((0, 0), (1, 1), (1, 1), (0, 0)))
    box = sum(xp[:, ky:ky + h, kx:kx + w] for ky in range(3) for kx in range(3)) / 9
    want = np.repeat(np.repeat(box, 2, axis=1), 2, axis=2)
    assert ulp_close(f16(out), want, ulps=2)


def test_convex_with_one_dominant_weight_picks_that_neighbour():
    n, h, w, c = 1, 4, 5, 2
    x = f16(rng.uniform(-1, 1, (n, h, w, c)))
    wt = np.zeros((n, h, w, 40), np.float32)
    pick = {(0, 0): 0, (0, 1): 5, (1, 0): 7, (1, 1): 4}  # sub-pixel (sy, sx) -> neighbour k
    for (sy, sx), k in pick.items():
        wt[..., 4 + k * 4 + sy * 2 + sx] = 40.0  # a view at channel offset 4
    out = val(oracle.convex(f16(wt), x, c, wt_c0=4))
    xp = np.pad(val(x), ((0, 0), (1, 1), (1, 1), (0, 0)))
    for (sy, sx), k in pick.items():
        ky, kx = divmod(k, 3)
        assert np.array_equal(out[:, sy::2, sx::2], xp[:, ky:ky + h, kx:kx + w])


# ---- film_modulate (shaders/film.wgsl) ---------------------------------------------------------------------------

def test_film_identity_scale_and_shift_per_image():
    n, h, w, c = 2, 3, 4, 5
    hv = f16(rng.uniform(-1, 1, (n, h, w, c + 2)))
    g = np.zeros((n, 2 * c), np.float32)
    assert np.array_equal(oracle.film(hv, f16(g), c, c0=2), hv[..., 2:])
    g[0, :c] = 1.0  # image 0: doubled
    g[1, c:] = np.arange(c) / 4  # image 1: shifted per channel
    out = val(oracle.film(hv, f16(g), c, c0=2))
    assert np.array_equal(out[0], 2 * val(hv)[0, ..., 2:])
    assert ulp_close(f16(out[1]), val(hv)[1, ..., 2:] + np.arange(c, dtype=np.float32) / 4)


# ---- blend_weights and blendmix (shaders/blend.wgsl, blendmix.wgsl) ---------------------------------------------------

def test_blend_weights_invariants():
    vis = np.zeros((2, 3, 4, 3), np.float32)
    out = val(oracle.blend(f16(vis)))
    assert ulp_close(f16(out), np.full(out.shape, 0.5, np.float32))  # equal logits: 1/3 + 1/6 each
    vis[0, ..., 0] = 12.0  # class A dominates, read at scale 2
    vis[1, ..., 2] = 12.0  # the shared class dominates
    out = val(oracle.blend(f16(vis), scale=2.0))
    assert np.all(out[0, ..., 0] > 0.999) and np.all(out[0, ..., 1] < 1e-3)
    assert ulp_close(f16(out[1]), np.full(out[1].shape, 0.5, np.float32))
    rnd = val(oracle.blend(f16(rng.normal(0, 3, (1, 8, 8, 3)))))
    assert np.allclose(rnd.sum(-1), 1.0, atol=2e-3) and np.all(rnd >= 0)


def test_blendmix_is_the_blend_of_the_two_images():
    n, h, w = 1, 6, 5
    wa, wb = f16(rng.uniform(0, 1, (n, h, w, 3))), f16(rng.uniform(0, 1, (n, h, w, 3)))
    vis = np.zeros((n, h, w, 4), np.float32)
    vis[:, :3, :, 1] = 30.0  # rows 0-2: class A (view c0 = 1); rows 3-5: class B
    vis[:, 3:, :, 2] = 30.0
    out = val(oracle.blendmix(wa, wb, f16(vis), vis_c0=1))
    assert np.array_equal(out[:, :3], val(wa)[:, :3])
    assert np.array_equal(out[:, 3:], val(wb)[:, 3:])
    logits = f16(rng.normal(0, 2, (n, h, w, 3)))
    bw = val(oracle.blend(logits))
    mix = val(oracle.blendmix(wa, wb, logits))
    want = val(wa) * bw[..., :1] + val(wb) * bw[..., 1:2]
    assert np.allclose(mix, want, atol=2e-3)


# ---- avgpool (shaders/avgpool.wgsl) ------------------------------------------------------------------------------

@pytest.mark.parametrize("k", [1, 2, 4])
def test_avgpool_is_the_block_mean(k):
    n, h, w, c = 2, 9, 14, 3  # h, w not multiples of k: the remainder rows and columns are dropped
    x = f16(rng.uniform(-1, 1, (n, h, w, c + 1)))
    out = oracle.avgpool(x, c, k, c0=1)
    oh, ow = h // k, w // k
    blocks = val(x)[:, :oh * k, :ow * k, 1:].reshape(n, oh, k, ow, k, c).mean(axis=(2, 4))
    if k == 1:
        assert np.array_equal(out, x[..., 1:])
    assert ulp_close(out, blocks)


# ---- interpolate (shaders/interp.wgsl) ---------------------------------------------------------------------------

def _torch_resize(x, c, oh, ow, aa):
    torch = pytest.importorskip("torch")
    t = torch.from_numpy(val(x)[..., :c].copy()).permute(0, 3, 1, 2)
    y = torch.nn.functional.interpolate(t, size=(oh, ow), mode="bilinear", align_corners=False, antialias=aa)
    return y.permute(0, 2, 3, 1).numpy()


@pytest.mark.parametrize("ih,iw,oh,ow,aa", [(8, 12, 16, 24, False), (30, 54, 60, 108, False), (13, 7, 5, 3, False),
                                            (120, 216, 30, 54, True), (24, 40, 12, 20, True), (17, 23, 5, 11, True)])
def test_interp_matches_torch_bilinear(ih, iw, oh, ow, aa):
    x = f16(rng.uniform(-1, 1, (2, ih, iw, 3)))
    out = oracle.interp(x, 3, oh, ow, aa=aa)
    assert ulp_close(out, _torch_resize(x, 3, oh, ow, aa), ulps=2)


def test_interp_same_size_is_a_copy_and_scale_applies():
    x = f16(rng.uniform(-1, 1, (1, 7, 9, 4)))
    assert np.array_equal(oracle.interp(x, 4, 7, 9), x)
    assert np.array_equal(oracle.interp(x, 2, 7, 9, aa=True, c0=1), x[..., 1:3])  # triangle of width 1 at scale 1
    assert np.array_equal(val(oracle.interp(x, 4, 7, 9, scale=0.5)), val(x) * 0.5)


# ---- elementwise: binary, unary, chcopy (shaders/binary.wgsl, unary.wgsl, chcopy.wgsl) ----------------------------
# The f32 operation of each element is one IEEE operation (or two) followed by one RTNE rounding, which numpy's
# float32 arithmetic and float16 conversion perform identically: these are exact checks.

def test_binary_add_mul_and_broadcast_match_numpy_float32():
    a, b = f16(rng.uniform(-4, 4, (2, 5, 7, 6))), f16(rng.uniform(-4, 4, (2, 5, 7, 3)))
    A, B = val(a)[..., 1:5], val(b)[..., 2:3]
    got = oracle.binary(a, b, 4, op=0, a_c0=1, a_scale=0.5, b_c0=2, b_scale=-2.0, cb=1)
    want = (A * np.float32(0.5) + B * np.float32(-2.0)).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    got = oracle.binary(a, b, 3, op=1, b_c0=0)
    want = (val(a)[..., :3] * val(b)[..., :3]).astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_unary_ops_match_their_closed_forms():
    x = f16(rng.uniform(-6, 6, (1, 4, 9, 3)))
    v = val(x) * np.float32(2.0)
    assert np.array_equal(oracle.unary(x, 3, 0, a=0.25, scale=2.0), (v * np.float32(0.25)).astype(np.float16).view(np.uint16))
    assert np.array_equal(oracle.unary(x, 3, 1, a=-1.0, b=1.5, scale=2.0), np.clip(v, -1, 1.5).astype(np.float16).view(np.uint16))
    assert np.array_equal(oracle.unary(x, 3, 3, scale=2.0), (-v).astype(np.float16).view(np.uint16))
    aff = val(oracle.unary(x, 3, 2))
    assert np.allclose(aff, np.tanh(val(x) / 2), atol=1e-3)  # 2 sigmoid(v) - 1 = tanh(v / 2)
    assert np.all(np.abs(aff) <= 1)


def test_chcopy_copies_bits_at_scale_one_and_rounds_scaled_values():
    x = np.ascontiguousarray(rng.integers(0, 0x7C00, (1, 3, 4, 6)).astype(np.uint16))  # finite f16 patterns
    assert np.array_equal(oracle.chcopy(x, 4, c0=2), x[..., 2:])
    got = oracle.chcopy(x, 3, c0=1, scale=0.125)
    assert np.array_equal(got, (val(x)[..., 1:4] * np.float32(0.125)).astype(np.float16).view(np.uint16))


# ---- render_pix (shaders/render.wgsl) ------------------------------------------------------------------------------

def _render_maps(hq, wq, flow=(0.0, 0.0, 0.0, 0.0), logits=(0.0, 0.0, 0.0), r=0.0):
    fl = np.zeros((1, hq, wq, 4), np.float32) + np.asarray(flow, np.float32)
    vis = np.zeros((1, hq, wq, 3), np.float32) + np.asarray(logits, np.float32)
    return f16(fl), f16(vis), f16(np.full((1, hq, wq, 3), r, np.float32))


@pytest.mark.parametrize("cubic", [False, True])
def test_render_of_still_equal_pictures_is_the_picture_plus_the_residual(cubic):
    h, w = 16, 24
    pic = f16(rng.uniform(0.1, 0.8, (1, h, w, 3)))
    fl, vis, rt = _render_maps(h // 4, w // 4)
    assert np.array_equal(oracle.render(pic, pic, fl, vis, rt, h // 4, w // 4, cubic=cubic), pic)  # cubw(0) = e1
    fl, vis, rt = _render_maps(h // 4, w // 4, r=0.125)
    got = val(oracle.render(pic, pic, fl, vis, rt, h // 4, w // 4, cubic=cubic))
    assert ulp_close(f16(got), np.minimum(val(pic) + np.float32(0.125), 1))


@pytest.mark.parametrize("cubic", [False, True])
def test_render_warp_matches_torch_grid_sample(cubic):
    """render.wgsl:6-7 names its sampler: torch.grid_sample with align_corners=True and border padding (bicubic: Keys
    a = -0.75, which does not reproduce linear ramps, so a library check rather than a closed form)."""
    torch = pytest.importorskip("torch")
    h, w = 20, 28
    pic = f16(rng.uniform(0.05, 0.95, (1, h, w, 3)))
    fx, fy = 1.3, -0.6
    fl, vis, rt = _render_maps(h // 4, w // 4, flow=(fx, fy, 0.0, 0.0), logits=(40.0, 0.0, 0.0))
    got = val(oracle.render(pic, pic, fl, vis, rt, h // 4, w // 4, cubic=cubic))
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    grid = np.stack([-1 + 2 * (xx + fx) / (w - 1), -1 + 2 * (yy + fy) / (h - 1)], -1)[None]
    t = torch.from_numpy(val(pic).astype(np.float64)).permute(0, 3, 1, 2)
    ref = torch.nn.functional.grid_sample(t, torch.from_numpy(grid), mode="bicubic" if cubic else "bilinear",
                                          padding_mode="border", align_corners=True)
    want = np.clip(ref.permute(0, 2, 3, 1).numpy(), 0, 1)
    assert np.allclose(got, want, atol=2e-3)


@pytest.mark.parametrize("cubic", [False, True])
def test_render_in_row_bands_on_threads_equals_one_pass(cubic):
    """The render's row bands (each output pixel computed alone) on several threads give the one-pass result bit for
    bit, bands of unequal length and random maps included."""
    h, w, hq, wq = 150, 44, 37, 11
    a, b = f16(rng.uniform(0, 1, (1, h, w, 3))), f16(rng.uniform(0, 1, (1, h, w, 3)))
    fl, vis, rt = f16(rng.uniform(-3, 3, (1, hq, wq, 4))), f16(rng.uniform(-2, 2, (1, hq, wq, 3))), \
        f16(rng.uniform(-0.1, 0.1, (1, hq, wq, 3)))
    one = oracle.render(a, b, fl, vis, rt, hq, wq, cubic=cubic, fsx=1.5, fsy=0.75)
    for threads in (2, 3, 7):
        assert np.array_equal(oracle.render(a, b, fl, vis, rt, hq, wq, cubic=cubic, fsx=1.5, fsy=0.75,
                                            threads=threads), one)


def test_render_visibility_picks_the_dominant_picture_and_clamps():
    h, w = 8, 8
    a, b = f16(np.full((1, h, w, 3), 0.25, np.float32)), f16(np.full((1, h, w, 3), 0.75, np.float32))
    for logits, want in (((30.0, 0.0, 0.0), 0.25), ((0.0, 30.0, 0.0), 0.75), ((0.0, 0.0, 30.0), 0.5)):
        fl, vis, rt = _render_maps(2, 2, logits=logits)
        assert ulp_close(oracle.render(a, b, fl, vis, rt, 2, 2), np.full((1, h, w, 3), want, np.float32))
    fl, vis, rt = _render_maps(2, 2, r=0.5)
    assert np.all(val(oracle.render(b, b, fl, vis, rt, 2, 2)) == 1.0)  # 0.75 + 0.5 clamps to 1


def test_render_decisive_blend_takes_the_trusted_picture_where_they_disagree():
    h, w = 8, 8
    a, b = f16(np.full((1, h, w, 3), 0.2, np.float32)), f16(np.full((1, h, w, 3), 0.8, np.float32))
    fl, vis, rt = _render_maps(2, 2, logits=(1.0, 0.0, 0.0), r=0.05)
    soft = val(oracle.render(a, b, fl, vis, rt, 2, 2))
    hard = val(oracle.render(a, b, fl, vis, rt, 2, 2, flags=1))
    assert np.all(soft > 0.3) and np.allclose(hard, 0.2, atol=1e-3)  # |A - B| = 0.6 >> 0.12: k = 1, no residual


def _stripes(h, w, lo, hi):
    """A still picture whose columns alternate lo / hi (all 3 channels)."""
    col = np.where(np.arange(w) % 2 == 0, lo, hi).astype(np.float32)
    return f16(np.broadcast_to(col[None, None, :, None], (1, h, w, 3)))


def test_render_still_test_keeps_a_still_picture_where_the_flow_disagrees():
    """render.wgsl:134-148 (flags bit 1). A == B, so es = 0 < 0.03 and own = A. A's flow moves one column, B's none:
    on stripes of 0.2 / 0.8 the two warped pictures differ by 0.6 >= 0.04, so stillw = 1 and the output is the still
    picture itself (the plain blend would give 0.5 grey); at the last column both warps read the same pixel, ef = 0,
    and the blend is the picture too."""
    h, w = 8, 12
    pic = _stripes(h, w, 0.2, 0.8)
    fl, vis, rt = _render_maps(2, 3, flow=(1.0, 0.0, 0.0, 0.0))
    got = oracle.render(pic, pic, fl, vis, rt, 2, 3, cubic=False, flags=2)
    assert np.array_equal(got, pic)
    plain = val(oracle.render(pic, pic, fl, vis, rt, 2, 3, cubic=False, flags=0))
    assert np.allclose(plain[:, :, :-1], 0.5, atol=1e-3)


def test_render_still_test_weight_ramps_with_the_flow_disagreement():
    """stillw = clamp((ef - es) / 0.04, 0, 1): stripes 0.49 / 0.51 give ef = |0.49 - 0.51| (their f16 values), about
    half of 0.04, so the output is the blend (0.5 with equal logits) mixed halfway toward the picture."""
    h, w = 6, 10
    pic = _stripes(h, w, 0.49, 0.51)
    fl, vis, rt = _render_maps(2, 2, flow=(1.0, 0.0, 0.0, 0.0))
    got = val(oracle.render(pic, pic, fl, vis, rt, 2, 2, cubic=False, flags=2))[0, :, :-1, 0]
    p = val(pic)[0, :, :-1, 0].astype(np.float64)
    q = val(pic)[0, :, 1:, 0].astype(np.float64)     # A warped one column
    ef = np.abs(q - p)
    stillw = np.clip(ef / 0.04, 0, 1)
    blend = 0.5 * q + 0.5 * p
    want = blend * (1 - stillw) + p * stillw
    assert 0.3 < stillw.min() and stillw.max() < 0.7
    assert ulp_close(f16(got), want.astype(np.float32), ulps=1)


def test_render_still_test_is_off_where_the_pictures_differ():
    """es >= 0.03 (A and B differ by 0.1 everywhere) makes stillw 0: the still test changes nothing."""
    h, w = 8, 12
    a = f16(rng.uniform(0.1, 0.8, (1, h, w, 3)))
    b = f16(val(a) + np.float32(0.1))
    fl, vis, rt = _render_maps(2, 3, flow=(0.7, -0.4, -0.3, 0.5), logits=(0.5, -0.2, 0.1), r=0.02)
    for cubic in (False, True):
        assert np.array_equal(oracle.render(a, b, fl, vis, rt, 2, 3, cubic=cubic, flags=2),
                              oracle.render(a, b, fl, vis, rt, 2, 3, cubic=cubic, flags=0))


def test_render_at_a_non_integer_ratio_upsamples_and_scales_the_flow():
    """The internal-size render (net/build.rs:717-736): maps at hq x wq, the output at a padded frame size about 9x
    larger per axis (the 1080p case is 120 x 216 -> 1088 x 1920), the flow's x scaled by fsx and y by fsy. A flow
    that is linear in x at map resolution upsamples to F(x) = a * ix + b with ix = (x + 0.5) * wq / w - 0.5 (away
    from the clamped border), and a bilinear warp of a linear ramp picture is exact, so the output is the ramp at
    x + fsx * F(x) (y: a constant flow times fsy over a picture constant in y)."""
    hq, wq, h, w = 6, 11, 56, 96
    fsx, fsy = 2.25, 2.0
    a_, b_ = 0.25, 0.5
    qx = np.arange(wq, dtype=np.float32)
    fl = np.zeros((1, hq, wq, 4), np.float32)
    fl[..., 0] = a_ * qx[None, None, :] + b_
    fl[..., 1] = 0.75
    c, d = 1.0 / 256, 0.125
    xs = np.arange(w, dtype=np.float32)
    pic = f16(np.broadcast_to((c * xs + d)[None, None, :, None], (1, h, w, 3)))
    vis = f16(np.zeros((1, hq, wq, 3), np.float32) + np.asarray((40.0, 0.0, 0.0), np.float32))
    rt = f16(np.zeros((1, hq, wq, 3), np.float32))
    got = val(oracle.render(pic, pic, f16(fl), vis, rt, hq, wq, cubic=False, fsx=fsx, fsy=fsy))[0]
    ix = (xs.astype(np.float64) + 0.5) * wq / w - 0.5
    F = a_ * ix + b_
    want = c * (xs + fsx * F) + d
    inner = (ix >= 0) & (ix <= wq - 1) & (xs + fsx * F <= w - 1)
    assert inner.sum() > w // 2
    assert np.allclose(got[:, inner, 0], want[None, inner], atol=2e-3)
    # a y-flow scaled by fsx instead of fsy, or the map ratio taken from the wrong size, fails the check above or
    # this one: the y flow over a picture constant in y changes nothing
    assert np.allclose(got[:, inner, 1], want[None, inner], atol=2e-3)


def test_render_at_the_1080p_internal_ratio_matches_torch_grid_sample():
    """The internal-size render at the 1080p ratios (maps 120 x 216, output 1088 x 1920 rows scaled down by 8 to keep
    the check fast: 15 x 27 -> 136 x 240) with a constant flow: torch's grid_sample (bicubic, align_corners, border)
    of the picture at (x + fx * fsx, y + fy * fsy)."""
    torch = pytest.importorskip("torch")
    hq, wq, h, w = 15, 27, 136, 240
    fsx, fsy = 1920 / 864, 1088 / 480
    fx, fy = 1.5, -0.75
    pic = f16(rng.uniform(0.05, 0.95, (1, h, w, 3)))
    fl, vis, rt = _render_maps(hq, wq, flow=(fx, fy, 0.0, 0.0), logits=(40.0, 0.0, 0.0))
    got = val(oracle.render(pic, pic, fl, vis, rt, hq, wq, cubic=True, fsx=fsx, fsy=fsy))
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float64)
    gx, gy = xx + fx * np.float32(fsx), yy + fy * np.float32(fsy)
    grid = np.stack([-1 + 2 * gx / (w - 1), -1 + 2 * gy / (h - 1)], -1)[None]
    t = torch.from_numpy(val(pic).astype(np.float64)).permute(0, 3, 1, 2)
    ref = torch.nn.functional.grid_sample(t, torch.from_numpy(grid), mode="bicubic", padding_mode="border",
                                          align_corners=True)
    want = np.clip(ref.permute(0, 2, 3, 1).numpy(), 0, 1)
    assert np.allclose(got, want, atol=2e-3)


# ---- the host's 8-bit frames (shaders/rgba_in.wgsl, rgba_out.wgsl) ---------------------------------------------------

def _rgba(r, g, b, a=255):
    return (np.uint32(r) | (np.uint32(g) << 8) | (np.uint32(b) << 16) | (np.uint32(a) << 24)).astype(np.uint32)


def test_rgba_in_is_bgr_over_255_for_every_byte():
    """Channel 0 is blue (bits 16-23), 1 green, 2 red; each is the f16 of byte / 255 (numpy's float16 rounding of
    the exact quotient, every byte); alpha is ignored."""
    v = np.arange(256, dtype=np.uint32)
    frames = np.stack([_rgba(v, 0, 0, 7), _rgba(0, v, 0, 0), _rgba(0, 0, v, 255)])[:, None, :]  # (3, 1, 256)
    x = oracle.rgba_in(frames, 1, 256)
    unit = (v.astype(np.float64) / 255.0).astype(np.float16).view(np.uint16)
    zero = np.zeros(256, np.uint16)
    assert np.array_equal(x[0, 0, :, 2], unit) and np.array_equal(x[0, 0, :, :2], np.stack([zero, zero], -1))
    assert np.array_equal(x[1, 0, :, 1], unit) and np.array_equal(x[1, 0, :, 0], zero)
    assert np.array_equal(x[2, 0, :, 0], unit) and np.array_equal(x[2, 0, :, 1], zero)


def test_rgba_in_replicates_the_last_row_and_column_into_the_padding():
    f = rng.integers(0, 2 ** 32, (1, 5, 7), dtype=np.uint64).astype(np.uint32)
    x = oracle.rgba_in(f, 8, 12)
    assert np.array_equal(x[:, :5, :7], oracle.rgba_in(f, 5, 7))
    assert np.array_equal(x[:, 5:, :7], np.broadcast_to(x[:, 4:5, :7], (1, 3, 7, 3)))
    assert np.array_equal(x[:, :, 7:], np.broadcast_to(x[:, :, 6:7], (1, 8, 5, 3)))


def test_rgba_out_quantizes_every_f16_and_round_trips_every_byte():
    """q(v) = floor(clamp(v, 0, 1) * 255 + 0.5) for every non-NaN f16 pattern (WGSL leaves clamp of a NaN to the
    implementation; a rendered picture holds none), the BGR -> R | G << 8 | B << 16 packing with alpha 255, and
    rgba_out(rgba_in(f)) == f with alpha 255 for every byte in every channel."""
    pats = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = np.zeros((1, 256, 256, 3), np.uint16)
    x[..., 0] = pats.reshape(256, 256)
    got = oracle.rgba_out(x, 256, 256)[0].ravel()
    v = pats.view(np.float16).astype(np.float64)
    q = np.floor(np.clip(np.nan_to_num(v, nan=0.0), 0, 1) * 255 + 0.5).astype(np.uint32)
    ok = ~np.isnan(v)
    assert ok.sum() == 65536 - 2046
    assert np.array_equal(got[ok], ((q << 16) | 0xff000000)[ok])
    b = np.arange(256, dtype=np.uint32)
    f = _rgba(b, b[::-1], (b * 7) % 256, 3)[None, None, :]
    assert np.array_equal(oracle.rgba_out(oracle.rgba_in(f, 1, 256), 1, 256), f | np.uint32(0xff000000))


def test_rgba_out_crops_the_padding():
    f = rng.integers(0, 2 ** 32, (2, 5, 7), dtype=np.uint64).astype(np.uint32)
    x = oracle.rgba_in(f, 32, 32, cs=4)
    assert np.array_equal(oracle.rgba_out(x, 5, 7), f | np.uint32(0xff000000))
