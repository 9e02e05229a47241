"""Bit-exact padding, stride and indexing of every conv kernel family on the GPU, by closed forms (no oracle):

- delta input (one input pixel of one channel is 1, the rest 0; bias 0, no activation): each output is the one
  weight tap that pixel meets, f16(1 * w) = w exactly, or +0 where it meets none;
- delta weight (one tap of one input channel into one output channel is 1): that output channel is the input
  channel shifted by the tap (zero where the tap falls in the padding), every other channel +0;
- all ones (input and weights 1): each output is cin times the number of taps inside the image (4, 6 or 9 at the
  borders and inside), an integer summed exactly in f32 and rounded once to f16;
- the residual epilogue on the delta input: f16(f32(w) + f32(r)) (shaders/conv_tiled.wgsl:57-61).

Every variant fhc_variant_list offers runs (direct one-tile, resident /p, wave-stream /w, kernel-row split /rows,
the deep-layer gemm, the chunked igemm, split-K), at stride 1 and 2 and 1x1, plus the fused pairs on all ones."""
import numpy as np
import pytest

from fhtest import Case, fhconv

pytestmark = pytest.mark.gpu

# (n, h, w, cin, cout, k, stride): 3x3 stride 1 and 2 at odd and even sizes, channels of the frame's direct,
# kernel-row-split and deep-layer variants, and the 1x1
SHAPES = [(1, 17, 23, 32, 48, 3, 1), (2, 21, 30, 36, 72, 3, 2), (1, 20, 26, 3, 36, 3, 2), (1, 12, 20, 96, 48, 3, 1),
          (1, 18, 26, 14, 24, 3, 1), (1, 9, 16, 155, 48, 3, 1), (1, 10, 14, 128, 64, 1, 1)]


def say(*a):
    print(*a, flush=True)


def f16(a):
    return np.ascontiguousarray(np.asarray(a, np.float32).astype(np.float16)).view(np.uint16)


def case(shape, seed, residual=False):
    n, h, w, cin, cout, k, s = shape
    c = Case(n, h, w, cin, cout, k=k, stride=s, act=0, residual=residual, seed=seed)
    c.bias = f16(np.zeros(cout))
    return c


def codes(c):
    return [0] + list(fhconv.variant_list(c.fhc_desc()))


def name(code):
    return fhconv.variant_name(code) if code else "planner"


def taps(c, oy, ox):
    """(ky, kx, iy, ix) of every tap of output pixel (oy, ox), inside or outside the image."""
    out = []
    for ky in range(c.k):
        for kx in range(c.k):
            out.append((ky, kx, oy * c.stride + ky - c.pad, ox * c.stride + kx - c.pad))
    return out


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_delta_input_gives_the_weights_bit_exact(shape):
    c = case(shape, seed=71)
    rng = np.random.default_rng(72)
    img, ci = c.n - 1, c.cin - 1
    py, px = c.h // 2, c.w - 1  # an interior row and the last column
    x = np.zeros((c.n, c.h, c.w, c.cin), np.float32)
    x[img, py, px, ci] = 1.0
    c.x = f16(x)
    wt = rng.normal(0, 0.5, (c.cout, c.cin, c.k, c.k))
    c.wt = f16(wt)
    wv = c.wt.view(np.float16)
    want = np.zeros((c.n, c.hout, c.wout, c.cout), np.float16)
    for oy in range(c.hout):
        for ox in range(c.wout):
            for ky, kx, iy, ix in taps(c, oy, ox):
                if (iy, ix) == (py, px):
                    want[img, oy, ox] = wv[:, ci, ky, kx]
    want = want.view(np.uint16)
    for code in codes(c):
        got = c.run_gpu(variant=code)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (name(code), len(bad), bad[0].tolist())
    say("delta input", shape, len(codes(c)), "variants")


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_delta_weight_gives_the_shifted_channel_bit_exact(shape):
    c = case(shape, seed=73)
    co, ci = c.cout // 2, c.cin // 2
    ky, kx = (c.k - 1, 0)  # the bottom-left tap: a shift by (+1, -1) in 3x3
    wt = np.zeros((c.cout, c.cin, c.k, c.k), np.float32)
    wt[co, ci, ky, kx] = 1.0
    c.wt = f16(wt)
    xv = c.x.view(np.float16)
    want = np.zeros((c.n, c.hout, c.wout, c.cout), np.float16)
    for oy in range(c.hout):
        iy = oy * c.stride + ky - c.pad
        for ox in range(c.wout):
            ix = ox * c.stride + kx - c.pad
            if 0 <= iy < c.h and 0 <= ix < c.w:
                want[:, oy, ox, co] = xv[:, iy, ix, ci]
    want = want.view(np.uint16)
    for code in codes(c):
        got = c.run_gpu(variant=code)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (name(code), len(bad), bad[0].tolist())
    say("delta weight", shape, len(codes(c)), "variants")


def ones_count(c):
    cnt = np.zeros((c.hout, c.wout), np.float64)
    for oy in range(c.hout):
        for ox in range(c.wout):
            cnt[oy, ox] = sum(1 for _, _, iy, ix in taps(c, oy, ox) if 0 <= iy < c.h and 0 <= ix < c.w)
    return cnt


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_all_ones_gives_the_border_counts_bit_exact(shape):
    c = case(shape, seed=74)
    c.x = f16(np.ones((c.n, c.h, c.w, c.cin)))
    c.wt = f16(np.ones((c.cout, c.cin, c.k, c.k)))
    want = np.broadcast_to((ones_count(c) * c.cin).astype(np.float16)[None, :, :, None],
                           (c.n, c.hout, c.wout, c.cout)).view(np.uint16)
    for code in codes(c):
        got = c.run_gpu(variant=code)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (name(code), len(bad), bad[0].tolist())
    say("all ones", shape, len(codes(c)), "variants")


@pytest.mark.parametrize("shape", [s for s in SHAPES if s[6] == 1 and s[3] == s[4] or s[3] in (32, 14)],
                         ids=lambda s: "x".join(map(str, s)))
def test_delta_input_with_the_residual_rounds_twice(shape):
    n, h, w, cin, cout, k, s = shape
    c = case((n, h, w, cin, cout, k, s), seed=75, residual=True)
    rng = np.random.default_rng(76)
    x = np.zeros((c.n, c.h, c.w, c.cin), np.float32)
    x[0, 1, 1, 0] = 1.0
    c.x = f16(x)
    c.wt = f16(rng.normal(0, 0.5, (c.cout, c.cin, c.k, c.k)))
    wv = c.wt.view(np.float16)
    acc = np.zeros((c.n, c.hout, c.wout, c.cout), np.float16)
    for oy in range(c.hout):
        for ox in range(c.wout):
            for ky, kx, iy, ix in taps(c, oy, ox):
                if (iy, ix) == (1, 1):
                    acc[0, oy, ox] = wv[:, 0, ky, kx]
    want = (acc.astype(np.float32) + c.res.view(np.float16).astype(np.float32)).astype(np.float16).view(np.uint16)
    for code in codes(c):
        got = c.run_gpu(variant=code)
        bad = np.argwhere(got != want)
        assert bad.size == 0, (name(code), len(bad), bad[0].tolist())


# fused pairs on all ones: A's output (border counts * cin, exact) is B's input; B's weights are 2^-6 (exact in f16),
# so B sums multiples of 2^-6 below 2^12 over its taps and channels in f32 (exact: under 2^24 units) and rounds once
# to f16; every expected value is finite (all ones would reach 9 * 72 * 324 = 209,952 > 65,504 at 36 -> 72 -> 72)
PAIR_SHAPES = [(2, 20, 30, 3, 36, 36, 2, "mid"), (1, 16, 30, 36, 72, 72, 2, "mid"), (1, 14, 28, 48, 48, 48, 1, None),
               (1, 13, 29, 14, 24, 24, 1, None), (1, 13, 29, 24, 24, 3, 1, None), (1, 24, 40, 48, 64, 64, 1, None)]
# the loops each shape's channels instantiate (kPairCfgs, conv_kernels.h): 1 one workgroup per tile, 2 a resident
# grid, 3 a resident grid with A and B on separate waves; 36 -> 72 -> 72 has the one-tile loop only, and
# 48 -> 64 -> 64 (four 16-channel blocks) the two resident loops only
PAIR_LOOPS = {(2, 20, 30, 3, 36, 36, 2, "mid"): (1, 2, 3), (1, 16, 30, 36, 72, 72, 2, "mid"): (1,),
              (1, 14, 28, 48, 48, 48, 1, None): (1, 2, 3), (1, 13, 29, 14, 24, 24, 1, None): (1, 2, 3),
              (1, 13, 29, 24, 24, 3, 1, None): (1, 2, 3), (1, 24, 40, 48, 64, 64, 1, None): (2, 3)}
B_WEIGHT = 2.0 ** -6


# A's K order: with at most 8 (16) input channels the taps share K-steps by default (8 or 16 channels a tap), and
# FHC_PAIR_TAP32 keeps one tap a step; both are run for those shapes
PAIR_RUNS = [(p, loop, tap32) for p in PAIR_SHAPES for loop in PAIR_LOOPS[p] for tap32 in
             ((False, True) if p[3] <= 16 else (False,))]


@pytest.mark.parametrize("p,loop,tap32", PAIR_RUNS,
                         ids=lambda v: "x".join(map(str, v[:7])) if isinstance(v, tuple) else
                         ("tap32" if v is True else "packed" if v is False else f"loop{v}"))
def test_fused_pair_all_ones_bit_exact(p, loop, tap32):
    import torch
    n, h, w, cin, cmid, cout, sa, res = p
    A = Case(n, h, w, cin, cmid, stride=sa, act=0, seed=77)
    B = Case(n, A.hout, A.wout, cmid, cout, act=0, residual=res is not None, seed=78)
    A.x, A.wt, A.bias = f16(np.ones(A.x.shape)), f16(np.ones(A.wt.shape)), f16(np.zeros(cmid))
    B.wt, B.bias = f16(np.full(B.wt.shape, B_WEIGHT)), f16(np.zeros(cout))
    ya = (ones_count(A) * cin).astype(np.float16)                                   # A's output, f16
    pa = np.pad(ya.astype(np.float64), 1)
    sb = sum(pa[dy:dy + A.hout, dx:dx + A.wout] for dy in range(3) for dx in range(3)) * cmid * B_WEIGHT
    assert np.all(sb < 2.0 ** 12) and np.all(sb == np.round(sb / B_WEIGHT) * B_WEIGHT)  # exact f32 sums
    yb = sb.astype(np.float16)
    if res == "mid":
        yb = (yb.astype(np.float32) + ya.astype(np.float32)).astype(np.float16)
    assert np.isfinite(yb).all() and np.isfinite(ya).all()
    want = np.broadcast_to(yb[None, :, :, None], (n, A.hout, A.wout, cout)).view(np.uint16)
    plan = fhconv.ConvPairPlan(A.fhc_desc(), A.wt, A.bias, None, B.fhc_desc(), B.wt, B.bias, None,
                               res_mid=res == "mid", loop=loop, tap32=tap32)
    d = plan.describe()
    assert d["a_channels_per_tap"] == (32 if tap32 or cin > 16 else 8 if cin <= 8 else 16), d["name"]
    dev = torch.device("cuda", 0)
    x = torch.from_numpy(np.ascontiguousarray(A.x).view(np.int16)).to(dev)
    y = torch.zeros((n, A.hout, A.wout, cout), dtype=torch.int16, device=dev)
    plan.run(x, y, None)
    got = y.cpu().numpy().view(np.uint16)
    say("pair all ones", p[:7], "loop", loop, d["name"], "A K-steps", d["a_ksteps"])
    bad = np.argwhere(got != want)
    assert bad.size == 0, (plan.describe()["name"], len(bad), bad[0].tolist())


# fused pairs with a delta input: unit inputs at scattered pixels and channels (at least 4 input pixels apart, so an
# output of A meets at most one of them), random f16 weights for A, B the identity (its centre tap of input channel
# co into output channel co is 1): every output of A is the one weight its delta meets, exactly, and B (with A's
# output as its residual where the pair has one) passes it on exactly, doubled with the residual. A wrong (tap,
# channel) position in A's K order, packed or one tap a step, moves a weight to another pixel or channel.
DELTA_PAIRS = [((2, 22, 34, 3, 36, 36, 2, "mid"), (1, 2, 3)), ((1, 17, 29, 14, 24, 24, 1, None), (1, 2, 3)),
               ((1, 19, 27, 8, 24, 24, 1, None), (1,)), ((1, 21, 33, 16, 24, 24, 1, None), (1,))]
DELTA_RUNS = [(p, loop, tap32) for p, loops in DELTA_PAIRS for loop in loops for tap32 in (False, True)]


@pytest.mark.parametrize("p,loop,tap32", DELTA_RUNS,
                         ids=lambda v: "x".join(map(str, v[:7])) if isinstance(v, tuple) else
                         ("tap32" if v is True else "packed" if v is False else f"loop{v}"))
def test_fused_pair_delta_input_bit_exact(p, loop, tap32):
    import torch
    n, h, w, cin, cmid, cout, sa, res = p
    rng = np.random.default_rng(90 + cin + loop)
    A = Case(n, h, w, cin, cmid, stride=sa, act=0, seed=91)
    B = Case(n, A.hout, A.wout, cmid, cout, act=0, residual=res is not None, seed=92)
    x = np.zeros((n, h, w, cin), np.float32)
    deltas = [(i, yy, xx, int(rng.integers(cin))) for i in range(n) for yy in range(1, h, 4) for xx in range(2, w, 4)]
    for i, yy, xx, ch in deltas:
        x[i, yy, xx, ch] = 1.0
    A.x, A.bias = f16(x), f16(np.zeros(cmid))
    A.wt = f16(rng.uniform(-1, 1, (cmid, cin, 3, 3)))
    wid = np.zeros((cout, cmid, 3, 3), np.float32)
    for co in range(cout):
        wid[co, co, 1, 1] = 1.0
    B.wt, B.bias = f16(wid), f16(np.zeros(cout))
    wa = A.wt.view(np.float16).astype(np.float32)
    ya = np.zeros((n, A.hout, A.wout, cmid), np.float32)
    for i, yy, xx, ch in deltas:
        for ky in range(3):
            for kx in range(3):
                oy, ox = yy + 1 - ky, xx + 1 - kx  # the output whose tap (ky, kx) meets the delta
                if oy % sa or ox % sa:
                    continue
                oy, ox = oy // sa, ox // sa
                if 0 <= oy < A.hout and 0 <= ox < A.wout:
                    assert ya[i, oy, ox].max() == 0 and ya[i, oy, ox].min() == 0, "deltas too close"
                    ya[i, oy, ox] = wa[:, ch, ky, kx]
    yb = ya * 2 if res == "mid" else ya  # f16 values doubled: exact
    want = f16(yb)
    plan = fhconv.ConvPairPlan(A.fhc_desc(), A.wt, A.bias, None, B.fhc_desc(), B.wt, B.bias, None,
                               res_mid=res == "mid", loop=loop, tap32=tap32)
    d = plan.describe()
    # the packed configurations: 8 channels a tap for the stride-2 encoder pair, 16 for the stride-1 refine pair
    assert d["a_channels_per_tap"] == (32 if tap32 else 8 if sa == 2 else 16), d["name"]
    dev = torch.device("cuda", 0)
    xd = torch.from_numpy(np.ascontiguousarray(A.x).view(np.int16)).to(dev)
    y = torch.zeros((n, A.hout, A.wout, cout), dtype=torch.int16, device=dev)
    plan.run(xd, y, None)
    got = y.cpu().numpy().view(np.uint16)
    say("pair delta", p[:7], "loop", loop, d["name"], len(deltas), "deltas")
    bad = np.argwhere(got != want)
    assert bad.size == 0, (d["name"], len(bad), bad[0].tolist())
