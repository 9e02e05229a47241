"""Parity of the HIP conv path (through the C ABI) with the CPU oracle, on the GPU.

Bar (north star): per element |diff| <= 1e-2 * max|ref| for f16 results with f32 accumulation; indexing,
padding and stride are checked bit-exactly by closed forms; the untouched parts of views must stay untouched.
"""
import os

import numpy as np
import pytest

from fhtest import Case, as_f64, f16_bits, fhconv, oracle, oracle_rows, parity, ulp_dist

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "conv_vectors.npz")


def say(*a):
    print(*a, flush=True)


def test_mfma_fragment_layout():
    import torch
    rng = np.random.default_rng(1)
    a = f16_bits(rng.uniform(-1, 1, (16, 32)))
    b = f16_bits(rng.uniform(-1, 1, (32, 16)))
    da = torch.from_numpy(a.view(np.int16)).cuda()
    db = torch.from_numpy(b.view(np.int16)).cuda()
    dd = torch.zeros((16, 16), dtype=torch.float32, device="cuda")
    fhconv.probe_mfma_layout(da, db, dd)
    torch.cuda.synchronize()
    want = as_f64(a) @ as_f64(b)
    assert np.abs(dd.cpu().numpy() - want).max() < 1e-5


def test_mfma_rate_probe():
    # the sustained-rate probe runs and reports a plausible dense f16 rate: between 50% and 110% of 2.5 PFLOP/s
    # (16 independent chains per wave at 4 waves per SIMD keep the MFMA pipe busy; compiled well it reaches ~90%)
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(cus * 4 * 1024, dtype=torch.float32, device="cuda")
    fhconv.probe_mfma_rate(cus * 4, 16, out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    flops = fhconv.probe_mfma_rate(cus * 4, 1024, out)
    e1.record()
    e1.synchronize()
    tflops = flops / (e0.elapsed_time(e1) * 1e-3) / 1e12
    say("mfma rate", round(tflops), "TFLOP/s")
    assert 1250 < tflops < 2750
    assert torch.isfinite(out).all()


def test_golden_vectors_on_the_gpu():
    z = np.load(GOLDEN)
    names = sorted({k.split(".")[0] for k in z.files})
    for nm in names:
        n, h, w, cin, cout, k, s, pad, act, res, xcs, xc0, ycs, yc0, rcs, rc0 = [int(v) for v in z[nm + ".meta"]]
        say("golden", nm)
        c = Case(n, h, w, cin, cout, k=k, stride=s, act=act, alpha=float(z[nm + ".alpha"][0]), residual=res,
                 xv=(xcs, xc0), yv=(ycs, yc0), rv=(rcs, rc0))
        c.x, c.wt, c.bias, c.slope = z[nm + ".x"], z[nm + ".w"], z[nm + ".bias"], z[nm + ".slope"]
        c.res, c.y0 = z[nm + ".res"], z[nm + ".y0"]
        got = c.run_gpu()
        want = z[nm + ".y"]
        ok, md, mref = parity(got, want)
        assert ok, (nm, md, mref)
        assert ulp_dist(got, want).max() <= 4, nm
        # channels outside the output view keep their prior contents
        mask = np.ones(ycs, bool)
        mask[yc0:yc0 + cout] = False
        assert np.array_equal(got[..., mask], c.y0[..., mask])


SHAPES = [
    # n, h, w, cin, cout, k, stride, act, residual
    (1, 9, 11, 5, 7, 3, 1, 1, 0),
    (1, 10, 13, 3, 6, 3, 2, 1, 0),
    (1, 20, 37, 14, 24, 3, 1, 1, 1),
    (2, 17, 23, 36, 36, 3, 1, 1, 1),
    (1, 33, 35, 36, 72, 3, 2, 1, 0),
    (1, 30, 54, 72, 72, 3, 1, 1, 1),
    (1, 30, 54, 279, 96, 3, 1, 1, 0),
    (1, 30, 54, 96, 12, 3, 1, 0, 0),
    (1, 60, 108, 155, 48, 3, 1, 1, 0),
    (1, 60, 108, 48, 7, 3, 1, 0, 0),
    (1, 60, 108, 48, 36, 3, 1, 0, 0),
    (1, 120, 216, 24, 3, 3, 1, 0, 0),
    (1, 120, 216, 3, 36, 3, 2, 1, 0),
    (1, 68, 120, 128, 64, 1, 1, 0, 0),
    (1, 13, 29, 40, 130, 1, 1, 2, 1),
    (1, 136, 240, 32, 32, 3, 1, 2, 0),
    (1, 1, 1, 9, 4, 3, 1, 1, 0),
    (1, 7, 1, 6, 5, 3, 2, 1, 0),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_planner_choice_matches_the_oracle(shape):
    n, h, w, cin, cout, k, s, act, res = shape
    c = Case(n, h, w, cin, cout, k=k, stride=s, act=act, residual=res, seed=sum(shape))
    got, plan = c.run_gpu(return_plan=True)
    say("shape", shape, plan.describe()["name"])
    ok, md, mref = parity(got, c.run_oracle(threads=8))
    assert ok, (md, mref)


VARIANT_SHAPES = [(1, 20, 37, 40, 72, 3, 1), (1, 19, 35, 24, 40, 3, 2), (1, 18, 33, 48, 40, 1, 1), (1, 9, 21, 279, 40, 3, 1),
                  (1, 12, 20, 130, 100, 3, 1), (1, 17, 35, 90, 44, 3, 1)]


@pytest.mark.parametrize("shape", VARIANT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_every_variant_matches_the_oracle(shape):
    n, h, w, cin, cout, k, s = shape
    c = Case(n, h, w, cin, cout, k=k, stride=s, act=1, residual=True, seed=7)
    want = c.run_oracle(threads=8)
    codes = fhconv.variant_list(c.fhc_desc())
    assert codes
    for code in codes:
        say("variant", shape, fhconv.variant_name(code))
        ok, md, mref = parity(c.run_gpu(variant=code), want)
        assert ok, (fhconv.variant_name(code), md, mref)


def test_views_with_poisoned_neighbours():
    # NaN in the input channels outside the view must never reach the result; NaN in the output channels outside
    # the view must stay there; unaligned strides take the scalar load / store paths
    # the planner's choice and every persistent variant: with aligned views these run the buffer-load loop (the
    # input group at channel 16 holds 4 channels of the view next to 4 poisoned ones), with unaligned ones they fall
    # back to one workgroup per tile
    for xv, yv, rv in [((48, 8), (80, 16), (40, 4)), ((37, 3), (35, 1), (33, 5)), ((24, 0), (24, 0), (24, 0))]:
        c = Case(1, 21, 30, 20, 24, act=1, residual=True, xv=xv, yv=yv, rv=rv, poison=True, seed=11)
        want = c.run_oracle()
        persistent = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).endswith("/p")]
        assert persistent
        for code in [0] + persistent:
            say("views", xv, yv, rv, fhconv.variant_name(code) if code else "planner")
            got = c.run_gpu(variant=code)
            sl = slice(yv[1], yv[1] + 24)
            ok, md, mref = parity(got, want, view=sl)
            assert ok, (code, md, mref)
            mask = np.ones(yv[0], bool)
            mask[sl] = False
            assert np.array_equal(got[..., mask], c.y0[..., mask])


PADDED_SHAPES = [(2, 24, 40, 3, 36, 2), (1, 12, 40, 279, 96, 1), (1, 20, 36, 14, 24, 1), (1, 14, 35, 155, 48, 1)]


@pytest.mark.parametrize("shape", PADDED_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_padded_channel_stride_views(shape):
    # the frame's odd channel counts in buffers whose channel stride is padded to 8: the partial last group loads
    # as one 16-byte group and its channels past cin (NaN here) are masked; every variant against the oracle
    n, h, w, cin, cout, s = shape
    cx, cy = (cin + 7) // 8 * 8, (cout + 7) // 8 * 8
    c = Case(n, h, w, cin, cout, stride=s, act=1, residual=(s == 1 and cin == cout), xv=(cx, 0), yv=(cy, 0),
             rv=(cy, 0), poison=True, seed=23)
    want = c.run_oracle(threads=8)
    sl = slice(0, cout)
    for code in [0] + list(fhconv.variant_list(c.fhc_desc())):
        say("padded", shape, fhconv.variant_name(code) if code else "planner")
        got = c.run_gpu(variant=code)
        ok, md, mref = parity(got, want, view=sl)
        assert ok, (fhconv.variant_name(code) if code else "planner", md, mref)
        assert np.array_equal(got[..., cout:], c.y0[..., cout:])


def test_batch_images_are_independent():
    c = Case(3, 22, 35, 24, 40, act=1, residual=True, seed=12)
    batched = c.run_gpu()
    for i in range(3):
        one = Case(1, 22, 35, 24, 40, act=1, residual=True, seed=12)
        one.x, one.res, one.y0 = c.x[i:i + 1], c.res[i:i + 1], c.y0[i:i + 1]
        one.wt, one.bias, one.slope = c.wt, c.bias, c.slope
        assert np.array_equal(one.run_gpu(), batched[i:i + 1])


@pytest.mark.parametrize("ks", [1, 2, 4, 8])
def test_split_k_deep_small_spatial(ks):
    # the deep 1080p/16 layer: 128 -> 128 at 68 x 120, K = 1152, split 1 / 2 / 4 / 8 ways (f32 partials)
    c = Case(1, 68, 120, 128, 128, act=1, seed=13)
    got, plan = c.run_gpu(ksplit=ks, return_plan=True)
    d = plan.describe()
    say("split", ks, d["name"], d["ksplit"])
    assert d["ksplit"] == ks
    ok, md, mref = parity(got, c.run_oracle(threads=8))
    assert ok, (md, mref)
    # the same conv split differently differs only by f32 reassociation
    ref = as_f64(c.run_gpu(ksplit=1))
    assert np.abs(as_f64(got) - ref).max() <= 4e-3 * np.abs(ref).max()


def test_known_answer_closed_form_conv_on_the_gpu():
    # crates/flyhigh-cli/src/cli/coop_tests.rs:337-346 and :612 (max|d| < 0.1 against unrounded f32 values)
    import torch
    cin, cout, h, w = 208, 64, 46, 80
    x_chw = (((np.arange(cin * h * w) % 17) - 8) * 0.05).reshape(cin, h, w)
    wv = (((np.arange(cout * cin * 9) % 13) - 6) * 0.04).reshape(cout, cin, 3, 3)
    b = (np.arange(cout) % 5 - 2) * 0.1
    want = torch.nn.functional.conv2d(torch.from_numpy(x_chw[None]), torch.from_numpy(wv), padding=1)[0].numpy()
    want = want + b[:, None, None]
    want = np.where(want > 0, want, 0.1 * want)
    c = Case(1, h, w, cin, cout, act=1, seed=14)
    c.x = f16_bits(x_chw.transpose(1, 2, 0)[None])
    c.wt, c.bias, c.slope = f16_bits(wv), f16_bits(b), f16_bits(np.full(cout, 0.1))
    got = c.run_gpu()
    assert np.abs(as_f64(got)[0].transpose(2, 0, 1) - want).max() < 0.1
    ok, md, mref = parity(got, c.run_oracle(threads=8))
    assert ok, (md, mref)


def test_full_size_ladder_rows():
    # the 1080p/4 ladder at full size, chained on the GPU; every layer checked on three row bands against the
    # oracle run on the very input the GPU layer read
    import torch
    layers = [(544, 960, 32, 64, 2, 0), (272, 480, 64, 64, 1, 0), (272, 480, 64, 64, 1, 0), (272, 480, 64, 64, 1, 1)]
    x = None
    first_out = None
    for i, (h, w, cin, cout, s, res) in enumerate(layers):
        c = Case(1, h, w, cin, cout, stride=s, act=1, residual=res, seed=20 + i)
        if x is not None:
            c.x = x
        if res:
            c.res = first_out
        say("ladder layer", i, (h, w, cin, cout, s, res))
        got = c.run_gpu()
        for r0 in (0, c.hout // 2 - 3, c.hout - 6):
            ok, md, mref = parity(got[0, r0:r0 + 6], oracle_rows(c, r0, r0 + 6, threads=8))
            assert ok, (i, r0, md, mref)
        x = got
        if i == 0:
            first_out = got


def test_graph_capture_replays_match_eager():
    import torch
    c = Case(1, 40, 64, 32, 32, act=2, seed=15)
    plan = fhconv.ConvPlan(c.fhc_desc(), c.wt, c.bias, None)
    x = torch.from_numpy(c.x.view(np.int16)).cuda()
    y = torch.zeros_like(torch.from_numpy(c.y0.view(np.int16))).cuda()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        plan.run(x, y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    eager = y.clone()
    g = torch.cuda.CUDAGraph()
    y.zero_()
    with torch.cuda.graph(g):
        plan.run(x, y)
    for i in range(4):
        y.fill_(i + 1)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), i


def test_plan_lifecycle_and_describe():
    c = Case(1, 16, 16, 8, 8, act=1, seed=16)
    for _ in range(50):
        p = fhconv.ConvPlan(c.fhc_desc(), c.wt, c.bias, c.slope)
        d = p.describe()
        assert d["hout"] == 16 and d["wout"] == 16 and d["flops"] == 2 * 16 * 16 * 8 * 8 * 9
        p.close()
    p = fhconv.ConvPlan(c.fhc_desc(), c.wt, c.bias, c.slope)
    with pytest.raises(fhconv.FhcError):
        p.run(None, None)


def test_autotune_picks_a_listed_variant_and_records_it():
    import torch
    fhconv.tune_clear()
    try:
        c = Case(1, 40, 70, 48, 48, act=1, residual=True, seed=17)
        d = c.fhc_desc()
        host = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).cuda()  # noqa: E731
        x, y, r = host(c.x), host(c.y0), host(c.res)
        code, us = fhconv.autotune(d, c.wt, c.bias, c.slope, x, y, r, reps=5)
        say("autotune", fhconv.variant_name(code), us)
        assert code in fhconv.variant_list(d) and us > 0
        assert fhconv.tune_get(48, 48, 40, 70, 1) == code
        got, plan = c.run_gpu(return_plan=True)
        assert plan.describe()["variant"] == code
        ok, md, mref = parity(got, c.run_oracle())
        assert ok, (md, mref)
    finally:
        fhconv.tune_clear()


@pytest.mark.parametrize("shape", [(1, 272, 480, 64, 64, 1), (1, 544, 960, 32, 64, 2)], ids=["s1", "s2"])
def test_persistent_variants_full_size(shape):
    # the persistent variants loop over more tiles than workgroups at the 1080p/4 sizes: rows checked in bands
    n, h, w, cin, cout, s = shape
    c = Case(n, h, w, cin, cout, stride=s, act=1, residual=(s == 1), seed=18)
    codes = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).endswith("/p")]
    assert codes
    bands = {r0: oracle_rows(c, r0, r0 + 4, threads=8) for r0 in (0, c.hout // 2 - 2, c.hout - 4)}
    for code in codes:
        got, plan = c.run_gpu(variant=code, return_plan=True)
        d = plan.describe()
        say("persistent", d["name"], d["grid"], d["tiles"])
        assert d["grid"][0] < d["tiles"]
        for r0, want in bands.items():
            ok, md, mref = parity(got[0, r0:r0 + 4], want)
            assert ok, (d["name"], r0, md, mref)


WAVE_SHAPES = [(2, 37, 53, 32, 40, 1, 1, None, None), (1, 29, 71, 64, 64, 1, 2, None, None),
               (1, 33, 47, 48, 24, 1, 0, (80, 8), (44, 4)), (1, 41, 67, 32, 64, 2, 1, None, None),
               (1, 31, 45, 96, 96, 1, 1, None, None)]


@pytest.mark.parametrize("shape", WAVE_SHAPES, ids=lambda s: "x".join(map(str, s[:7])))
def test_wave_variants_match_the_oracle(shape):
    # the wave-stream variants ("/w": halos by LDS DMA, one tile stream per wave): ragged tiles, several channel
    # tiles with a partial last one, every activation, stride 2, and views inside poisoned wider tensors
    n, h, w, cin, cout, s, act, xv, yv = shape
    c = Case(n, h, w, cin, cout, stride=s, act=act, xv=xv, yv=yv, poison=xv is not None, seed=31)
    want = c.run_oracle(threads=8)
    codes = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).endswith("/w")]
    assert codes
    sl = slice(c.yc0, c.yc0 + cout)
    for code in codes:
        got, plan = c.run_gpu(variant=code, return_plan=True)
        say("wave", shape[:7], plan.describe()["name"], plan.describe()["grid"])
        ok, md, mref = parity(got, want, view=sl)
        assert ok, (fhconv.variant_name(code), md, mref)
        mask = np.ones(c.ycs, bool)
        mask[sl] = False
        assert np.array_equal(got[..., mask], c.y0[..., mask])


def test_wave_variant_unaligned_input_falls_back():
    # an input pointer off 16-byte alignment cannot take the LDS DMA: the launcher runs the one-tile kernel instead
    import torch
    c = Case(1, 21, 34, 32, 32, act=1, seed=32)
    want = c.run_oracle()
    code = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).endswith("/w")][0]
    plan = fhconv.ConvPlan(c.fhc_desc(code), c.wt, c.bias, c.slope)
    dev = torch.device("cuda", 0)
    xb = torch.zeros(c.x.size + 4, dtype=torch.int16, device=dev)
    xb[4:] = torch.from_numpy(c.x.ravel().view(np.int16)).to(dev)
    y = torch.from_numpy(c.y0.view(np.int16)).to(dev)
    plan.run(xb[4:], y)
    torch.cuda.synchronize()
    ok, md, mref = parity(y.cpu().numpy().view(np.uint16), want)
    assert ok, (md, mref)


@pytest.mark.parametrize("shape", [(1, 272, 480, 64, 64, 1, 1), (1, 544, 960, 32, 64, 2, 1), (1, 136, 240, 32, 32, 1, 2)],
                         ids=["s1", "s2", "c1"])
def test_wave_variants_full_size(shape):
    # the 1080p/4 and /8 sizes: every wave runs several rounds of its two-buffer loop; rows checked in bands
    n, h, w, cin, cout, s, act = shape
    c = Case(n, h, w, cin, cout, stride=s, act=act, seed=19)
    codes = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).endswith("/w")]
    assert codes
    bands = {r0: oracle_rows(c, r0, r0 + 4, threads=8) for r0 in (0, c.hout // 2 - 2, c.hout - 4)}
    for code in codes:
        got, plan = c.run_gpu(variant=code, return_plan=True)
        d = plan.describe()
        say("wave", d["name"], d["grid"], d["tiles"])
        for r0, want in bands.items():
            ok, md, mref = parity(got[0, r0:r0 + 4], want)
            assert ok, (d["name"], r0, md, mref)


# fused pairs: n, h, w, cin, cmid, cout, A's stride, A's and B's activation, B's residual (None, "mid": A's
# output, "ext": a tensor), A's input view, B's output view
PAIR_CASES = [(2, 50, 90, 3, 36, 36, 2, 1, 1, "mid", (8, 0), None),
              (1, 33, 61, 48, 48, 48, 1, 1, 1, None, None, None),
              (1, 41, 75, 14, 24, 24, 1, 1, 1, None, (16, 0), None),
              (1, 37, 53, 24, 24, 3, 1, 1, 0, None, None, (8, 0)),
              (1, 30, 44, 48, 48, 48, 1, 2, 1, "ext", None, None)]
# the encoder's second pair (36 -> 72 -> 72, stride 2, A's output as B's residual): tiles of 1 or 2 rows
PAIR_CASES_E3 = [(2, 61, 107, 36, 72, 72, 2, 1, 1, "mid", (40, 0), None),
                 (1, 19, 29, 36, 72, 72, 2, 1, 1, "mid", None, (80, 8))]
# A's K order: cases with at most 16 input channels pack taps into K-steps at one wave row (8 or 16 channels a
# tap), and run once more with one tap a step (FHC_PAIR_TAP32); at two wave rows only one tap a step is instantiated
PAIR_RUNS = [(c, th, wm, False) for c in PAIR_CASES for th, wm in ((2, 1), (4, 1), (2, 2), (4, 2))] + \
    [(c, th, 1, True) for c in PAIR_CASES if c[3] <= 16 for th in (2, 4)] + \
    [(c, th, 1, False) for c in PAIR_CASES_E3 for th in (1, 2)]


@pytest.mark.parametrize("case,th,wm,tap32", PAIR_RUNS,
                         ids=lambda v: "x".join(map(str, v[:7])) + (f"-{v[9]}" if v[9] else "")
                         if isinstance(v, tuple) else ("tap32" if v is True else "" if v is False else str(v)))
def test_pair_matches_the_two_convs(case, th, wm, tap32):
    # the fused pair against the oracle run twice (A, then B on A's f16 output): ragged tiles, stride 2, a residual
    # from A's output or from a tensor, a padded input view with NaN past cin, an output view inside a wider tensor
    import torch
    n, h, w, cin, cmid, cout, sa, act_a, act_b, res, xv, yv = case
    A = Case(n, h, w, cin, cmid, stride=sa, act=act_a, xv=xv, poison=xv is not None, seed=41)
    ya = A.run_oracle(threads=8)
    B = Case(n, A.hout, A.wout, cmid, cout, act=act_b, residual=res is not None, yv=yv, poison=yv is not None, seed=42)
    B.x = ya
    if res == "mid":
        B.res = ya
    want = B.run_oracle(threads=8)
    plan = fhconv.ConvPairPlan(A.fhc_desc(), A.wt, A.bias, A.slope if act_a == 1 else None, B.fhc_desc(), B.wt, B.bias,
                               B.slope if act_b == 1 else None, res_mid=res == "mid", tile_rows=th, wave_rows=wm,
                               tap32=tap32)
    d = plan.describe()
    say("pair", case, d["name"], d["grid"], d["tiles"])
    assert d["family"] == "pair" and d["tile_rows"] == th and d["wave_rows"] == wm
    packed = not tap32 and wm == 1 and cin <= 16
    assert d["a_channels_per_tap"] == ((8 if cin <= 8 else 16) if packed else 32), d["name"]
    dev = torch.device("cuda", 0)
    x = torch.from_numpy(np.ascontiguousarray(A.x).view(np.int16)).to(dev)
    y = torch.from_numpy(np.ascontiguousarray(B.y0).view(np.int16)).to(dev)
    r = torch.from_numpy(np.ascontiguousarray(B.res).view(np.int16)).to(dev) if res == "ext" else None
    plan.run(x, y, r)
    torch.cuda.synchronize()
    got = y.cpu().numpy().view(np.uint16)
    sl = slice(B.yc0, B.yc0 + cout)
    ok, md, mref = parity(got, want, view=sl)
    assert ok, (d["name"], md, mref)
    mask = np.ones(B.ycs, bool)
    mask[sl] = False
    assert np.array_equal(got[..., mask], B.y0[..., mask])


# the deep-layer kernel ("gemm.": weights and halos through LDS by DMA, chunks of 32 or 64 input channels):
# n, h, w, cin, cout, act, residual, input view, output view
GEMM_SHAPES = [(1, 30, 54, 279, 96, 1, 0, (280, 0), None),
               (1, 27, 45, 155, 48, 1, 1, (160, 0), None),
               (2, 19, 37, 128, 128, 2, 1, (136, 8), (136, 4)),
               (1, 17, 33, 96, 12, 0, 0, None, None),
               (1, 11, 18, 64, 100, 1, 0, None, (104, 0))]


@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: "x".join(map(str, s[:7])))
def test_gemm_variants_match_the_oracle(shape):
    # every deep-layer configuration and split: partial last channel groups with NaN past cin in the tensor, ragged
    # tiles, partial channel tiles, a residual, every activation, views inside poisoned wider tensors
    n, h, w, cin, cout, act, res, xv, yv = shape
    c = Case(n, h, w, cin, cout, act=act, residual=res, xv=xv, yv=yv, poison=xv is not None or yv is not None,
             seed=51)
    want = c.run_oracle(threads=8)
    codes = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).startswith("gemm")]
    assert codes
    sl = slice(c.yc0, c.yc0 + cout)
    for code in codes:
        got, plan = c.run_gpu(variant=code, return_plan=True)
        d = plan.describe()
        say("gemm", shape[:7], d["name"], d["grid"], d["ksplit"])
        assert d["family"] == "gemm"
        ok, md, mref = parity(got, want, view=sl)
        assert ok, (d["name"], md, mref)
        mask = np.ones(c.ycs, bool)
        mask[sl] = False
        assert np.array_equal(got[..., mask], c.y0[..., mask])


def test_gemm_variant_unaligned_input_falls_back():
    # an input pointer off 16-byte alignment cannot take the LDS DMA: the launcher runs the chunked kernel on the
    # same packed weights instead, with and without a split
    import torch
    c = Case(1, 21, 34, 155, 48, act=1, xv=(160, 0), seed=52)
    want = c.run_oracle()
    names = {fhconv.variant_name(k): k for k in fhconv.variant_list(c.fhc_desc())}
    for name in ("gemm.t8x16.n64.f4x2.w2x2.c32.p3", "gemm.t8x16.n64.f4x2.w2x2.c32.p2/k2",
                 "gemm.t8x16.n32.f2x2.w4x1.c64.p2"):
        plan = fhconv.ConvPlan(c.fhc_desc(names[name]), c.wt, c.bias, c.slope)
        dev = torch.device("cuda", 0)
        xb = torch.zeros(c.x.size + 4, dtype=torch.int16, device=dev)
        xb[4:] = torch.from_numpy(c.x.ravel().view(np.int16)).to(dev)
        y = torch.from_numpy(c.y0.view(np.int16)).to(dev)
        ws = torch.empty(plan.workspace_bytes // 4 + 4, dtype=torch.float32, device=dev) if plan.workspace_bytes else None
        say("gemm fallback", name)
        plan.run(xb[4:], y, None, ws)
        torch.cuda.synchronize()
        ok, md, mref = parity(y.cpu().numpy().view(np.uint16), want)
        assert ok, (name, md, mref)


@pytest.mark.parametrize("shape", [(1, 68, 120, 128, 128, 1, 0), (8, 30, 54, 279, 96, 1, 0)], ids=["deep", "c1x8"])
def test_gemm_variants_full_size(shape):
    # the 1080p/16 deep layer and the batched 279-channel layer: rows checked in bands of the first image
    n, h, w, cin, cout, act, res = shape
    c = Case(n, h, w, cin, cout, act=act, residual=res, xv=((cin + 7) // 8 * 8, 0), seed=53)
    codes = [k for k in fhconv.variant_list(c.fhc_desc()) if fhconv.variant_name(k).startswith("gemm")]
    assert codes
    bands = {r0: oracle_rows(c, r0, r0 + 4, threads=8) for r0 in (0, c.hout // 2 - 2, c.hout - 4)}
    for code in codes:
        got, plan = c.run_gpu(variant=code, return_plan=True)
        d = plan.describe()
        say("gemm", d["name"], d["grid"], d["ksplit"])
        for r0, want in bands.items():
            ok, md, mref = parity(got[0, r0:r0 + 4], want)
            assert ok, (d["name"], r0, md, mref)


# the resident-grid pair (weights loaded once, tiles looped over): cases with more tiles than the grid holds, so
# every workgroup runs several iterations. n, h, w, cin, cmid, cout, A's stride, A's and B's activation, B's
# residual, A's input view, B's output view
PAIR_P_CASES = [(4, 64, 200, 48, 64, 64, 1, 1, 1, None, (56, 0), None),
                (4, 61, 203, 48, 48, 48, 1, 1, 1, "ext", None, None),
                (24, 50, 90, 3, 36, 36, 2, 1, 1, "mid", (8, 0), None),
                (4, 120, 216, 14, 24, 24, 1, 1, 1, None, (16, 0), None),
                (4, 119, 213, 24, 24, 3, 1, 2, 0, None, None, (8, 0))]


def run_pair(A, B, res, **kw):
    import torch
    plan = fhconv.ConvPairPlan(A.fhc_desc(), A.wt, A.bias, A.slope if A.act == 1 else None, B.fhc_desc(), B.wt,
                               B.bias, B.slope if B.act == 1 else None, res_mid=res == "mid", **kw)
    dev = torch.device("cuda", 0)
    x = torch.from_numpy(np.ascontiguousarray(A.x).view(np.int16)).to(dev)
    y = torch.from_numpy(np.ascontiguousarray(B.y0).view(np.int16)).to(dev)
    r = torch.from_numpy(np.ascontiguousarray(B.res).view(np.int16)).to(dev) if res == "ext" else None
    plan.run(x, y, r)
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16), plan


# the resident-grid loops (tile rows, wave rows, loop) instantiated per case: 4 rows x 2 wave rows and the
# warp-specialised loop at 4 rows for every pair; 4 rows x 1 wave row, 8 rows x 2 and the warp-specialised loop at 8
# rows only for the 14/24-channel refine-head pairs
PAIR_P_LOOPS = {(4, 1, 2): "t4w1", (4, 2, 2): "t4w2", (8, 2, 2): "t8w2", (4, 1, 3): "t4ws", (8, 1, 3): "t8ws"}
PAIR_P_PARAMS = [pytest.param(c, *t, id=PAIR_P_LOOPS[t] + "-" + "x".join(map(str, c[:7])) + (f"-{c[9]}" if c[9] else ""))
                 for c in PAIR_P_CASES for t in PAIR_P_LOOPS
                 if c[4] <= 24 or t in ((4, 2, 2), (4, 1, 3))]


@pytest.mark.parametrize("case,th,wm,loop", PAIR_P_PARAMS)
def test_resident_pair_matches_the_two_convs(case, th, wm, loop):
    # loop 2: both stages on every wave; loop 3: A and B on separate waves, pipelined across tiles
    n, h, w, cin, cmid, cout, sa, act_a, act_b, res, xv, yv = case
    A = Case(n, h, w, cin, cmid, stride=sa, act=act_a, xv=xv, poison=xv is not None, seed=61)
    ya = A.run_oracle(threads=8)
    B = Case(n, A.hout, A.wout, cmid, cout, act=act_b, residual=res is not None, yv=yv, poison=yv is not None, seed=62)
    B.x = ya
    if res == "mid":
        B.res = ya
    want = B.run_oracle(threads=8)
    got, plan = run_pair(A, B, res, tile_rows=th, wave_rows=wm, loop=loop)
    d = plan.describe()
    say("pair/p", case[:7], d["name"], d["grid"], d["tiles"])
    assert d["persistent"] == loop - 1 and d["tile_rows"] == th and d["grid"][0] < d["tiles"]
    sl = slice(B.yc0, B.yc0 + cout)
    ok, md, mref = parity(got, want, view=sl)
    assert ok, (d["name"], md, mref)
    mask = np.ones(B.ycs, bool)
    mask[sl] = False
    assert np.array_equal(got[..., mask], B.y0[..., mask])


@pytest.mark.parametrize("loop", [2, 3], ids=["p", "ws"])
def test_resident_pair_full_size_ladder(loop):
    # the 1080p/4 ladder's two 64 -> 64 convs as one resident-grid pair, rows checked in bands: B's rows
    # [r0, r0 + 4) from the oracle of A's rows [r0 - 1, r0 + 5)
    import copy
    A = Case(1, 272, 480, 64, 64, act=1, seed=63)
    B = Case(1, 272, 480, 64, 64, act=1, seed=64)
    got, plan = run_pair(A, B, None, loop=loop)
    d = plan.describe()
    say("pair/p", d["name"], d["grid"], d["tiles"])
    assert d["persistent"] == loop - 1
    for r0 in (0, 134, 268):
        a0, a1 = max(0, r0 - 1), min(272, r0 + 5)
        band = copy.copy(B)
        band.h = band.hout = a1 - a0
        band.x = oracle_rows(A, a0, a1, threads=8)
        band.y0 = np.zeros((1, a1 - a0, 480, 64), np.uint16)
        want = band.run_oracle(threads=8)[:, r0 - a0:r0 - a0 + 4]
        ok, md, mref = parity(got[:, r0:r0 + 4], want)
        assert ok, (r0, md, mref)
