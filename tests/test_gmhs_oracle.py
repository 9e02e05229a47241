"""The periodic-structure repair (GMHS, crates/flyhigh-engine/src/gmhs.rs) in the oracle, pinned on the CPU.

The reference holds no numeric vectors for this stage, so the oracle (oracle/fh_ops_oracle.c) is pinned by
  - the parameter words of the reference's golden plans (every gm_* dispatch: grids, FitP, CostP, BoxP, SelP),
    against the oracle's and the library's derivation of them;
  - closed forms: an exactly affine flow is recovered by the fit; a constant map is its own box mean; identical
    pictures under zero motion cost nothing; a known displacement difference is its Euclidean length; the select
    rewrites exactly the cells whose three conditions hold, with the affine motion at the cell;
  - a float64 restatement of the reweighted least squares (independent of the summation order);
  - the stage's purpose: in a striped scene whose flow is one stripe period off inside a blob, the blob takes the
    global motion and the rest of the flow is untouched.
"""
import json
import math
import os

import numpy as np
import pytest

from fhtest import oracle  # noqa: F401 (puts oracle/ and the package on the path)
import fhops  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
STEPS = os.path.join(HERE, "golden", "ref_plan_steps.json")


def f32bits(v):
    return int(np.float32(v).view(np.uint32))


def pad32(v):
    return (v + 31) // 32 * 32


def f16(a):
    return np.asarray(a, np.float32).astype(np.float16).view(np.uint16)


def golden_gm_plans():
    plans = json.load(open(STEPS))
    return sorted(n for n, p in plans.items() if any(s[0].startswith("gm_") for s in p["steps"]))


@pytest.mark.parametrize("name", golden_gm_plans())
def test_parameters_match_the_golden_plans(name):
    """Every gm_* dispatch of the golden plan (grid and parameter words) from (network, padded frame width,
    level), through the oracle's and the library's derivation (gmhs.rs:149-206)."""
    p = json.load(open(STEPS))[name]
    hdr = p["header"]
    frame = hdr.split()[1] if not hdr.startswith("cpu-") else hdr.split()[0][4:]
    full_w = pad32(int(frame.split("x")[0]))
    level = 2 if "repair=2" in hdr else 1
    gm = [s for s in p["steps"] if s[0].startswith("gm_")]
    cost = next(s for s in gm if s[0] == "gm_cost")
    h8, w8, h, w = cost[2][:4]  # the network the graph ran at (CostP)
    assert (h8, w8) == (h // 8, w // 8)
    for par in (oracle.gm_params(h, w, full_w, level), fhops.gmhs_params(h, w, full_w, level)):
        hc, wc = par["hc"], par["wc"]
        want = []
        for it in range(4):
            want.append(["gm_fit_reduce", [32, 1, 1], [h8, w8, 32, int(it > 0), f32bits(par["delta"]), 0, 0, 0]])
            want.append(["gm_fit_solve", [1, 1, 1], [32, 0, 0, 0]])
        g = [-(-wc // 8), -(-hc // 8)]
        want.append(["gm_cost", g + [1], [h8, w8, h, w, hc, wc, f32bits(2.0), 0]])
        for c, r in ((5, par["r_blk"]), (3, par["r_dwin"])):
            want.append(["gm_box_h", g + [c], [c, hc, wc, r]])
            want.append(["gm_box_v", g + [c], [c, hc, wc, r]])
        want.append(["gm_select", [-(-w8 // 8), -(-h8 // 8), 1],
                     [h8, w8, hc, wc, f32bits(par["eps"]), f32bits(par["dmin"]), f32bits(par["tex"]), 0]])
        assert [list(s) for s in gm] == want, name


def test_parameters_closed_form():
    """s = w / (full_w / 2); radii round(10 s) and round(16 s), half away from zero; dmin 8 s (0 at level 2)."""
    p = oracle.gm_params(480, 864, 1920)
    assert (p["hc"], p["wc"], p["r_blk"], p["r_dwin"]) == (240, 432, 9, 14)
    assert np.float32(p["s"]) == np.float32(864) / np.float32(960)
    p = oracle.gm_params(480, 864, 1280, 2)
    assert (p["r_blk"], p["r_dwin"], p["dmin"]) == (14, 22, 0.0)  # 10 s = 13.5 rounds up
    p = oracle.gm_params(7, 9, 1000)
    assert (p["hc"], p["wc"], p["r_blk"], p["r_dwin"]) == (4, 5, 1, 1)  # radii at least 1
    lib = fhops.gmhs_params(7, 9, 1000)
    assert all(lib[k] == p[k] for k in p)


# ---- the fit -------------------------------------------------------------------------------------------------------

def grid(h8, w8):
    yy, xx = np.mgrid[0:h8, 0:w8].astype(np.float64)
    return yy, xx


def norm_coords(h8, w8):
    yy, xx = grid(h8, w8)
    return -1 + 2 * xx / max(w8 - 1, 1), -1 + 2 * yy / max(h8 - 1, 1)


def flow_of(chans):
    """(1, h8, w8, 4) f16 bits from 4 float arrays (exactly representable ones stay exact)."""
    return np.ascontiguousarray(f16(np.stack(chans, -1))[None])


def test_fit_recovers_an_affine_flow():
    h8, w8 = 60, 108
    yy, xx = grid(h8, w8)
    pqr = [(3.5, 0.25, -0.5), (-2.0, 0.0, 0.125), (0.75, -0.5, 0.25), (1.0, 0.125, 0.0)]
    chans = [p + q * xx + r * yy for p, q, r in pqr]
    flow = flow_of(chans)
    assert np.array_equal(flow[0].view(np.float16).astype(np.float64), np.stack(chans, -1))  # exact in f16
    coef = oracle.gm_fit(flow, delta=1.35)
    for c, (p, q, r) in enumerate(pqr):
        want = [p + q * (w8 - 1) / 2 + r * (h8 - 1) / 2, q * (w8 - 1) / 2, r * (h8 - 1) / 2]
        assert np.allclose(coef[c, :3], want, rtol=1e-4, atol=1e-4), (c, coef[c], want)
        assert coef[c, 3] == 0


def irls64(f, h8, w8, delta, iters=4):
    """Reweighted least squares in float64: the normal equations of f ~ a0 + a1 x + a2 y with weights 1, then
    delta / max(delta, |residual|), a ridge of 1e-6 on the diagonal (gm_fit_solve.wgsl:13)."""
    x, y = norm_coords(h8, w8)
    x, y, f = x.ravel(), y.ravel(), f.ravel()
    A = np.stack([np.ones_like(x), x, y], 1)
    a = np.zeros(3)
    out = []
    for it in range(iters):
        wt = np.ones_like(f) if it == 0 else delta / np.maximum(delta, np.abs(f - A @ a))
        M = (A * wt[:, None]).T @ A + np.diag([1e-6, 1e-6, 1e-6])
        a = np.linalg.solve(M, (A * wt[:, None]).T @ f)
        out.append(a.copy())
    return out


def test_fit_is_the_reweighted_least_squares_and_ignores_a_blob():
    """The oracle's fit equals a float64 restatement of the reweighted least squares to f32 accuracy, and the
    reweighting pulls the fit off an outlier blob: after 4 rounds the global motion is recovered far better than
    by the plain least squares of the first round (the blob, 9 % of the cells 16 px off, keeps a weight of about
    delta / 16 each, so a bias of about 0.15 px remains)."""
    rng = np.random.default_rng(3)
    h8, w8 = 60, 108
    yy, xx = grid(h8, w8)
    truth = [(-3.0, 0.5, 0.2), (0.5, 0.0, -0.3), (3.0, -0.5, -0.2), (-0.5, 0.1, 0.3)]
    x, y = norm_coords(h8, w8)
    chans = []
    for a0, a1, a2 in truth:
        f = a0 + a1 * x + a2 * y + rng.normal(0, 0.05, (h8, w8))
        f[10:30, 20:50] += 16.0  # one stripe period off inside a blob
        chans.append(f)
    flow = flow_of(chans)
    fq = flow[0].view(np.float16).astype(np.float64)
    for iters in (1, 4):
        coef = oracle.gm_fit(flow, delta=1.35, iters=iters)
        for c in range(4):
            ref = irls64(fq[..., c], h8, w8, 1.35, iters)[-1]
            assert np.allclose(coef[c, :3], ref, rtol=2e-4, atol=2e-4), (iters, c, coef[c], ref)
    plain, robust = oracle.gm_fit(flow, 1.35, iters=1), oracle.gm_fit(flow, 1.35, iters=4)
    for c, t in enumerate(truth):
        e_plain, e_rob = np.abs(plain[c, :3] - t).max(), np.abs(robust[c, :3] - t).max()
        assert e_rob < 0.2 * e_plain and e_rob < 0.25, (c, e_plain, e_rob)


def test_fit_of_a_constant_flow():
    flow = flow_of([np.full((9, 13), v) for v in (2.5, -1.0, 0.0, 7.0)])
    coef = oracle.gm_fit(flow, 3.0)
    assert np.allclose(coef[:, 0], [2.5, -1.0, 0.0, 7.0], atol=1e-5) and np.allclose(coef[:, 1:3], 0, atol=1e-5)


# ---- the box windows -----------------------------------------------------------------------------------------------

def box64(src, r, vert):
    src = np.asarray(src, np.float64)
    ax = 1 if vert else 2
    pad = [(0, 0)] * 3
    pad[ax] = (r, r)
    p = np.pad(src, pad, mode="edge")
    n = src.shape[ax]
    return sum(np.take(p, np.arange(d, d + n), axis=ax) for d in range(2 * r + 1)) / (2 * r + 1)


@pytest.mark.parametrize("r", [1, 3, 9, 40])
def test_box_is_the_edge_replicated_mean(r):
    rng = np.random.default_rng(r)
    src = rng.uniform(0, 1, (3, 23, 37)).astype(np.float32)
    for vert in (0, 1):
        got = oracle.gm_box(src, r, vert)
        # a sequential f32 sum of 2r + 1 terms in [0, 1]: relative error below (2r + 1) 2^-24
        assert np.allclose(got, box64(src, r, vert), rtol=(2 * r + 2) * 2.0 ** -24, atol=1e-7)
    const = np.full((2, 5, 6), 0.375, np.float32)
    assert np.array_equal(oracle.gm_box(const, r, 0), const) and np.array_equal(oracle.gm_box(const, r, 1), const)


# ---- the cost maps -------------------------------------------------------------------------------------------------

def pictures(rng, h, w, n=1):
    return f16(rng.uniform(0, 1, (n, h, w, 4)).astype(np.float32))


def luma64(pic):
    p = pic.view(np.float16).astype(np.float64)
    return 0.299 * p[..., 2] + 0.587 * p[..., 1] + 0.114 * p[..., 0]


@pytest.mark.parametrize("h,w", [(48, 64), (33, 45)])
def test_cost_of_identical_pictures_and_no_motion(h, w):
    """A == B, zero flow and zero coefficients: no mismatch, no displacement difference; the luma map is the mean
    of each 2 x 2 block (the last row / column replicated where h, w are odd)."""
    rng = np.random.default_rng(h)
    a = pictures(rng, h, w)
    flow = np.zeros((1, h // 8 or 1, w // 8 or 1, 4), np.uint16)
    hc, wc = (h + 1) // 2, (w + 1) // 2
    maps = oracle.gm_cost(a, a, flow, np.zeros((4, 4), np.float32), hc, wc)
    assert not maps[:3].any()
    lum = np.pad(luma64(a[0]), ((0, 2 * hc - h), (0, 2 * wc - w)), mode="edge")
    blk = (lum[0::2, 0::2] + lum[0::2, 1::2] + lum[1::2, 0::2] + lum[1::2, 1::2]) / 4
    assert np.allclose(maps[3], blk, atol=2e-6)
    assert np.allclose(maps[4], maps[3].astype(np.float64) ** 2, rtol=1e-6)


def test_cost_under_the_true_translation_is_zero():
    """B is A moved by (dx, dy) whole pixels: the flow (0, 0, dx, dy) and the same affine motion match exactly away
    from the borders (mismatch 0 under both, displacement difference 0); an affine motion that leaves the picture
    costs what the flow costs."""
    rng = np.random.default_rng(5)
    h, w, dx, dy = 64, 96, 5, -3
    a = pictures(rng, h, w)
    b = np.roll(a, (dy, dx), axis=(1, 2))  # b(p) = a(p - d)
    h8, w8 = h // 8, w // 8
    flow = flow_of([np.zeros((h8, w8)), np.zeros((h8, w8)), np.full((h8, w8), dx), np.full((h8, w8), dy)])
    coef = np.zeros((4, 4), np.float32)
    coef[2, 0], coef[3, 0] = dx, dy
    hc, wc = h // 2, w // 2
    maps = oracle.gm_cost(a, b, flow, coef, hc, wc)
    inner = (slice(4, hc - 4), slice(4, wc - 4))
    assert not maps[0][inner].any() and not maps[1][inner].any() and not maps[2].any()
    coef[0, 0] = 1e4
    maps2 = oracle.gm_cost(a, b, flow, coef, hc, wc)
    assert np.array_equal(maps2[1], maps2[0])


def test_cost_displacement_difference():
    """(g1 - g0) - (f1 - f0) under zero flow and constant hypotheses (3, 0) towards a, (-1, 3) towards b: (-4, 3),
    length 5 exactly."""
    rng = np.random.default_rng(6)
    a = pictures(rng, 32, 32)
    coef = np.zeros((4, 4), np.float32)
    coef[0, 0], coef[2, 0], coef[3, 0] = 3.0, -1.0, 3.0
    maps = oracle.gm_cost(a, a, np.zeros((1, 4, 4, 4), np.uint16), coef, 16, 16)
    assert np.all(maps[2] == 5.0)


# ---- the select ----------------------------------------------------------------------------------------------------

def affine_f16(coef, h8, w8):
    j = np.arange(w8, dtype=np.float32)[None, :]
    i = np.arange(h8, dtype=np.float32)[:, None]
    xn = np.float32(-1) + np.float32(2) * j / np.float32(max(w8 - 1, 1))
    yn = np.float32(-1) + np.float32(2) * i / np.float32(max(h8 - 1, 1))
    c = coef.astype(np.float32)
    return np.stack([c[k, 0] + c[k, 1] * xn + c[k, 2] * yn for k in range(4)], -1).astype(np.float16).view(np.uint16)


def test_select_rewrites_exactly_the_cells_that_pass():
    h8, w8 = 12, 20
    hc, wc = 4 * h8, 4 * w8
    coef = np.array([[1.5, 0.25, -0.5, 0], [0.1, 0, 0.2, 0], [-2, 1, 0, 0], [0.5, -0.25, 0.75, 0]], np.float32)
    flow = f16(np.random.default_rng(1).normal(0, 3, (1, h8, w8, 8)))
    maps = np.zeros((5, hc, wc), np.float32)
    maps[0], maps[1], maps[2], maps[3], maps[4] = 1.0, 0.5, 10.0, 0.5, 0.5  # sd = 0.5
    allsel = oracle.gm_select(maps, coef, flow, 0.0, 7.2, 0.015)
    assert np.array_equal(allsel[0, ..., :4], affine_f16(coef, h8, w8))
    assert np.array_equal(allsel[..., 4:], flow[..., 4:])  # channels past the flow's 4 untouched
    for k, v in ((1, 1.0), (2, 7.2), (4, 0.25)):  # cost not lower / no jump / flat texture (sd 0)
        m = maps.copy()
        m[k] = v
        assert np.array_equal(oracle.gm_select(m, coef, flow, 0.0, 7.2, 0.015), flow), k
    # the nearest cell: E8 cell (i, j) reads cell (4 i + 2, 4 j + 2)
    m = maps.copy()
    m[1] = 2.0
    m[1][4 * 5 + 2, 4 * 7 + 2] = 0.5
    got = oracle.gm_select(m, coef, flow, 0.0, 7.2, 0.015)
    changed = np.argwhere((got != flow).any(-1)[0])
    assert changed.tolist() == [[5, 7]]


# ---- the whole stage -----------------------------------------------------------------------------------------------

def striped_scene(h, w, dx, seed=0):
    """A picture of vertical stripes (period 16) under a faint smooth texture, and the same picture moved dx
    pixels right; BGR f16 (1, h, w, 4)."""
    rng = np.random.default_rng(seed)
    yy, xx = np.mgrid[0:h + 8, 0:w + 64].astype(np.float64)
    tex = sum(rng.uniform(0.01, 0.03) * np.sin(xx * rng.uniform(0.02, 0.06) + yy * rng.uniform(0.02, 0.06) +
                                               rng.uniform(0, 6)) for _ in range(4))
    base = 0.5 + 0.3 * np.sign(np.sin(2 * np.pi * xx / 16)) * 0.5 + tex
    pic = np.stack([base * 0.9, base, base * 0.8, np.zeros_like(base)], -1)
    a = pic[4:4 + h, 32:32 + w]
    b = pic[4:4 + h, 32 - dx:32 - dx + w]
    return f16(a[None]), f16(b[None])


def test_stage_repairs_a_blob_one_period_off():
    """Frames of a striped wall panned 6 px, the flow right (-3, 0 towards a; 3, 0 towards b) except in a blob
    where it is one stripe period (16 px) off, where the stripes match as well as anywhere: the stage puts the
    blob back on the global motion (the fitted affine motion, whose displacement is the pan's 6 px, not the blob's
    -10) and leaves the rest of the flow as it was."""
    h, w = 256, 384
    a, b = striped_scene(h, w, 6)
    h8, w8 = h // 8, w // 8
    f = [np.full((h8, w8), v) for v in (-3.0, 0.0, 3.0, 0.0)]
    blob = (slice(8, 16), slice(10, 22))
    f[0][blob], f[2][blob] = 5.0, -5.0  # relative displacement -10 instead of 6: 16 px off
    flow = np.zeros((1, h8, w8, 8), np.uint16)
    flow[0, ..., :4] = flow_of(f)[0]
    out, coef, maps = oracle.gmhs(a, b, flow, full_w=2 * w)  # s = 1: dmin 8 px
    assert np.allclose(coef[:, 0], [-3, 0, 3, 0], atol=0.15) and np.allclose(coef[:, 1:3], 0, atol=0.15)
    got = out[0, ..., :4]
    inner = (slice(10, 14), slice(12, 20))
    assert np.array_equal(got[inner], affine_f16(coef, h8, w8)[inner])
    disp = got[inner].view(np.float16).astype(np.float32)
    assert np.all(np.abs((disp[..., 2] - disp[..., 0]) - 6) < 0.6)
    mask = np.ones((h8, w8), bool)
    mask[blob] = False
    assert np.array_equal(out[0][mask], flow[0][mask])
    assert np.array_equal(out[..., 4:], flow[..., 4:])
    p2 = oracle.gm_params(h, w, 2 * w, 2)
    assert p2["dmin"] == 0.0 and math.isclose(p2["delta"], 1.5)


def test_select_cells_closed_form():
    """The cost cell the select reads: 4i + 2 on the 1080p network's grids (hc = 4 h8), the nearest cell centre
    otherwise (floor((i + 1/2) hc / h8), exact in f32 at these sizes)."""
    assert np.array_equal(oracle.gm_select_cells(60, 240), 4 * np.arange(60) + 2)
    for n8, nc in [(12, 50), (9, 45), (1, 7), (18, 75)]:
        want = np.floor((np.arange(n8) + 0.5) * nc / n8).astype(np.int64)
        assert np.array_equal(oracle.gm_select_cells(n8, nc), np.clip(want, 0, nc - 1))


def test_stages_compose_to_the_stage():
    """gmhs_stages (the steps called one by one, the decision values gathered at the select's cells) against the
    whole stage: the same flow and coefficients, maps 3-4 untouched by the decision window, and the decision values
    the final maps hold at the select's cells."""
    rng = np.random.default_rng(5)
    h, w = 100, 150
    a = f16(rng.uniform(0, 1, (1, h, w, 4)))
    b = np.roll(a, (2, -3), axis=(1, 2)).copy()
    h8, w8 = h // 8, w // 8
    flow = f16(rng.normal(0, 3, (1, h8, w8, 8)))
    for level in (1, 2):
        out, coef, maps = oracle.gmhs(a, b, flow, 160, level)
        out2, coef2, tex, dec = oracle.gmhs_stages(a, b, flow, 160, level)
        assert np.array_equal(out, out2) and np.array_equal(coef.view(np.uint32), coef2.view(np.uint32))
        assert np.array_equal(tex[3:].view(np.uint32), maps[3:].view(np.uint32))
        p = oracle.gm_params(h, w, 160, level)
        ys, xs = oracle.gm_select_cells(h8, p["hc"]), oracle.gm_select_cells(w8, p["wc"])
        assert dec.shape == (5, h8, w8)
        assert np.array_equal(dec.view(np.uint32), maps[:, ys[:, None], xs[None, :]].view(np.uint32))
        # the texture window alone: the oracle's box of the cost maps
        raw = oracle.gm_cost(a, b, flow, coef, p["hc"], p["wc"])
        want = oracle.gm_box(oracle.gm_box(raw, p["r_blk"], 0), p["r_blk"], 1)
        assert np.array_equal(tex.view(np.uint32), want.view(np.uint32))
