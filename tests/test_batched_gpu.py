"""The batched configuration (8 independent 3840x2160 frame pairs at the 864x480 network, 3 mid() phases each) on the
GPU: every conv launch of its step at its real batch (the encoders at 16 images, the pair-stage convs at 8, the
mid-stage convs at 24), with the committed MI355X choice table and the fused pairs the bench runs, checked against
the oracle on the first and the last image of the batch (the parity bar |diff| <= 1e-2 * max|ref|); and the
batch-independence invariant, bit-exact, for every kernel family the step uses: image i of a batched launch equals
the same variant run on that image alone."""
import copy
import os

import numpy as np
import pytest

from fhtest import Case, fhconv, parity
import flyhighfg

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
TABLE = os.path.join(HERE, "..", "flyhigh-engine_amd", "tune_mi355x.txt")
LAYERS = {L.name: L for L in flyhighfg.batched_layers(8, 3)}
# the fused pairs of the batched step and the loop each runs (the bench's fastest: the warp-specialised resident
# grid for the encoders' first pair and the fine block, the resident grid for the refine head)
PAIRS = [("enc.e1.ab", "enc.e2.ab", "mid", dict(tile_rows=4, wave_rows=1, loop=3)),
         ("fine.r2", "fine.r3", None, dict(tile_rows=4, wave_rows=1, loop=3)),
         ("refine.q1", "refine.q2", None, dict(tile_rows=8, wave_rows=2, loop=2))]
IN_PAIRS = {a for a, _, _, _ in PAIRS} | {b for _, b, _, _ in PAIRS}


def say(*a):
    print(*a, flush=True)


def pad8(c):
    return (c + 7) // 8 * 8


def layer_case(L, seed, n=None):
    return Case(n or L.n, L.h, L.w, L.cin, L.cout, stride=L.stride, act=L.act, residual=L.residual,
                xv=(pad8(L.cin), 0), yv=(pad8(L.cout), 0), rv=(pad8(L.cout), 0), seed=seed)


def image(c, i):
    """The case restricted to image i (same weights)."""
    one = copy.copy(c)
    one.n = 1
    one.x, one.res, one.y0 = c.x[i:i + 1], c.res[i:i + 1], c.y0[i:i + 1]
    return one


@pytest.fixture(scope="module", autouse=True)
def committed_table():
    fhconv.tune_clear()
    fhconv.parse_tune(open(TABLE).read())
    yield
    fhconv.tune_clear()


@pytest.mark.parametrize("name", [n for n in LAYERS if n not in IN_PAIRS])
def test_batched_conv_matches_the_oracle_on_first_and_last_image(name):
    L = LAYERS[name]
    c = layer_case(L, seed=300 + len(name))
    got, plan = c.run_gpu(return_plan=True)
    d = plan.describe()
    say("batched", name, L.n, d["name"])
    for i in (0, L.n - 1):
        ok, md, mref = parity(got[i:i + 1], image(c, i).run_oracle(threads=8), view=slice(0, L.cout))
        assert ok, (name, i, d["name"], md, mref)


def _run_pair(A, B, res, kw):
    import torch
    plan = fhconv.ConvPairPlan(A.fhc_desc(), A.wt, A.bias, A.slope if A.act == 1 else None, B.fhc_desc(), B.wt,
                               B.bias, B.slope if B.act == 1 else None, res_mid=res == "mid", **kw)
    dev = torch.device("cuda", 0)
    x = torch.from_numpy(np.ascontiguousarray(A.x).view(np.int16)).to(dev)
    y = torch.from_numpy(np.ascontiguousarray(B.y0).view(np.int16)).to(dev)
    plan.run(x, y, None)
    torch.cuda.synchronize()
    return y.cpu().numpy().view(np.uint16), plan


def _pair_cases(a, b, res):
    La, Lb = LAYERS[a], LAYERS[b]
    A = layer_case(La, seed=400)
    B = layer_case(Lb, seed=401)
    return La, Lb, A, B


@pytest.mark.parametrize("a,b,res,kw", PAIRS, ids=[f"{a}+{b}" for a, b, _, _ in PAIRS])
def test_batched_fused_pair_matches_the_oracle_on_first_and_last_image(a, b, res, kw):
    La, Lb, A, B = _pair_cases(a, b, res)
    got, plan = _run_pair(A, B, res, kw)
    d = plan.describe()
    say("batched pair", a, b, La.n, d["name"])
    for i in (0, La.n - 1):
        ai = image(A, i)
        ya = ai.run_oracle(threads=8)
        bi = image(B, i)
        bi.x = ya
        if res == "mid":
            bi.res = ya
        ok, md, mref = parity(got[i:i + 1], bi.run_oracle(threads=8), view=slice(0, Lb.cout))
        assert ok, (a, b, i, d["name"], md, mref)


# one layer per kernel family of the batched step (the committed table's choice for it), each run batched and on
# its first and last image alone with the same variant: bit-identical
FAMILY_LAYERS = ["enc.e3.ab", "enc.e4.ab", "coarse.head", "fine.out", "film.h1", "refine.q3"]


@pytest.mark.parametrize("name", FAMILY_LAYERS)
def test_batch_independence_per_family(name):
    L = LAYERS[name]
    c = layer_case(L, seed=500)
    got, plan = c.run_gpu(return_plan=True)
    code = plan.describe()["variant"]
    say("independence", name, L.n, fhconv.variant_name(code))
    for i in (0, L.n - 1):
        alone = image(c, i).run_gpu(variant=code)
        assert np.array_equal(alone, got[i:i + 1]), (name, i, fhconv.variant_name(code))


@pytest.mark.parametrize("a,b,res,kw", PAIRS, ids=[f"{a}+{b}" for a, b, _, _ in PAIRS])
def test_batch_independence_of_the_fused_pairs(a, b, res, kw):
    La, Lb, A, B = _pair_cases(a, b, res)
    got, plan = _run_pair(A, B, res, kw)
    say("independence", a, b, plan.describe()["name"])
    for i in (0, La.n - 1):
        alone, _ = _run_pair(image(A, i), image(B, i), res, kw)
        assert np.array_equal(alone, got[i:i + 1]), (a, b, i)
