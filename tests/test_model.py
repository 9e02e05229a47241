"""The model ABI (include/fhc_model.h) on the CPU: the loader against the reference's own model files, the
validation of damaged ones, and the static plan against the reference's golden plans step by step.

The model files are read where they lie (the reference checkout of the build container); nothing of them is copied
into this repository, and these tests are skipped where the checkout is absent. The golden plans are the fixture
tests/golden/ref_plan_steps.json (every dispatch of the reference's 27 golden plans: pipeline and grid, extracted by
tests/golden/extract_ref_plans.py) with ref_conv_plans.json (every conv's dispatch words)."""
import json
import os
import re

import numpy as np
import pytest

from fhtest import fhconv
import fhmodel
import fhops

HERE = os.path.dirname(os.path.abspath(__file__))
MODEL_DIR = "/root/reference/models"
STEPS = os.path.join(HERE, "golden", "ref_plan_steps.json")
have_model = pytest.mark.skipif(not os.path.exists(os.path.join(MODEL_DIR, "graph.json")),
                                reason="the reference's model files are not in this environment")


@pytest.fixture(scope="module")
def model():
    return fhmodel.Model.load(MODEL_DIR)


@have_model
def test_loader_reads_the_reference_model(model):
    info = model.info()
    # models/flyhighfg.json meta: 62 tensors, 775,811 parameters, bicubic render, format 1 (README.md:214)
    assert info == dict(model="FlyHighFG", train_step=110000, graph_ops=83, tensors=62, params=775811,
                        render_sampling="bicubic", format_version=1, default_k=2)
    man = json.load(open(os.path.join(MODEL_DIR, "flyhighfg.json")))
    raw = np.fromfile(os.path.join(MODEL_DIR, "flyhighfg.bin"), dtype="<u2")
    for name, t in man["tensors"].items():
        assert model.shape(name) == tuple(t["shape"]), name
        n = int(np.prod(t["shape"]))
        assert np.array_equal(model.weight(name).ravel(), raw[t["offset"]:t["offset"] + n]), name
    assert model.shape("no.such.tensor") is None
    with pytest.raises(fhconv.FhcError, match="no tensor"):
        model.weight("no.such.tensor")


def _parts():
    g = open(os.path.join(MODEL_DIR, "graph.json"), "rb").read()
    m = open(os.path.join(MODEL_DIR, "flyhighfg.json"), "rb").read()
    b = open(os.path.join(MODEL_DIR, "flyhighfg.bin"), "rb").read()
    return g, m, b


@have_model
def test_loader_rejects_damaged_files():
    """Model::from_shared's checks (model/mod.rs:57-119, model/graph.rs:17-47): each damage is an error status with
    a message, never a crash."""
    g, m, b = _parts()
    man, graph = json.loads(m), json.loads(g)
    assert fhmodel.Model.from_bytes(g, m, b).info()["params"] == 775811

    def bad(gj, mj, blob, msg):
        with pytest.raises(fhconv.FhcError, match=msg):
            fhmodel.Model.from_bytes(gj, mj, blob)

    bad(g, m, b[:-2], "runs past the end")                                     # the blob one element short
    t = json.loads(m)
    t["tensors"]["enc.e1.0.bias"]["shape"] = [0]
    bad(g, json.dumps(t).encode(), b, "zero dimension")
    t = json.loads(m)
    t["tensors"]["enc.e1.0.bias"]["offset"] = -1
    bad(g, json.dumps(t).encode(), b, "offset is not an unsigned integer")
    t = json.loads(m)
    t["meta"]["format_version"] = 2
    bad(g, json.dumps(t).encode(), b, "format_version 2")
    t = json.loads(m)
    del t["tensors"]["coarse.c1.0.weight"]
    bad(g, json.dumps(t).encode(), b, "reads tensor coarse.c1.0.weight")
    t = json.loads(m)
    del t["tensors"]["film.film.2.bias"]
    bad(g, json.dumps(t).encode(), b, "film")
    gr = json.loads(g)
    gr["ops"][3]["in"] = [5]
    bad(json.dumps(gr).encode(), m, b, "non-string entry")
    bad(g[:100], m, b, "JSON")
    bad(json.dumps({"ops": []}).encode(), m, b, "no ops")
    assert man["meta"]["n_params"] == 775811 and len(graph["ops"]) == 83


# ---- the static plan against the golden plans --------------------------------------------------------------------

def wg(w, h, c):
    return [(w + 7) // 8, (h + 7) // 8, c]


def dispatches(plan, coop, f32):
    """The reference dispatches (pipeline, grid) of a static plan's steps: each op's Gpu method's grid (ops/*.rs),
    the conv's through the reference planner restated (fhc_ref_conv_steps); the session's frame steps and the host
    film_mlp are left out."""
    bufs = plan["buffers"]

    def dims(v):
        b = bufs[v["buf"]]
        return b["h"], b["w"]

    out = []
    for s in plan["steps"]:
        op, o = s["op"], s["out"]
        h, w = dims(o)
        if op in ("rgba_in", "rgba_out", "film_mlp"):
            continue
        if op == "conv":
            x = s["in"][0]
            xh, xw = dims(x)
            for name, grid, _, _ in fhconv.ref_conv_steps(s["cin"], s["cout"], xh, xw, s["stride"],
                                                          residual=s["residual"] is not None, coop=coop,
                                                          f32_mode=f32):
                out.append((name, list(grid), s["stage"]))
        elif op in ("mat", "concat"):
            hw2 = h * w // 2
            ins = s["in"]
            for k in range(0, len(ins), 7):
                c = sum(v["c"] for v in ins[k:k + 7])
                out.append(("chcopy", [(c * hw2 + 255) // 256, 1, 1], s["stage"]))
        elif op in ("luma", "luma_grad", "blend", "blendmix", "render"):
            out.append(({"luma_grad": "grad"}.get(op, op), wg(w, h, 1), s["stage"]))
        elif op == "sad":
            out.append(("sad", wg(w, h, (2 * s["radius"] + 1) ** 2), s["stage"]))
        elif op == "gmhs":  # gm_steps' 14 dispatches (gmhs.rs:161-198)
            ah, aw = dims(s["in"][0])
            par = fhops.gmhs_params(ah, aw, s["full_w"], s["level"])
            cg = [-(-par["wc"] // 8), -(-par["hc"] // 8)]
            for _ in range(4):
                out += [("gm_fit_reduce", [32, 1, 1], s["stage"]), ("gm_fit_solve", [1, 1, 1], s["stage"])]
            out.append(("gm_cost", cg + [1], s["stage"]))
            for pipe, c in (("gm_box_h", 5), ("gm_box_v", 5), ("gm_box_h", 3), ("gm_box_v", 3)):
                out.append((pipe, cg + [c], s["stage"]))
            out.append(("gm_select", wg(w, h, 1), s["stage"]))
        else:  # interp, avgpool, warp, binary, unary, film, convex: one lane per output element of 8 x 8 tiles
            out.append((op, wg(w, h, o["c"]), s["stage"]))
    return out


SESSION = {"tex_in", "tex_out", "rgba_in", "rgba_out"}


def golden_configs():
    plans = json.load(open(STEPS))
    out = []
    for name, p in sorted(plans.items()):
        hdr = p["header"]
        if "static=true" in hdr or "fast=true" in hdr or "cadence" in hdr:
            continue  # static protection, the fast render path and cadence are not part of this plan
        out.append(name)
    return out


@have_model
@pytest.mark.parametrize("name", golden_configs())
def test_static_plan_reproduces_the_golden_plan(model, name):
    """Every dispatch of the reference's golden plan (crates/flyhigh-engine/tests/golden/<name>.txt), in order and
    with its grid, from the static plan: the walk's order, shapes, views and their materialisation, the dead-op
    rule, both peepholes, the repeat, the internal-size mode and the periodic-structure repair's place and grids
    (its parameter words are checked in test_gmhs_oracle.py). The session's frame steps are left out on the golden
    side."""
    p = json.load(open(STEPS))[name]
    hdr = p["header"]
    m = re.match(r"\S+ (\d+)x(\d+) k=(\d+)(?: internal=(\d+)x(\d+))?", hdr)
    if m:
        fw, fh, k = int(m.group(1)), int(m.group(2)), int(m.group(3))
        nw, nh = (int(m.group(4)), int(m.group(5))) if m.group(4) else (fw, fh)
    else:  # "cpu-256x192 k=1 t=0.5": the frame is the network
        mm = re.match(r"cpu-(\d+)x(\d+) k=(\d+)", hdr)
        fw, fh, k = int(mm.group(1)), int(mm.group(2)), int(mm.group(3))
        nw, nh = fw, fh
    cls = name.rsplit(".", 1)[1]
    rm = re.search(r"repair=(\d)", hdr)
    plan = model.plan(k, (fw, fh), (nw, nh), repair=int(rm.group(1)) if rm else 1)
    got = dispatches(plan, coop=cls.startswith("tc"), f32=cls.endswith("f32"))
    want = [(s[0], s[1]) for s in p["steps"] if s[0] not in SESSION]
    assert [(n, g) for n, g, _ in got] == want
    # the pair / mid boundary (mid_start, model/graph.rs:182) falls where the golden plan's "# mid" does
    if p["mid"] is not None:
        pre = [s for s in p["steps"][:p["mid"]] if s[0] not in SESSION]
        assert [st for _, _, st in got].index("mid") == len(pre)


@have_model
def test_plan_at_1080p_matches_the_frame_program(model):
    """The 1080p plan (frames 1920 x 1080, network 856 x 480 -> 864 x 480): padded 1920 x 1088, internal mode, the
    flow scaled by 1920 / 864 and 1088 / 480 in the frame-size render, and the conv sequence of the hand-written
    frame program's layer table (flyhighfg.flyhighfg_layers, encoders unbatched)."""
    import flyhighfg
    plan = model.plan(1, (1920, 1080), (856, 480))
    assert plan["padded"] == [1920, 1088] and plan["network"] == [864, 480] and plan["internal"]
    rend = [s for s in plan["steps"] if s["op"] == "render"]
    assert len(rend) == 1
    assert rend[0]["fsx"] == pytest.approx(float(np.float32(1920) / np.float32(864)), rel=1e-7)
    assert rend[0]["fsy"] == pytest.approx(float(np.float32(1088) / np.float32(480)), rel=1e-7)
    bufs = plan["buffers"]
    convs = [(s["cin"], s["cout"], bufs[s["in"][0]["buf"]]["h"], bufs[s["in"][0]["buf"]]["w"], s["stride"],
              s["act"], s["residual"] is not None) for s in plan["steps"] if s["op"] == "conv"]
    layers = flyhighfg.flyhighfg_layers(864, 480, k=1, batch_encoders=False)
    order = {name: i for i, name in enumerate(L.name for L in layers)}
    # the layer table lists the encoders per picture, then the rest in graph order
    want = [(L.cin, L.cout, L.h, L.w, L.stride, 1 if L.act == 1 else 0, L.residual) for L in
            sorted(layers, key=lambda L: order[L.name])]
    # fine.out's add of the flow is two slices in the graph (no fused residual there) and up.w sits before the
    # convex upsample in the graph's mid stage
    assert sorted(convs) == sorted((c[0], c[1], c[2], c[3], c[4], c[5], c[6] if c[1] != 7 else False)
                                   for c in want)


# ---- the plan replayed: the hand-written frame program's wiring, and the trained model ----------------------------

def _frames(w, h, dx, dy=0):
    import flyhighfg_net as net
    return np.stack([net.procedural_frame(w, h), net.procedural_frame(w, h, dx, dy)])


@have_model
@pytest.mark.parametrize("frame,network", [((256, 128), (256, 128)), ((500, 250), (256, 128))],
                         ids=["network-size", "internal-size"])
def test_graph_replay_equals_the_frame_program(model, frame, network):
    """The graph's own op sequence (the static plan replayed op by op over the oracle) and the hand-written frame
    program (flyhighfg_net.FlyHighFG: batched encoders, fused chains composed op by op, the fine loop's add as a
    residual) over the same oracle give bit-identical results: the program's wiring is the graph's."""
    import flyhighfg_net as net
    from frame_oracle import CpuBackend
    W = net.make_weights(9)
    fr = _frames(*frame, dx=5, dy=2)
    plan = model.plan(1, frame, network)
    g = net.GraphProgram(CpuBackend(W), plan)
    g.frames[...] = fr
    g.run(0.5, W)
    f = net.FlyHighFG(CpuBackend(W), plan["network"][0], plan["network"][1], frame=frame)
    f.frames[...] = fr
    f.pair()
    f.mid(0.5, W)
    assert f.internal == plan["internal"]
    assert np.array_equal(g.named["up7"][..., :7], f.up7[..., :7])
    assert np.array_equal(g.named["R_t"][..., :3], f.Rt[..., :3])
    assert np.array_equal(g.rgba, f.rgba)


def _capi_frame(dx, w=256, h=192):
    """The scene of the reference's C-API test (crates/flyhigh-capi/tests/core.rs:69-83): three sine patterns in
    f32, truncated to bytes, moved dx pixels to the right; alpha 255. As RGBA8 words (h, w)."""
    yy, xx = np.mgrid[0:h, 0:w].astype(np.float32)
    u = (xx - np.float32(dx)) * np.float32(0.07)
    v = yy * np.float32(0.05)
    r = (np.float32(128) + np.float32(100) * np.sin(u)).astype(np.uint32)
    g = (np.float32(128) + np.float32(100) * np.cos(u * np.float32(0.7) + v)).astype(np.uint32)
    b = (np.float32(128) + np.float32(90) * np.sin(u + v)).astype(np.uint32)
    return (r | g << 8 | b << 16 | np.uint32(0xFF000000)).astype(np.uint32)


@have_model
def test_trained_model_generates_the_inbetween(model):
    """The reference's own in-between check (crates/flyhigh-capi/tests/core.rs:85-94, the session at its default K
    on 256 x 192 frames): with the trained weights (models/flyhighfg.bin, read in place) the frame generated at
    t = 0.5 between the scene and the scene moved 8 px has a mean absolute byte error to the scene moved 4 px below
    its error to either input frame, and below 6. The whole graph, its weights and the oracle's arithmetic together."""
    import flyhighfg_net as net
    from frame_oracle import CpuBackend
    W = net.weights_from_model(model)
    f0, f1, mid = _capi_frame(0), _capi_frame(8), _capi_frame(4)
    plan = model.plan(model.info()["default_k"], (256, 192), (256, 192))
    g = net.GraphProgram(CpuBackend(W), plan)
    g.frames[...] = np.stack([f0, f1])
    g.run(0.5, W)

    def mae(a, b):
        bytes_ = lambda f: np.stack([(f >> s) & 0xFF for s in (0, 8, 16, 24)], -1).astype(np.float64)  # noqa: E731
        return float(np.abs(bytes_(a) - bytes_(b)).mean())

    got = g.rgba[0]
    to_mid, to_f0, to_f1 = mae(got, mid), mae(got, f0), mae(got, f1)
    print(f"MAE to the true middle {to_mid:.2f}, to f0 {to_f0:.2f}, to f1 {to_f1:.2f}")
    assert to_mid < to_f0 and to_mid < to_f1 and to_mid < 6.0


# ---- discovery of the plan's conv shapes, and their autotune -------------------------------------------------------

@have_model
def test_conv_shapes_are_the_golden_plans_convs(model):
    """The distinct conv shapes of the plan at the 856 x 480 network, in plan order, are those of the reference's
    golden plan at that network with the full graph (rt-720p-default: every conv it records,
    tests/golden/ref_conv_plans.json), keyed as the reference's discovery build keys them (cin, cout, h, w, stride,
    autotune.rs:214-217); the frame size does not change them (1280 x 720 and 1920 x 1080 alike)."""
    recs = json.load(open(os.path.join(HERE, "golden", "ref_conv_plans.json")))
    want = []
    for r in recs:
        if r["source"].startswith("rt-720p-default.tc-f16:"):
            c = r["conv"]
            key = (c["cin"], c["cout"], c["h"], c["w"], c["stride"])
            if key not in want:
                want.append(key)
    got = model.conv_shapes(1, (1280, 720), (856, 480))
    assert [s[:5] for s in got] == want
    assert model.conv_shapes(1, (1920, 1080), (856, 480)) == got
    assert all(s[5:] == (1, 3) for s in got)
    assert [s[5] for s in model.conv_shapes(1, (1920, 1080), (856, 480), n=8)] == [8] * len(got)


def synthetic_model(rng):
    """A small model of this library's own making (three convs and the render, random weights): graph.json,
    manifest and blob bytes in the reference's formats (model/graph.rs, model/mod.rs:57-119)."""
    layers = [("s.c1", 3, 16, True), ("s.c2", 16, 16, True), ("s.c3", 16, 10, False)]
    tensors, blob, off = {}, [], 0
    for name, cin, cout, act in layers:
        parts = [(f"{name}.0.weight" if act else f"{name}.weight", [cout, cin, 3, 3]),
                 (f"{name}.0.bias" if act else f"{name}.bias", [cout])]
        if act:
            parts.append((f"{name}.1.weight", [cout]))
        for tname, shape in parts:
            n = int(np.prod(shape))
            tensors[tname] = {"shape": shape, "offset": off}
            blob.append(rng.normal(0, 0.2, n).astype(np.float16).view(np.uint16))
            off += n
    ops = [{"in": ["A"], "out": ["x1"], "w": ["s.c1.0.weight", "s.c1.0.bias", "s.c1.1.weight"], "stride": 2,
            "op": "conv"},
           {"in": ["x1"], "out": ["x2"], "w": ["s.c2.0.weight", "s.c2.0.bias", "s.c2.1.weight"], "op": "conv"},
           {"in": ["x2"], "out": ["x3"], "w": ["s.c3.weight", "s.c3.bias"], "op": "conv2d"},
           {"in": ["x3"], "out": ["f"], "a": 0, "b": 4, "op": "slice"},
           {"in": ["x3"], "out": ["v"], "a": 4, "b": 7, "op": "slice"},
           {"in": ["x3"], "out": ["r"], "a": 7, "b": 10, "op": "slice"},
           {"in": ["A", "B", "f", "v", "r"], "out": ["render"], "output": True, "op": "render_pix"}]
    graph = json.dumps({"meta": {}, "ops": ops}).encode()
    manifest = json.dumps({"meta": {"model": "synthetic", "format_version": 1, "train_step": 0,
                                    "render_sampling": "bilinear", "n_params": off},
                           "tensors": tensors}).encode()
    return graph, manifest, np.concatenate(blob).astype("<u2").tobytes()


def test_synthetic_model_plans_its_convs():
    g, m, b = synthetic_model(np.random.default_rng(0))
    mdl = fhmodel.Model.from_bytes(g, m, b)
    assert mdl.conv_shapes(1, (64, 64), (64, 64)) == [(3, 16, 64, 64, 2, 1, 3), (16, 16, 32, 32, 1, 1, 3),
                                                     (16, 10, 32, 32, 1, 1, 3)]


@pytest.mark.gpu
def test_autotune_of_a_model_fills_the_choice_table():
    """fhc_model_autotune times every discovered shape and records its choice under the shape's key, at batch 1
    and 2 (a synthetic model: the reference's model files stay where they lie)."""
    g, m, b = synthetic_model(np.random.default_rng(1))
    mdl = fhmodel.Model.from_bytes(g, m, b)
    for n in (1, 2):
        shapes = mdl.conv_shapes(1, (64, 64), (64, 64), n=n)
        assert mdl.autotune(1, (64, 64), (64, 64), n=n, reps=3) == len(shapes) == 3
        for s in shapes:
            assert fhconv.load().fhc_tune_get_ex(*s) >= 0, s


# ---- a model of this library's own making whose plan holds every step kind (tests/synthetic_graph.py) ------------

@pytest.mark.parametrize("frame", [(128, 64), (300, 140)], ids=["network-size", "internal-size"])
def test_synthetic_plan_holds_every_step_kind(frame):
    """The plan walk over the synthetic model emits every step kind (frame input and, in the internal-size mode,
    its downscale; convs with and without activation and residual; views materialised; concat with a zeros buffer;
    the ops; the repair; the frame output), the repeat body K = 2 times, the pair / mid boundary at film_mlp."""
    import synthetic_graph as sg
    g, m, b = sg.model_bytes(0)
    mdl = fhmodel.Model.from_bytes(g, m, b)
    plan = mdl.plan(2, frame, (128, 64), repair=1)
    kinds = {s["op"] for s in plan["steps"]}
    assert kinds == sg.STEP_KINDS, kinds ^ sg.STEP_KINDS
    assert plan["internal"] == (frame != (128, 64))
    convs = [s for s in plan["steps"] if s["op"] == "conv"]
    assert sum(s["weight"] == "s.rd.weight" for s in convs) == 2                  # the repeat body twice
    assert [s["weight"] for s in convs if s["residual"]] == ["s.e2.0.weight", "s.rd.weight", "s.rd.weight"]
    stages = [s["stage"] for s in plan["steps"]]
    first_mid = stages.index("mid")
    assert "mid" not in stages[:first_mid] and "pair" not in stages[first_mid:]
    assert plan["steps"][first_mid]["op"] in ("gmhs", "film_mlp")
    assert [s["op"] for s in plan["steps"] if s["op"] in ("film_mlp", "gmhs")] == ["gmhs", "film_mlp"]
    assert sum(s["op"] == "interp" for s in plan["steps"]) == (4 if plan["internal"] else 2)


def test_synthetic_plan_replays_over_the_oracle():
    """GraphProgram takes the synthetic model's own convs (names and shapes from the plan, weights from the model)
    and runs every step over the oracle backend: finite maps, a whole RGBA8 frame."""
    import synthetic_graph as sg
    import flyhighfg_net as net
    from frame_oracle import CpuBackend
    g, m, b = sg.model_bytes(0)
    mdl = fhmodel.Model.from_bytes(g, m, b)
    plan = mdl.plan(2, (300, 140), (128, 64), repair=1)
    W = net.weights_from_model(mdl, plan)
    assert set(W) == {"s.e1", "s.e2", "s.h0", "s.fl", "s.vi", "s.hh", "s.rd", "s.fd", "s.vc", "up.w", "s.r1", "s.r2",
                      "film"}
    gp = net.GraphProgram(CpuBackend(W), plan)
    gp.frames[...] = net.pair_frames(300, 140, 3, shift=5)
    gp.run(0.4, W)
    for name in ("up7", "rt", "flow", "hh", "cin"):
        assert np.isfinite(gp.named[name].view(np.float16)).all(), name
    assert np.all(gp.rgba >> 24 == 255) and len(np.unique(gp.rgba)) > 1000
