"""A model of this library's own making whose static plan holds every step kind the plan walk produces (the frames
in and the downscale, conv and conv2d, the residual peephole, views and their materialisation, zeros, concat,
avgpool, luma, sad_volume, warp, a repeat body carrying the flow, the pair / mid boundary, film_mlp and
film_modulate, mul_t, add, convex_upsample with its up.w conv, blend_weights with the blendmix peephole, luma_grad,
affine_out, render_pix, and, when asked, the repair), in the reference's model formats (graph.json ops,
flyhighfg.json manifest of f16 tensor offsets, flyhighfg.bin; crates/flyhigh-engine/src/model/graph.rs,
model/mod.rs:57-119). Small channel counts; random weights. Test data only."""
import json

import numpy as np

# (weight stem, cin, cout, activation): "conv" layers carry a PReLU slope (stem.0.weight, .0.bias, .1.weight),
# "conv2d" layers none (stem.weight, stem.bias)
LAYERS = [("s.e1", 6, 16, True), ("s.e2", 16, 16, True), ("s.h0", 27, 16, True), ("s.fl", 16, 4, False),
          ("s.vi", 16, 3, False), ("s.hh", 16, 48, True), ("s.rd", 19, 4, False), ("s.fd", 48, 5, False),
          ("s.vc", 3, 3, False), ("up.w", 48, 36, False), ("s.r1", 10, 8, True), ("s.r2", 8, 3, False)]


def _w(stem, act):
    return [f"{stem}.0.weight", f"{stem}.0.bias", f"{stem}.1.weight"] if act else [f"{stem}.weight", f"{stem}.bias"]


def _conv(stem, inp, out, stride=1):
    act = next(a for s, _, _, a in LAYERS if s == stem)
    op = {"op": "conv" if act else "conv2d", "in": [inp], "out": [out], "w": _w(stem, act)}
    if stride != 1:
        op["stride"] = stride
    return op


def ops():
    sl = lambda src, out, a, b: {"op": "slice", "in": [src], "out": [out], "a": a, "b": b}  # noqa: E731
    pair = [
        {"op": "interpolate", "in": ["A"], "out": ["aq"], "scale": 0.25, "antialias": True},
        {"op": "interpolate", "in": ["B"], "out": ["bq"], "scale": 0.25, "antialias": True},
        {"op": "concat", "in": ["aq", "bq"], "out": ["ab"]},
        _conv("s.e1", "ab", "e1", stride=2),
        _conv("s.e2", "e1", "e2"),
        {"op": "add", "in": ["e2", "e1"], "out": ["e2r"]},                     # the residual peephole
        {"op": "avgpool", "in": ["aq"], "out": ["a8"], "k": 2},
        {"op": "avgpool", "in": ["bq"], "out": ["b8"], "k": 2},
        {"op": "luma", "in": ["a8"], "out": ["la"]},
        {"op": "luma", "in": ["b8"], "out": ["lb"]},
        {"op": "sad_volume", "in": ["la", "lb"], "out": ["cv"], "radius": 1},
        {"op": "zeros", "in": ["e1"], "out": ["z2"], "ch": 2},
        {"op": "copy", "in": ["e2r"], "out": ["e2c"]},
        {"op": "concat", "in": ["e2c", "cv", "z2"], "out": ["cin"]},
        _conv("s.h0", "cin", "h0"),
        _conv("s.fl", "h0", "flow"),
        _conv("s.vi", "h0", "vis"),
        _conv("s.hh", "h0", "hh"),
        {"op": "repeat", "times": "K", "body": [                                # the flow refined K times
            sl("flow", "fa", 0, 2),
            {"op": "warp", "in": ["a8", "fa"], "out": ["wa8"]},
            {"op": "concat", "in": ["wa8", "h0"], "out": ["fx"]},
            _conv("s.rd", "fx", "d"),
            {"op": "add", "in": ["d", "flow"], "out": ["flow"]}]},
    ]
    mid = [
        {"op": "film_mlp", "in": ["t"], "out": ["g"]},                          # the pair / mid boundary
        {"op": "film_modulate", "in": ["hh", "g"], "out": ["hm"]},
        _conv("s.fd", "hm", "fd"),
        sl("flow", "ff", 0, 2), sl("flow", "fb", 2, 4),
        {"op": "mul_t", "in": ["ff"], "out": ["ftf"], "mode": "fwd"},
        {"op": "mul_t", "in": ["fb"], "out": ["ftb"], "mode": "bwd"},
        {"op": "concat", "in": ["ftf", "ftb"], "out": ["ft4"]},
        sl("fd", "dfl", 0, 4),
        {"op": "add", "in": ["ft4", "dfl"], "out": ["flt"]},
        {"op": "neg", "in": ["vis"], "out": ["vn"]},
        _conv("s.vc", "vn", "vc"),                                               # reads a scaled view: mat
        {"op": "concat", "in": ["flt", "vc"], "out": ["x7"]},
        {"op": "convex_upsample", "in": ["hh", "x7"], "out": ["up7"]},
        sl("up7", "fq", 0, 4), sl("up7", "vq", 4, 7), sl("fq", "fqa", 0, 2), sl("fq", "fqb", 2, 4),
        {"op": "warp", "in": ["aq", "fqa"], "out": ["wa"]},
        {"op": "warp", "in": ["bq", "fqb"], "out": ["wb"]},
        {"op": "blend_weights", "in": ["vq"], "out": ["bw0", "bw1"]},           # the blendmix peephole
        {"op": "mul", "in": ["wa", "bw0"], "out": ["m1"]},
        {"op": "mul", "in": ["wb", "bw1"], "out": ["m2"]},
        {"op": "add", "in": ["m1", "m2"], "out": ["bl"]},
        {"op": "luma_grad", "in": ["bl"], "out": ["lg"]},
        {"op": "concat", "in": ["wa", "wb", "vq", "lg"], "out": ["rx"]},
        _conv("s.r1", "rx", "r1"),
        _conv("s.r2", "r1", "r2"),
        {"op": "affine_out", "in": ["r2"], "out": ["rt"]},
        {"op": "scale", "in": ["fq"], "out": ["fr"], "factor": 4.0},
        {"op": "render_pix", "in": ["A", "B", "fr", "vq", "rt"], "out": ["render"], "output": True},
    ]
    return pair + mid


def model_bytes(seed=0, render_sampling="bicubic", k=2):
    """(graph.json, flyhighfg.json, flyhighfg.bin) bytes of the model, random f16 weights from seed."""
    rng = np.random.default_rng(seed)
    tensors, blob, off = {}, [], 0

    def add(name, arr):
        nonlocal off
        a = np.asarray(arr, np.float32).astype(np.float16).view(np.uint16).reshape(-1)
        tensors[name] = {"shape": list(np.shape(arr)), "offset": off}
        blob.append(a)
        off += a.size

    for stem, cin, cout, act in LAYERS:
        names = _w(stem, act)
        add(names[0], rng.normal(0, np.sqrt(1.0 / (9 * cin)), (cout, cin, 3, 3)))
        add(names[1], rng.normal(0, 0.01, cout))
        if act:
            add(names[2], rng.uniform(0.05, 0.3, cout))
    add("film.film.0.weight", rng.normal(0, 1, (64, 1)))
    add("film.film.0.bias", rng.normal(0, 0.1, 64))
    add("film.film.2.weight", rng.normal(0, 0.1, (96, 64)))
    add("film.film.2.bias", rng.normal(0, 0.01, 96))
    graph = json.dumps({"meta": {}, "ops": ops()}).encode()
    manifest = json.dumps({"meta": {"model": "synthetic-every-step", "format_version": 1, "train_step": 0,
                                    "render_sampling": render_sampling, "n_params": off, "default_K": k},
                           "tensors": tensors}).encode()
    return graph, manifest, np.concatenate(blob).astype("<u2").tobytes()


# the step kinds of a plan of this model (frame input, network and mid ops, repair, frame output)
STEP_KINDS = {"rgba_in", "interp", "conv", "mat", "concat", "avgpool", "luma", "sad", "warp", "binary", "unary",
              "film_mlp", "film", "convex", "blendmix", "luma_grad", "render", "rgba_out", "gmhs"}
