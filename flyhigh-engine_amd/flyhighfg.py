"""The conv layers of the FlyHighFG graph and of the benchmark configurations, as the planner walks them.

The FlyHighFG table restates the conv ops of the reference graph (models/graph.json:68-1244, the weight shapes of
models/flyhighfg.json) as the planner's conv arm sees them (crates/flyhigh-engine/src/net/build.rs:209-278):
``conv`` ops carry a PReLU slope, ``conv2d`` ops and the convex-upsample conv (build.rs:379-416) have none, and a
following ``add`` of a plain same-shape tensor is fused as the residual (build.rs:222-237). The pair / mid split
is the graph's mid_start (crates/flyhigh-engine/src/model/graph.rs:182). Layer input sizes follow from the
network size: the encoder reads the quarter-resolution image and halves it twice (stride-2 e1 and e3); the
coarse block works at 1/16, the fine block and FiLM at 1/8, the refine block at 1/4.
"""
from __future__ import annotations

import math

from dataclasses import dataclass
from typing import List, Optional


@dataclass(frozen=True)
class ConvLayer:
    name: str
    stage: str            # "pair" or "mid"
    cin: int
    cout: int
    h: int                # input height / width
    w: int
    stride: int = 1
    k: int = 3
    act: int = 1          # 1 PReLU (graph op conv), 0 identity (conv2d), 2 LeakyReLU(alpha)
    alpha: float = 0.0
    residual: bool = False
    n: int = 1            # batch: images this conv runs on (the A and B encoders share their weights)
    chain: Optional[str] = None  # the conv whose output is this conv's input (None: a non-conv op feeds it)
    res_from: Optional[str] = None  # the conv whose output is the fused residual (None: another op's output)
    weight: str = ""      # weight tensor name in the model manifest

    @property
    def hout(self):
        pad = 1 if self.k == 3 else 0
        return (self.h + 2 * pad - self.k) // self.stride + 1

    @property
    def wout(self):
        pad = 1 if self.k == 3 else 0
        return (self.w + 2 * pad - self.k) // self.stride + 1

    @property
    def flops(self):
        return 2 * self.n * self.hout * self.wout * self.cout * self.cin * self.k * self.k

    @property
    def bytes(self):
        """Algorithmic bytes: f16 input + output + weights + bias + slope (+ residual), each touched once."""
        out = self.n * self.hout * self.wout * self.cout
        return 2 * (self.n * self.h * self.w * self.cin + out + self.cout * self.cin * self.k * self.k + self.cout
                    + (self.cout if self.act == 1 else 0) + (out if self.residual else 0))


def default_internal(w: int, h: int):
    """The network resolution of a frame size: the frame itself up to 960 px on the long side, above that the
    480-line rung, aspect kept, multiples of 8 (crates/flyhigh-engine/src/options.rs:347-356)."""
    if max(w, h) <= 960:
        return (w, h)
    s = min(480.0 / h, 1.0)
    rw = max(int(math.floor(w * s / 8.0 + 0.5)) * 8, 64)  # f64::round: half away from zero
    rh = max(int(math.floor(h * s / 8.0 + 0.5)) * 8, 64)
    return (min(rw, w), min(rh, h))


def pad32(v: int) -> int:
    return (v + 31) // 32 * 32


def flyhighfg_layers(net_w: int = 864, net_h: int = 480, k: int = 1, batch_encoders: bool = True) -> List[ConvLayer]:
    """Conv layers of one pair() and one mid() at a padded network size (default: 1080p's 856x480 -> 864x480).
    batch_encoders: the A and B encoders (the same weights on the two frames, models/graph.json enc.* ops) run as
    one batch-2 conv per layer instead of two convs; the work is the same."""
    qw, qh = net_w // 4, net_h // 4
    e8w, e8h = (qw + 2 - 3) // 2 + 1, (qh + 2 - 3) // 2 + 1
    e16w, e16h = (e8w + 2 - 3) // 2 + 1, (e8h + 2 - 3) // 2 + 1
    L = []
    for side in (("ab",) if batch_encoders else ("a", "b")):
        n = 2 if side == "ab" else 1
        L += [
            ConvLayer(f"enc.e1.{side}", "pair", 3, 36, qh, qw, 2, n=n, weight="enc.e1.0.weight"),
            ConvLayer(f"enc.e2.{side}", "pair", 36, 36, e8h, e8w, residual=True, n=n, chain=f"enc.e1.{side}",
                      res_from=f"enc.e1.{side}", weight="enc.e2.0.weight"),
            ConvLayer(f"enc.e3.{side}", "pair", 36, 72, e8h, e8w, 2, n=n, chain=f"enc.e2.{side}",
                      weight="enc.e3.0.weight"),
            ConvLayer(f"enc.e4.{side}", "pair", 72, 72, e16h, e16w, residual=True, n=n, chain=f"enc.e3.{side}",
                      res_from=f"enc.e3.{side}", weight="enc.e4.0.weight"),
        ]
    L += [
        ConvLayer("coarse.c1", "pair", 279, 96, e16h, e16w, weight="coarse.c1.0.weight"),
        ConvLayer("coarse.c2", "pair", 96, 96, e16h, e16w, chain="coarse.c1", weight="coarse.c2.0.weight"),
        ConvLayer("coarse.c3", "pair", 96, 96, e16h, e16w, residual=True, chain="coarse.c2",
                  res_from="coarse.c1", weight="coarse.c3.0.weight"),
        ConvLayer("coarse.c4", "pair", 96, 96, e16h, e16w, chain="coarse.c3", weight="coarse.c4.0.weight"),
        ConvLayer("coarse.head", "pair", 96, 12, e16h, e16w, act=0, chain="coarse.c4",
                  weight="coarse.head.weight"),
    ]
    for i in range(k):
        sfx = f".{i}" if k > 1 else ""
        L += [
            ConvLayer(f"fine.r1{sfx}", "pair", 155, 48, e8h, e8w, weight="fine.r1.0.weight"),
            ConvLayer(f"fine.r2{sfx}", "pair", 48, 48, e8h, e8w, chain=f"fine.r1{sfx}", weight="fine.r2.0.weight"),
            ConvLayer(f"fine.r3{sfx}", "pair", 48, 48, e8h, e8w, chain=f"fine.r2{sfx}", weight="fine.r3.0.weight"),
            ConvLayer(f"fine.out{sfx}", "pair", 48, 7, e8h, e8w, act=0, residual=True, chain=f"fine.r3{sfx}",
                      weight="fine.out.weight"),  # flow, vis += its output: the add fused as the residual
        ]
    L += [
        ConvLayer("film.h1", "mid", 48, 48, e8h, e8w, weight="film.h1.0.weight"),
        ConvLayer("film.h2", "mid", 48, 48, e8h, e8w, chain="film.h1", weight="film.h2.0.weight"),
        ConvLayer("film.out", "mid", 48, 5, e8h, e8w, act=0, chain="film.h2", weight="film.out.weight"),
        ConvLayer("up.w", "mid", 48, 36, e8h, e8w, act=0, weight="up.w.weight"),
        ConvLayer("refine.q1", "mid", 14, 24, qh, qw, weight="refine.q1.0.weight"),
        ConvLayer("refine.q2", "mid", 24, 24, qh, qw, chain="refine.q1", weight="refine.q2.0.weight"),
        ConvLayer("refine.q3", "mid", 24, 24, qh, qw, chain="refine.q2", weight="refine.q3.0.weight"),
        ConvLayer("refine.q4", "mid", 24, 3, qh, qw, act=0, chain="refine.q3", weight="refine.q4.weight"),
    ]
    return L


# Consecutive convs of models/graph.json whose intermediate tensor has no other reader (enc.e1's and enc.e3's outputs
# are also the residuals that enc.e2's and enc.e4's "add" take: the pair's second conv adds the first's output),
# and of the 1080p/4 ladder configuration (one of its two overlapping pairs runs fused): each pair can run as one fused
# launch (fhc_conv_pair_plan_create). (first conv, second conv, second's residual is the first's output)
FUSIBLE_PAIRS = [("enc.e1", "enc.e2", True), ("enc.e3", "enc.e4", True), ("fine.r2", "fine.r3", False),
                 ("film.h1", "film.h2", False), ("c2.b1", "c2.b2", False), ("c2.b2", "c2.b3", False),
                 ("refine.q1", "refine.q2", False), ("refine.q3", "refine.q4", False)]


def fusible_pairs(layers: List[ConvLayer]):
    """(first, second, res_mid) layer pairs of `layers` that FUSIBLE_PAIRS names (by prefix: enc.e1.ab, fine.r2.0)."""
    by = {L.name: L for L in layers}
    out = []
    for a_pre, b_pre, res_mid in FUSIBLE_PAIRS:
        for L in layers:
            if L.name == a_pre or L.name.startswith(a_pre + "."):
                b_name = b_pre + L.name[len(a_pre):]
                B = by.get(b_name)
                if B is not None and B.chain == L.name and (not res_mid or B.res_from == L.name):
                    out.append((L, B, res_mid))
    return out


def batched_layers(pairs: int = 8, mids_per_pair: int = 3, net_w: int = 864, net_h: int = 480) -> List[ConvLayer]:
    """The frame's conv layers batched over `pairs` independent frame pairs with `mids_per_pair` mid() phases each:
    pair-stage convs on pairs images (the encoders on 2 * pairs: A and B), mid-stage convs on pairs * mids_per_pair.
    8 pairs of 3840x2160 frames run at the same network size as 1080p (default_internal(3840, 2160) = (856, 480),
    tests/defaults.rs:12)."""
    import dataclasses
    return [dataclasses.replace(L, n=L.n * (pairs if L.stage == "pair" else pairs * mids_per_pair))
            for L in flyhighfg_layers(net_w, net_h)]


def config_layers(cfg: int) -> List[ConvLayer]:
    """The single-layer / ladder benchmark configurations C1-C3 (batch 1, NHWC f16)."""
    if cfg == 1:  # 3x3 32->32 at 1080p/8, LeakyReLU(0.1)
        return [ConvLayer("c1.conv", "pair", 32, 32, 136, 240, act=2, alpha=0.1)]
    if cfg == 2:  # 1080p/4 ladder: s2 32->64 from 544x960, three 64->64, residual (the s2 output) on the last
        return [
            ConvLayer("c2.down", "pair", 32, 64, 544, 960, 2),
            ConvLayer("c2.b1", "pair", 64, 64, 272, 480, chain="c2.down"),
            ConvLayer("c2.b2", "pair", 64, 64, 272, 480, chain="c2.b1"),
            ConvLayer("c2.b3", "pair", 64, 64, 272, 480, residual=True, chain="c2.b2", res_from="c2.down"),
        ]
    if cfg == 3:  # deep small-spatial 1080p/16: 128->128 (split-K) and 1x1 128->64 on the same input
        return [
            ConvLayer("c3.deep", "pair", 128, 128, 68, 120),
            ConvLayer("c3.pw", "pair", 128, 64, 68, 120, k=1, act=0),
        ]
    raise ValueError(f"unknown configuration {cfg}")


@dataclass
class NetOp:
    """One non-conv op instance of models/graph.json as the planner runs it (net/build.rs:199-450): its kind, batch
    (the A and B branches run as a batch of 2 per frame pair), NHWC input shapes (h, w, c), output shape, and
    parameters (radius, pool k, resize size and antialias)."""
    name: str
    op: str
    n: int
    ins: List[tuple]
    out: tuple
    kw: dict

    @property
    def bytes(self):
        """Algorithmic HBM bytes: every input read once and the output written once (f16)."""
        return 2 * self.n * (sum(h * w * c for h, w, c in self.ins) + self.out[0] * self.out[1] * self.out[2])


def network_ops(net_w: int = 864, net_h: int = 480, pairs: int = 1, mids: int = 1) -> List[NetOp]:
    """The non-conv ops of pair() (per frame pair) and mid() (per mid phase) at a padded network size, fine loop
    k = 1; `pairs` frame pairs and `mids` mid() phases in total. The graph's slices, scales and concats are views (no
    launch); its film_mlp is a 64-wide MLP of the scalar t on the host (net/build.rs:331-357); render_pix, rgba_in /
    rgba_out and affine_out sit outside the network (frame I/O) and are not listed."""
    qw, qh = net_w // 4, net_h // 4
    e8w, e8h = (qw + 2 - 3) // 2 + 1, (qh + 2 - 3) // 2 + 1
    e16w, e16h = (e8w + 2 - 3) // 2 + 1, (e8h + 2 - 3) // 2 + 1
    ab, m = 2 * pairs, mids
    return [
        NetOp("interp A,B -> aq,bq", "interp", ab, [(net_h, net_w, 3)], (qh, qw, 3), dict(oh=qh, ow=qw, aa=True)),
        NetOp("avgpool aq -> i8", "avgpool", ab, [(qh, qw, 3)], (qh // 2, qw // 2, 3), dict(k=2)),
        NetOp("avgpool i8 -> i16", "avgpool", ab, [(e8h, e8w, 3)], (e8h // 2, e8w // 2, 3), dict(k=2)),
        NetOp("luma i16", "luma", ab, [(e16h, e16w, 3)], (e16h, e16w, 1), dict(grad=False)),
        NetOp("sad_volume r3", "sad", pairs, [(e16h, e16w, 1), (e16h, e16w, 1)], (e16h, e16w, 49), dict(r=3)),
        NetOp("interp flow16", "interp", pairs, [(e16h, e16w, 4)], (e8h, e8w, 4), dict(oh=e8h, ow=e8w, aa=False)),
        NetOp("interp vis16", "interp", pairs, [(e16h, e16w, 3)], (e8h, e8w, 3), dict(oh=e8h, ow=e8w, aa=False)),
        NetOp("warp f8a,f8b", "warp", ab, [(e8h, e8w, 36), (e8h, e8w, 2)], (e8h, e8w, 36), {}),
        NetOp("warp i8a,i8b", "warp", ab, [(e8h, e8w, 3), (e8h, e8w, 2)], (e8h, e8w, 3), {}),
        NetOp("luma ia,ib", "luma", ab, [(e8h, e8w, 3)], (e8h, e8w, 1), dict(grad=False)),
        NetOp("sad_volume r2", "sad", pairs, [(e8h, e8w, 1), (e8h, e8w, 1)], (e8h, e8w, 25), dict(r=2)),
        NetOp("film_modulate", "film", m, [(e8h, e8w, 48), (1, 1, 96)], (e8h, e8w, 48), {}),
        NetOp("convex_upsample", "convex", m, [(e8h, e8w, 36), (e8h, e8w, 7)], (qh, qw, 7), {}),
        NetOp("warp aq,bq (refine)", "warp", 2 * m, [(qh, qw, 3), (qh, qw, 2)], (qh, qw, 3), {}),
        NetOp("blendmix", "blendmix", m, [(qh, qw, 3), (qh, qw, 3), (qh, qw, 3)], (qh, qw, 3), {}),
        NetOp("luma_grad", "luma", m, [(qh, qw, 3)], (qh, qw, 1), dict(grad=True)),
    ]
