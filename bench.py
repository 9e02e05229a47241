#!/usr/bin/env python3
"""Benchmark of the FlyHigh frame path on one MI355X.

Workload (one step): one 1080p pair() + mid(0.5) as the reference's Session runs it: two 1920x1080 RGBA8 frames
resident in HBM -> rgba_in and the antialiased downscale to the 864x480 network -> every op of the FlyHighFG graph
(the convs, fused conv pairs, the network ops) -> render_pix at 1920x1088 and rgba_out -> the RGBA8 in-between frame.
Random weights of the architecture, synthetic frames (a procedural picture and the same moved 12 px). The frame is
captured once as a HIP graph and replayed; value = frames/s = 1e6 / us per frame (wall clock over the timed replays,
synchronised on both sides).

Alongside (the last stdout line is one compact JSON record; the full record goes to --detail): every launch of the
frame timed alone against its roofline, the dominant one cold; the conv-only step (every conv of pair()+mid(), one
graph) with per-layer warm/cold time and roofline fraction (each launch captured R times in a graph, median of G
replays; "cold" rotates buffer sets larger than the 256 MB MALL); the single-layer configurations (3x3 32->32 at
1080p/8; the 1080p/4 stride-2 ladder; the 1080p/16 deep layer and 1x1); the frame over 8 rotating sets of frames
and buffers (each replay reading what another wrote, beyond the MALL); the batched workload (8 independent 3840x2160
RGBA8 frame pairs through the whole graph with 3 mid() phases each, 24 generated frames a step, one HIP graph), and
its convs alone; the sustained MFMA rate; and the CPU baseline: the same frame through the oracle (a C restatement of
the reference's arithmetic) on the host's cores.

    python bench.py [--steps K] [--warmup W] [--no-cpu] [--no-configs] [--no-batched] [--no-fuse] [--ops]
    python bench.py --only-frame | --only-ops | --only-batched
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flyhigh-engine_amd"))


METRIC = "1080p frames/s (pair+mid); per-conv-layer % of MFMA or HBM roofline"
# the reference's published time for the same workload (1080p frames, network 856x480, k = 1, repair 1): pair 1.61 ms +
# mid 0.81 ms per generated frame on an RTX 4060 Ti (README.md:160 of the reference)
PUBLISHED_MS_PER_FRAME = 2.41
HBM_PEAK = 8.0e12       # B/s
MFMA_F16_PEAK = 2.5e15  # FLOP/s, dense


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def pad8(c):
    return (c + 7) // 8 * 8


def roof(flops, nbytes):
    t_hbm, t_mfma = nbytes / HBM_PEAK, flops / MFMA_F16_PEAK
    return ("hbm", t_hbm) if t_hbm >= t_mfma else ("mfma", t_mfma)


class Net:
    """Plans and resident buffers of a list of conv layers, chained as the graph chains them. With `tune`, each
    conv shape is autotuned on its buffers before its plan is made (the reference's conv_pick with autotune on)."""

    def __init__(self, layers, seed, torch, np, fhconv, tune=True, slope=None):
        self.layers = layers
        self.plans, self.bufs, self.tuned, self.params = {}, {}, {}, {}
        self.pairs = {}  # first layer's name -> (pair plan, second layer)
        dev = torch.device("cuda", 0)
        rng = np.random.default_rng(seed)
        f16 = lambda a: torch.from_numpy(np.asarray(a, np.float32).astype(np.float16))  # noqa: E731
        for L in layers:
            wt = f16(rng.normal(0, np.sqrt(2.0 / (L.k * L.k * L.cin)), (L.cout, L.cin, L.k, L.k)))
            b = f16(rng.normal(0, 0.01, L.cout))
            s = (f16(np.full(L.cout, slope)) if slope is not None else f16(rng.uniform(0.05, 0.3, L.cout))) \
                if L.act == 1 else None
            # activations are NHWC with the channel stride padded to 8 halves (16 bytes): the concat buffers the
            # graph's convs read (279, 155, 14 channels ...) are allocated that way, and the convs read views
            cx, cy = pad8(L.cin), pad8(L.cout)
            d = fhconv.make_desc(L.n, L.h, L.w, L.cin, L.cout, k=L.k, stride=L.stride, act=L.act, alpha=L.alpha,
                                 residual=L.residual, x_cstride=cx, y_cstride=cy, r_cstride=cy if L.residual else 0)
            x = self.bufs[L.chain][1] if L.chain else \
                f16(rng.uniform(-1, 1, (L.n, L.h, L.w, cx))).to(dev)
            y = torch.zeros((L.n, L.hout, L.wout, cy), dtype=torch.float16, device=dev)
            if L.residual:
                r = self.bufs[L.res_from][1] if L.res_from else \
                    f16(rng.uniform(-1, 1, (L.n, L.hout, L.wout, cy))).to(dev)
            else:
                r = None
            if tune:
                key = (L.n, L.cin, L.cout, L.h, L.w, L.stride, L.k)
                if key not in self.tuned:
                    code, us = fhconv.autotune(d, wt, b, s, x, y, r, reps=20)
                    self.tuned[key] = (fhconv.variant_name(code), round(us, 3))
            p = fhconv.ConvPlan(d, wt, b, s)
            ws = torch.empty(p.workspace_bytes // 4 + 4, dtype=torch.float32, device=dev) \
                if p.workspace_bytes else None
            self.plans[L.name] = p
            self.bufs[L.name] = (x, y, r, ws)
            self.params[L.name] = (d, wt, b, s)

    def fuse(self, pairs, torch, fhconv, stream, time_fn, default_tile=False, always=False):
        """Pair plans for (first, second, res_mid) layer pairs: the second's output buffer, the first's input; every
        instantiated tile height (1, 2, 4 or 8 rows), wave rows (1 or 2) and loop (one workgroup per tile, a
        resident grid, or a resident grid with the two stages on separate waves) timed on the real buffers, the fastest kept (default_tile: the pair planner's own choice, no
        timing), and only where it beats the two separate launches (always: every pair the library instantiates, with
        the default tile and no timing, as the frame program fuses them). A pair that shares a conv with one fused
        before it is skipped."""
        used = set()
        for A, B, res_mid in pairs:
            if A.name in used or B.name in used:
                continue
            if always:
                da, wa, ba, sa = self.params[A.name]
                db, wb, bb, sb = self.params[B.name]
                try:
                    pp = fhconv.ConvPairPlan(da, wa, ba, sa, db, wb, bb, sb, res_mid=res_mid)
                except fhconv.FhcError:
                    continue
                self.pairs[A.name] = (pp, B, None, res_mid)
                used |= {A.name, B.name}
                continue
            sep = time_fn(lambda i=0: (self.run_one(A, stream=stream), self.run_one(B, stream=stream)))
            da, wa, ba, sa = self.params[A.name]
            db, wb, bb, sb = self.params[B.name]
            x = self.bufs[A.name][0]
            _, y, r, _ = self.bufs[B.name]
            rx = None if res_mid else r
            best = None
            combos = [(0, 0, 0)] if default_tile else \
                [(th, wm, lp) for lp in (1, 2) for th, wm in ((1, 1), (2, 1), (4, 1), (2, 2), (4, 2), (8, 2))] + \
                [(th, 1, 3) for th in (4, 8)]
            for th, wm, lp in combos:
                try:
                    pp = fhconv.ConvPairPlan(da, wa, ba, sa, db, wb, bb, sb, res_mid=res_mid, tile_rows=th,
                                             wave_rows=wm, loop=lp)
                except fhconv.FhcError:
                    continue  # not instantiated for these channels
                us = time_fn(lambda i=0, pp=pp: pp.run(x, y, rx, stream=stream))
                if best is None or us < best[1]:
                    best = (pp, us)
            if best is not None and best[1] < sep:
                self.pairs[A.name] = (best[0], B, round(best[1], 3), res_mid)
                used |= {A.name, B.name}

    def run_one(self, L, stream=None):
        x, y, r, ws = self.bufs[L.name]
        self.plans[L.name].run(x, y, r, ws, stream=stream)

    def run(self, names=None, fused=False):
        skip = {B.name for _, B, _, _ in self.pairs.values()} if fused else set()
        for L in self.layers:
            if names is not None and L.name not in names:
                continue
            if fused and L.name in self.pairs:
                pp, B, _, res_mid = self.pairs[L.name]
                x = self.bufs[L.name][0]
                _, y, r, _ = self.bufs[B.name]
                pp.run(x, y, None if res_mid else r)
            elif L.name not in skip:
                x, y, r, ws = self.bufs[L.name]
                self.plans[L.name].run(x, y, r, ws)


def time_graph(torch, fn, reps, graphs, stream):
    """Median over `graphs` replays of a graph holding `reps` calls of fn, per call, in microseconds. Capture,
    replays and events all run on `stream`."""
    g = torch.cuda.CUDAGraph()
    ts = []
    with torch.cuda.stream(stream):
        fn()  # warm the path outside the capture
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            for i in range(reps):
                fn(i)
        g.replay()
        for _ in range(graphs):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            g.replay()
            e1.record(stream)
            e1.synchronize()
            ts.append(e0.elapsed_time(e1) * 1e3 / reps)
    return statistics.median(ts)


def layer_timing(torch, np, fhconv, net, L, reps, graphs, cold_bytes, stream):
    """Warm and cold per-launch time of one layer (graph of `reps` launches)."""
    p = net.plans[L.name]
    x, y, r, ws = net.bufs[L.name]
    warm = time_graph(torch, lambda i=0: p.run(x, y, r, ws), reps, graphs, stream)
    # cold: rotate through enough distinct x / y / res sets to exceed the MALL
    per = x.numel() * 2 + y.numel() * 2 + (r.numel() * 2 if r is not None else 0)
    nsets = max(2, min(4096, -(-cold_bytes // per)))
    creps = -(-max(reps, nsets) // nsets) * nsets
    sets = [(torch.empty_like(x).uniform_(-1, 1), torch.empty_like(y),
             torch.empty_like(r).uniform_(-1, 1) if r is not None else None) for _ in range(nsets)]
    cold = time_graph(torch, lambda i=0: p.run(sets[i % nsets][0], sets[i % nsets][1], sets[i % nsets][2], ws),
                      creps, graphs, stream)
    del sets
    bound, t_roof = roof(L.flops, L.bytes)
    d = p.describe()
    return dict(name=L.name, variant=d["name"], cin=L.cin, cout=L.cout, h=L.h, w=L.w, stride=L.stride, k=L.k,
                us_warm=round(warm, 3), us_cold=round(cold, 3), flops=L.flops, bytes=L.bytes, bound=bound,
                roof_us=round(t_roof * 1e6, 3), frac_cold=round(t_roof * 1e6 / cold, 4),
                frac_warm=round(t_roof * 1e6 / warm, 4),
                tflops_cold=round(L.flops / cold / 1e6, 2), gbs_cold=round(L.bytes / cold / 1e3, 1),
                cold_sets=nsets)


def pair_timing(torch, net, a_name, reps, graphs, cold_bytes, stream):
    """Warm and cold per-launch time of a fused pair (graph of `reps` launches), with its algorithmic work: both
    convs' FLOPs; bytes of the first's input, the second's output and residual, both weights (the intermediate
    stays on chip)."""
    pp, B, _, res_mid = net.pairs[a_name]
    x = net.bufs[a_name][0]
    _, y, r, _ = net.bufs[B.name]
    r = None if res_mid else r
    warm = time_graph(torch, lambda i=0: pp.run(x, y, r), reps, graphs, stream)
    per = x.numel() * 2 + y.numel() * 2 + (r.numel() * 2 if r is not None else 0)
    nsets = max(2, min(4096, -(-cold_bytes // per)))
    creps = -(-max(reps, nsets) // nsets) * nsets
    sets = [(torch.empty_like(x).uniform_(-1, 1), torch.empty_like(y),
             torch.empty_like(r).uniform_(-1, 1) if r is not None else None) for _ in range(nsets)]
    cold = time_graph(torch, lambda i=0: pp.run(sets[i % nsets][0], sets[i % nsets][1], sets[i % nsets][2]),
                      creps, graphs, stream)
    del sets
    d = pp.describe()
    flops, nbytes = d["flops"], d["bytes"]
    bound, t_roof = roof(flops, nbytes)
    return dict(name=a_name + "+" + B.name, variant=d["name"], us_warm=round(warm, 3), us_cold=round(cold, 3),
                flops=flops, bytes=nbytes, bound=bound, roof_us=round(t_roof * 1e6, 3),
                frac_cold=round(t_roof * 1e6 / cold, 4), frac_warm=round(t_roof * 1e6 / warm, 4),
                tflops_cold=round(flops / cold / 1e6, 2), gbs_cold=round(nbytes / cold / 1e3, 1), cold_sets=nsets)


def net_op_call(fh, op, ins, out, stream):
    """One launch of the network op `op` (flyhighfg.NetOp) on device tensors ins -> out."""
    k = op.kw
    if op.op == "interp":
        return fh.interp(ins[0], k["oh"], k["ow"], k["aa"], out=out, stream=stream)
    if op.op == "avgpool":
        return fh.avgpool(ins[0], k["k"], out=out, stream=stream)
    if op.op == "luma":
        return fh.luma(ins[0], k["grad"], out=out, stream=stream)
    if op.op == "sad":
        return fh.sad(ins[0], ins[1], k["r"], out=out, stream=stream)
    if op.op == "warp":
        return fh.warp(ins[0], ins[1], out=out, stream=stream)
    if op.op == "film":
        return fh.film(ins[0], ins[1], out=out, stream=stream)
    if op.op == "convex":
        return fh.convex(ins[0], ins[1], out=out, stream=stream)
    if op.op == "blendmix":
        return fh.blendmix(ins[0], ins[1], ins[2], out=out, stream=stream)
    raise ValueError(op.op)


def net_ops_timing(torch, fhops, ops, reps, graphs, cold_bytes, stream):
    """Warm and cold per-launch time of each network op instance (graph of `reps` launches) against its HBM
    roofline: the algorithmic bytes (inputs read once, output written once) at 8 TB/s."""
    rows = []
    for op in ops:
        def make():
            ins = [torch.empty((op.n,) + s, dtype=torch.float16, device="cuda").uniform_(0, 1) for s in op.ins]
            return ins, torch.empty((op.n,) + op.out, dtype=torch.float16, device="cuda")
        i0, o0 = make()
        warm = time_graph(torch, lambda i=0: net_op_call(fhops, op, i0, o0, stream), reps, graphs, stream)
        nsets = max(2, min(4096, -(-cold_bytes // op.bytes)))
        creps = -(-max(reps, nsets) // nsets) * nsets
        sets = [make() for _ in range(nsets)]
        cold = time_graph(torch, lambda i=0: net_op_call(fhops, op, *sets[i % nsets], stream), creps, graphs, stream)
        del sets
        roof_us = op.bytes / HBM_PEAK * 1e6
        rows.append(dict(name=op.name, op=op.op, n=op.n, bytes=op.bytes, us_warm=round(warm, 3),
                         us_cold=round(cold, 3), roof_us=round(roof_us, 3), frac_cold=round(roof_us / cold, 4),
                         frac_warm=round(roof_us / warm, 4), gbs_cold=round(op.bytes / cold / 1e3, 1),
                         cold_sets=nsets))
        log("net op", json.dumps(rows[-1]))
    return rows


def net_ops_report(args, torch, flyhighfg, stream, net_w, net_h):
    """The network ops of one frame (1 pair, 1 mid) and of the batched workload (8 pairs, 3 mids each)."""
    import fhops
    frame = net_ops_timing(torch, fhops, flyhighfg.network_ops(net_w, net_h, 1, 1), args.reps, args.graphs,
                           args.cold_mb << 20, stream)
    batched = net_ops_timing(torch, fhops, flyhighfg.network_ops(net_w, net_h, 8, 24), args.reps, args.graphs,
                             args.cold_mb << 20, stream)
    torch.cuda.empty_cache()
    return dict(frame=frame, frame_us_warm_sum=round(sum(r["us_warm"] for r in frame), 3),
                batched=batched, batched_us_warm_sum=round(sum(r["us_warm"] for r in batched), 3),
                batched_workload="8 frame pairs (A/B ops over 16 frames) and 24 mid() phases at network 864x480")


def eager_frames(args, torch, np, stream, t=0.5):
    """The 1080p frame of frame_1080p (committed MI355X choices, repair on) run args.eager_frames times eagerly with
    no timing and no graph: one dispatch per launch, for profilers' counter passes."""
    import fhconv
    import flyhighfg_net as fnet
    if not args.tune:
        fhconv.parse_tune(open(os.path.join(ROOT, "flyhigh-engine_amd", "tune_mi355x.txt")).read())
    W = fnet.make_weights(7)
    be = fnet.GpuBackend(W, stream=stream, fuse=not args.no_fuse)
    f = fnet.FlyHighFG(be, 864, 480, frame=(1920, 1080), repair=1)
    be.upload_frames(f.frames, np.stack([fnet.procedural_frame(1920, 1080), fnet.procedural_frame(1920, 1080, 12, 0)]))
    be.set_g(fnet.film_mlp(W, t))
    with torch.cuda.stream(stream):
        for _ in range(args.eager_frames):
            f.pair_mid(t)
    stream.synchronize()
    log(f"bench: {args.eager_frames} eager 1080p frames done")
    return 0


def frame_1080p(args, torch, np, stream, t=0.5, repair=1, per_launch=True):
    """The headline workload: one 1080p pair() + mid(t) as the reference's Session runs it (net/session.rs:26-66,
    Internal::Auto): two 1920x1080 RGBA8 frames (the procedural picture and the same moved 12 px) resident in HBM ->
    rgba_in + antialiased downscale to the 864x480 network (one launch) -> every op of the graph (convs, fused pairs,
    the network ops and chains) -> render_pix at 1920x1088 + rgba_out to the RGBA8 frame (one launch). Random weights
    of the architecture (seed 7). Captured as one HIP graph on `stream`; args.steps replays after args.warmup,
    bracketed by a device synchronisation on both sides (wall clock; events on the stream beside it). Then (with
    per_launch) every launch of the frame alone, a graph of args.reps launches, median of args.graphs replays
    (warm). repair: the periodic-structure repair's level (1, the engine's default; 0 for the frame without it)."""
    import flyhighfg_net as fnet
    W = fnet.make_weights(7)
    be = fnet.GpuBackend(W, stream=stream, fuse=not args.no_fuse)
    net_w, net_h = 864, 480
    f = fnet.FlyHighFG(be, net_w, net_h, frame=(1920, 1080), repair=repair)
    be.upload_frames(f.frames, np.stack([fnet.procedural_frame(1920, 1080), fnet.procedural_frame(1920, 1080, 12, 0)]))
    be.set_g(fnet.film_mlp(W, t))
    with torch.cuda.stream(stream):
        for _ in range(2):  # plans are made on the first run
            f.pair_mid(t)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            f.pair_mid(t)
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    us, ev_us = wall * 1e6 / args.steps, e0.elapsed_time(e1) * 1e3 / args.steps
    rgba = be.host_frames(f.rgba)
    ok = bool(np.all(rgba >> 24 == 255)) and len(np.unique(rgba)) > 1000
    if not per_launch:
        return dict(us_per_frame=round(us, 3), event_us_per_frame=round(ev_us, 3), output_ok=ok), (be, f, None)
    # every launch of the frame, timed alone (the recorder re-issues each with the frame's own buffers)
    be.record = []  # each launch re-issued alone
    with torch.cuda.stream(stream):
        f.pair_mid(t)
        stream.synchronize()
    rec, be.record = be.record, None
    launches = []
    for i, r in enumerate(rec):
        us_l = time_graph(torch, lambda j=0, fn=r["fn"]: fn(), args.reps, args.graphs, stream)
        bound, t_roof = roof(r["flops"], r["bytes"])
        launches.append(dict(i=i, label=r["label"], kind=r["kind"], us_warm=round(us_l, 3), bytes=r["bytes"],
                             flops=r["flops"], bound=bound, roof_us=round(t_roof * 1e6, 4),
                             frac_warm=round(t_roof * 1e6 / us_l, 4), kernels=r.get("kernels", 1)))
        log("frame launch", json.dumps(launches[-1]))
    res = dict(us_per_frame=round(us, 3), frames_per_s=round(1e6 / us, 2), event_us_per_frame=round(ev_us, 3),
               steps=args.steps, warmup=args.warmup, network=f"{net_w}x{net_h}", frame="1920x1080",
               launches=sum(x.get("kernels", 1) for x in rec),
               launch_us_sum=round(sum(x["us_warm"] for x in launches), 3),
               output_ok=ok, launch_table=launches,
               workload="1080p pair()+mid(0.5), two 1920x1080 RGBA8 frames to the RGBA8 in-between frame: "
                        "rgba_in+downscale to 864x480, every graph op, GMHS repair (level 1), bicubic render_pix at "
                        "1920x1088 + rgba_out; one HIP graph; random weights, synthetic frames (12 px shift)")
    return res, (be, f, rec)


def frame_rotating(args, torch, np, stream, sets=8, t=0.5):
    """The 1080p frame (frame_1080p's program, repair on) over `sets` independent frame pairs, each with its own
    buffers and HIP graph, replayed in turn: every replay reads frames and intermediates another replay wrote last
    (about 70 MB a set, more than the 256 MB MALL over the sets), as a stream of new frame pairs would. Microseconds
    per frame (wall clock over args.steps replays)."""
    import flyhighfg_net as fnet
    W = fnet.make_weights(7)
    be = fnet.GpuBackend(W, stream=stream, fuse=not args.no_fuse)
    progs, graphs = [], []
    with torch.cuda.stream(stream):
        for k in range(sets):
            f = fnet.FlyHighFG(be, 864, 480, frame=(1920, 1080), repair=1)
            be.upload_frames(f.frames, fnet.pair_frames(1920, 1080, 100 + k, shift=16))
            be.set_g(fnet.film_mlp(W, t))
            f.pair_mid(t)
            stream.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=stream):
                f.pair_mid(t)
            progs.append(f)
            graphs.append(g)
        for i in range(max(args.warmup, sets)):
            graphs[i % sets].replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            graphs[i % sets].replay()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    del graphs, progs
    return wall * 1e6 / args.steps


def batched_frames(args, torch, np, stream, pairs=8, phases=(0.25, 0.5, 0.75), steps=20, warmup=3):
    """The batched configuration as written: `pairs` independent 3840x2160 RGBA8 frame pairs (seeded textures, a
    per-pair translation in [-32, 32] px) resident in HBM -> the downscale to the 864x480 network (the internal size
    of 2160p) -> every op of pair() (the repair on) -> mid(t) at each of `phases` -> the bicubic render of every
    in-between frame at 3840x2176 and rgba_out: pairs x phases RGBA8 frames per step. Every conv runs once per layer
    over the whole batch (16, 8 or 24 images); one HIP graph per step. Random weights (seed 7)."""
    import flyhighfg_net as fnet
    W = fnet.make_weights(7)
    be = fnet.GpuBackend(W, stream=stream, fuse=not args.no_fuse)
    f = fnet.FlyHighFG(be, 864, 480, frame=(3840, 2160), repair=1, pairs=pairs, mids=len(phases))
    t0 = time.perf_counter()
    be.upload_frames(f.frames, np.concatenate([fnet.pair_frames(3840, 2160, p) for p in range(pairs)]))
    log(f"bench: {pairs} 3840x2160 frame pairs generated in {time.perf_counter() - t0:.1f} s")
    for j, t in enumerate(phases):
        be.set_g(f.film_vectors(W, t), j)
    with torch.cuda.stream(stream):
        for _ in range(2):  # plans are made on the first run
            f.run(phases)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        be.record = []
        with torch.cuda.graph(g, stream=stream):
            f.run(phases)
        rec, be.record = be.record, None
        for _ in range(warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(steps):
            g.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    step_us, ev_us = wall * 1e6 / steps, e0.elapsed_time(e1) * 1e3 / steps
    rgba = be.host_frames(f.rgba)
    ok = bool(np.all(rgba >> 24 == 255)) and all(len(np.unique(rgba[i, ::64, ::64])) > 100 for i in range(len(rgba)))
    n_out = pairs * len(phases)
    flops = sum(r["flops"] for r in rec)
    kinds = {}
    for r in rec:
        k = r["label"].split(" ")[0]
        kinds[k] = kinds.get(k, 0) + r.get("kernels", 1)
    log(f"bench: batched {pairs} pairs x {len(phases)} phases at 3840x2160: {step_us:.1f} us per step, "
        f"{n_out / step_us * 1e6:.0f} generated frames/s, {sum(kinds.values())} launches")
    del g, f
    return dict(workload=f"{pairs} independent 3840x2160 RGBA8 frame pairs (seeded textures, per-pair translation in "
                         f"[-32, 32] px) -> downscale to the 864x480 network -> pair() with the repair -> mid(t) at "
                         f"t = {', '.join(str(t) for t in phases)} -> bicubic render at 3840x2176 + rgba_out: "
                         f"{n_out} RGBA8 frames per step; every conv batched over the pairs (encoders over both "
                         "frames) or pairs x phases; one HIP graph; random weights",
                step_us=round(step_us, 2), event_step_us=round(ev_us, 2),
                generated_frames_per_s=round(n_out / step_us * 1e6, 1), pairs_per_s=round(pairs / step_us * 1e6, 1),
                step_tflops=round(flops / step_us / 1e6, 2), launches=sum(kinds.values()), launch_kinds=kinds,
                steps=steps, output_ok=ok)


def render_cold(args, torch, be, f, reps, graphs, cold_bytes, stream):
    """The frame-size render (fhc_render_rgba) over rotating sets of input frames and output frames larger than the
    MALL, so every launch reads its frames from HBM: per-launch microseconds."""
    per = 3 * f.frames.numel() // 2 * 4
    nsets = max(2, min(512, -(-cold_bytes // per)))
    sets = [(torch.randint_like(f.frames, -2 ** 31, 2 ** 31 - 1), torch.empty_like(f.rgba)) for _ in range(nsets)]
    fh = be.fh
    vf, vv, vr = fh.View(f.up7, 0), fh.View(f.up7, 4), fh.View(f.Rt, 0)

    def call(i=0):
        fr, out = sets[i % nsets]
        fh.render_rgba(fr[0:1], fr[1:2], vf, vv, vr, f.hp, f.wp, f.cubic, f.render_flags, f.fsx, f.fsy, out=out,
                       stream=stream)
    creps = -(-max(reps, nsets) // nsets) * nsets
    us = time_graph(torch, call, creps, graphs, stream)
    del sets
    return us, nsets


def cpu_frame_baseline(np, frames_n=3):
    """Seconds per 1080p pair()+mid() of the CPU oracle composition (the same program over oracle/: its C
    restatement of the reference's WGSL arithmetic, the convs multithreaded over rows), median of `frames_n` frames,
    inputs generated outside the timing."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import flyhighfg_net as fnet
    from frame_oracle import CpuBackend
    W = fnet.make_weights(7)
    be = CpuBackend(W)
    fr = np.stack([fnet.procedural_frame(1920, 1080), fnet.procedural_frame(1920, 1080, 12, 0)])
    secs = []
    for _ in range(frames_n):
        f = fnet.FlyHighFG(be, 864, 480, frame=(1920, 1080))
        be.upload_frames(f.frames, fr)
        t0 = time.perf_counter()
        f.pair_mid(0.5, W)
        secs.append(time.perf_counter() - t0)
    return statistics.median(secs), be.threads


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def batched_workload(args, torch, np, fhconv, flyhighfg, stream, pairs=8, mids=3):
    """The convs alone of the batched configuration: the frame's convs over 8 independent frame pairs (network
    856x480) with 3 mid() phases each, one batched conv (or fused pair) per layer; the convs' step time and TFLOP/s,
    and each launch's warm and cold time against its roofline (the whole configuration is batched_frames)."""
    layers = flyhighfg.batched_layers(pairs, mids)
    net = Net(layers, 3, torch, np, fhconv, tune=not (args.no_autotune or args.tune))
    fused = not args.no_fuse
    if fused:
        net.fuse(flyhighfg.fusible_pairs(layers), torch, fhconv, stream,
                 lambda fn: time_graph(torch, fn, 20, 3, stream), default_tile=bool(args.tune))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        net.run(fused=fused)
        stream.synchronize()
        with torch.cuda.graph(g, stream=stream):
            net.run(fused=fused)
        for _ in range(3):
            g.replay()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 20
        a.record(stream)
        for _ in range(n):
            g.replay()
        b.record(stream)
        b.synchronize()
    step_us = a.elapsed_time(b) * 1e3 / n
    fused_b = {B.name for _, B, _, _ in net.pairs.values()}
    launches = []
    for L in layers:
        if L.name in net.pairs:
            launches.append(pair_timing(torch, net, L.name, 20, 3, args.cold_mb << 20, stream))
        elif L.name not in fused_b:
            launches.append(layer_timing(torch, np, fhconv, net, L, 20, 3, args.cold_mb << 20, stream))
        else:
            continue
        log("batched", json.dumps(launches[-1]))
    flops = sum(L.flops for L in layers)
    log(f"bench: batched convs ({pairs} pairs x {mids} mids): {step_us:.1f} us per step of the convs alone, "
        f"{flops / step_us / 1e6:.1f} TFLOP/s over the step")
    return dict(workload=f"the convs alone of {pairs} independent frame pairs (network 856x480), {mids} mid() phases "
                         "each: pair-stage convs batched over the pairs (encoders over both frames), mid-stage convs "
                         "over pairs x mids; synthetic inputs, random weights",
                convs_step_us=round(step_us, 2), step_tflops=round(flops / step_us / 1e6, 2),
                launches=launches, fused_pairs=[f"{a}+{B.name}" for a, (_, B, _, _) in net.pairs.items()],
                tune_table=fhconv.format_tune().splitlines())


def mfma_rate_probe(torch, fhconv, stream):
    """The sustained dense f16 MFMA rate of this device (TFLOP/s): the library's register-only MFMA probe, 16
    independent chains per wave at 4 workgroups (4 waves each) per CU, best of 3 timed launches on `stream`."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    blocks, iters = cus * 4, 1024
    out = torch.empty(blocks * 1024, dtype=torch.float32, device="cuda")
    best = 0.0
    with torch.cuda.stream(stream):
        fhconv.probe_mfma_rate(blocks, 16, out, stream)
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            flops = fhconv.probe_mfma_rate(blocks, iters, out, stream)
            e1.record(stream)
            e1.synchronize()
            best = max(best, flops / (e0.elapsed_time(e1) * 1e-3) / 1e12)
    return best


COPY_BYTES = 256 << 20  # the calibration copy of the traffic passes


def pmc_workload(args, torch, fhconv, flyhighfg, net, stream):
    """One layer, or one fused pair ("first+second", the pair planner's default tile, the same in both counter
    passes), over rotating buffer sets (> 512 MB, so every launch reads from HBM), then a device copy of COPY_BYTES
    the same number of times: rocprofv3 --pmc runs this to read FETCH_SIZE / WRITE_SIZE per dispatch."""
    if "+" in args.pmc_layer:
        a_name, b_name = args.pmc_layer.split("+")
        pair = [(A, B, rm) for A, B, rm in flyhighfg.fusible_pairs(net.layers) if A.name == a_name and B.name == b_name]
        if not pair:
            raise SystemExit(f"{args.pmc_layer} is not a fusible pair of the frame")
        A, B, res_mid = pair[0]
        da, wa, ba, sa = net.params[A.name]
        db, wb, bb, sb = net.params[B.name]
        p = fhconv.ConvPairPlan(da, wa, ba, sa, db, wb, bb, sb, res_mid=res_mid)
        x, ws = net.bufs[A.name][0], None
        _, y, r, _ = net.bufs[B.name]
        r = None if res_mid else r
    else:
        L = [L for L in net.layers if L.name == args.pmc_layer][0]
        p = net.plans[L.name]
        x, y, r, ws = net.bufs[L.name]
    per = x.numel() * 2 + y.numel() * 2 + (r.numel() * 2 if r is not None else 0)
    nsets = max(2, -(-(600 << 20) // per))
    sets = [(torch.empty_like(x).uniform_(-1, 1), torch.empty_like(y),
             torch.empty_like(r).uniform_(-1, 1) if r is not None else None) for _ in range(nsets)]
    src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device="cuda").uniform_(-1, 1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(args.pmc_reps):
            sx, sy, sr = sets[i % nsets]
            p.run(sx, sy, sr, ws, stream)
        for _ in range(args.pmc_reps):
            dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps(dict(pmc_layer=args.pmc_layer, variant=p.describe()["name"], reps=args.pmc_reps,
                          cold_sets=nsets, copy_bytes=COPY_BYTES)), flush=True)
    return 0


POOL_BYTES = 2 << 30  # the counter workload's rotating buffer pool


def conv_launches(args, torch, np, fhconv, flyhighfg, stream):
    """Every conv launch the counter workload measures, as (group, label, plan, x, y, r, ws, flops, bytes): the 1080p
    frame's convs (the committed choices; every instantiated pair fused with the pair planner's default tile, as the
    frame program runs them), the single-layer configurations (3x3 32 -> 32 at 1080p/8, the 1080p/4 ladder, the
    1080p/16 deep layer and 1x1), and the batched workload's convs (8 pairs, 3 phases) fused the same way. Nothing
    is chosen by timing, so every counter pass runs the same launches."""
    out = []
    tf = lambda fn: time_graph(torch, fn, 20, 3, stream)  # noqa: E731
    groups = [("frame", flyhighfg.flyhighfg_layers(864, 480, k=1), 1, None, True)]
    groups += [(f"C{c}", flyhighfg.config_layers(c), 100 + c, 0.25, False) for c in (1, 2, 3)]
    groups += [("batched", flyhighfg.batched_layers(8, 3), 3, None, True)]
    nets = []
    for group, layers, seed, slope, fuse in groups:
        net = Net(layers, seed, torch, np, fhconv, tune=False, slope=slope)
        if fuse:
            net.fuse(flyhighfg.fusible_pairs(layers), torch, fhconv, stream, tf, default_tile=True, always=True)
        nets.append(net)
        skip = {B.name for _, B, _, _ in net.pairs.values()}
        for L in layers:
            if L.name in net.pairs:
                pp, B, _, res_mid = net.pairs[L.name]
                _, y, r, _ = net.bufs[B.name]
                d = pp.describe()
                out.append((group, L.name + "+" + B.name, pp, net.bufs[L.name][0], y, None if res_mid else r, None,
                            d["flops"], d["bytes"]))
            elif L.name not in skip:
                x, y, r, ws = net.bufs[L.name]
                out.append((group, L.name, net.plans[L.name], x, y, r, ws, L.flops, L.bytes))
    return out, nets


def pmc_convs(args, torch, np, fhconv, flyhighfg, stream):
    """The counter workload of every conv launch (conv_launches): each launch --pmc-reps times, every call on a set
    of input, output and residual buffers of its own carved from one pre-filled 2 GiB pool (so each call reads
    tensors no earlier call of it touched: HBM or the MALL, never the L2, which the acquire at every kernel boundary
    invalidates), then a device copy of COPY_BYTES as many times. Prints one JSON line per launch (its order, variant
    and kernels per call), the manifest --counters-from attributes the dispatches by."""
    items, nets = conv_launches(args, torch, np, fhconv, flyhighfg, stream)
    pool = torch.empty(POOL_BYTES // 2, dtype=torch.float16, device="cuda").uniform_(-1, 1)
    src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device="cuda").uniform_(-1, 1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    manifest = []
    al = 128  # elements between carved tensors (256-byte alignment)
    with torch.cuda.stream(stream):
        off = 0
        for order, (group, label, plan, x, y, r, ws, flops, nbytes) in enumerate(items):
            d = plan.describe()
            kernels = 2 if d.get("ksplit", 1) > 1 else 1
            for i in range(args.pmc_reps):
                views = []
                for t in (x, y, r):
                    if t is None:
                        views.append(None)
                        continue
                    n = -(-t.numel() // al) * al
                    if off + n > pool.numel():
                        off = 0
                    views.append(pool[off:off + t.numel()].view(t.shape))
                    off += n
                if ws is None:
                    plan.run(views[0], views[1], views[2], stream=stream)
                else:
                    plan.run(views[0], views[1], views[2], ws, stream=stream)
            manifest.append(dict(order=order, group=group, label=label, variant=d["name"], kernels=kernels,
                                 reps=args.pmc_reps, flops=int(flops), bytes=int(nbytes)))
        # the calibration of the MFMA counters: the register-only MFMA probe (16 independent chains per wave, 4
        # workgroups of 4 waves per CU), whose rate the bench times on its own
        blocks = torch.cuda.get_device_properties(0).multi_processor_count * 4
        pout = torch.empty(blocks * 1024, dtype=torch.float32, device="cuda")
        for _ in range(args.pmc_reps):
            pflops = fhconv.probe_mfma_rate(blocks, 256, pout, stream)
        manifest.append(dict(order=len(manifest), group="calibration", label="mfma_probe", variant="probe",
                             kernels=1, reps=args.pmc_reps, flops=int(pflops), bytes=0))
        for _ in range(args.pmc_reps):
            dst.copy_(src)
    torch.cuda.synchronize()
    for m in manifest:
        print(json.dumps(dict(pmc_conv=m)), flush=True)
    print(json.dumps(dict(pmc_copy=dict(reps=args.pmc_reps, copy_bytes=COPY_BYTES))), flush=True)
    return 0


def _dispatches(csv_path):
    """[(dispatch id, kernel name, {counter: value})] of a rocprofv3 counter_collection.csv, in dispatch order: the
    SQ and TCC counters summed over their instances, GRBM_GUI_ACTIVE (one per XCD) the largest of them, as rocprof's
    own derived metrics reduce them; of a kernel_trace.csv, the duration in ns as "duration"."""
    import csv
    import collections
    rows = collections.OrderedDict()
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            k = int(row["Dispatch_Id"])
            if k not in rows:
                rows[k] = (row["Kernel_Name"], collections.defaultdict(float))
            c = rows[k][1]
            if "Counter_Name" not in row:
                c["duration"] = float(row["End_Timestamp"]) - float(row["Start_Timestamp"])
            elif row["Counter_Name"].startswith("GRBM_"):
                c[row["Counter_Name"]] = max(c[row["Counter_Name"]], float(row["Counter_Value"]))
            else:
                c[row["Counter_Name"]] += float(row["Counter_Value"])
    return [(k, rows[k][0], rows[k][1]) for k in sorted(rows)]


def counters_from(args):
    """profiles/conv_counters.txt from the three counter passes over the --pmc-convs workload (FETCH_SIZE;
    WRITE_SIZE; the SQ/GRBM group) and that run's stdout (the manifest): per conv launch, HBM bytes per call (the
    two size counters scaled by what they read for the copy of COPY_BYTES) against its algorithmic bytes, MFMA busy
    cycles over GRBM active cycles x 1024 SIMDs (rocprof's MfmaUtil), the MFMA FLOPs executed (512 per
    SQ_INSTS_VALU_MFMA_MOPS_F16) against the algorithmic FLOPs (K padding and halo recompute show as a ratio above
    1), and VALU instructions per wave."""
    f_csv, w_csv, q_csv, t_csv, man = args.counters_from
    manifest = [json.loads(line)["pmc_conv"] for line in open(man) if line.startswith('{"pmc_conv"')]
    for path in (f_csv, w_csv, q_csv, t_csv):  # every pass ran the same launches (its stdout beside its folder)
        other = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(path))),
                             os.path.basename(os.path.dirname(os.path.abspath(path))) + ".out")
        if os.path.exists(other):
            om = [json.loads(line)["pmc_conv"] for line in open(other) if line.startswith('{"pmc_conv"')]
            if [(m["label"], m["variant"], m["kernels"]) for m in om] != \
                    [(m["label"], m["variant"], m["kernels"]) for m in manifest]:
                raise SystemExit(f"{other} ran other launches than {man}")
    reps = manifest[0]["reps"]

    def ours(csv_path):
        ds = _dispatches(csv_path)
        need = sum(m["kernels"] * m["reps"] for m in manifest)
        # the workload's calls are the last library dispatches (set-up launches, such as the pair planner's timing,
        # come before them), and the copies follow them
        conv = [d for d in ds if "fhc::" in d[1]][-need:]
        copy = [d for d in ds if "copybuffer" in d[1].lower()][-reps:]
        if len(conv) != need or len(copy) != reps or conv[-1][0] > copy[0][0]:
            raise SystemExit(f"{csv_path}: {len(conv)} library dispatches for {need} expected, {len(copy)} copies")
        return conv, copy

    passes = {name: ours(path) for name, path in (("fetch", f_csv), ("write", w_csv), ("sq", q_csv),
                                                    ("trace", t_csv))}
    cf = sum(d[2]["FETCH_SIZE"] for d in passes["fetch"][1]) / reps
    cw = sum(d[2]["WRITE_SIZE"] for d in passes["write"][1]) / reps
    f_scale, w_scale = COPY_BYTES / (cf * 1024.0), COPY_BYTES / (cw * 1024.0)
    # MI355X's engine clock: the MFMA busy cycles are SIMD cycles at it (the MFMA probe, 82% of the dense peak by its
    # FLOPs, reads 0.82 so); the dispatch's GRBM_GUI_ACTIVE as reported is the sum of its 8 XCDs' counters
    f_clk, xcds = 2.4e9, 8
    lines = []
    pos = 0
    for m in manifest:
        n = m["kernels"] * m["reps"]
        seg = {k: v[0][pos:pos + n] for k, v in passes.items()}
        pos += n
        first = seg["fetch"][0][1]
        kern = first.split("(")[0].replace("void ", "").strip()[:90]
        fetch = sum(d[2]["FETCH_SIZE"] for d in seg["fetch"]) / m["reps"] * 1024.0 * f_scale
        write = sum(d[2]["WRITE_SIZE"] for d in seg["write"]) / m["reps"] * 1024.0 * w_scale
        sq = seg["sq"]
        busy = sum(d[2]["SQ_VALU_MFMA_BUSY_CYCLES"] for d in sq)
        active = sum(d[2]["GRBM_GUI_ACTIVE"] for d in sq)
        mops = sum(d[2]["SQ_INSTS_VALU_MFMA_MOPS_F16"] for d in sq) / m["reps"]
        waves = sum(d[2]["SQ_WAVES"] for d in sq) / m["reps"]
        valu = sum(d[2]["SQ_INSTS_VALU"] for d in sq) / m["reps"]
        t_call = sum(d[2]["duration"] for d in seg["trace"]) / m["reps"] * 1e-9
        busy_call = busy / m["reps"]
        lines.append(f"{m['group']} {m['label']} variant={m['variant']} kernel={kern.replace(' ', '')} "
                     f"calls={m['reps']} kernels_per_call={m['kernels']} flops={m['flops']} bytes={m['bytes']} "
                     f"us={t_call * 1e6:.3f} traffic={fetch + write:.0f} fetch={fetch:.0f} write={write:.0f} "
                     f"traffic_ratio={(fetch + write) / max(m['bytes'], 1):.3f} "
                     f"mfma_util={busy * xcds / (active * 1024):.4f} "
                     f"mfma_busy={busy_call / (1024 * f_clk * t_call):.4f} "
                     f"mfma_flops={mops * 512:.0f} mfma_pad={mops * 512 / max(m['flops'], 1):.3f} "
                     f"mfma_tflops={mops * 512 / t_call / 1e12:.1f} "
                     f"waves={waves:.0f} valu_per_wave={valu / max(waves, 1):.1f}")
    tune = f" --tune {os.path.relpath(args.tune, ROOT)}" if args.tune else ""
    cmd = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && timeout -s KILL 300 rocprofv3 {c} "
           "-d gpurun_out/{d} -o run --output-format csv -- python3 bench.py" + tune +
           f" --pmc-convs --pmc-reps {reps} > gpurun_out/{{d}}.out")
    head = ["# Counters of every conv launch (MI355X): four passes over the same workload, then on any host",
            "# " + cmd.format(c="--pmc FETCH_SIZE", d="pmc_cf"), "# " + cmd.format(c="--pmc WRITE_SIZE", d="pmc_cw"),
            "# " + cmd.format(c="--pmc SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_WAVES SQ_INSTS_VALU "
                                "GRBM_GUI_ACTIVE", d="pmc_cq"),
            "# " + cmd.format(c="--kernel-trace", d="pmc_ct"),
            f"# python3 bench.py{tune} --counters-from gpurun_out/pmc_cf/run_counter_collection.csv "
            "gpurun_out/pmc_cw/run_counter_collection.csv gpurun_out/pmc_cq/run_counter_collection.csv "
            "gpurun_out/pmc_ct/run_kernel_trace.csv gpurun_out/pmc_cf.out",
            "# per call (of its 'calls' calls, each on tensors of its own): us = kernel duration in the trace pass; "
            "traffic = FETCH_SIZE x fetch_scale + WRITE_SIZE x write_scale (KiB), the scales making the copy of "
            f"{COPY_BYTES} bytes read and write that; mfma_util = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE x 1024 "
            "SIMDs / 8 XCDs: the reported GRBM value sums the XCDs), rocprof's MfmaUtil over the counted dispatch's "
            "active window (which the counting stretches for short kernels); mfma_busy = the same busy cycles over the "
            "kernel's own duration (1024 SIMDs at 2.4 GHz); mfma_flops = 512 x SQ_INSTS_VALU_MFMA_MOPS_F16 (what the "
            "MFMAs compute, padding included), mfma_pad = that over the algorithmic FLOPs; the MFMA probe (the "
            "calibration line) checks the busy scale against its FLOP rate",
            f"# fetch_scale {f_scale:.4f} write_scale {w_scale:.4f}"]
    text = "\n".join(head + lines) + "\n"
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    with open(os.path.join(ROOT, "profiles", "conv_counters.txt"), "w") as f:
        f.write(text)
    print(text, end="")
    return 0


def conv_counters():
    """{(group, label): {key: value}} from profiles/conv_counters.txt, or {} where it was not recorded."""
    path = os.path.join(ROOT, "profiles", "conv_counters.txt")
    if not os.path.exists(path):
        return {}
    out = {}
    for line in open(path).read().splitlines():
        if not line or line[0] == "#":
            continue
        group, label, *kv = line.split(" ")
        out[(group, label)] = dict(x.split("=", 1) for x in kv)
    return out


def pmc_render(args, torch, np, stream):
    """The 1080p frame's render (fhc_render_rgba, as the frame runs it) --pmc-reps times over rotating sets of input
    and output frames (> 512 MB, so every launch reads its frames from HBM), after one eager frame that fills the
    quarter maps, then a device copy of COPY_BYTES as many times: the workload of the render's FETCH_SIZE /
    WRITE_SIZE passes (the eager frame's own render is the kernel's first dispatch, left out of the mean)."""
    import flyhighfg_net as fnet
    W = fnet.make_weights(7)
    be = fnet.GpuBackend(W, stream=stream)
    f = fnet.FlyHighFG(be, 864, 480, frame=(1920, 1080), repair=1)
    be.upload_frames(f.frames, np.stack([fnet.procedural_frame(1920, 1080), fnet.procedural_frame(1920, 1080, 12, 0)]))
    be.set_g(fnet.film_mlp(W, 0.5))
    with torch.cuda.stream(stream):
        f.pair_mid(0.5)
    torch.cuda.synchronize()
    per = 3 * f.frames.numel() // 2 * 4
    nsets = max(2, -(-(600 << 20) // per))
    sets = [(torch.randint_like(f.frames, -2 ** 31, 2 ** 31 - 1), torch.empty_like(f.rgba)) for _ in range(nsets)]
    fh = be.fh
    vf, vv, vr = fh.View(f.up7, 0), fh.View(f.up7, 4), fh.View(f.Rt, 0)
    src = torch.empty(COPY_BYTES // 2, dtype=torch.float16, device="cuda").uniform_(-1, 1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for i in range(args.pmc_reps):
            fr, out = sets[i % nsets]
            fh.render_rgba(fr[0:1], fr[1:2], vf, vv, vr, f.hp, f.wp, f.cubic, f.render_flags, f.fsx, f.fsy, out=out,
                           stream=stream)
        for _ in range(args.pmc_reps):
            dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps(dict(pmc_layer=args.pmc_layer, variant="render_rgba (one frame pixel per lane)",
                          reps=args.pmc_reps, cold_sets=nsets, copy_bytes=COPY_BYTES)), flush=True)
    return 0


def _counter_per_dispatch(csv_path, counter, skip_first=()):
    """{kernel name: mean counter value per dispatch} from a rocprofv3 counter_collection.csv; for the kernels whose
    name contains one of skip_first, the first dispatch is left out."""
    import csv
    import collections
    vals = collections.defaultdict(lambda: collections.defaultdict(float))
    with open(csv_path) as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            vals[row["Kernel_Name"]][int(row["Dispatch_Id"])] += float(row["Counter_Value"])
    out = {}
    for k, d in vals.items():
        ids = sorted(d)
        if any(s in k for s in skip_first) and len(ids) > 1:
            ids = ids[1:]
        out[k] = sum(d[i] for i in ids) / len(ids)
    return out


def traffic_from(args):
    """HBM bytes per launch of --pmc-layer's conv kernel from the FETCH_SIZE and WRITE_SIZE passes (KiB per
    dispatch), each scaled by what the same counter reads for the copy of COPY_BYTES; written to
    profiles/traffic_<layer>.txt."""
    render = args.pmc_layer == "frame_render"
    skip = ("render_rgba",) if render else ()
    fetch = _counter_per_dispatch(args.traffic_from[0], "FETCH_SIZE", skip)
    write = _counter_per_dispatch(args.traffic_from[1], "WRITE_SIZE", skip)
    conv = [k for k in fetch if ("render_rgba" in k if render else "conv" in k)]
    copy = [k for k in fetch if "copybuffer" in k.lower()]  # the runtime's device-to-device copy kernel
    if len(conv) != 1 or len(copy) != 1:
        raise SystemExit(f"expected one {'render' if render else 'conv'} and one copy kernel, got {conv} / {copy}")
    fk, wk = conv[0], copy[0]
    f_scale = COPY_BYTES / (fetch[wk] * 1024.0)
    w_scale = COPY_BYTES / (write[wk] * 1024.0)
    traffic = fetch[fk] * 1024.0 * f_scale + write[fk] * 1024.0 * w_scale
    if len(args.traffic_from) > 2:
        # the variant the counted workload ran: its JSON line in the third file (a pair's tile is chosen by timing)
        runs = [json.loads(line) for line in open(args.traffic_from[2]) if line.startswith("{")]
        variant = [r["variant"] for r in runs if r.get("pmc_layer") == args.pmc_layer][-1]
    else:
        # the variant the planner gives this layer under the same choice table (no GPU needed)
        import fhconv
        import flyhighfg
        if args.tune:
            with open(args.tune) as f:
                fhconv.parse_tune(f.read())
        L = [L for L in flyhighfg.flyhighfg_layers(864, 480, k=1) if L.name == args.pmc_layer][0]
        desc = fhconv.make_desc(L.n, L.h, L.w, L.cin, L.cout, k=L.k, stride=L.stride, act=L.act, alpha=L.alpha,
                                residual=L.residual, x_cstride=pad8(L.cin), y_cstride=pad8(L.cout),
                                r_cstride=pad8(L.cout) if L.residual else 0)
        variant = fhconv.plan_dry(desc)["name"]
    tune = f" --tune {os.path.relpath(args.tune, ROOT)}" if args.tune else ""
    cmd = ("cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT && timeout -s KILL 120 rocprofv3 --pmc "
           "{counter} -d gpurun_out/{d} -o run --output-format csv -- python3 bench.py" + tune +
           f" --pmc-layer {args.pmc_layer} > gpurun_out/{{d}}.out")
    text = (f"# HBM traffic per launch from two counter passes (MI355X), then on any host:\n"
            f"# {cmd.format(counter='FETCH_SIZE', d='pmc_fetch')}\n"
            f"# {cmd.format(counter='WRITE_SIZE', d='pmc_write')}\n"
            f"# python3 bench.py{tune} --pmc-layer {args.pmc_layer} --traffic-from "
            f"gpurun_out/pmc_fetch/*/run_counter_collection.csv gpurun_out/pmc_write/*/run_counter_collection.csv"
            f"{' gpurun_out/pmc_fetch.out' if len(args.traffic_from) > 2 else ''}\n"
            f"layer {args.pmc_layer}\nvariant {variant}\nkernel {fk}\n"
            f"fetch_kib_per_launch {fetch[fk]:.1f}\nwrite_kib_per_launch {write[fk]:.1f}\n"
            f"copy_kernel {wk}\ncopy_bytes {COPY_BYTES}\n"
            f"copy_fetch_kib {fetch[wk]:.1f}\ncopy_write_kib {write[wk]:.1f}\n"
            f"fetch_scale {f_scale:.4f}\nwrite_scale {w_scale:.4f}\n"
            f"traffic_bytes_per_launch {traffic:.0f}\n")
    os.makedirs(os.path.join(ROOT, "profiles"), exist_ok=True)
    with open(os.path.join(ROOT, "profiles", f"traffic_{args.pmc_layer}.txt"), "w") as f:
        f.write(text)
    print(text, end="")
    return 0


def traffic_name(label):
    """The file stem of a launch's traffic record: its label up to the first space ("frame_render", "enc.e3+enc.e4")."""
    return label.split(" ")[0]


def measured_traffic(label, variant=None):
    """(bytes per launch, source) from profiles/traffic_<name>.txt when it was measured (on this variant's kernel, when
    a variant is named), else (None, reason)."""
    path = os.path.join(ROOT, "profiles", f"traffic_{traffic_name(label)}.txt")
    if not os.path.exists(path):
        return None, "no counter passes recorded for this launch"
    kv = dict(line.split(" ", 1) for line in open(path).read().splitlines() if " " in line and line[0] != "#")
    if variant is not None and kv.get("variant") != variant:
        return None, f"{os.path.relpath(path, ROOT)} was measured on {kv.get('variant')}, this run uses {variant}"
    return int(float(kv["traffic_bytes_per_launch"])), f"{os.path.relpath(path, ROOT)} ({kv['kernel'][:80]})"


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--reps", type=int, default=100, help="launches per timing graph (per-layer timing)")
    ap.add_argument("--graphs", type=int, default=20, help="graph replays per per-layer timing (median)")
    ap.add_argument("--cold-mb", type=int, default=600, help="buffer bytes rotated by the cold timing")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true", help="skip the single-layer configurations")
    ap.add_argument("--no-layers", action="store_true", help="skip the per-layer timing of the frame workload")
    ap.add_argument("--no-autotune", action="store_true", help="plan with the heuristic only (no per-shape timing)")
    ap.add_argument("--no-fuse", action="store_true", help="one launch per conv (no fused conv pairs)")
    ap.add_argument("--no-batched", action="store_true", help="skip the batched workload (8 pairs, 3 mids each)")
    ap.add_argument("--only-batched", action="store_true",
                    help="only time the batched workload (8 3840x2160 pairs, 3 phases each, every op, one HIP graph) "
                         "and print it as one JSON line")
    ap.add_argument("--ops", action="store_true", help="also time each network op instance over rotating buffers "
                                                        "(frame and batched shapes)")
    ap.add_argument("--only-ops", action="store_true",
                    help="only time the network ops (frame and batched shapes) and print them as one JSON line")
    ap.add_argument("--only-frame", action="store_true",
                    help="only time the 1080p frame (RGBA8 in, every op of pair() + mid(), RGBA8 out, one HIP graph) "
                         "and print it as one JSON line")
    ap.add_argument("--tune", help="plan with this choice table (cin,cout,h,w,stride=code lines) instead of autotuning")
    ap.add_argument("--pmc-layer", help="only run this frame layer (or fused pair, or frame_render: the frame-size "
                                        "render) --pmc-reps times over rotating (cold) buffers, then a copy of "
                                        "known size as many times: the workload of the rocprofv3 --pmc FETCH_SIZE / "
                                        "WRITE_SIZE passes")
    ap.add_argument("--pmc-reps", type=int, default=64)
    ap.add_argument("--pmc-convs", action="store_true",
                    help="only run every conv launch (the frame's conv step, the single-layer configurations, the "
                         "batched convs) --pmc-reps times over carved cold buffers, then a copy of known size: the "
                         "workload of the conv counter passes")
    ap.add_argument("--counters-from", nargs=5, metavar="FILE",
                    help="turn the --pmc-convs passes' counter_collection.csv files (FETCH_SIZE, WRITE_SIZE, the SQ "
                         "group), its kernel_trace.csv and that run's stdout into profiles/conv_counters.txt")
    ap.add_argument("--eager-frames", type=int, default=0,
                    help="only run the 1080p frame (as --only-frame builds it) this many times eagerly, untimed: the "
                         "workload of rocprofv3 counter passes over the frame's kernels")
    ap.add_argument("--detail", default=os.path.join("gpurun_out", "bench_detail.json"),
                    help="file for the full record (per-launch tables, configurations, batched launches, choice "
                         "table); '' for none")
    ap.add_argument("--traffic-from", nargs="+", metavar="CSV",
                    help="with --pmc-layer: turn the two passes' counter_collection.csv files (FETCH, WRITE) into "
                         "profiles/traffic_<layer>.txt (HBM bytes per launch, copy-calibrated); a third file, the "
                         "counted run's stdout, names the variant it ran (needed for a fused pair)")
    args = ap.parse_args()
    if args.traffic_from:
        return traffic_from(args)
    if args.counters_from:
        return counters_from(args)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported (the conv path shards "
              "by frame pair, one independent pipeline per GPU, so N GPUs run N of these)", file=sys.stderr)
        return 2

    import numpy as np
    import torch
    import fhconv
    import flyhighfg

    torch.cuda.init()
    dev = torch.device("cuda", 0)
    stream = torch.cuda.Stream(device=dev)
    if args.tune:
        with open(args.tune) as f:
            n_tune = fhconv.parse_tune(f.read())
        log(f"bench: {n_tune} choices from {args.tune}")
    net_w, net_h = 864, 480  # default_internal(1920, 1080) = (856, 480), padded to a multiple of 32
    assert flyhighfg.default_internal(1920, 1080) == (856, 480)
    if args.eager_frames:
        return eager_frames(args, torch, np, stream)
    if args.pmc_convs:
        fhconv.parse_tune(open(args.tune or os.path.join(ROOT, "flyhigh-engine_amd", "tune_mi355x.txt")).read())
        return pmc_convs(args, torch, np, fhconv, flyhighfg, stream)
    if args.pmc_layer == "frame_render" and not args.traffic_from:
        fhconv.parse_tune(open(os.path.join(ROOT, "flyhigh-engine_amd", "tune_mi355x.txt")).read())
        return pmc_render(args, torch, np, stream)
    if args.only_frame:
        if not args.tune:  # no autotuning here: the frame's convs take the committed MI355X choices
            fhconv.parse_tune(open(os.path.join(ROOT, "flyhigh-engine_amd", "tune_mi355x.txt")).read())
        frame, _ = frame_1080p(args, torch, np, stream)
        frame["no_repair"], _ = frame_1080p(args, torch, np, stream, repair=0, per_launch=False)
        frame["rotating_us_per_frame"] = round(frame_rotating(args, torch, np, stream), 3)
        print(json.dumps({k: v for k, v in frame.items() if k != "launch_table"}), flush=True)
        return 0
    if args.only_batched:
        if not args.tune:
            fhconv.parse_tune(open(os.path.join(ROOT, "flyhigh-engine_amd", "tune_mi355x.txt")).read())
        print(json.dumps(dict(batched=batched_frames(args, torch, np, stream))), flush=True)
        return 0
    if args.only_ops:
        print(json.dumps(dict(net_ops=net_ops_report(args, torch, flyhighfg, stream, net_w, net_h))), flush=True)
        return 0
    layers = flyhighfg.flyhighfg_layers(net_w, net_h, k=1)
    pair = [L for L in layers if L.stage == "pair"]
    mid = [L for L in layers if L.stage == "mid"]
    log(f"bench: FlyHighFG conv layers at {net_w}x{net_h}: {len(pair)} pair + {len(mid)} mid launches "
        f"(the two encoders batched)")
    net = Net(layers, 1, torch, np, fhconv, tune=not (args.no_autotune or args.tune))
    log(f"bench: autotuned {len(net.tuned)} conv shapes")
    tune_table = fhconv.format_tune().splitlines()  # the frame's choices (later workloads add their own)
    torch.cuda.synchronize()
    if args.pmc_layer:
        return pmc_workload(args, torch, fhconv, flyhighfg, net, stream)
    fused = not args.no_fuse
    if fused:
        # with a committed choice table the pairs take the pair planner's default tile: the run is then repeatable
        # (a profiler's own overhead cannot change the variants it traces)
        net.fuse(flyhighfg.fusible_pairs(layers), torch, fhconv, stream,
                 lambda fn: time_graph(torch, fn, 50, 5, stream), default_tile=bool(args.tune))
        log(f"bench: {len(net.pairs)} conv pairs fused: " +
            ", ".join(f"{a}+{B.name} ({pp.describe()['name']})" for a, (pp, B, _, _) in net.pairs.items()))
    launches = len(layers) - len(net.pairs)

    # the fused step against the one-launch-per-conv step: the pairs' outputs (and everything after them) agree
    # within the parity bar (a pair computes each conv as its separate launch does, up to the f32 summation order)
    fuse_check = None
    if fused:
        with torch.cuda.stream(stream):
            net.run()
            stream.synchronize()
            ref = {L.name: net.bufs[L.name][1].float().clone() for L in layers if L.name not in net.pairs}
            net.run(fused=True)
            stream.synchronize()
        worst = 0.0
        for name, want in ref.items():
            got = net.bufs[name][1].float()
            worst = max(worst, float((got - want).abs().max()) / max(float(want.abs().max()), 1e-30))
        fuse_check = dict(max_rel_diff=round(worst, 6), tol=1e-2, ok=worst <= 1e-2)
        log(f"bench: fused step vs one launch per conv: max |diff| / max |ref| = {worst:.2e}")
        del ref

    # one graph per step (pair then mid: one launch per frame), and one per stage for the stage split
    gs, gp, gm, gu = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        net.run(fused=fused)
        stream.synchronize()
        with torch.cuda.graph(gs, stream=stream):
            net.run(fused=fused)
        with torch.cuda.graph(gp, stream=stream):
            net.run({L.name for L in pair}, fused=fused)
        with torch.cuda.graph(gm, stream=stream):
            net.run({L.name for L in mid}, fused=fused)
        with torch.cuda.graph(gu, stream=stream):
            net.run()
        for _ in range(args.warmup):
            gs.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            gs.replay()
        e1.record(stream)
        t_submit = time.perf_counter() - t0
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps
    ev_ms = e0.elapsed_time(e1) / args.steps
    log(f"bench: {ms_per_step * 1e3:.2f} us per pair+mid (wall), {ev_ms * 1e3:.2f} us (events), "
        f"{t_submit * 1e6 / args.steps:.2f} us to submit one replay")

    def stage_us(g, n=200):
        with torch.cuda.stream(stream):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            for _ in range(n):
                g.replay()
            b.record(stream)
            b.synchronize()
        return a.elapsed_time(b) * 1e3 / n

    pair_us, mid_us, unfused_us = stage_us(gp), stage_us(gm), stage_us(gu)
    log(f"bench: pair {pair_us:.2f} us + mid {mid_us:.2f} us; one launch per conv: {unfused_us:.2f} us")

    per_layer = []
    if not args.no_layers:
        for L in layers:
            per_layer.append(layer_timing(torch, np, fhconv, net, L, args.reps, args.graphs,
                                          args.cold_mb << 20, stream))
            log("layer", json.dumps(per_layer[-1]))
    per_pair = []
    if not args.no_layers:
        for a_name in net.pairs:
            per_pair.append(pair_timing(torch, net, a_name, args.reps, args.graphs, args.cold_mb << 20, stream))
            log("pair", json.dumps(per_pair[-1]))
    cfg_layers, cfg_pairs = [], []
    if not args.no_configs:
        for c in (1, 2, 3):
            cl = flyhighfg.config_layers(c)
            # the configurations' PReLU slopes are 0.25 (the He-normal ladder of the 1080p/4 configuration)
            cnet = Net(cl, 100 + c, torch, np, fhconv, tune=not args.no_autotune, slope=0.25)
            for L in cl:
                cfg_layers.append(dict(config=c, **layer_timing(torch, np, fhconv, cnet, L, args.reps,
                                                                args.graphs, args.cold_mb << 20, stream)))
                log("config layer", json.dumps(cfg_layers[-1]))
            # the ladder's consecutive 64 -> 64 convs also as a fused pair (one launch, the intermediate on chip)
            if not args.no_fuse:
                cnet.fuse(flyhighfg.fusible_pairs(cl), torch, fhconv, stream,
                          lambda fn: time_graph(torch, fn, 20, 3, stream), default_tile=bool(args.tune))
                for a_name in cnet.pairs:
                    cfg_pairs.append(dict(config=c, **pair_timing(torch, cnet, a_name, args.reps, args.graphs,
                                                                  args.cold_mb << 20, stream)))
                    log("config pair", json.dumps(cfg_pairs[-1]))
            del cnet
            torch.cuda.empty_cache()

    # the headline: the whole 1080p frame from RGBA8 to RGBA8; its conv plans come from the choice table the
    # conv step's autotuning filled (or --tune); the batched workload's choices sit under keys of their own (the
    # table's key holds the batch)
    frame, (fbe, fobj, frec) = frame_1080p(args, torch, np, stream)
    frame["no_repair"], _ = frame_1080p(args, torch, np, stream, repair=0, per_launch=False)
    frame["rotating_us_per_frame"] = round(frame_rotating(args, torch, np, stream), 3)
    log(f"bench: 1080p frame {frame['us_per_frame']:.2f} us ({frame['frames_per_s']:.0f} frames/s), "
        f"{frame['launches']} launches, per-launch sum {frame['launch_us_sum']:.1f} us; without the repair "
        f"{frame['no_repair']['us_per_frame']:.2f} us; over 8 rotating frame sets {frame['rotating_us_per_frame']:.2f} us")
    net_ops = net_ops_report(args, torch, flyhighfg, stream, net_w, net_h) if args.ops else None

    batched = batched_convs = None
    if not args.no_batched:
        batched = batched_frames(args, torch, np, stream)
        torch.cuda.empty_cache()
        batched_convs = batched_workload(args, torch, np, fhconv, flyhighfg, stream)
        torch.cuda.empty_cache()

    mfma_rate = mfma_rate_probe(torch, fhconv, stream)
    log(f"bench: sustained dense f16 MFMA rate {mfma_rate:.0f} TFLOP/s")

    # the dominant kernel of the frame: the launch with the largest time alone (warm); its achieved rate is its
    # algorithmic bytes (or FLOPs) per launch over its per-launch time, cold (inputs from HBM) where the launch can
    # be rotated over fresh buffers: the frame-size render, a conv layer or fused pair of the conv step
    dom = max((r for r in frame["launch_table"] if r["kernels"] == 1), key=lambda r: r["us_warm"])
    us_cold, cold_note = None, "warm only"
    if dom["label"].startswith("frame_render"):
        us_cold, nsets = render_cold(args, torch, fbe, fobj, args.reps, args.graphs, args.cold_mb << 20, stream)
        cold_note = f"cold: {nsets} rotating sets of input and output frames"
    elif dom["kind"] == "conv":
        rows = [r for r in per_layer + per_pair if r["name"].replace(".ab", "") == dom["label"]]
        if rows:
            us_cold, cold_note = rows[0]["us_cold"], "cold: the conv step's rotating buffer sets"
    us = us_cold if us_cold is not None else dom["us_warm"]
    if dom["bound"] == "hbm":
        unit, achieved, peak = "GB/s", dom["bytes"] / us / 1e3, HBM_PEAK / 1e9
    else:
        unit, achieved, peak = "TFLOP/s", dom["flops"] / us / 1e6, MFMA_F16_PEAK / 1e12
    traffic, traffic_note = measured_traffic(dom["label"], None)
    roofline = dict(bound=dom["bound"], achieved=round(achieved, 2), peak=peak, unit=unit, frac=round(achieved / peak, 4),
                    traffic=traffic, kernel=dom["label"], us_warm=dom["us_warm"],
                    us_cold=None if us_cold is None else round(us_cold, 3), timing=cold_note,
                    per_launch_bytes=dom["bytes"], per_launch_flops=dom["flops"], traffic_source=traffic_note,
                    sustained_mfma_tflops=round(mfma_rate, 1))
    if dom["label"].startswith("frame_render"):
        # 1920 x 1088 lanes of bicubic sampling in the reference's f32 order: the SQ counters put it at ~900 VALU
        # instructions per wave over 32,400 waves, the VALU issue rate of the chip, far below the HBM roofline
        roofline["note"] = "VALU issue-bound: ~509 VALU instructions per wave, 32,400 waves (SQ counter pass)"
    log("bench: dominant launch", json.dumps(roofline))

    cpu = None
    if not args.no_cpu:
        secs, threads = cpu_frame_baseline(np)
        cpu = dict(value=round(1.0 / secs, 4), unit="frames/s", cores=threads, kind="port",
                   sample="one 1080p pair()+mid(0.5) from two RGBA8 frames through the oracle composition (the C "
                          "restatement of the reference's WGSL ops and conv arithmetic, convs multithreaded over "
                          "rows), not lavapipe; median of 3 frames",
                   seconds=round(secs, 3), cpu_model=cpu_model(), host_cpus=os.cpu_count())
        log(f"bench: CPU baseline {secs:.3f} s per frame on {threads} threads")

    conv_roof = conv_roofline(per_layer, per_pair, net, cfg_layers, batched_convs)
    log("bench: conv roofline", json.dumps(conv_roof))

    conv_step = dict(
        workload="FlyHighFG conv layers of one pair()+mid() at 1080p (network 856x480 padded to 864x480), NHWC "
                 "f16, conv-only; the A/B encoders run as batch-2 convs"
                 + ("; consecutive convs whose intermediate has no other reader run as fused pairs"
                    if net.pairs else ""),
        us_per_step=round(ms_per_step * 1e3, 3), frames_per_s=round(1000.0 / ms_per_step, 2), conv_layers=25,
        conv_launches=launches, fused_pairs=[f"{a}+{B.name}" for a, (_, B, _, _) in net.pairs.items()],
        pair_us=round(pair_us, 3), mid_us=round(mid_us, 3), unfused_step_us=round(unfused_us, 3),
        fuse_check=fuse_check, event_ms_per_step=round(ev_ms, 6),
        submit_us_per_step=round(t_submit * 1e6 / args.steps, 3))
    detail = dict(frame=frame, conv_step=conv_step, roofline=roofline, conv_roofline=conv_roof, cpu_baseline=cpu,
                  layers=per_layer,
                  pairs=per_pair, config_layers=cfg_layers, config_pairs=cfg_pairs, batched=batched,
                  batched_convs=batched_convs, net_ops=net_ops,
                  tune_table=tune_table)
    return emit(args, frame, conv_step, roofline, cpu, batched, detail)


def conv_roofline(per_layer, per_pair, net, cfg_layers, batched_convs):
    """The conv layers' roofline in brief: the dominant conv launch of the frame's conv step (the largest warm time
    among its launches: the fused pairs and the convs not fused), its cold roofline fraction and bound, with the MFMA
    busy fraction, MFMA padding and HBM traffic ratio its counter passes recorded (profiles/conv_counters.txt, when
    they ran on the same variant); the least and median cold fraction over the step's launches; each single-layer
    configuration's fraction; the batched convs' dominant launch likewise."""
    if not per_layer:
        return None
    ctr = conv_counters()

    def counted(group, r):
        c = ctr.get((group, r["name"]))
        if c is None or c.get("variant") != r["variant"]:
            return {}
        return dict(mfma_busy=float(c["mfma_busy"]), mfma_pad=float(c["mfma_pad"]),
                    traffic_ratio=float(c["traffic_ratio"]))

    fused_b = {B.name for _, B, _, _ in net.pairs.values()}
    step = [r for r in per_pair] + [r for r in per_layer if r["name"] not in net.pairs and r["name"] not in fused_b]
    if not step:
        return None
    fr = sorted(r["frac_cold"] for r in step)
    dom = max(step, key=lambda r: r["us_warm"])
    out = dict(dominant=dict(name=dom["name"], variant=dom["variant"], bound=dom["bound"], frac=dom["frac_cold"],
                             us_cold=dom["us_cold"], roof_us=dom["roof_us"], **counted("frame", dom)),
               frame_frac_min=fr[0], frame_frac_median=fr[len(fr) // 2], frame_launches=len(step),
               configs={f"C{r['config']} {r['name']}": dict(frac=r["frac_cold"], bound=r["bound"],
                                                           **{k: v for k, v in counted(f"C{r['config']}", r).items()
                                                              if k == "mfma_busy"})
                        for r in cfg_layers},
               counters="profiles/conv_counters.txt")
    if batched_convs:
        bl = batched_convs["launches"]
        bd = max(bl, key=lambda r: r["us_warm"])
        out["batched_dominant"] = dict(name=bd["name"], variant=bd["variant"], bound=bd["bound"],
                                       frac=bd["frac_cold"], us_cold=bd["us_cold"], **counted("batched", bd))
    return out


def emit(args, frame, conv_step, roofline, cpu, batched, detail):
    """Write the whole record to args.detail and print the one compact JSON line (under 4 KB) that is the bench's
    result: the headline is the whole frame (frame), with the conv-only step, the roofline of the dominant kernel,
    the CPU baseline and the batched workload's summary beside it."""
    if args.detail:
        os.makedirs(os.path.dirname(os.path.abspath(args.detail)), exist_ok=True)
        with open(args.detail, "w") as f:
            json.dump(detail, f, indent=1)
        log(f"bench: full record in {args.detail}")
    keep_roof = ("bound", "achieved", "peak", "unit", "frac", "traffic", "kernel", "us_cold", "us_warm", "timing",
                 "per_launch_bytes", "per_launch_flops", "sustained_mfma_tflops", "note")
    line = dict(
        metric=METRIC, value=frame["frames_per_s"], unit="frames/s", n_gpus=1, steps=frame["steps"],
        warmup=frame["warmup"], ms_per_step=round(frame["us_per_frame"] / 1e3, 6), higher_is_better=True,
        scaling="weak", vs_baseline=round(frame["frames_per_s"] * PUBLISHED_MS_PER_FRAME / 1e3, 3), dtype="f16",
        data="synthetic",
        config=dict(workload=frame["workload"], frame="1920x1080", network=frame["network"],
                    launches=frame.get("launches"), parallelism="single GPU"),
        frame_without_repair_us=frame.get("no_repair", {}).get("us_per_frame"),
        frame_rotating_us=frame.get("rotating_us_per_frame"),
        roofline=None if roofline is None else {k: roofline[k] for k in keep_roof if k in roofline},
        cpu_baseline=cpu,
        conv_step=None if conv_step is None else {k: conv_step[k] for k in ("us_per_step", "frames_per_s",
                                                                            "conv_launches", "pair_us", "mid_us")},
        batched=None if batched is None else {k: batched[k] for k in ("step_us", "generated_frames_per_s",
                                                                      "pairs_per_s", "launches", "output_ok")},
        batched_convs_step_us=(detail.get("batched_convs") or {}).get("convs_step_us"),
        conv_roofline=detail.get("conv_roofline"),
        detail=args.detail or None)
    text = json.dumps(line)
    if len(text) > 4000:
        line["config"]["workload"] = line["config"]["workload"][:200]
        text = json.dumps(line)
    print(text, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
