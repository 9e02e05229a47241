"""The static plan (fhc_model_plan) replayed on the GPU: flyhighfg_net.GraphProgram over the GPU backend (every plan
step one library call: the convs through fhc_conv.h plans, the ops through fhc_ops.h, no fused chains or pairs)
against the same program over the oracle backend, for a model of this library's own making whose plan holds every
step kind (tests/synthetic_graph.py; the reference's model files stay where they lie). The network's tensors are
held to the conv path's bar (1e-2 max|ref|: the convs' f32 summation order differs from the oracle's); the render
step to the oracle's render of the GPU's own inputs (bit-exact but for expf's last bit) and rgba_out exactly; the
repair step (a threshold decision, so compared on its own inputs) bit-exactly on the GPU's own pictures and flow."""
import numpy as np
import pytest

import fhtest  # noqa: F401  (the package and the oracle on the import path)
import fhmodel
import flyhighfg_net as net
import synthetic_graph as sg
from frame_oracle import CpuBackend

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _setup(frame, repair):
    g, m, b = sg.model_bytes(0)
    mdl = fhmodel.Model.from_bytes(g, m, b)
    plan = mdl.plan(2, frame, (128, 64), repair=repair)
    return plan, net.weights_from_model(mdl, plan), net.pair_frames(frame[0], frame[1], 3, shift=5)


def _host_view(gb, prog, v):
    return net.V(gb.host(prog.bufs[v["buf"]]).copy(), v["c0"], v["scale"])


@pytest.mark.parametrize("frame", [(128, 64), (300, 140)], ids=["network-size", "internal-size"])
def test_graph_replay_on_the_gpu_matches_the_oracle(frame):
    import torch
    say("graph replay", frame)
    plan, W, fr = _setup(frame, repair=0)
    gb = net.GpuBackend(W, stream=torch.cuda.current_stream())
    gpu = net.GraphProgram(gb, plan)
    gb.upload_frames(gpu.frames, fr)
    gpu.run(0.4, W)
    torch.cuda.synchronize()
    cpu = net.GraphProgram(CpuBackend(W), plan)
    cpu.frames[...] = fr
    cpu.run(0.4, W)
    render = [i for i, s in enumerate(plan["steps"]) if s["op"] == "render"][-1]
    rbuf = plan["steps"][render]["out"]["buf"]
    checked = 0
    for i, (info, gbuf, cbuf) in enumerate(zip(plan["buffers"], gpu.bufs, cpu.bufs)):
        if i == rbuf or info["h"] * info["w"] == 0:
            continue
        g = gb.host(gbuf)[..., :info["c"]].view(np.float16).astype(np.float64)
        r = cbuf[..., :info["c"]].view(np.float16).astype(np.float64)
        err, tol = np.abs(g - r).max(), 1e-2 * max(np.abs(r).max(), 1e-6)
        assert np.isfinite(g).all() and err <= tol, (info["name"], i, err, tol)
        checked += 1
    say(f"  {checked} buffers within the conv path's bar")
    # the render step on the GPU's own inputs, then rgba_out
    s = plan["steps"][render]
    ins = [_host_view(gb, gpu, v) for v in s["in"]]
    cb = CpuBackend(W)
    want = cb.zeros(*gpu.bufs[rbuf].shape)
    cb.render(*ins, net.V(want), gpu.cubic, gpu.render_flags, s["fsx"], s["fsy"])
    got = gb.host(gpu.bufs[rbuf])[..., :3].view(np.float16).astype(np.float64)
    d = np.abs(got - want[..., :3].view(np.float16).astype(np.float64))
    say(f"  render of its own inputs: max |diff| {d.max():.3g}, {np.mean(d == 0):.5f} identical")
    assert d.max() <= 1e-3 and np.mean(d == 0) >= 0.999
    h, w = gpu.rgba.shape[1:]
    import oracle
    assert np.array_equal(gb.host_frames(gpu.rgba), oracle.rgba_out(gb.host(gpu.bufs[rbuf]), h, w))


def _repairable_flow(a, b, f, full_w, level, motion):
    """A flow the stage rewrites somewhere, for the pictures a, b: the frames' own translation (network pixels, both
    directions, at a few magnitudes and signs) with a wrong jump of 8 network pixels in a patch; the candidate the
    oracle's stage repairs most cells of (a random net's own flow may need no repair)."""
    import oracle
    best = None
    c0 = f.c0
    for sgn in (1.0, -1.0):
        for mag in (0.25, 0.5, 1.0):
            x = f.buf.copy()
            fx, fy = sgn * mag * motion[0], sgn * mag * motion[1]
            fl = np.zeros(x.shape[:3] + (4,), np.float32) + np.float32([fx, fy, -fx, -fy])
            fl[:, 2:6, 4:12] += np.float32([8.0, 8.0, -8.0, -8.0])
            x[..., c0:c0 + 4] = fl.astype(np.float16).view(np.uint16)
            out, _, _ = oracle.gmhs(a.buf, b.buf, x, full_w, level, a_c0=a.c0, b_c0=b.c0, flow_c0=c0)
            n = int((out[..., c0:c0 + 4] != x[..., c0:c0 + 4]).any(-1).sum())
            if best is None or n > best[0]:
                best = (n, x, out)
    return best


def test_graph_replay_repair_step_on_the_gpus_own_flow():
    """The plan's repair step (level 1, on the pair's flow, the padded frame width) run by the GPU backend equals the
    oracle's stage on the same pictures and flow, bit for bit: the GPU's own pictures, and a flow in the step's
    buffer that the stage does rewrite in places (the synthetic net's own flow needs no repair); the rest of the
    plan then runs to a whole frame."""
    import torch
    say("graph replay, repair")
    plan, W, fr = _setup((300, 140), repair=1)
    gb = net.GpuBackend(W, stream=torch.cuda.current_stream())
    gpu = net.GraphProgram(gb, plan)
    gb.upload_frames(gpu.frames, fr)
    k = [i for i, s in enumerate(plan["steps"]) if s["op"] == "gmhs"][0]
    gpu.run(0.4, W, steps=range(k))
    s = plan["steps"][k]
    a, b, f = (_host_view(gb, gpu, v) for v in s["in"])
    dx, dy = np.random.default_rng(1000 + 3).integers(-5, 6, 2)  # pair_frames(300, 140, 3, shift=5)'s motion
    scale = np.float32(a.buf.shape[2]) / np.float32(plan["padded"][0])
    n, flow_in, want = _repairable_flow(a, b, f, s["full_w"], s["level"], (dx * scale, dy * scale))
    assert n > 0, "no candidate flow gets repaired"
    gpu.bufs[s["in"][2]["buf"]].copy_(torch.from_numpy(flow_in.view(np.int16)))
    gpu.run(0.4, W, steps=range(k, k + 1))
    got = gb.host(gpu.bufs[s["out"]["buf"]])
    say(f"  cells repaired: {n} of {f.buf.shape[1] * f.buf.shape[2]}, full_w {s['full_w']}")
    assert np.array_equal(got[..., f.c0:f.c0 + 4], want[..., f.c0:f.c0 + 4])
    gpu.run(0.4, W, steps=range(k + 1, len(plan["steps"])))
    rgba = gb.host_frames(gpu.rgba)
    assert np.all(rgba >> 24 == 255) and len(np.unique(rgba)) > 1000
