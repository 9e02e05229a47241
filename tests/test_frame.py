"""The end-to-end FlyHighFG pair() + mid() program (flyhigh-engine_amd/flyhighfg_net.py).

On the CPU: the program's wiring runs over the oracle backend at a small network size (shapes, slices, every op
called with views it accepts, finite outputs, a FiLM vector that depends on t). On the GPU: the same program through
libfhconv.so (fused conv pairs, the network ops) against the oracle composition with the same weights and inputs,
per output tensor |diff| <= 1e-2 * max|ref| (the conv path's bar; the ops themselves are bit-exact or within an ulp,
and the convs' f32 summation order differs from the oracle's, so differences propagate through ~20 layers).
"""
import numpy as np
import pytest

from fhtest import f16_bits
from frame_oracle import CpuBackend
import flyhighfg_net as net

OUTPUTS = [("out", 3), ("up7", 7), ("Rt", 3), ("state_out", 76), ("o", 12), ("h", 48), ("cin", 279)]


def inputs(seed, net_w, net_h):
    rng = np.random.default_rng(seed)
    ab = np.zeros((2, net_h, net_w, 4), np.float32)
    yy, xx = np.mgrid[0:net_h, 0:net_w] / 16.0
    base = 0.5 + 0.25 * np.sin(xx)[..., None] * np.cos(yy)[..., None] + 0.1 * rng.uniform(-1, 1, (net_h, net_w, 3))
    ab[0, ..., :3] = base
    ab[1, ..., :3] = np.roll(base, 12, axis=1)  # B: the same picture moved 12 pixels right
    return f16_bits(ab)


def run(be, W, net_w, net_h, ab, t=0.5):
    f = net.FlyHighFG(be, net_w, net_h)
    if isinstance(f.AB, np.ndarray):
        f.AB[...] = ab
    else:
        f.AB.copy_(be.upload(ab))
    f.pair()
    f.mid(t, W)
    return f


def test_program_runs_on_the_oracle_backend():
    W = net.make_weights(1)
    f = run(CpuBackend(W), W, 128, 64, inputs(1, 128, 64))
    for name, c in OUTPUTS:
        v = getattr(f, name)[..., :c].view(np.float16)
        assert np.all(np.isfinite(v)), name
    assert np.any(f.Rt[..., :3] != 0) and np.any(f.up7[..., :7] != 0)
    assert np.all(f.cin[..., 150:230] == 0)  # side and state enter as zeros
    assert np.all(f.fx[..., 82:130] == 0)    # h enters the fine loop as zeros
    assert not np.array_equal(net.film_mlp(W, 0.25), net.film_mlp(W, 0.75))


@pytest.mark.gpu
@pytest.mark.parametrize("net_w,net_h,fuse", [(256, 128, True), (256, 128, False), (864, 480, True)])
def test_gpu_frame_matches_the_oracle_composition(net_w, net_h, fuse):
    import torch
    print("frame", net_w, net_h, "fused" if fuse else "unfused", flush=True)
    W = net.make_weights(2)
    ab = inputs(2, net_w, net_h)
    ref = run(CpuBackend(W), W, net_w, net_h, ab)
    gb = net.GpuBackend(W, stream=torch.cuda.current_stream(), fuse=fuse)
    got = run(gb, W, net_w, net_h, ab)
    torch.cuda.synchronize()
    for name, c in OUTPUTS:
        g = gb.host(getattr(got, name))[..., :c].view(np.float16).astype(np.float64)
        r = getattr(ref, name)[..., :c].view(np.float16).astype(np.float64)
        err, tol = np.abs(g - r).max(), 1e-2 * np.abs(r).max()
        print(f"  {name}: max|diff| {err:.3g} (bar {tol:.3g}, max|ref| {np.abs(r).max():.3g})", flush=True)
        assert err <= tol, name


@pytest.mark.gpu
def test_fused_chains_equal_their_ops_on_the_gpu():
    """The four fused op chains (pyramid, fine input, flow_t / vis_t, refine input) against the same chains run op
    by op on the GPU, in the whole frame: the same f32 operations and roundings, so every output is bit-identical."""
    import torch
    W = net.make_weights(3)
    ab = inputs(3, 256, 128)
    outs = []
    for chains in (True, False):
        gb = net.GpuBackend(W, stream=torch.cuda.current_stream(), chains=chains)
        f = run(gb, W, 256, 128, ab, t=0.3)
        extra = [("fx", 155), ("rx", 14), ("i8", 3), ("l16", 2), ("l8", 2), ("fv", 7), ("ftvt", 7), ("d", 7),
                 ("dfilm", 5), ("wt36", 36), ("f16", 72)]
        outs.append({name: gb.host(getattr(f, name))[..., :c].copy() for name, c in OUTPUTS + extra})
    diffs = []
    for name in outs[0]:
        bad = np.argwhere(outs[0][name] != outs[1][name])
        if bad.size:
            diffs.append(f"{name}: {len(bad)} differ, first at {bad[0].tolist()}")
    assert not diffs, "; ".join(diffs)
