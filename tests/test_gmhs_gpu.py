"""Parity of the periodic-structure repair (fhc_gmhs, include/fhc_ops.h) with the oracle's GMHS, on the GPU.

Bar: bit-exact. The affine coefficients, the five cost maps after the texture window (every cell), the five values
each E8 cell decides on (the decision window at the cells the select reads) and the repaired flow equal the
oracle's (oracle/fh_ops_oracle.c, gmhs.rs and its shaders restated) bit for bit: the fit keeps the reference's 32
workgroups of 256 strided lanes and their pairwise lane tree, every other value is the same f32 operations in the
same order, and the square roots and quotients are correctly rounded on both sides. Cases: the 1080p network (864 x 480 of
1920-wide frames), a network as wide as its frame (the largest windows), ragged sizes whose cost grid is no multiple
of the 16-cell tiles, the E8 flow as a view of a wider buffer, a flow grid coarser than E8, level 2, a striped scene
where the select fires, and a workspace full of NaN (nothing in it is read before it is written).
"""
import numpy as np
import pytest

from fhtest import oracle
from test_gmhs_oracle import f16, striped_scene

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to("cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def fhops():
    import fhops as m  # noqa: E402
    return m


def smooth_flow(rng, h8, w8, cs, amp=4.0):
    """A smooth random E8 flow (4 channels at c0 0 of a cs-channel buffer) with a blob 16 px off and some noise."""
    yy, xx = np.mgrid[0:h8, 0:w8].astype(np.float64)
    chans = []
    for c in range(4):
        a = rng.uniform(-amp, amp) + rng.uniform(-1, 1) * xx / max(w8, 1) + rng.uniform(-1, 1) * yy / max(h8, 1)
        chans.append(a + rng.normal(0, 0.3, (h8, w8)))
    by, bx = h8 // 3, w8 // 3
    chans[0][by:by + max(h8 // 4, 1), bx:bx + max(w8 // 4, 1)] += 16.0
    out = rng.normal(0, 1, (1, h8, w8, cs))
    out[0, ..., :4] = np.stack(chans, -1)
    return f16(out)


def run(a, b, flow, full_w, level, poison=True):
    import torch
    fh = fhops()
    _, h, w, _ = a.shape
    p = fh.gmhs_params(h, w, full_w, level)
    ws = torch.empty(p["ws_bytes"], dtype=torch.uint8, device="cuda")
    if poison:
        ws.view(torch.float32)[:p["ws_bytes"] // 4].fill_(float("nan"))
    fd = dev(flow)
    fh.gmhs(dev(a), dev(b), fd, full_w, level, ws=ws)
    _, h8, w8, _ = flow.shape
    coef, maps, dec = fh.gmhs_results(ws, h, w, full_w, level, h8, w8)
    return host(fd).view(np.uint16), host(coef), host(maps), host(dec)


def check(a, b, flow, full_w, level, what):
    got_flow, got_coef, got_maps, got_dec = run(a, b, flow, full_w, level)
    want_flow, want_coef, want_maps, want_dec = oracle.gmhs_stages(a, b, flow, full_w, level)
    assert np.array_equal(got_coef.view(np.uint32), want_coef.view(np.uint32)), f"{what}: coef {got_coef} {want_coef}"
    for k in range(5):
        bad = np.argwhere(got_maps[k].view(np.uint32) != want_maps[k].view(np.uint32))
        assert bad.size == 0, f"{what}: map {k}: {len(bad)} cells differ, first at {bad[0].tolist()}"
        bad = np.argwhere(got_dec[k].view(np.uint32) != want_dec[k].view(np.uint32))
        assert bad.size == 0, f"{what}: decision value {k}: {len(bad)} cells differ, first at {bad[0].tolist()}"
    bad = np.argwhere(got_flow != want_flow)
    assert bad.size == 0, f"{what}: flow: {len(bad)} elements differ, first at {bad[0].tolist()}"
    return (want_flow != flow).any(-1).sum()


CASES = [  # network h, w, padded frame width, flow cstride, level
    (480, 864, 1920, 8, 1),   # the 1080p frame's network (s 0.9: windows 9 and 14)
    (192, 256, 256, 4, 1),    # network = frame (s 2: windows 20 and 32, the largest)
    (100, 150, 160, 8, 1),    # ragged: cost grid 50 x 75, flow 12 x 18
    (70, 90, 128, 6, 2),      # level 2 (no jump gate), odd grids
]


@pytest.mark.parametrize("h,w,full_w,cs,level", CASES)
def test_gmhs_matches_the_oracle(h, w, full_w, cs, level):
    say("gmhs", h, w, full_w, cs, level)
    rng = np.random.default_rng(h * w)
    a = f16(rng.uniform(0, 1, (1, h, w, 4)))
    b = np.roll(a, (2, -3), axis=(1, 2)).copy()
    flow = smooth_flow(rng, h // 8, w // 8, cs)
    check(a, b, flow, full_w, level, f"random {h}x{w}")


def test_gmhs_with_a_coarser_flow_matches_the_oracle():
    """A flow grid of 1/16 the network (the select's cells 8 cost cells apart, where the reference's E8 grid puts
    them 4 apart), at the largest decision window: the select's sampled rows and columns follow the flow's grid."""
    say("gmhs coarse flow")
    h, w = 192, 256
    rng = np.random.default_rng(7)
    a = f16(rng.uniform(0, 1, (1, h, w, 4)))
    b = np.roll(a, (3, 2), axis=(1, 2)).copy()
    check(a, b, smooth_flow(rng, h // 16, w // 16, 4), w, 1, "coarse flow")


def test_gmhs_repairs_the_striped_scene_as_the_oracle():
    say("gmhs striped scene")
    h, w = 256, 384
    a, b = striped_scene(h, w, 6)
    h8, w8 = h // 8, w // 8
    f = [np.full((h8, w8), v) for v in (-3.0, 0.0, 3.0, 0.0)]
    f[0][8:16, 10:22], f[2][8:16, 10:22] = 5.0, -5.0
    flow = np.zeros((1, h8, w8, 8), np.uint16)
    flow[0, ..., :4] = f16(np.stack(f, -1))
    changed = check(a, b, flow, 2 * w, 1, "striped")
    assert changed > 20  # the select fired on the blob


def test_gmhs_level_0_and_errors():
    import torch
    fh = fhops()
    a = dev(np.zeros((1, 32, 32, 4), np.uint16))
    flow = dev(np.full((1, 4, 4, 4), 0x3C00, np.uint16))
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    fh.gmhs(a, a, flow, 64, 0, ws=ws)  # off: nothing launched, nothing checked
    assert np.all(host(flow).view(np.uint16) == 0x3C00)
    with pytest.raises(fh.FhcError, match="workspace"):
        fh.gmhs(a, a, flow, 64, 1, ws=ws)
    with pytest.raises(fh.FhcError, match="wider than the padded frame"):
        fh.gmhs(a, a, flow, 16, 1)
    with pytest.raises(fh.FhcError, match="repair level"):
        fh.gmhs_params(32, 32, 64, 3)


@pytest.mark.parametrize("h,w,full_w,cs,level,striped", [(100, 150, 160, 8, 1, False), (256, 384, 768, 8, 1, True),
                                                         (70, 90, 128, 6, 2, False)])
def test_gmhs_n_repairs_each_pair_as_the_oracle(h, w, full_w, cs, level, striped):
    """Three pairs in one fhc_gmhs_n (pictures A0 B0 A1 B1 A2 B2 in one buffer, the flows in another, the workspaces
    NaN-poisoned): each pair's coefficients, maps, decision values and flow equal the oracle's stage on that pair."""
    import torch
    say("gmhs_n", h, w, full_w, cs, level, striped)
    fh = fhops()
    rng = np.random.default_rng(h + w)
    pics, flows = [], []
    for k in range(3):
        if striped and k == 1:
            a, b = striped_scene(h, w, 6)
            f = [np.full((h // 8, w // 8), v) for v in (-3.0, 0.0, 3.0, 0.0)]
            f[0][8:16, 10:22], f[2][8:16, 10:22] = 5.0, -5.0
            fl = np.zeros((1, h // 8, w // 8, cs), np.uint16)
            fl[0, ..., :4] = f16(np.stack(f, -1))
        else:
            a = f16(rng.uniform(0, 1, (1, h, w, 4)))
            b = np.roll(a, (k + 1, -2 * k - 1), axis=(1, 2)).copy()
            fl = smooth_flow(rng, h // 8, w // 8, cs)
        pics += [a, b]
        flows.append(fl)
    ab, fd = dev(np.concatenate(pics)), dev(np.concatenate(flows))
    ws = fh.gmhs_workspace(h, w, full_w, level, "cuda", 3)
    ws.view(torch.float32)[:ws.numel() // 4].fill_(float("nan"))
    fh.gmhs_n(ab, fd, full_w, level, ws=ws)
    got_flow = host(fd).view(np.uint16)
    stride = fh.gmhs_ws_stride(h, w, full_w, level)
    changed = 0
    for k in range(3):
        coef, maps, dec = (host(x) for x in fh.gmhs_results(ws[k * stride:], h, w, full_w, level, h // 8, w // 8))
        want_flow, want_coef, want_maps, want_dec = oracle.gmhs_stages(pics[2 * k], pics[2 * k + 1], flows[k],
                                                                       full_w, level)
        assert np.array_equal(coef.view(np.uint32), want_coef.view(np.uint32)), f"pair {k}: coef"
        for m in range(5):
            assert np.array_equal(maps[m].view(np.uint32), want_maps[m].view(np.uint32)), f"pair {k}: map {m}"
            assert np.array_equal(dec[m].view(np.uint32), want_dec[m].view(np.uint32)), f"pair {k}: decision {m}"
        bad = np.argwhere(got_flow[k:k + 1] != want_flow)
        assert bad.size == 0, f"pair {k}: flow: {len(bad)} elements differ, first at {bad[0].tolist()}"
        changed += (want_flow != flows[k]).any(-1).sum()
    if striped:
        assert changed > 20  # the select fired on the striped pair
    with pytest.raises(fh.FhcError, match="workspace"):
        fh.gmhs_n(ab, fd, full_w, level, ws=ws[:2 * stride])
