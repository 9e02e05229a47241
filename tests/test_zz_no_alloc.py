"""fhc_conv_run_noalloc: the split-K plans' partials in the library's static device scratch instead of a caller
workspace. Against fhc_conv_run with a workspace (the same kernels and partial order: bit-identical) and against
the oracle (the parity bar), on two calls in a row, the second with a smaller input, then a plan without scratch,
and a plan whose scratch exceeds the static array (refused with an error, nothing launched)."""
import ctypes

import numpy as np
import pytest

from fhtest import Case, fhconv, parity


def say(*a):
    print(*a, flush=True)


def _run_both(c, ksplit, variant=0):
    import torch
    dev = torch.device("cuda", 0)
    plan = fhconv.ConvPlan(c.fhc_desc(variant=variant, ksplit=ksplit), c.wt, c.bias, c.slope if c.act == 1 else None)
    host = lambda a: torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev)  # noqa: E731
    x, r = host(c.x), host(c.res) if c.residual else None
    y_ws, y_na = host(c.y0), host(c.y0)
    ws = torch.empty(plan.workspace_bytes // 2 + 8, dtype=torch.int16, device=dev) if plan.workspace_bytes else None
    plan.run(x, y_ws, r, ws)
    plan.run_noalloc(x, y_na, r)
    torch.cuda.synchronize()
    return plan, y_ws.cpu().numpy().view(np.uint16), y_na.cpu().numpy().view(np.uint16)


@pytest.mark.gpu
def test_noalloc_matches_the_workspace_entry_point():
    cases = [(Case(1, 68, 120, 128, 128, act=1, seed=31), 4),   # the 1080p/16 deep layer, split 4
             (Case(1, 20, 36, 96, 48, act=1, residual=True, seed=32), 2)]  # smaller, with a residual, split 2
    for c, ks in cases:
        say("noalloc", c.n, c.h, c.w, c.cin, c.cout, "ksplit", ks)
        plan, y_ws, y_na = _run_both(c, ks)
        d = plan.describe()
        say("  ", d["name"], "workspace", plan.workspace_bytes)
        assert d["ksplit"] == ks and plan.workspace_bytes > 0
        assert np.array_equal(y_ws, y_na), "noalloc differs from the workspace entry point"
        ok, md, mref = parity(y_na, c.run_oracle(threads=8))
        assert ok, (md, mref)


@pytest.mark.gpu
def test_noalloc_without_scratch_and_beyond_its_limit():
    c = Case(1, 24, 40, 32, 32, act=1, seed=33)
    say("noalloc without scratch")
    plan, y_ws, y_na = _run_both(c, 0)
    assert plan.workspace_bytes == 0 and np.array_equal(y_ws, y_na)
    # a split-K plan whose partials exceed the static array: refused before any launch, on real input and output
    # buffers of the plan's shape (the output keeps its sentinel: nothing ran)
    import torch
    big = Case(1, 272, 480, 128, 128, act=1, seed=34)
    plan = fhconv.ConvPlan(big.fhc_desc(ksplit=4), big.wt, big.bias, big.slope)
    limit = 32 << 20
    say("noalloc beyond the limit:", plan.workspace_bytes, "bytes")
    assert plan.workspace_bytes > limit
    dev = torch.device("cuda", 0)
    x = torch.zeros((1, 272, 480, 128), dtype=torch.int16, device=dev)
    y = torch.full((1, 272, 480, 128), 0x7E00, dtype=torch.int16, device=dev)
    rc = fhconv.load().fhc_conv_run_noalloc(plan.handle, ctypes.c_void_p(x.data_ptr()),
                                            ctypes.c_void_p(y.data_ptr()), None, None)
    assert rc < 0 and "static scratch" in fhconv.last_error()
    torch.cuda.synchronize()
    assert bool((y == 0x7E00).all())
