"""Pins the CPU oracle before it is trusted as the checker of the GPU path.

Each check is independent of the oracle's own formula: numpy's f16 conversion, torch.nn.functional.conv2d in
float64 (golden vectors), closed forms (delta inputs, delta weights, border counts), a constructed case whose f32
result depends on the split-K grouping, and the reference's own closed-form known-answer conv
(crates/flyhigh-cli/src/cli/coop_tests.rs:340-346, tolerance :612).
"""
import os

import numpy as np
import pytest

from fhtest import Case, as_f64, f16_bits, oracle, ulp_dist

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "conv_vectors.npz")


def test_f16_to_f32_all_patterns_match_numpy():
    a = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(a)
    want = a.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_f32_to_f16_matches_numpy_rounding():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(10 ** 6) * 10.0 ** rng.integers(-9, 6, 10 ** 6)).astype(np.float32)
    edge = np.array([65504, 65519.99, 65520, 1e-8, 5.96e-8, 2.98e-8, 2.9802322e-08, 6.1e-5, -0.0, 0.0,
                     np.inf, -np.inf, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2049.0, 2051.0], dtype=np.float32)
    x = np.concatenate([x, edge, -edge])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f32_to_f16(x), want)


def _golden_cases():
    z = np.load(GOLDEN)
    return z, sorted({k.split(".")[0] for k in z.files})


@pytest.mark.parametrize("order", [oracle.ORDER_TILED, oracle.ORDER_NAIVE, oracle.ORDER_SPLITK])
def test_oracle_matches_float64_golden_vectors(order):
    z, names = _golden_cases()
    for nm in names:
        n, h, w, cin, cout, k, s, pad, act, res, xcs, xc0, ycs, yc0, rcs, rc0 = [int(v) for v in z[nm + ".meta"]]
        d = oracle.make_desc(n, h, w, cin, cout, k=k, stride=s, pad=pad, act=act, alpha=float(z[nm + ".alpha"][0]),
                             residual=res, x_cstride=xcs, x_c0=xc0, y_cstride=ycs, y_c0=yc0, r_cstride=rcs, r_c0=rc0)
        y = z[nm + ".y0"].copy().ravel()
        oracle.conv(d, z[nm + ".x"], z[nm + ".w"], z[nm + ".bias"], z[nm + ".slope"], z[nm + ".res"], y=y,
                    order=order, ksplit=3)
        want = z[nm + ".y"].ravel()
        # f32 accumulation may round across an f16 boundary the f64 result did not: 1 ulp, 2 through a residual
        assert ulp_dist(y, want).max() <= (2 if res else 1), nm
        assert (y == want).mean() >= 0.98, nm


@pytest.mark.parametrize("stride", [1, 2])
def test_delta_input_gives_the_weights_back(stride):
    # a single 1 in the input: every output that sees it equals the weight of the tap it sits under
    h, w, cin, cout = 9, 10, 3, 4
    c = Case(1, h, w, cin, cout, stride=stride, act=0, seed=3)
    c.bias[:] = 0
    x = np.zeros((1, h, w, cin))
    y0, x0, c0 = 4, 5, 2
    x[0, y0, x0, c0] = 1.0
    c.x = f16_bits(x)
    y = as_f64(c.run_oracle())
    wt = as_f64(c.wt)
    want = np.zeros_like(y)
    for oy in range(c.hout):
        for ox in range(c.wout):
            ky, kx = y0 - (oy * stride - 1), x0 - (ox * stride - 1)
            if 0 <= ky < 3 and 0 <= kx < 3:
                want[0, oy, ox, :] = wt[:, c0, ky, kx]
    assert np.array_equal(y, want)


@pytest.mark.parametrize("stride", [1, 2])
def test_delta_weight_gives_a_shifted_copy(stride):
    h, w, cin, cout = 7, 9, 3, 2
    c = Case(1, h, w, cin, cout, stride=stride, act=0, seed=4)
    c.bias[:] = 0
    wt = np.zeros((cout, cin, 3, 3))
    co, ci, ky, kx = 1, 2, 0, 2
    wt[co, ci, ky, kx] = 1.0
    c.wt = f16_bits(wt)
    y = c.run_oracle()
    x = as_f64(c.x)
    want = np.zeros((1, c.hout, c.wout, cout))
    for oy in range(c.hout):
        for ox in range(c.wout):
            iy, ix = oy * stride + ky - 1, ox * stride + kx - 1
            if 0 <= iy < h and 0 <= ix < w:
                want[0, oy, ox, co] = x[0, iy, ix, ci]
    assert np.array_equal(as_f64(y), want)


@pytest.mark.parametrize("h,w,stride", [(6, 7, 1), (7, 8, 2), (8, 9, 2), (1, 5, 1), (2, 2, 2)])
def test_all_ones_counts_the_window_inside_the_image(h, w, stride):
    cin, cout = 5, 3
    c = Case(1, h, w, cin, cout, stride=stride, act=0, seed=5)
    c.x[:] = f16_bits(1.0)
    c.wt[:] = f16_bits(1.0)
    c.bias[:] = 0
    y = as_f64(c.run_oracle())
    for oy in range(c.hout):
        for ox in range(c.wout):
            rows = sum(1 for ky in range(3) if 0 <= oy * stride + ky - 1 < h)
            cols = sum(1 for kx in range(3) if 0 <= ox * stride + kx - 1 < w)
            assert np.all(y[0, oy, ox] == rows * cols * cin)


def test_split_k_result_depends_on_the_z_grouping():
    # 1x1 image: only the centre tap (k = ci*9 + 4) is inside. cin 7 -> K 63, kp 64, 4 K-steps of 16; ksplit 2 puts
    # ci 0..3 in z = 0 and ci 4..6 in z = 1 (conv_tiled.wgsl:94-97). In f32: sequential 2^24 + 1 + 1 + 0 + 1 + 1
    # - 2^24 = 0 (every +1 absorbed), grouped (2^24 + 1 + 1 + 0) + (1 + 1 - 2^24) = 2^24 + (-16777214) = 2.
    c = Case(1, 1, 1, 7, 1, act=0, seed=6)
    c.bias[:] = 0
    x = np.array([4096, 1, 1, 0, 1, 1, 4096], dtype=np.float64)
    wc = np.array([4096, 1, 1, 0, 1, 1, -4096], dtype=np.float64)
    c.x = f16_bits(x.reshape(1, 1, 1, 7))
    wt = np.zeros((1, 7, 3, 3))
    wt[0, :, 1, 1] = wc
    c.wt = f16_bits(wt)
    assert as_f64(c.run_oracle(order=oracle.ORDER_TILED)).item() == 0.0
    assert as_f64(c.run_oracle(order=oracle.ORDER_NAIVE)).item() == 0.0
    assert as_f64(c.run_oracle(order=oracle.ORDER_SPLITK, ksplit=2)).item() == 2.0
    assert as_f64(c.run_oracle(order=oracle.ORDER_SPLITK, ksplit=1)).item() == 0.0


def test_epilogue_rounds_before_the_residual_add():
    # act(acc + b) = 1 + 2^-11 rounds to 1.0 in f16 (tie to even); + residual 2^-11 then gives f16(1 + 2^-11) = 1.0.
    # Without the first rounding the sum would be 1 + 2^-10, which f16 holds exactly.
    c = Case(1, 1, 1, 1, 1, act=0, residual=True, seed=8)
    c.x[:] = f16_bits(1.0)
    wt = np.zeros((1, 1, 3, 3))
    wt[0, 0, 1, 1] = 1.0
    c.wt = f16_bits(wt)
    c.bias[:] = f16_bits(2.0 ** -11)
    c.res[:] = f16_bits(2.0 ** -11)
    assert as_f64(c.run_oracle()).item() == 1.0


def test_prelu_and_leaky_select():
    c = Case(1, 1, 1, 1, 2, act=1, seed=9)
    c.x[:] = f16_bits(1.0)
    wt = np.zeros((2, 1, 3, 3))
    wt[0, 0, 1, 1], wt[1, 0, 1, 1] = -2.0, 3.0
    c.wt = f16_bits(wt)
    c.bias[:] = 0
    c.slope[:] = f16_bits([0.25, 0.5])
    assert list(as_f64(c.run_oracle()).ravel()) == [-0.5, 3.0]
    c.act, c.alpha = 2, 0.125
    assert list(as_f64(c.run_oracle()).ravel()) == [-0.25, 3.0]
    c.act = 0
    assert list(as_f64(c.run_oracle()).ravel()) == [-2.0, 3.0]


def test_known_answer_closed_form_conv():
    # crates/flyhigh-cli/src/cli/coop_tests.rs:337-346: 208 -> 64 at 80 x 46, x[i] = ((i % 17) - 8) * 0.05 in CHW
    # order, w[i] = ((i % 13) - 6) * 0.04 in OIHW order, bias (i % 5 - 2) * 0.1, PReLU slope 0.1; the reference
    # accepts max|d| < 0.1 against an f32 CPU conv of the unrounded values (:554-579, :612).
    import torch
    cin, cout, h, w = 208, 64, 46, 80
    xi = np.arange(cin * h * w)
    x_chw = (((xi % 17) - 8) * 0.05).reshape(cin, h, w)
    wv = (((np.arange(cout * cin * 9) % 13) - 6) * 0.04).reshape(cout, cin, 3, 3)
    b = (np.arange(cout) % 5 - 2) * 0.1
    want = torch.nn.functional.conv2d(torch.from_numpy(x_chw[None]), torch.from_numpy(wv), padding=1)[0].numpy()
    want = want + b[:, None, None]
    want = np.where(want > 0, want, 0.1 * want)
    c = Case(1, h, w, cin, cout, act=1, seed=10)
    c.x = f16_bits(x_chw.transpose(1, 2, 0)[None])
    c.wt = f16_bits(wv)
    c.bias = f16_bits(b)
    c.slope = f16_bits(np.full(cout, 0.1))
    y = as_f64(c.run_oracle(threads=8))[0].transpose(2, 0, 1)
    assert np.abs(y - want).max() < 0.1


@pytest.mark.parametrize("bad", [dict(stride=0), dict(cin=0), dict(x_cstride=2), dict(y_c0=7)])
def test_oracle_rejects_bad_descriptors(bad):
    d = oracle.make_desc(1, 4, 4, 3, 3)
    d.update(bad)
    x = np.zeros(4 * 4 * 3, np.uint16)
    with pytest.raises(ValueError):
        oracle.conv(d, x, np.zeros(81, np.uint16), np.zeros(3, np.uint16), np.zeros(3, np.uint16))


def test_multithreaded_oracle_equals_single_threaded():
    c = Case(2, 13, 17, 12, 10, stride=1, act=1, residual=True, seed=11)
    assert np.array_equal(c.run_oracle(), c.run_oracle(threads=5))


@pytest.mark.parametrize("k,stride,h", [(3, 1, 23), (3, 2, 24), (3, 2, 25), (1, 1, 19)])
def test_row_bands_equal_the_whole_oracle(k, stride, h):
    from fhtest import oracle_rows
    c = Case(1, h, 14, 6, 5, k=k, stride=stride, act=1, residual=True, seed=12)
    full = c.run_oracle()
    for r0, r1 in [(0, 4), (3, 7), (c.hout - 4, c.hout), (0, c.hout)]:
        assert np.array_equal(oracle_rows(c, r0, r1), full[0, r0:r1]), (r0, r1)
