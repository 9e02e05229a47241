"""The planner: the reference's choices restated (pinned by its golden plans and logic tests), and the MI355X
planner's own choices, variant codes and choice table. Host logic only, no GPU."""
import json
import os

import pytest

from fhtest import fhconv

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_conv_plans.json")


def test_reference_golden_plans_are_reproduced():
    # every conv of the 27 golden plans (crates/flyhigh-engine/tests/golden/*, 3 device classes x 9 sessions):
    # kernel, grid, packed-weight bytes, the 16 ImplicitGemmParams words, the split-K reduce and the residual add
    recs = json.load(open(GOLDEN))
    assert len(recs) == 639
    seen = set()
    for r in recs:
        c, cls = r["conv"], r["cls"]
        got = fhconv.ref_conv_steps(c["cin"], c["cout"], c["h"], c["w"], c["stride"], residual=c["residual"],
                                    coop=cls.startswith("tc"), f32_mode=cls.endswith("f32"))
        want = [(s[0], tuple(s[1]), s[2], s[3]) for s in r["steps"]]
        assert got == want, r["source"]
        seen.update(s[0] for s in want)
    # the golden plans exercise every path of the restatement
    assert {"fused", "fused2", "fdirect32", "xshift", "tconv", "tconv32", "skreduce", "binary"} <= seen


def has(lst, kind):
    return any(c & 15 == kind for c in lst)


def test_portable_candidates_for_a_wide_conv():
    # crates/flyhigh-engine/tests/logic.rs:33-45
    lst = fhconv.cand_list(False, 64, 60, 108, False)
    assert has(lst, fhconv.CAND_TILED) and has(lst, fhconv.CAND_TILED8) and has(lst, fhconv.CAND_TILED88)
    assert not has(lst, fhconv.CAND_TC) and not has(lst, fhconv.CAND_DIRECT)
    assert not has(lst, fhconv.CAND_TILED16) and not has(lst, fhconv.CAND_TILEDN8)
    for ks in (1, 2, 4):
        assert fhconv.CAND_TILED | ks << 4 in lst


def test_narrow_candidates_for_a_small_conv():
    # logic.rs:47-52
    lst = fhconv.cand_list(False, 16, 120, 216, False)
    assert has(lst, fhconv.CAND_TILED) and has(lst, fhconv.CAND_TILED16) and has(lst, fhconv.CAND_TILEDN8)
    assert not has(lst, fhconv.CAND_TILED8) and not has(lst, fhconv.CAND_TILED88)


def test_tensor_core_candidates_need_the_feature_and_direct_needs_its_shape():
    # logic.rs:54-61
    tc = fhconv.cand_list(True, 64, 60, 108, False)
    assert has(tc, fhconv.CAND_TC) and not has(tc, fhconv.CAND_DIRECT)
    direct = fhconv.cand_list(True, 64, 60, 112, True)
    assert has(direct, fhconv.CAND_TC) and has(direct, fhconv.CAND_DIRECT)
    assert has(tc, fhconv.CAND_TILED)


def test_try_all_adds_the_kernels_that_never_won():
    base = fhconv.cand_list(True, 64, 60, 112, True)
    full = fhconv.cand_list(True, 64, 60, 112, True, try_all=True)
    assert not has(base, fhconv.CAND_DIRECT64) and has(full, fhconv.CAND_DIRECT64)
    assert has(full, fhconv.CAND_TILEDM32) and has(full, fhconv.CAND_TILED8P)


def test_candidate_names():
    assert fhconv.cand_name(fhconv.CAND_TILED) == "tiled"
    assert fhconv.cand_name(fhconv.CAND_TILED | 4 << 4) == "tiled/k4"
    assert fhconv.cand_name(fhconv.CAND_DIRECT) == "direct"
    with pytest.raises(fhconv.FhcError):
        fhconv.cand_name(12)


def test_forced_split_and_env_override_in_the_reference_planner():
    # kernels.rs:157-170: a forced split (candidate nibble) is capped by the K-step count; FH_KSPLIT overrides it;
    # the partials stay under 32 MB
    steps = fhconv.ref_conv_steps(36, 36, 60, 108, 1, coop=False, cand=fhconv.CAND_TILED | 4 << 4)
    assert steps[0][1] == (1, 102, 4) and steps[1][0] == "skreduce"
    steps = fhconv.ref_conv_steps(3, 36, 120, 216, 2, coop=False, cand=fhconv.CAND_TILED | 4 << 4)
    assert steps[0][1][2] == 2  # kp 32 -> 2 K-steps
    steps = fhconv.ref_conv_steps(36, 36, 60, 108, 1, coop=False, ksplit_env=3)
    assert steps[0][1][2] == 3
    big = fhconv.ref_conv_steps(32, 32, 1088, 1920, 1, coop=False, cand=fhconv.CAND_TILED | 4 << 4)
    assert big[0][1][2] == 1 and len(big) == 1  # 4 * 32 * 2088960 * 4 bytes > 32 MB


def test_tune_table_round_trips_and_skips_garbage():
    # crates/flyhigh-engine/tests/defaults.rs:55-64, on the MI355X table (same key and text format)
    fhconv.tune_clear()
    try:
        text = "96,96,60,108,1=18\nnot a line\n36,36,180,320,1=2\n1,2,3=4\n48,48,60,108,1=x\n"
        assert fhconv.parse_tune(text) == 2
        assert fhconv.tune_get(96, 96, 60, 108, 1) == 18
        assert fhconv.tune_get(36, 36, 180, 320, 1) == 2
        assert fhconv.tune_get(48, 48, 60, 108, 1) is None
        out = fhconv.format_tune()
        assert out == "36,36,180,320,1=2\n96,96,60,108,1=18"
        fhconv.tune_clear()
        assert fhconv.parse_tune(out) == 2 and fhconv.format_tune() == out
        fhconv.tune_clear()
        assert fhconv.parse_tune("") == 0 and fhconv.parse_tune("garbage") == 0
    finally:
        fhconv.tune_clear()


# the conv layers the planner has to serve: the configs' layers and the FlyHighFG layer shapes
SHAPES = [
    (1, 136, 240, 32, 32, 3, 1), (1, 544, 960, 32, 64, 3, 2), (1, 272, 480, 64, 64, 3, 1),
    (1, 68, 120, 128, 128, 3, 1), (1, 68, 120, 128, 64, 1, 1), (1, 120, 216, 3, 36, 3, 2),
    (1, 60, 108, 36, 36, 3, 1), (1, 60, 108, 36, 72, 3, 2), (1, 30, 54, 72, 72, 3, 1), (1, 30, 54, 279, 96, 3, 1),
    (1, 30, 54, 96, 96, 3, 1), (1, 30, 54, 96, 12, 3, 1), (1, 60, 108, 155, 48, 3, 1), (1, 60, 108, 48, 48, 3, 1),
    (1, 60, 108, 48, 7, 3, 1), (1, 60, 108, 48, 5, 3, 1), (1, 60, 108, 48, 36, 3, 1), (1, 120, 216, 14, 24, 3, 1),
    (1, 120, 216, 24, 24, 3, 1), (1, 120, 216, 24, 3, 3, 1), (8, 120, 216, 3, 36, 3, 2),
]


def test_direct_kernel_where_the_channels_fit():
    # small-channel layers go to the direct kernel (weights resident), deep ones to the deep-layer kernel where the
    # input view has 16-byte channel groups, else to the chunked kernel
    assert fhconv.plan_dry(fhconv.make_desc(1, 136, 240, 32, 32))["family"] == "direct"
    assert fhconv.plan_dry(fhconv.make_desc(1, 544, 960, 32, 64, stride=2))["family"] == "direct"
    assert fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 64, k=1))["family"] == "direct"
    deep = fhconv.plan_dry(fhconv.make_desc(1, 30, 54, 279, 96))  # one kernel row of K per wave
    assert deep["family"] == "direct" and deep["cc"] == 288 and deep["waves"][2] == 3
    assert fhconv.plan_dry(fhconv.make_desc(1, 60, 108, 72, 36, stride=2))["family"] == "igemm"
    assert fhconv.plan_dry(fhconv.make_desc(1, 30, 54, 300, 96))["family"] == "igemm"  # 300 % 8: no DMA path
    assert fhconv.plan_dry(fhconv.make_desc(1, 30, 54, 300, 96, x_cstride=304))["family"] == "gemm"
    assert fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 128))["name"] == "gemm.t8x16.n48.f2x3.w4x1.c32.p2"
    d = fhconv.plan_dry(fhconv.make_desc(1, 60, 108, 36, 36))
    assert d["family"] == "direct" and d["cc"] == 64 and d["tile_channels"] == 48 and d["ntn"] == 1


@pytest.mark.parametrize("shape", SHAPES)
def test_mi355x_plan_covers_the_output(shape):
    n, h, w, cin, cout, k, s = shape
    p = fhconv.plan_dry(fhconv.make_desc(n, h, w, cin, cout, k=k, stride=s))
    assert p["hout"] == (h + 2 * (k == 3) - k) // s + 1 and p["wout"] == (w + 2 * (k == 3) - k) // s + 1
    tiles = -(-p["hout"] // p["tile_rows"]) * -(-p["wout"] // 16) * n
    assert p["tiles"] == tiles
    assert p["ntn"] * p["tile_channels"] >= cout > (p["ntn"] - 1) * p["tile_channels"]
    assert p["cc"] % 8 == 0 and p["cc"] * p["nchunks"] >= cin and p["cc"] * (p["nchunks"] - 1) < cin
    if p["family"] == "igemm":
        assert p["grid"][0] == tiles * p["ntn"]
        assert p["ksteps"] * 32 >= k * k * p["cc"]
    elif p["family"] == "gemm":  # deep-layer kernel: one workgroup per tile and channel tile, chunks of 32 or 64
        assert p["grid"] == [tiles, p["ntn"], 1] and k == 3 and s == 1
        assert p["cc"] in (32, 64) and p["ksteps"] * 32 == 9 * p["cc"]
    else:
        assert p["grid"][1] == p["ntn"] and 1 <= p["grid"][0] <= tiles
        assert p["cc"] % 32 == 0 and p["ksteps"] * 32 == k * k * p["cc"] and p["nchunks"] == 1
    assert p["lds"] <= 64 * 1024
    assert p["flops"] == 2 * n * p["hout"] * p["wout"] * cout * cin * k * k
    name = fhconv.variant_name(p["variant"])
    assert name == p["name"]


def test_variant_list_and_forced_variants():
    d = fhconv.make_desc(1, 68, 120, 128, 128)
    codes = fhconv.variant_list(d)
    assert len(codes) >= 4 and len(set(codes)) == len(codes)
    for code in codes:
        p = fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 128, variant=code))
        assert p["variant"] == code
    split = [c for c in codes if c < 128 and c >> 5]
    assert split, "a 68x120 layer has a small tile grid: split-K variants are listed"
    with pytest.raises(fhconv.FhcError):
        fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 128, variant=31))


def test_forced_split_k_and_reference_hint():
    p = fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 128, ksplit=4))
    np_ = -(-128 // p["tile_channels"]) * p["tile_channels"]
    assert p["ksplit"] == 4 and p["grid"][1 if p["family"] == "igemm" else 2] == 4
    assert p["workspace_bytes"] == 4 * 68 * 120 * np_ * 4  # f32 partials [z][pixel][np]
    assert p["nchunks"] % 4 == 0
    h = fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 128, ref_cand=fhconv.CAND_TILED | 2 << 4))
    assert h["ksplit"] == 2
    none = fhconv.plan_dry(fhconv.make_desc(1, 68, 120, 128, 128))
    assert none["ksplit"] == 1 and none["workspace_bytes"] == 0


def test_tune_table_keys_batch_and_kernel_size():
    # the batch and the kernel size extend the reference's key: the batch-1 3x3 entry keeps the reference's 5
    # fields, a batched or 1x1 entry carries n and k, and none of them overwrites another
    fhconv.tune_clear()
    try:
        text = "48,48,60,108,1=18\n48,48,60,108,1,24,3=17\n48,48,60,108,1,1,1=130\n48,48,60,108,1,0,3=5\n" \
               "48,48,60,108,1,2,5=5\n48,48,60,108,1,2=5\n"
        assert fhconv.parse_tune(text) == 3
        assert fhconv.tune_get(48, 48, 60, 108, 1) == 18
        assert fhconv.tune_get(48, 48, 60, 108, 1, n=24) == 17
        assert fhconv.tune_get(48, 48, 60, 108, 1, k=1) == 130
        assert fhconv.tune_get(48, 48, 60, 108, 1, n=8) is None
        out = fhconv.format_tune()
        assert out == "48,48,60,108,1,1,1=130\n48,48,60,108,1,24,3=17\n48,48,60,108,1=18"
        fhconv.tune_clear()
        assert fhconv.parse_tune(out) == 3 and fhconv.format_tune() == out
        # the planner looks the descriptor's own batch up
        d1, d24 = fhconv.make_desc(1, 60, 108, 48, 48), fhconv.make_desc(24, 60, 108, 48, 48)
        codes = fhconv.variant_list(d24)
        fhconv.tune_clear()
        fhconv.parse_tune(f"48,48,60,108,1,24,3={codes[0]}\n48,48,60,108,1={codes[1]}")
        assert fhconv.plan_dry(d24)["variant"] == codes[0]
        assert fhconv.plan_dry(d1)["variant"] == codes[1]
    finally:
        fhconv.tune_clear()


def test_the_table_steers_the_planner():
    fhconv.tune_clear()
    try:
        d = fhconv.make_desc(1, 136, 240, 32, 32)
        default = fhconv.plan_dry(d)["variant"]
        other = [c for c in fhconv.variant_list(d) if c != default][0]
        fhconv.parse_tune(f"32,32,136,240,1={other}")
        assert fhconv.plan_dry(d)["variant"] == other
    finally:
        fhconv.tune_clear()


def test_tune_table_takes_variant_names():
    # a committed table names variants (stable across builds); the parser maps each name to this build's code
    fhconv.tune_clear()
    try:
        d = fhconv.make_desc(1, 60, 108, 48, 48)
        names = {fhconv.variant_name(c): c for c in fhconv.variant_list(d)}
        name = sorted(names)[0]
        assert fhconv.parse_tune(f"48,48,60,108,1={name}\n48,48,60,108,2=no.such.variant\n") == 1
        assert fhconv.tune_get(48, 48, 60, 108, 1) == names[name]
        assert fhconv.tune_get(48, 48, 60, 108, 2) is None
        assert f"48,48,60,108,1={names[name]}" in fhconv.format_tune()
        assert fhconv.plan_dry(d)["name"] == name
    finally:
        fhconv.tune_clear()


def test_committed_choice_table_parses():
    # every line of the shipped MI355X table names a variant this build has
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "flyhigh-engine_amd", "tune_mi355x.txt")
    text = open(path).read()
    fhconv.tune_clear()
    try:
        assert fhconv.parse_tune(text) == len([ln for ln in text.splitlines() if ln.strip()])
    finally:
        fhconv.tune_clear()
