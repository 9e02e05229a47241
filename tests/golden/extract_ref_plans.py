"""Extracts the conv dispatches from the reference's golden plans into a compact fixture.

Reads /root/reference/crates/flyhigh-engine/tests/golden/<config>.<class>.txt (data files the reference's own
test, tests/golden_plans.rs:125-154, compares plans against) and writes ref_conv_plans.json beside this script:
one record per conv the planner recorded, holding the conv's inputs (cin, cout, input h/w, stride, whether a
residual add was fused) and the dispatches the reference recorded for it (pipeline, grid, packed-weight bytes,
parameter words). The planner restatement (fhc_ref_conv_steps) must reproduce the dispatches from the inputs.
Also writes ref_plan_steps.json: every plan's whole step sequence (pipeline names and grids, the mid stage's first
step, and the parameter words of the periodic-structure repair's gm_* steps), against which the static plan of
fhc_model_plan is checked step by step.

Line format of the reference files (ops/step.rs:51-88): "idx pipeline (gx,gy,gz) [bindings] <u32 words as hex>".
Run in the build container only (the reference is not present on the GPU box):
    python tests/golden/extract_ref_plans.py
"""
import glob
import json
import os
import re

REF = "/root/reference/crates/flyhigh-engine/tests/golden"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_conv_plans.json")
OUT_STEPS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_plan_steps.json")

CONV = {"fused", "fused2", "fdirect", "fdirect32", "fdirect64", "tconv", "tconv8", "tconv88", "tconv8p",
        "tconvm32", "tconv16", "tconv32", "tconvn8"}
LINE = re.compile(r"^\s*(\d+) (\S+) \((\d+),(\d+),(\d+)\) \[([^\]]*)\]((?: [0-9a-f]{8})*)\s*$")


def parse(path):
    steps = []
    for ln in open(path):
        m = LINE.match(ln)
        if not m:
            continue
        binds = m.group(6).split()
        words = [int(v, 16) for v in m.group(7).split()]
        steps.append(dict(name=m.group(2), grid=[int(m.group(3)), int(m.group(4)), int(m.group(5))],
                          binds=binds, words=words))
    return steps


def buf_bytes(tok):
    return int(tok[3:]) if tok.startswith("buf") else 0


def main():
    records = []
    for path in sorted(glob.glob(os.path.join(REF, "*.txt"))):
        base = os.path.basename(path)[:-4]
        config, cls = base.rsplit(".", 1)
        steps = parse(path)
        i = 0
        while i < len(steps):
            s = steps[i]
            group = []
            if s["name"] == "xshift" and i + 1 < len(steps) and steps[i + 1]["name"].startswith("fdirect"):
                group = [s, steps[i + 1]]
                conv = steps[i + 1]
            elif s["name"] in CONV:
                group = [s]
                conv = s
            else:
                i += 1
                continue
            p = conv["words"]
            cin, h, w, hout, wout, stride = p[0], p[1], p[2], p[3], p[4], p[5]
            cout = p[9]
            residual = 0
            j = i + len(group)
            if conv["name"].startswith("tconv"):
                if p[13] <= 1:
                    residual = p[14]
                elif j < len(steps) and steps[j]["name"] == "skreduce":
                    residual = steps[j]["words"][3]
                    group.append(steps[j])
            else:
                # tensor-core / direct kernels: a fused residual is a separate binary add of the conv output
                # (ops/conv/autotune.rs:135-139), reading the conv's output binding first
                out_bind = conv["binds"][5]
                if j < len(steps) and steps[j]["name"] == "binary":
                    b = steps[j]
                    if (b["binds"][0] == out_bind and b["words"][:8] == [cout, hout, wout, cout, 0, 0, 0, 0]
                            and b["words"][8:10] == [0x3F800000, 0x3F800000]):
                        residual = 1
                        group.append(b)
            rec = dict(source=f"{base}:{i}", config=config, cls=cls,
                       conv=dict(cin=cin, cout=cout, h=h, w=w, stride=stride, residual=residual),
                       steps=[])
            for g in group:
                wb = buf_bytes(g["binds"][1]) if g["name"] in CONV or g["name"].startswith("fdirect") else 0
                rec["steps"].append([g["name"], g["grid"], wb, g["words"]])
            records.append(rec)
            i += len(group)
    with open(OUT, "w") as f:
        json.dump(records, f, separators=(",", ":"))
        f.write("\n")
    print(f"{len(records)} conv records from {len(glob.glob(os.path.join(REF, '*.txt')))} golden plans -> {OUT}")
    # the whole step sequence of every golden plan: pipeline names and grids, and where the mid stage starts
    plans = {}
    for path in sorted(glob.glob(os.path.join(REF, "*.txt"))):
        base = os.path.basename(path)[:-4]
        header, mid = "", None
        steps = []
        for ln in open(path):
            if ln.startswith("# ") and not header:
                header = ln[2:].strip()
            elif ln.strip() == "# mid":
                mid = len(steps)
            m = LINE.match(ln)
            if m:
                step = [m.group(2), [int(m.group(3)), int(m.group(4)), int(m.group(5))]]
                if m.group(2).startswith("gm_"):  # the repair's parameter words (FitP, CostP, BoxP, SelP)
                    step.append([int(v, 16) for v in m.group(7).split()])
                steps.append(step)
        plans[base] = dict(header=header, mid=mid, steps=steps)
    with open(OUT_STEPS, "w") as f:
        json.dump(plans, f, separators=(",", ":"))
        f.write("\n")
    print(f"{len(plans)} step sequences -> {OUT_STEPS}")


if __name__ == "__main__":
    main()
