"""GPU: the traced training step (ptmi_model_train_step_trace) and the
host trace API behind pt_enable_trace (pitorch/pt.c:322-364,
pitorch/profiler/trace.c).

* The traced step runs the same kernels (eagerly, behind a busy kernel): its loss and
  updated weights equal the untraced step's exactly.
* Its span sequence (name, cat, layer, depth, in the order trace.c records
  them) is the reference's own traced pt_train_step's
  (tests/golden/trace_spans.json, written from oracle/_ref), plus one span
  the reference does not have: "weight_grads", the grouped launch of the
  layers' weight gradients, which the reference computes inside each
  layer's spans.  Every span lies inside its parent.
* pt_demo (a C caller of pt.h) writes trace.json / meta.json as the
  reference's dev/host/test_train_profiled.c does.
"""
import json
import os
import subprocess

import numpy as np
import pytest

import pitorch_amd as pa

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FX = json.load(open(os.path.join(ROOT, "tests", "golden", "trace_spans.json")))
CFG = tuple(FX["config"])
PER_LAYER = ["layer", "qkv", "attention", "wo", "ffn", "transpose"]
EXTRA = ("weight_grads", "bwd", -1, 2)          # ours only, just before the backward "embedding"


def expected_spans():
    spans = [tuple(sp) for sp in FX["spans"]]
    i = spans.index(("embedding", "bwd", -1, 2))
    return spans[:i] + [EXTRA] + spans[i:]


def expected_names(L):
    assert L == CFG[2]
    return sorted(sp[0] for sp in expected_spans())


def check_nesting(spans, slack):
    """spans in end order, each with depth/start/dur: every span of depth d > 0
    lies inside the next span (in end order) of depth d - 1."""
    for i, s in enumerate(spans):
        if s["depth"] == 0:
            continue
        parent = next(p for p in spans[i + 1:] if p["depth"] == s["depth"] - 1)
        assert parent["start"] - slack <= s["start"], (s, parent)
        assert s["start"] + s["dur"] <= parent["start"] + parent["dur"] + slack, (s, parent)


def test_traced_step_equals_untraced_and_spans_nest():
    blob = pa.synth_model(CFG, FX["model_seed"], 0.05)
    tokens = pa.seed_tokens(FX["token_seed"], FX["T"], CFG[5])
    a, b = pa.Model(blob.copy(), max_T=FX["T"]), pa.Model(blob.copy(), max_T=FX["T"])
    for _ in range(2):
        la, spans = a.train_step_trace(tokens, FX["lr"])
        lb = b.train_step(tokens, FX["lr"])
        assert la == lb
    assert np.array_equal(a.read_weights(), b.read_weights())
    assert [(s["name"], s["cat"], s["layer"], s["depth"]) for s in spans] == expected_spans()
    assert spans[-1]["name"] == "train_step" and spans[-1]["depth"] == 0 and spans[-1]["start_us"] == 0.0
    check_nesting([dict(depth=s["depth"], start=s["start_us"], dur=s["dur_us"]) for s in spans], 1e-3)
    for s in spans:
        assert s["dur_us"] >= 0.0
        if s["name"] in ("qkv", "attention", "ffn", "weight_grads", "loss", "cls_weight_grad"):
            assert s["dur_us"] > 0.0, s
    depth1 = sum(s["dur_us"] for s in spans if s["depth"] == 1)
    assert depth1 <= spans[-1]["dur_us"] + 1e-3
    with pytest.raises(pa.PtmiError):
        a.train_step_trace(tokens, FX["lr"], max_spans=3)         # buffer smaller than the step's spans
    a.close()
    b.close()


def test_c_caller_writes_trace_json(tmp_path):
    demo = os.path.join(pa.lib_dir(), "pt_demo")
    args = [demo, "train", *map(str, CFG), "33", "34", "16", "0.05", "2"]
    out = tmp_path / "trace"                   # created by pt_demo, as the reference's profiled test does
    plain = subprocess.run(args, capture_output=True, text=True, timeout=120)
    traced = subprocess.run(args + [str(out)], capture_output=True, text=True, timeout=120)
    assert plain.returncode == 0 and traced.returncode == 0, traced.stderr[-2000:]
    losses = lambda out: [ln for ln in out.splitlines() if ln.startswith("loss ")]
    assert losses(plain.stdout) == losses(traced.stdout)
    # a trace that cannot be written is an error, not a silent success
    bad = subprocess.run(args + [str(tmp_path / "no" / "such" / "dir")], capture_output=True, text=True, timeout=120)
    assert bad.returncode != 0 and "could not write" in bad.stderr
    ev = json.load(open(out / "trace.json"))
    L = CFG[2]
    assert len(ev) == 2 * len(expected_spans())
    names = sorted(e["name"].split("_", 1)[1] if e["name"][0] == "L" and e["name"][1].isdigit() else e["name"]
                   for e in ev[: len(ev) // 2])
    assert names == expected_names(L)
    assert all(e["ph"] == "X" and e["cat"] in ("train", "fwd", "bwd") for e in ev)
    assert {e["name"] for e in ev if e["name"].startswith("L")} == {f"L{l}_{n}" for l in range(L) for n in PER_LAYER}
    steps = [e for e in ev if e["name"] == "train_step"]
    assert len(steps) == 2 and steps[0]["ts"] + steps[0]["dur"] <= steps[1]["ts"] + 1
    meta = json.load(open(out / "meta.json"))
    assert meta["steps"] == 2 and meta["layers"] == L and meta["device"] == "mi355x"
