"""GPU: the C host layer (pitorch_amd/host/pt.h) driven from C.

pitorch_amd/lib/pt_demo is a C program in the shape of the reference's
examples/generate.c and examples/train.c (pt_gpu_init in place of
pt_pi_init).  It runs as a child process; its greedy ids, from both
pt_generate_ids and a pt_forward_step loop, must equal the reference
build's tokens (tests/golden/decode_stories15M.json), and its 18 training
losses must stay within 1e-4 of the reference's curve
(tests/golden/train_stories15M.json).
"""
import json
import os
import subprocess

import pytest

import pitorch_amd as pa

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DEMO = os.path.join(pa.lib_dir(), "pt_demo")


def run_demo(*args):
    assert os.path.exists(DEMO), "pt_demo not built: run __graft_entry__.build()"
    r = subprocess.run([DEMO, *map(str, args)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    return r.stdout.splitlines()


def ids(lines, tag):
    line = next(ln for ln in lines if ln.startswith(tag + ":"))
    return [int(v) for v in line.split(":", 1)[1].split()]


def test_c_generate_matches_reference_tokens():
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "decode_stories15M.json")))
    cfg = pa.STORIES["stories15M"]
    n_tok = len(fx["tokens"])
    lines = run_demo("generate", *cfg, pa.SEED_MODEL["stories15M"], pa.SEED_PROMPT, pa.N_PROMPT, n_tok)
    assert ids(lines, "prompt") == fx["prompt"]
    assert ids(lines, "generate") == fx["tokens"]
    assert ids(lines, "forward_step") == fx["tokens"]


def test_c_train_matches_reference_losses():
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "train_stories15M.json")))
    cfg = pa.STORIES["stories15M"]
    lines = run_demo("train", *cfg, pa.SEED_MODEL["stories15M"], fx["train_seed"], fx["T"], fx["lr"],
                     len(fx["losses"]))
    losses = [float(ln.split()[2]) for ln in lines if ln.startswith("loss ")]
    assert len(losses) == len(fx["losses"])
    assert max(abs(a - b) for a, b in zip(losses, fx["losses"])) < 1e-4, list(zip(losses, fx["losses"]))


def test_c_demo_fails_loudly_on_bad_usage():
    r = subprocess.run([DEMO, "generate", "1"], capture_output=True, text=True, timeout=30)
    assert r.returncode == 2 and "usage" in r.stderr
