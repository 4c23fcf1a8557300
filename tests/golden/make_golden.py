"""Write the golden decode/training fixtures from the reference's own build.

Runs masonwang025/pitorch's host C path (oracle/_ref/libptref.so, built from
the reference sources by oracle/Makefile) on the seeded synthetic models of
the benchmark configurations:

* decode_tokens.json — pt_forward_step (pitorch/pt.c:267-271) greedy tokens:
  the 8 seeded prompt ids are forced at positions 0..6 (pt_text.c:344-347),
  argmax afterwards; 256 positions (15M) / 1024 (42M, 110M).
* train_losses.json — pt_train_step (pitorch/pt.c:339-364) losses, 15M,
  T=256 seeded ids, lr=1e-3, 18 steps.
* logits_<config>.json — logits of pt_forward_step at chosen positions
  across the attention's position chunks (pitorch/model/llama2.c:153-177
  scans t <= pos), teacher-forced on the golden tokens: the top-16
  (id, logit), logits at 16 seeded ids, max |logit|, the top-1/top-2 margin,
  and the fp64 sum and sum of squares of all logits.
* trace_spans.json — the span sequence (name, cat, layer, depth, in the
  order trace.c records them) of one traced pt_train_step
  (pt_enable_trace, pitorch/pt.c:322-364; pt_train.c:171-866) on a small
  seeded model.

Usage: python tests/golden/make_golden.py [decode15|decode42|decode110|train15|trace|logits15|logits42|logits110 ...]
"""
import ctypes
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import pitorch_amd as pa  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))


def ref_lib():
    L = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libptref.so"))
    vp = ctypes.c_void_p
    L.ref_ctx_new.restype = vp
    L.ref_ctx_new.argtypes = [vp, ctypes.c_int]
    L.ref_ctx_free.argtypes = [vp]
    L.ref_forward_step.restype = ctypes.c_int
    L.ref_forward_step.argtypes = [vp, ctypes.c_int]
    L.ref_train_step.restype = ctypes.c_float
    L.ref_train_step.argtypes = [vp, ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_float]
    return L


def blob_digest(blob):
    return hashlib.sha256(blob.tobytes()).hexdigest()


def decode(name):
    cfg = pa.STORIES[name]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    prompt = pa.seed_tokens(pa.SEED_PROMPT, pa.N_PROMPT, cfg[5])
    L = ref_lib()
    ctx = L.ref_ctx_new(blob.ctypes.data_as(ctypes.c_void_p), 0)
    out = []
    tok = int(prompt[0])
    for pos in range(pa.DECODE_POSITIONS[name]):
        nxt = L.ref_forward_step(ctx, tok)
        if pos < len(prompt) - 1:
            nxt = int(prompt[pos + 1])
        out.append(int(nxt))
        tok = nxt
        if pos % 64 == 0:
            print(name, pos, flush=True)
    L.ref_ctx_free(ctx)
    return {"config": name, "model_seed": pa.SEED_MODEL[name], "blob_sha256": blob_digest(blob),
            "prompt": [int(t) for t in prompt], "tokens": out}


def train(name="stories15M", T=256, steps=18, lr=1e-3):
    cfg = pa.STORIES[name]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    tokens = pa.seed_tokens(pa.SEED_TRAIN, T, cfg[5])
    L = ref_lib()
    ctx = L.ref_ctx_new(blob.ctypes.data_as(ctypes.c_void_p), T)
    losses = []
    for s in range(steps):
        losses.append(float(L.ref_train_step(ctx, tokens.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), T, lr)))
        print("train step", s, losses[-1], flush=True)
    L.ref_ctx_free(ctx)
    return {"config": name, "model_seed": pa.SEED_MODEL[name], "blob_sha256": blob_digest(pa.synth_model(cfg, pa.SEED_MODEL[name])),
            "T": T, "lr": lr, "train_seed": pa.SEED_TRAIN, "losses": losses}


LOGIT_POSITIONS = {"stories15M": [0, 7, 63, 64, 127, 128, 191, 255],
                   "stories42M": [7, 127, 128, 511, 512, 1023],
                   "stories110M": [7, 127, 128, 511, 512, 1023]}
N_TOP, N_SPOT, SPOT_SEED = 16, 16, 77


def logits(name):
    """Teacher-forced decode through the reference build: the input at
    position p is the golden token chosen after p-1 (prompt[0] at p = 0)."""
    fx = json.load(open(os.path.join(HERE, f"decode_{name}.json")))
    cfg = pa.STORIES[name]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    assert blob_digest(blob) == fx["blob_sha256"]
    L = ref_lib()
    L.ref_logits.restype = ctypes.POINTER(ctypes.c_float)
    L.ref_logits.argtypes = [ctypes.c_void_p]
    ctx = L.ref_ctx_new(blob.ctypes.data_as(ctypes.c_void_p), 0)
    V = cfg[5]
    spot = np.random.default_rng(SPOT_SEED).choice(V, N_SPOT, replace=False)
    want = set(LOGIT_POSITIONS[name])
    rows = []
    for pos in range(max(want) + 1):
        tok = fx["prompt"][0] if pos == 0 else fx["tokens"][pos - 1]
        L.ref_forward_step(ctx, tok)
        if pos not in want:
            continue
        lg = np.ctypeslib.as_array(L.ref_logits(ctx), shape=(V,)).copy()
        order = np.argsort(-lg, kind="stable")[:N_TOP]
        lg64 = lg.astype(np.float64)
        rows.append({"pos": pos, "input": int(tok), "top_ids": [int(i) for i in order],
                     "top_logits": [float(lg[i]) for i in order], "spot_ids": [int(i) for i in spot],
                     "spot_logits": [float(lg[i]) for i in spot], "max_abs": float(np.max(np.abs(lg))),
                     "margin": float(lg[order[0]] - lg[order[1]]), "sum": float(lg64.sum()),
                     "sumsq": float((lg64 * lg64).sum())})
        print(name, "logits at", pos, flush=True)
    L.ref_ctx_free(ctx)
    return {"config": name, "blob_sha256": fx["blob_sha256"], "positions": rows}


TRACE_CFG = (64, 160, 2, 4, 4, 1024, 32)     # V >= 4*D + 3*H: the reference's w_transpose (pt_train.c:405-407)
TRACE_SEED, TRACE_TOK_SEED, TRACE_T, TRACE_LR = 31, 32, 16, 0.05


def trace():
    from tests._oracle import Trace, ref, trace_spans
    R = ref()
    blob = pa.synth_model(TRACE_CFG, TRACE_SEED, 0.05)
    tokens = pa.seed_tokens(TRACE_TOK_SEED, TRACE_T, TRACE_CFG[5])
    ctx = R.ref_ctx_new(blob.ctypes.data_as(ctypes.c_void_p), TRACE_T)
    R.ref_enable_trace(ctx)
    R.ref_train_step(ctx, tokens.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), TRACE_T, TRACE_LR)
    tr = ctypes.cast(R.ref_trace(ctx), ctypes.POINTER(Trace)).contents
    spans = trace_spans(tr)
    R.ref_ctx_free(ctx)
    return {"config": list(TRACE_CFG), "model_seed": TRACE_SEED, "token_seed": TRACE_TOK_SEED, "T": TRACE_T,
            "lr": TRACE_LR, "spans": [list(sp) for sp in spans]}


def main(args):
    jobs = args or ["decode15", "decode42", "decode110", "train15", "trace", "logits15", "logits42", "logits110"]
    for j in jobs:
        if j == "trace":
            res = trace()
            path = os.path.join(HERE, "trace_spans.json")
        elif j.startswith("logits"):
            name = {"logits15": "stories15M", "logits42": "stories42M", "logits110": "stories110M"}[j]
            res = logits(name)
            path = os.path.join(HERE, f"logits_{name}.json")
        elif j.startswith("decode"):
            name = {"decode15": "stories15M", "decode42": "stories42M", "decode110": "stories110M"}[j]
            res = decode(name)
            path = os.path.join(HERE, f"decode_{name}.json")
        else:
            res = train()
            path = os.path.join(HERE, "train_stories15M.json")
        with open(path, "w") as f:
            json.dump(res, f)
        print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1:])
