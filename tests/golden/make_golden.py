"""Write the golden decode/training fixtures from the reference's own build.

Runs masonwang025/pitorch's host C path (oracle/_ref/libptref.so, built from
the reference sources by oracle/Makefile) on the seeded synthetic models of
the benchmark configurations:

* decode_tokens.json — pt_forward_step (pitorch/pt.c:267-271) greedy tokens:
  the 8 seeded prompt ids are forced at positions 0..6 (pt_text.c:344-347),
  argmax afterwards; 256 positions (15M) / 1024 (42M, 110M).
* train_losses.json — pt_train_step (pitorch/pt.c:339-364) losses, 15M,
  T=256 seeded ids, lr=1e-3, 18 steps.

Usage: python tests/golden/make_golden.py [decode15|decode42|decode110|train15 ...]
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


def main(args):
    jobs = args or ["decode15", "decode42", "decode110", "train15"]
    for j in jobs:
        if j.startswith("decode"):
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
