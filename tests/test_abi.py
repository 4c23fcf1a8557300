"""C-ABI surface checks (CPU only: loading and symbol export, no compute)."""
import ctypes
import hashlib
import json
import os
import re

import numpy as np
import pytest

import pitorch_amd as pa
from tests._oracle import P, oracle, ref, ref_available

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared(header):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pt[a-z]*_[a-z0-9_]+)\s*\(", text)))


def test_libptmi_exports_every_declared_symbol():
    L = pa.load_ptmi()
    names = [n for n in declared(os.path.join(ROOT, "include", "ptmi.h")) if n.startswith("ptmi_")]
    assert len(names) >= 29
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_libpthost_exports_every_declared_symbol():
    H = ctypes.CDLL(os.path.join(pa.lib_dir(), "libpthost.so"))
    names = [n for n in declared(os.path.join(ROOT, "pitorch_amd", "host", "pt.h")) if n.startswith("pt_")]
    missing = [n for n in names if not hasattr(H, n)]
    assert not missing, missing


def test_no_gpu_is_an_error_not_a_fallback():
    """Without a device the library reports PTMI_ERR_NODEV; it never computes
    on the CPU."""
    L = pa.load_ptmi()
    st = L.ptmi_init(0)
    if st == 0:
        pytest.skip("a GPU is visible here")
    assert st == 5
    assert b"no HIP device" in L.ptmi_last_error()
    W = np.ones((4, 4), np.float32)
    y = np.zeros(4, np.float32)
    assert L.ptmi_matvec_checked(P(W), P(W[0]), P(y), 4, 4) == 5
    with pytest.raises(pa.PtmiError):
        pa.matvec(W, W[0])


def test_file_size_and_layout_agree_with_reference():
    for name, cfg in pa.STORIES.items():
        blob = pa.synth_model(cfg[:6] + (8,), 1) if name != "stories15M" else pa.synth_model(cfg, 1)
        H = pa.load_host()
        n = int(H.pt_file_size(P(blob)))
        assert n == blob.nbytes == oracle().po_file_size(P(blob))
        if ref_available():
            assert ref().pt_file_size(P(blob)) == n


def test_synthetic_model_is_deterministic_and_matches_fixture():
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", "decode_stories15M.json")))
    blob = pa.synth_model(pa.STORIES["stories15M"], pa.SEED_MODEL["stories15M"])
    assert hashlib.sha256(blob.tobytes()).hexdigest() == fx["blob_sha256"]
    w = np.frombuffer(blob.tobytes(), np.float32, offset=28)
    D, V = 288, 32000
    emb = w[: V * D]
    assert abs(emb.std() - 0.02) < 2e-4 and abs(emb.mean()) < 1e-4
    assert np.all(w[V * D: V * D + 6 * D] == 1.0)     # rms_att = 1
    assert list(pa.seed_tokens(pa.SEED_PROMPT, pa.N_PROMPT, V)) == fx["prompt"]
