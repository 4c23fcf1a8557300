"""GPU parity of the device-resident decode step (pt_forward_step drop-in).

Golden tokens come from the reference's own host build (tests/golden/
make_golden.py).  Greedy tokens must be IDENTICAL over the full runs
(256 positions for 15M, 1024 for 42M/110M); logits are compared with the
oracle at a relative tolerance (matvec reduction order differs).

Every decode path is held to this: the one-kernel step (the default for
every shape it supports), the captured multi-kernel step (PTMI_DECODE_STEP=0,
and the shapes the one kernel does not take; PTMI_DECODE_STEP is read when
a model is created) and the one kernel cut into launch windows
(PTMI_STEP_SPLIT).
"""
import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

import pitorch_amd as pa
from tests._oracle import OracleModel, P, greedy_tokens, ref, ref_available

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(params=["multi_kernel", "one_kernel", "windows"])
def decode_path(request, monkeypatch):
    """The captured multi-kernel step, the one-kernel step, and the
    one-kernel step cut into two launches per layer (PTMI_STEP_SPLIT=qo)."""
    monkeypatch.setenv("PTMI_DECODE_STEP", "0" if request.param == "multi_kernel" else "1")
    monkeypatch.setenv("PTMI_STEP_SPLIT", "qo" if request.param == "windows" else "")
    return request.param


def check_path(m, decode_path):
    """The model ran the decode path the test was parametrized for (one
    profiled step from position 0: "step" launches only on the one-kernel
    path, one per launch window of PTMI_STEP_SPLIT)."""
    m.reset_kv()
    prof = m.profile(1, 1)
    assert (prof["step"][1] >= 1) == (decode_path != "multi_kernel"), prof["step"]


def fixture(name):
    return json.load(open(os.path.join(ROOT, "tests", "golden", f"decode_{name}.json")))


def model_for(name):
    blob = pa.synth_model(pa.STORIES[name], pa.SEED_MODEL[name])
    assert hashlib.sha256(blob.tobytes()).hexdigest() == fixture(name)["blob_sha256"], \
        "synthetic model generator drifted on this host"
    return blob


def test_logits_track_oracle_15M(decode_path):
    """Every one of the 256 positions (4 attention chunks of 64 positions,
    so the multi-chunk softmax combine runs from position 64 on): logits
    within 1e-5 of max |logit| of the oracle's, same argmax."""
    blob = model_for("stories15M")
    m = pa.Model(blob)
    om = OracleModel(blob.copy())
    prompt = fixture("stories15M")["prompt"]
    tok = prompt[0]
    worst = 0.0
    for pos in range(256):
        a = m.forward_step(tok)
        b = om.forward_step(tok)
        lg, ref_lg = m.logits(), om.logits()
        err = np.max(np.abs(lg - ref_lg)) / np.max(np.abs(ref_lg))
        worst = max(worst, err)
        assert err < 1e-5, (pos, err)
        assert a == b == int(np.argmax(ref_lg))
        tok = prompt[pos + 1] if pos + 1 < len(prompt) else a
    assert m.pos() == 256
    check_path(m, decode_path)
    m.close()
    om.close()


@pytest.mark.parametrize("name", ["stories15M", "stories42M", "stories110M"])
def test_long_context_logits_match_reference(name, decode_path):
    """Logits at positions across the attention chunks (128 positions per
    chunk at seq_len 1024: 127 | 128 on either side of a chunk boundary,
    511/512, the full cache at 1023), teacher-forced on the golden tokens,
    against the reference build's (tests/golden/logits_<config>.json):
    every recorded logit (top 16, 16 seeded ids) within 1e-5 of max
    |logit|, the same argmax, and the fp64 sum / norm of all logits within
    1e-5 relative of the reference's."""
    fx = json.load(open(os.path.join(ROOT, "tests", "golden", f"logits_{name}.json")))
    golden = fixture(name)
    m = pa.Model(model_for(name))
    rows = {r["pos"]: r for r in fx["positions"]}
    for pos in range(max(rows) + 1):
        tok = golden["prompt"][0] if pos == 0 else golden["tokens"][pos - 1]
        m.forward_step(tok)
        if pos not in rows:
            continue
        r = rows[pos]
        lg = m.logits()
        tol = 1e-5 * r["max_abs"]
        for ids, vals in ((r["top_ids"], r["top_logits"]), (r["spot_ids"], r["spot_logits"])):
            err = np.max(np.abs(lg[np.array(ids)] - np.array(vals, np.float32)))
            assert err <= tol, (pos, err, tol)
        assert int(np.argmax(lg)) == r["top_ids"][0], pos
        assert abs(float(np.max(np.abs(lg))) - r["max_abs"]) <= tol
        lg64 = lg.astype(np.float64)
        norm, ref_norm = np.sqrt((lg64 * lg64).sum()), np.sqrt(r["sumsq"])
        assert abs(norm - ref_norm) <= 1e-5 * ref_norm, pos
        assert abs(lg64.sum() - r["sum"]) <= 1e-5 * np.sqrt(len(lg)) * ref_norm, pos
    check_path(m, decode_path)
    m.close()


@pytest.mark.parametrize("name", ["stories15M", "stories42M", "stories110M"])
def test_greedy_tokens_identical_to_reference(name, decode_path):
    fx = fixture(name)
    blob = model_for(name)
    m = pa.Model(blob)
    toks = m.generate(np.array(fx["prompt"], np.int32), pa.DECODE_POSITIONS[name], stop_on_eos=False)
    assert len(toks) == len(fx["tokens"])
    first_diff = next((i for i, (a, b) in enumerate(zip(toks, fx["tokens"])) if a != b), None)
    assert first_diff is None, f"first divergence at position {first_diff}"
    check_path(m, decode_path)
    m.close()


def test_forward_step_matches_generate_and_reset(decode_path):
    fx = fixture("stories15M")
    blob = model_for("stories15M")
    m = pa.Model(blob)
    toks = greedy_tokens(m.forward_step, fx["prompt"], 64)
    assert toks == fx["tokens"][:64]
    m.reset_kv()
    assert m.pos() == 0
    assert greedy_tokens(m.forward_step, fx["prompt"], 16) == fx["tokens"][:16]
    check_path(m, decode_path)
    m.close()


def test_generate_stop_and_clamp_semantics(decode_path):
    """pt_text.c:321-322 clamp, :344-347 forced prefill, :354 stop on 1/2."""
    cfg = (64, 160, 2, 4, 4, 512, 24)
    blob = pa.synth_model(cfg, 5, 0.3)
    om = OracleModel(blob.copy())
    prompt = np.array([3, 9, 27, 81], np.int32)
    out = np.zeros(64, np.int32)
    n = om.L.po_generate_greedy(om.h, prompt.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), 4, 100,
                                out.ctypes.data_as(ctypes.POINTER(ctypes.c_int)))
    m = pa.Model(blob)
    got = m.generate(prompt, 100, stop_on_eos=True)
    assert list(got) == list(out[:n])
    check_path(m, decode_path)
    m.close()
    om.close()


def test_argmax_keeps_index_0_when_first_logit_is_nan(decode_path):
    """pt_ops.c:65-70 starts from index 0 and no comparison with NaN is true:
    a classifier whose row 0 yields NaN makes every next token 0, while NaNs
    elsewhere never win.  Untied classifier (llama2.c's unshared layout) with
    row 0 and row 7 NaN; tokens against the oracle's."""
    from tests.test_gpu_train import untie
    cfg = (64, 160, 1, 4, 4, 512, 16)
    V, D = cfg[5], cfg[0]
    blob = untie(pa.synth_model(cfg, 7, 0.05), cfg, 8)
    w = blob[28:].view(np.float32)
    w[w.size - V * D: w.size - V * D + D] = np.nan          # wcls row 0
    w[w.size - V * D + 7 * D: w.size - V * D + 8 * D] = np.nan
    m = pa.Model(blob)
    om = OracleModel(blob.copy())
    tok = 5
    for _ in range(4):
        a, b = m.forward_step(tok), om.forward_step(tok)
        assert a == b == 0
        assert np.isnan(m.logits()[0]) and np.isnan(m.logits()[7])
        tok = a
    check_path(m, decode_path)
    m.close()
    om.close()


def test_errors_are_reported():
    cfg = (64, 160, 1, 4, 4, 512, 8)
    blob = pa.synth_model(cfg, 6)
    m = pa.Model(blob)
    with pytest.raises(pa.PtmiError):
        m.forward_step(512)                       # token out of range
    for _ in range(8):
        m.forward_step(1)
    with pytest.raises(pa.PtmiError) as e:
        m.forward_step(1)                         # KV cache full
    assert "seq_len" in str(e.value)
    with pytest.raises(pa.PtmiError):
        m.decode_async(1, 1)
    m.close()


@pytest.mark.skipif(not ref_available(), reason="oracle/_ref not built")
def test_reference_forward_with_ptmi_matvec_dropin():
    """The reference's own pt_forward_step (pitorch/pt.c:267-271) with
    ctx->matvec = ptmi_matvec, the drop-in binding a pitorch caller adds."""
    fx = fixture("stories15M")
    blob = model_for("stories15M")
    L = pa.load_ptmi()
    assert L.ptmi_register_weights(P(blob), blob.nbytes) == 0
    R = ref()
    ctx = R.ref_ctx_new(P(blob), 0)
    fn = ctypes.cast(L.ptmi_matvec, ctypes.c_void_p)
    R.ref_set_matvec(ctx, fn)
    try:
        toks = greedy_tokens(lambda t: R.ref_forward_step(ctx, t), fx["prompt"], 48)
        assert toks == fx["tokens"][:48]
    finally:
        R.ref_ctx_free(ctx)
        L.ptmi_unregister_weights(P(blob))


@pytest.mark.parametrize("mode", ["graph", "one_kernel", "split_qo", "split_qaofdc"])
def test_profile_roles_cover_every_launch(mode, monkeypatch):
    """The one-kernel step is one launch per token (role "step"), or one per
    launch window when PTMI_STEP_SPLIT cuts it before chosen stages of every
    layer; the multi-kernel step (PTMI_DECODE_STEP=0) is 5 launches per layer
    plus the classifier and the argmax."""
    monkeypatch.setenv("PTMI_DECODE_STEP", "0" if mode == "graph" else "1")
    split = mode[len("split_"):] if mode.startswith("split_") else ""
    monkeypatch.setenv("PTMI_STEP_SPLIT", split)
    cfg = pa.STORIES["stories15M"]
    blob = model_for("stories15M")
    m = pa.Model(blob)
    prof = m.profile(1, 4)
    Lyr = cfg[2]
    if mode != "graph":
        per_layer = sum(c in split for c in "qaofd")
        windows = 1 + per_layer * Lyr - ("q" in split) + ("c" in split)
        assert prof["step"][1] == 4 * windows and prof["step"][0] > 0
        assert all(cnt == 0 for r, (ms, cnt) in prof.items() if r != "step")
    else:
        assert prof["qkv"][1] == prof["attention"][1] == prof["wo"][1] == prof["w13"][1] == prof["w2"][1] == 4 * Lyr
        assert prof["classifier"][1] == prof["argmax"][1] == 4 and prof["step"][1] == 0
        assert all(ms > 0 for r, (ms, _) in prof.items() if r != "step")
    m.close()


def test_default_path_by_model_size(monkeypatch):
    """Without PTMI_DECODE_STEP the one-kernel step serves every shape it
    supports (stories15M, and a one-layer model of stories110M's widths);
    a shape it does not take (head_dim 128) gets the multi-kernel step."""
    monkeypatch.delenv("PTMI_DECODE_STEP", raising=False)
    monkeypatch.delenv("PTMI_STEP_SPLIT", raising=False)
    for cfg, one_kernel in [(pa.STORIES["stories15M"], True), ((768, 2048, 1, 12, 12, 512, 64), True),
                            ((256, 512, 1, 2, 2, 512, 64), False)]:
        m = pa.Model(pa.synth_model(cfg, 3))
        prof = m.profile(1, 1)
        assert (prof["step"][1] > 0) == one_kernel, (cfg, prof["step"])
        m.close()


def test_step_split_rejects_unknown_stage(monkeypatch):
    """PTMI_STEP_SPLIT takes only the stage letters q a o f d c."""
    monkeypatch.setenv("PTMI_DECODE_STEP", "1")
    monkeypatch.setenv("PTMI_STEP_SPLIT", "qx")
    with pytest.raises(pa.PtmiError):
        pa.Model(model_for("stories15M"))


def test_one_kernel_step_stage_stamps(monkeypatch):
    """PTMI_STEP_STAMPS=1: per workgroup, kernel start, then for every stage
    the end of its wait and the end of its work, in time order."""
    monkeypatch.setenv("PTMI_DECODE_STEP", "1")
    monkeypatch.setenv("PTMI_STEP_STAMPS", "1")
    cfg = pa.STORIES["stories15M"]
    m = pa.Model(model_for("stories15M"))
    m.forward_step(1)
    m.forward_step(5)
    st = m.step_stamps().astype(np.int64)
    L = cfg[2]
    assert st.shape[1] == 1 + 10 * L + 4 and st.shape[0] >= 64
    assert np.all(st[:, 0] > 0)
    for row in st:
        seen = row[row > 0]
        assert np.all(np.diff(seen) >= 0)          # a workgroup's stamps are in time order
    blocks_w13 = (2 * cfg[1] + 15) // 16            # 16 interleaved w1|w3 rows per workgroup pass
    took_w13 = st[:, 7 + 10 * (L - 1)] > 0
    assert took_w13.sum() == min(len(st), blocks_w13) and took_w13[:blocks_w13].all()
    assert st[0, 4 + 10 * L] > 0                   # workgroup 0 finished the step
    m.close()
    monkeypatch.setenv("PTMI_STEP_STAMPS", "0")
    m = pa.Model(model_for("stories15M"))
    with pytest.raises(pa.PtmiError):
        m.step_stamps()
    m.close()


def test_one_kernel_step_timeout_is_reported(monkeypatch):
    """A wait of the one-kernel step that runs out is an error of the call,
    forced here from the host with a one-tick wait bound: the kernel still
    exits normally (every wait is bounded and checks the shared error word;
    later steps of the same graph see the word and do nothing), the call
    raises, and the model stays usable for the next call."""
    monkeypatch.setenv("PTMI_DECODE_STEP", "1")
    monkeypatch.setenv("PTMI_STEP_WAIT_TICKS", "1")
    m = pa.Model(model_for("stories15M"))
    for _ in range(2):
        with pytest.raises(pa.PtmiError) as e:
            m.forward_step(1)
        assert "timed out" in str(e.value)
    with pytest.raises(pa.PtmiError):
        m.generate(np.array([1, 2, 3], np.int32), 8, stop_on_eos=False)
    # decode_async defers its errors to the next synchronising call
    m.reset_kv()
    m.decode_async(1, 4)
    with pytest.raises(pa.PtmiError) as e:
        m.sync()
    assert "timed out" in str(e.value)
    m.sync()                                        # reported once, then clear
    m.close()
    monkeypatch.delenv("PTMI_STEP_WAIT_TICKS")
    fx = fixture("stories15M")
    m = pa.Model(model_for("stories15M"))
    assert greedy_tokens(m.forward_step, fx["prompt"], 16) == fx["tokens"][:16]
    m.close()


def _oracle_decode(blob, n, prompt, paths=("0", "1")):
    """Greedy decode of n positions on each decode path against the oracle:
    tokens identical, logits within 1e-5 of max |logit| at every position.
    Returns the models' step plans."""
    plans = []
    for path in paths:
        os.environ["PTMI_DECODE_STEP"] = path
        try:
            m = pa.Model(blob)
        finally:
            os.environ.pop("PTMI_DECODE_STEP")
        plans.append(m.step_plan())
        om = OracleModel(blob.copy())
        tok = prompt[0]
        for pos in range(n):
            a, b = m.forward_step(tok), om.forward_step(tok)
            lg, ref_lg = m.logits(), om.logits()
            err = np.max(np.abs(lg - ref_lg)) / np.max(np.abs(ref_lg))
            assert err < 1e-5 and a == b, (path, pos, err, a, b)
            tok = prompt[pos + 1] if pos + 1 < len(prompt) else a
        m.close()
        om.close()
    return plans


def test_step_kernel_for_dim_256_matches_oracle():
    """dim 256 with head_dim 64 (4 heads), hidden 512, 64 positions: the
    shape that selects the one-kernel step's smallest multi-chunk
    instantiation (2 float4 per lane of a dim row, 2 of a hidden row, 2
    attention units of 32 positions per head).  Both decode paths, every
    position, against the oracle."""
    cfg = (256, 512, 2, 4, 4, 512, 64)
    blob = pa.synth_model(cfg, 7)
    prompt = [int(t) for t in pa.seed_tokens(5, 8, cfg[5])]
    assert _oracle_decode(blob, 64, prompt) == [-1, 0]


def test_step_merge_reads_only_the_records_it_polled():
    """A head's chunk-0 merge takes the statistics of the head's active
    chunks only.  With PTMI_STEP_POISON_LDS=1 every workgroup starts with
    its chunk-record LDS full of NaN, so a merge that let an inactive
    chunk's (unpolled) record into its sums would give NaN logits.
    stories15M shape, all 256 positions (8 units of 32 per head, 1 to 8
    active), against the oracle."""
    name = "stories15M"
    cfg = pa.STORIES[name]
    blob = pa.synth_model(cfg, pa.SEED_MODEL[name])
    prompt = [int(t) for t in pa.seed_tokens(pa.SEED_PROMPT, pa.N_PROMPT, cfg[5])]
    os.environ["PTMI_STEP_POISON_LDS"] = "1"
    try:
        assert _oracle_decode(blob, 256, prompt, paths=("1",)) == [0]
    finally:
        os.environ.pop("PTMI_STEP_POISON_LDS")


def test_wrapped_attention_units_take_the_multi_kernel_step():
    """48 heads of 16 over 1024 positions make 384 attention units, more
    than the 256 workgroups of the one-kernel step: the plan refuses it (a
    head's chunk-0 unit could wait behind another merge on its own
    workgroup), and the model decodes on the multi-kernel step, matching
    the oracle past position 896 where all eight chunks are active."""
    cfg = (768, 2048, 1, 48, 48, 512, 1024)
    blob = pa.synth_model(cfg, 9)
    prompt = [int(t) for t in pa.seed_tokens(6, 8, cfg[5])]
    assert pa.decode_step_plan(cfg, 256, 1)[0] == 2
    assert _oracle_decode(blob, 920, prompt, paths=("1",)) == [2]


def test_grouped_query_attention_is_refused():
    """n_kv_heads < n_heads is refused at model creation: the reference's
    rope() rotates k over dim floats while s->k holds kv_dim
    (pitorch/ops/core/pt_ops.c:33-49, pitorch/model/llama2.c:81,147), so
    it has no defined result to match."""
    blob = pa.synth_model((256, 512, 1, 4, 2, 512, 64), 3)
    with pytest.raises(pa.PtmiError) as e:
        pa.Model(blob)
    assert "grouped-query" in str(e.value)


def test_step_plan_of_the_stories_models(monkeypatch):
    """On the MI355X every stories model runs the one-kernel step (plan 0);
    PTMI_DECODE_STEP=0 forces the multi-kernel step (plan -1)."""
    monkeypatch.delenv("PTMI_DECODE_STEP", raising=False)
    for name in pa.STORIES:
        m = pa.Model(model_for(name))
        assert m.step_plan() == 0, name
        m.close()
    monkeypatch.setenv("PTMI_DECODE_STEP", "0")
    m = pa.Model(model_for("stories15M"))
    assert m.step_plan() == -1
    m.close()
