"""The host trace API (pitorch/profiler/trace.h:21-101 restated in
pitorch_amd/host/pt_trace.c), on the CPU: struct layout, span nesting, the
L<layer>_<name> naming, Chrome-Tracing JSON ("ph": "X" complete events) and
meta.json, and the disabled / reset behaviour of trace.c:28-66."""
import ctypes
import json

import pitorch_amd as pa


class Ev(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("cat", ctypes.c_char_p), ("ts_us", ctypes.c_uint32),
                ("dur_us", ctypes.c_uint32), ("layer", ctypes.c_int8), ("depth", ctypes.c_int8),
                ("hw_cycles", ctypes.c_uint32), ("hw_stall", ctypes.c_uint32)]


class Frame(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("cat", ctypes.c_char_p), ("ts_us", ctypes.c_uint32),
                ("layer", ctypes.c_int8)]


class Trace(ctypes.Structure):
    _fields_ = [("events", Ev * 4096), ("count", ctypes.c_int), ("enabled", ctypes.c_int),
                ("stack", Frame * 32), ("depth", ctypes.c_int)]


def test_trace_layout_nesting_and_json(tmp_path):
    H = pa._ffi.load_host()
    assert ctypes.sizeof(Trace) == H.pt_trace_size()
    t = Trace()
    p = ctypes.byref(t)
    H.pt_trace_init(p)
    assert t.enabled == 1 and t.count == 0
    H.pt_trace_begin(p, b"train_step", b"train", -1)
    H.pt_trace_begin(p, b"layer", b"fwd", 0)
    H.pt_trace_begin(p, b"qkv", b"fwd", 0)
    H.pt_trace_end(p)
    H.pt_trace_end(p)
    H.pt_trace_end(p)
    H.pt_trace_end(p)                                 # unmatched end: ignored
    H.pt_trace_add(p, b"attention", b"bwd", 3, 1, 1000, 250)
    assert t.count == 4 and t.depth == 0
    assert [t.events[i].depth for i in range(3)] == [2, 1, 0]
    path = tmp_path / "trace.json"
    H.pt_trace_write_json(p, str(path).encode())
    ev = json.load(open(path))
    assert [e["name"] for e in ev] == ["L0_qkv", "L0_layer", "train_step", "L3_attention"]
    assert all(e["ph"] == "X" and e["pid"] == 0 and e["tid"] == 0 and "args" not in e for e in ev)
    assert [e["cat"] for e in ev] == ["fwd", "fwd", "train", "bwd"]
    q, lay, top = ev[0], ev[1], ev[2]
    for inner, outer in ((q, lay), (lay, top)):       # children lie inside their parents
        assert outer["ts"] <= inner["ts"] and inner["ts"] + inner["dur"] <= outer["ts"] + outer["dur"]
    assert ev[3]["ts"] == 1000 and ev[3]["dur"] == 250
    # disabled: every call is a no-op; reset empties the record
    t.enabled = 0
    H.pt_trace_begin(p, b"forward", b"fwd", -1)
    H.pt_trace_end(p)
    H.pt_trace_add(p, b"x", b"fwd", -1, 0, 0, 0)
    assert t.count == 4 and t.depth == 0
    t.enabled = 1
    H.pt_trace_reset(p)
    assert t.count == 0 and t.enabled == 1
    H.pt_trace_write_json(p, str(tmp_path / "empty.json").encode())     # nothing recorded: no file
    assert not (tmp_path / "empty.json").exists()
    H.pt_trace_write_meta(str(tmp_path / "meta.json").encode(), b"run", b"stories15M", 288, 6, 32000, b"mi355x",
                          0, 18, 1e-3, 10.25, 1.5, b"note")
    meta = json.load(open(tmp_path / "meta.json"))
    assert meta["dim"] == 288 and meta["layers"] == 6 and meta["steps"] == 18 and meta["device"] == "mi355x"
    assert abs(meta["final_loss"] - 10.25) < 1e-6 and meta["notes"] == "note"


def _filled_trace():
    """One event array covering every branch of trace.c's writer: layer -1
    and >= 0 names, zero and non-zero V3D counters (the "args" object),
    timestamps near the uint32 range."""
    t = Trace()
    rows = [(b"train_step", b"train", -1, 0, 10, 900, 0, 0), (b"qkv", b"fwd", 0, 2, 20, 35, 0, 0),
            (b"attention", b"fwd", 11, 2, 55, 70, 1234, 0), (b"ffn", b"bwd", 3, 2, 4000000000, 5, 0, 77),
            (b"cls_weight_grad", b"bwd", -1, 2, 4294967295, 0, 4294967295, 4294967295),
            (b"sgd", b"train", -1, 1, 0, 0, 1, 1)]
    for i, (n, c, layer, depth, ts, dur, cyc, stall) in enumerate(rows):
        e = t.events[i]
        e.name, e.cat, e.layer, e.depth, e.ts_us, e.dur_us, e.hw_cycles, e.hw_stall = n, c, layer, depth, ts, dur, cyc, stall
    t.count = len(rows)
    t.enabled = 1
    return t


def test_trace_writers_byte_identical_to_reference(tmp_path):
    """pt_trace_write_json / pt_trace_write_meta of libpthost against the
    reference's own trace.c (oracle/_ref), fed the same event array: the
    files must be byte-identical (pitorch/profiler/trace.c:73-120)."""
    import pytest
    from tests._oracle import ref, ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built")
    R, H = ref(), pa._ffi.load_host()
    assert R.ref_trace_size() == H.pt_trace_size() == ctypes.sizeof(Trace)
    t = _filled_trace()
    a, b = tmp_path / "ours.json", tmp_path / "ref.json"
    H.pt_trace_write_json(ctypes.byref(t), str(a).encode())
    R.pt_trace_write_json(ctypes.byref(t), str(b).encode())
    assert a.read_bytes() == b.read_bytes()
    assert len(json.loads(a.read_text())) == t.count
    for notes in (b"a note", None):
        args = (b"run", b"stories110M", 768, 12, 32000, b"mi355x", 0, 18, 1e-3, 10.310569, 1.25, notes)
        H.pt_trace_write_meta(str(a).encode(), *args)
        R.pt_trace_write_meta(str(b).encode(), *args)
        assert a.read_bytes() == b.read_bytes()


def test_span_fixture_is_the_reference_traced_step():
    """tests/golden/trace_spans.json is what the reference's own traced
    pt_train_step records (regenerated here from oracle/_ref)."""
    import os
    import sys

    import pytest
    from tests._oracle import ref_available
    if not ref_available():
        pytest.skip("oracle/_ref not built")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path.insert(0, os.path.join(root, "tests", "golden"))
    import make_golden
    fx = json.load(open(os.path.join(root, "tests", "golden", "trace_spans.json")))
    assert make_golden.trace() == fx
