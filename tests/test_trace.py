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
