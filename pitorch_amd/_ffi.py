"""ctypes bindings for libptmi (include/ptmi.h) and libpthost (host/pt.h)."""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_c_float_p = ctypes.POINTER(ctypes.c_float)
_c_int_p = ctypes.POINTER(ctypes.c_int)
_vp = ctypes.c_void_p


class Span(ctypes.Structure):
    """ptmi_span_t (include/ptmi.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("cat", ctypes.c_char_p), ("layer", ctypes.c_int),
                ("depth", ctypes.c_int), ("start_us", ctypes.c_double), ("dur_us", ctypes.c_double)]


def lib_dir():
    return os.path.join(_HERE, "lib")


class PtmiError(RuntimeError):
    def __init__(self, status, msg):
        super().__init__(f"ptmi status {status}: {msg}")
        self.status = status


_ptmi = None
_host = None


def _sig(lib, name, res, args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = args
    return fn


def load_ptmi():
    """Load libptmi.so; raises if it has not been built."""
    global _ptmi
    if _ptmi is not None:
        return _ptmi
    path = os.path.join(lib_dir(), "libptmi.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} missing: run `python -c 'import __graft_entry__ as g; g.build()'`")
    L = ctypes.CDLL(path)
    i, f, sz = ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    _sig(L, "ptmi_init", i, [i])
    _sig(L, "ptmi_shutdown", None, [])
    _sig(L, "ptmi_last_error", ctypes.c_char_p, [])
    _sig(L, "ptmi_last_status", i, [])
    _sig(L, "ptmi_stream", _vp, [])
    _sig(L, "ptmi_sync", i, [])
    _sig(L, "ptmi_register_weights", i, [_vp, sz])
    _sig(L, "ptmi_invalidate", i, [_vp, sz])
    _sig(L, "ptmi_unregister_weights", i, [_vp])
    _sig(L, "ptmi_register_buffer", i, [_vp, sz])
    _sig(L, "ptmi_unregister_buffer", i, [_vp])
    _sig(L, "ptmi_matvec", None, [_vp, _vp, _vp, i, i])
    _sig(L, "ptmi_matvec_checked", i, [_vp, _vp, _vp, i, i])
    _sig(L, "ptmi_matvec_dev", i, [_vp, ctypes.c_long, _vp, _vp, i, i, _vp])
    _sig(L, "ptmi_matvec_dev_xreread", i, [_vp, ctypes.c_long, _vp, _vp, i, i, _vp])
    _sig(L, "ptmi_sgemm_rect", i, [_vp, _vp, _vp, i, i, i, i])
    _sig(L, "ptmi_sgemm_rect_tmu", None, [_vp, _vp, _vp, i, i, i, i, i])
    _sig(L, "ptmi_sgemm_cpu", None, [_vp, _vp, _vp, i, i, i])
    _sig(L, "ptmi_matmul_backward_weight_batched", None, [_vp, _vp, _vp, i, i, i])
    _sig(L, "ptmi_matmul_backward_weight_batched_checked", i, [_vp, _vp, _vp, i, i, i])
    _sig(L, "ptmi_matmul_backward_input_batched", i, [_vp, _vp, _vp, i, i, i, i])
    _sig(L, "ptmi_gemm_dev", i, [i, _vp, ctypes.c_long, _vp, ctypes.c_long, _vp, ctypes.c_long,
                                 i, i, i, i, _vp])
    _sig(L, "ptmi_gemm_dev_noalloc", i, [i, _vp, ctypes.c_long, _vp, ctypes.c_long, _vp, ctypes.c_long,
                                         i, i, i, i, _vp])
    _sig(L, "ptmi_model_create", i, [_vp, sz, i, ctypes.POINTER(_vp)])
    _sig(L, "ptmi_model_destroy", None, [_vp])
    _sig(L, "ptmi_model_config", i, [_vp, _c_int_p])
    _sig(L, "ptmi_model_reset_kv", i, [_vp])
    _sig(L, "ptmi_model_forward_step", i, [_vp, i, _c_int_p])
    _sig(L, "ptmi_model_logits", i, [_vp, _c_float_p])
    _sig(L, "ptmi_model_pos", i, [_vp])
    _sig(L, "ptmi_model_generate", i, [_vp, _c_int_p, i, i, i, _c_int_p, _c_int_p])
    _sig(L, "ptmi_model_decode_async", i, [_vp, i, i])
    _sig(L, "ptmi_model_sync", i, [_vp])
    _sig(L, "ptmi_model_profile", i, [_vp, i, i, _c_float_p, _c_int_p])
    _sig(L, "ptmi_model_step_stamps", i, [_vp, ctypes.POINTER(ctypes.c_uint64), sz, _c_int_p, _c_int_p])
    _sig(L, "ptmi_decode_step_plan", i, [_c_int_p, i, i, _c_int_p, _c_int_p, _c_int_p])
    _sig(L, "ptmi_model_step_plan", i, [_vp])
    _sig(L, "ptmi_model_train_step", i, [_vp, _c_int_p, i, f, _c_float_p])
    _sig(L, "ptmi_model_train_step_trace", i,
         [_vp, _c_int_p, i, f, _c_float_p, ctypes.POINTER(Span), i, ctypes.POINTER(i)])
    _sig(L, "ptmi_model_read_weights", i, [_vp, _vp, sz])
    _sig(L, "ptmi_model_read_grads", i, [_vp, _c_float_p, sz])
    _ptmi = L
    return L


def load_host():
    """Load libpthost.so (the C host layer); raises if not built."""
    global _host
    if _host is not None:
        return _host
    load_ptmi()
    path = os.path.join(lib_dir(), "libpthost.so")
    if not os.path.exists(path):
        raise RuntimeError(f"{path} missing: build first")
    H = ctypes.CDLL(path)
    u64 = ctypes.c_uint64
    _sig(H, "pt_synth_model_bytes", u64, [_c_int_p])
    _sig(H, "pt_synth_model", ctypes.c_int, [_c_int_p, u64, ctypes.c_float, _vp, u64])
    _sig(H, "pt_seed_tokens", None, [u64, ctypes.c_int, ctypes.c_int, _c_int_p])
    _sig(H, "pt_seed_uniform", None, [u64, u64, ctypes.c_float, ctypes.c_float, _c_float_p])
    _sig(H, "pt_file_size", u64, [_vp])
    cp, i, u32, f = ctypes.c_char_p, ctypes.c_int, ctypes.c_uint32, ctypes.c_float
    _sig(H, "pt_trace_size", ctypes.c_size_t, [])
    _sig(H, "pt_trace_init", None, [_vp])
    _sig(H, "pt_trace_begin", None, [_vp, cp, cp, i])
    _sig(H, "pt_trace_end", None, [_vp])
    _sig(H, "pt_trace_reset", None, [_vp])
    _sig(H, "pt_trace_add", None, [_vp, cp, cp, i, i, u32, u32])
    _sig(H, "pt_time_us", u32, [])
    _sig(H, "pt_trace_write_json", None, [_vp, cp])
    _sig(H, "pt_trace_write_meta", None, [cp, cp, cp, i, i, i, cp, i, i, f, f, f, cp])
    _host = H
    return H


def check(status):
    if status != 0:
        L = load_ptmi()
        raise PtmiError(status, L.ptmi_last_error().decode(errors="replace"))


def _ptr(a):
    return a.ctypes.data_as(_vp)


def model_bytes(cfg):
    H = load_host()
    c = (ctypes.c_int * 7)(*cfg)
    return int(H.pt_synth_model_bytes(c))


def synth_model(cfg, seed, std=0.02):
    """llama2.c .bin blob (numpy uint8) with N(0, std) weights from seed."""
    H = load_host()
    c = (ctypes.c_int * 7)(*cfg)
    n = int(H.pt_synth_model_bytes(c))
    blob = np.zeros(n, dtype=np.uint8)
    st = H.pt_synth_model(c, seed, std, _ptr(blob), n)
    if st:
        raise PtmiError(st, "pt_synth_model failed")
    return blob


def decode_step_plan(cfg, cus, per_cu):
    """ptmi_decode_step_plan for a 7-int model shape: (reason, grid, units);
    reason 0 = one kernel, 1 = shape not supported, 2 = grid not resident."""
    L = load_ptmi()
    c = (ctypes.c_int * 7)(*cfg)
    reason, grid, units = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    check(L.ptmi_decode_step_plan(c, int(cus), int(per_cu), ctypes.byref(reason), ctypes.byref(grid),
                                  ctypes.byref(units)))
    return reason.value, grid.value, units.value


def seed_tokens(seed, n, vocab):
    H = load_host()
    out = np.zeros(n, dtype=np.int32)
    H.pt_seed_tokens(seed, n, vocab, out.ctypes.data_as(_c_int_p))
    return out


def seed_uniform(seed, n, lo=-1.0, hi=1.0):
    H = load_host()
    out = np.zeros(n, dtype=np.float32)
    H.pt_seed_uniform(seed, n, lo, hi, out.ctypes.data_as(_c_float_p))
    return out


def matvec(W, x):
    """y = W @ x through the pt_matvec_fn drop-in (host arrays)."""
    L = load_ptmi()
    W = np.ascontiguousarray(W, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(W.shape[0], dtype=np.float32)
    check(L.ptmi_matvec_checked(_ptr(W), _ptr(x), _ptr(y), W.shape[0], W.shape[1]))
    return y


class Model:
    """Device-resident model over a llama2.c blob (numpy uint8 array).

    The blob must stay alive and unmoved while the model exists: libptmi
    resolves host pointers into it (pt_matvec_fn drop-in).
    """

    def __init__(self, blob, max_T=0):
        self.L = load_ptmi()
        self.blob = blob
        h = _vp()
        check(self.L.ptmi_model_create(_ptr(blob), blob.nbytes, max_T, ctypes.byref(h)))
        self.h = h
        cfg = (ctypes.c_int * 7)()
        check(self.L.ptmi_model_config(self.h, cfg))
        self.cfg = tuple(cfg)

    @property
    def vocab(self):
        return self.cfg[5]

    def close(self):
        if self.h:
            # the model's hold on the blob's registration ends here
            self.L.ptmi_model_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset_kv(self):
        check(self.L.ptmi_model_reset_kv(self.h))

    def forward_step(self, token):
        nxt = ctypes.c_int()
        check(self.L.ptmi_model_forward_step(self.h, int(token), ctypes.byref(nxt)))
        return nxt.value

    def logits(self):
        out = np.empty(self.vocab, dtype=np.float32)
        check(self.L.ptmi_model_logits(self.h, out.ctypes.data_as(_c_float_p)))
        return out

    def pos(self):
        return self.L.ptmi_model_pos(self.h)

    def generate(self, prompt, max_tokens, stop_on_eos=True):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(max_tokens, 1), dtype=np.int32)
        n = ctypes.c_int()
        check(self.L.ptmi_model_generate(self.h, prompt.ctypes.data_as(_c_int_p), len(prompt), max_tokens,
                                         int(stop_on_eos), out.ctypes.data_as(_c_int_p), ctypes.byref(n)))
        return out[: n.value]

    def decode_async(self, first_token, n_steps):
        check(self.L.ptmi_model_decode_async(self.h, int(first_token), int(n_steps)))

    def sync(self):
        """Wait for the model's enqueued steps; raises if one timed out."""
        check(self.L.ptmi_model_sync(self.h))

    ROLES = ("qkv", "attention", "wo", "w13", "w2", "classifier", "argmax", "step")

    def profile(self, first_token, n_steps):
        """Per-role (total ms, launches) over n_steps eager decode steps
        ("step": the whole step as one kernel, when it runs that way)."""
        ms = (ctypes.c_float * 8)()
        cnt = (ctypes.c_int * 8)()
        check(self.L.ptmi_model_profile(self.h, int(first_token), int(n_steps), ms, cnt))
        return {r: (ms[i], cnt[i]) for i, r in enumerate(self.ROLES)}

    def step_plan(self):
        """Why this model's decode step runs as one kernel (0) or not: 1 shape
        not supported, 2 grid not resident at once, -1 multi-kernel forced."""
        return self.L.ptmi_model_step_plan(self.h)

    def step_stamps(self):
        """Stage stamps of the last one-kernel decode step (model created
        with PTMI_STEP_STAMPS=1): uint64 array [workgroups][stamps]."""
        ns, nw = ctypes.c_int(), ctypes.c_int()
        self.L.ptmi_model_step_stamps(self.h, None, 0, ctypes.byref(ns), ctypes.byref(nw))
        out = np.zeros((nw.value, ns.value), dtype=np.uint64)
        check(self.L.ptmi_model_step_stamps(self.h, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)), out.size,
                                            ctypes.byref(ns), ctypes.byref(nw)))
        return out

    def train_step(self, tokens, lr):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        loss = ctypes.c_float()
        check(self.L.ptmi_model_train_step(self.h, tokens.ctypes.data_as(_c_int_p), len(tokens), lr,
                                           ctypes.byref(loss)))
        return loss.value

    def train_step_trace(self, tokens, lr, max_spans=4096):
        """The same step with its device-timed spans
        (ptmi_model_train_step_trace): (loss, [dict(name, cat, layer, depth,
        start_us, dur_us)]) in the order the spans end."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        loss = ctypes.c_float()
        buf = (Span * max_spans)()
        n = ctypes.c_int()
        check(self.L.ptmi_model_train_step_trace(self.h, tokens.ctypes.data_as(_c_int_p), len(tokens), lr,
                                                 ctypes.byref(loss), buf, max_spans, ctypes.byref(n)))
        spans = [dict(name=s.name.decode(), cat=s.cat.decode(), layer=s.layer, depth=s.depth,
                      start_us=s.start_us, dur_us=s.dur_us) for s in buf[:n.value]]
        return loss.value, spans

    def read_weights(self):
        out = np.empty_like(self.blob)
        check(self.L.ptmi_model_read_weights(self.h, _ptr(out), out.nbytes))
        return out

    def read_grads(self, n):
        out = np.empty(n, dtype=np.float32)
        check(self.L.ptmi_model_read_grads(self.h, out.ctypes.data_as(_c_float_p), n))
        return out
