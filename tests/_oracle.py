"""ctypes access to the test oracle (oracle/libptoracle.so) and to the
reference's own host build (oracle/_ref/libptref.so).  Test-only."""
import ctypes
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
vp = ctypes.c_void_p
fp = ctypes.POINTER(ctypes.c_float)
ip = ctypes.POINTER(ctypes.c_int)
_o = None
_r = None


def P(a):
    return a.ctypes.data_as(vp)


def oracle():
    global _o
    if _o is not None:
        return _o
    L = ctypes.CDLL(os.path.join(ROOT, "oracle", "libptoracle.so"))
    f, i = ctypes.c_float, ctypes.c_int
    for n in ("po_expf", "po_logf", "po_sinf", "po_cosf", "po_sqrtf"):
        getattr(L, n).restype = f
        getattr(L, n).argtypes = [f]
    sigs = {
        "po_rmsnorm": (None, [vp, vp, vp, i]), "po_softmax": (None, [vp, i]), "po_silu": (None, [vp, i]),
        "po_rope": (None, [vp, vp, i, i, i]), "po_vec_add": (None, [vp, vp, vp, i]),
        "po_vec_mul": (None, [vp, vp, vp, i]), "po_embedding_lookup": (None, [vp, vp, i, i]),
        "po_argmax": (i, [vp, i]), "po_smatvec": (None, [vp, vp, vp, i, i]),
        "po_sgemm": (None, [vp, vp, vp, i, i, i]), "po_sgemm_rect": (None, [vp, vp, vp, i, i, i, i]),
        "po_matmul_backward_input": (None, [vp, vp, vp, i, i]),
        "po_matmul_backward_weight": (None, [vp, vp, vp, i, i]),
        "po_matmul_backward_weight_batched": (None, [vp, vp, vp, i, i, i]),
        "po_rmsnorm_backward": (None, [vp, vp, vp, vp, vp, i]),
        "po_rope_backward": (None, [vp, vp, vp, vp, i, i, i]),
        "po_softmax_backward": (None, [vp, vp, vp, i]), "po_silu_backward": (None, [vp, vp, vp, i]),
        "po_embedding_backward": (None, [vp, vp, i, i]),
        "po_file_size": (ctypes.c_uint64, [vp]), "po_model_new": (vp, [vp, i]), "po_model_free": (None, [vp]),
        "po_reset_kv": (None, [vp]), "po_forward_step": (i, [vp, i]), "po_forward": (None, [vp, i, i]),
        "po_logits": (fp, [vp]), "po_residual": (fp, [vp]), "po_pos": (i, [vp]),
        "po_generate_greedy": (i, [vp, ip, i, i, ip]),
        "po_forward_train": (f, [vp, ip, i]), "po_backward": (None, [vp, ip, i]),
        "po_sgd_update": (None, [vp, f]), "po_train_step": (f, [vp, ip, i, f]),
        "po_zero_grads": (None, [vp]), "po_grads": (fp, [vp, ip]),
        "po_train_logits": (fp, [vp]), "po_train_x_final": (fp, [vp]),
    }
    for n, (r, a) in sigs.items():
        getattr(L, n).restype = r
        getattr(L, n).argtypes = a
    _o = L
    return L


def ref_available():
    return os.path.exists(os.path.join(ROOT, "oracle", "_ref", "libptref.so"))


def ref():
    """The reference's own build; None when it was not built."""
    global _r
    if _r is not None:
        return _r
    if not ref_available():
        return None
    L = ctypes.CDLL(os.path.join(ROOT, "oracle", "_ref", "libptref.so"))
    f, i = ctypes.c_float, ctypes.c_int
    for n in ("pt_expf", "pt_logf", "pt_sinf", "pt_cosf", "pt_sqrtf"):
        getattr(L, n).restype = f
        getattr(L, n).argtypes = [f]
    sigs = {
        "rmsnorm": (None, [vp, vp, vp, i]), "softmax": (None, [vp, i]), "silu": (None, [vp, i]),
        "rope": (None, [vp, vp, i, i, i]), "argmax": (i, [vp, i]), "smatvec_cpu": (None, [vp, vp, vp, i, i]),
        "matmul_backward_input": (None, [vp, vp, vp, i, i]),
        "matmul_backward_weight": (None, [vp, vp, vp, i, i]),
        "matmul_backward_weight_batched": (None, [vp, vp, vp, i, i, i]),
        "rmsnorm_backward": (None, [vp, vp, vp, vp, vp, i]), "rope_backward": (None, [vp, vp, vp, vp, i, i, i]),
        "softmax_backward": (None, [vp, vp, vp, i]), "silu_backward": (None, [vp, vp, vp, i]),
        "pt_file_size": (ctypes.c_uint, [vp]),
        "ref_ctx_new": (vp, [vp, i]), "ref_ctx_free": (None, [vp]), "ref_set_matvec": (None, [vp, vp]),
        "ref_forward_step": (i, [vp, i]), "ref_reset_kv": (None, [vp]), "ref_logits": (fp, [vp]),
        "ref_train_step": (f, [vp, ip, i, f]), "ref_grads": (fp, [vp, ip]), "ref_train_logits": (fp, [vp]),
        "ref_train_step_then": (f, [vp, ip, i, f, vp, vp, ctypes.c_size_t]),
        "ref_enable_trace": (None, [vp]), "ref_trace": (vp, [vp]), "ref_trace_size": (ctypes.c_size_t, []),
        "pt_trace_write_json": (None, [vp, ctypes.c_char_p]),
        "pt_trace_write_meta": (None, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, i, i, i, ctypes.c_char_p,
                                       i, i, f, f, f, ctypes.c_char_p]),
    }
    for n, (r, a) in sigs.items():
        getattr(L, n).restype = r
        getattr(L, n).argtypes = a
    _r = L
    return L


class TraceEvent(ctypes.Structure):
    """pt_trace_event_t (pitorch/profiler/trace.h:24-33)."""
    _fields_ = [("name", ctypes.c_char_p), ("cat", ctypes.c_char_p), ("ts_us", ctypes.c_uint32),
                ("dur_us", ctypes.c_uint32), ("layer", ctypes.c_int8), ("depth", ctypes.c_int8),
                ("hw_cycles", ctypes.c_uint32), ("hw_stall", ctypes.c_uint32)]


class TraceFrame(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("cat", ctypes.c_char_p), ("ts_us", ctypes.c_uint32),
                ("layer", ctypes.c_int8)]


class Trace(ctypes.Structure):
    """pt_trace_t (pitorch/profiler/trace.h:35-48): 4096 events, a stack of 32."""
    _fields_ = [("events", TraceEvent * 4096), ("count", ctypes.c_int), ("enabled", ctypes.c_int),
                ("stack", TraceFrame * 32), ("depth", ctypes.c_int)]


def trace_spans(tr):
    """(name, cat, layer, depth) of every recorded event, in record order."""
    return [(e.name.decode(), e.cat.decode(), int(e.layer), int(e.depth)) for e in tr.events[:tr.count]]


def arr(ptr, n):
    return np.ctypeslib.as_array(ptr, shape=(n,)).copy()


class OracleModel:
    """The restatement's model over a blob (numpy uint8, kept alive here)."""

    def __init__(self, blob, max_T=0):
        self.L = oracle()
        self.blob = blob
        self.h = self.L.po_model_new(P(blob), max_T)
        h = np.frombuffer(blob[:28].tobytes(), dtype=np.int32)
        self.vocab = abs(int(h[5]))
        self.dim = int(h[0])

    def close(self):
        if self.h:
            self.L.po_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def forward_step(self, tok):
        return self.L.po_forward_step(self.h, int(tok))

    def logits(self):
        return arr(self.L.po_logits(self.h), self.vocab)

    def train_step(self, tokens, lr):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        return self.L.po_train_step(self.h, t.ctypes.data_as(ip), len(t), lr)

    def grads(self):
        n = ctypes.c_int()
        p = self.L.po_grads(self.h, ctypes.byref(n))
        return arr(p, n.value)


def greedy_tokens(step_fn, prompt, n_pos):
    """Forced-prompt greedy protocol shared by fixtures and tests."""
    out = []
    tok = int(prompt[0])
    for pos in range(n_pos):
        nxt = step_fn(tok)
        if pos < len(prompt) - 1:
            nxt = int(prompt[pos + 1])
        out.append(int(nxt))
        tok = nxt
    return out
