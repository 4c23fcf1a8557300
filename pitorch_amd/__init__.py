"""pitorch_amd — MI355X (gfx950) projection hot path for pitorch-style LLaMA-2.

The product is two in-tree shared libraries built by ``pitorch_amd/Makefile``:

* ``lib/libptmi.so``  — HIP kernels behind the C-ABI in ``include/ptmi.h``
* ``lib/libpthost.so`` — the C host layer with pitorch's ``pt.h`` signatures

This package only binds them with ctypes for tests and the benchmark.  There
is no CPU fallback: if the libraries are missing, loading raises.
"""
from ._ffi import (  # noqa: F401
    PtmiError,
    Model,
    decode_step_plan,
    lib_dir,
    load_host,
    load_ptmi,
    matvec,
    model_bytes,
    seed_tokens,
    seed_uniform,
    synth_model,
)

# Seeds of the synthetic benchmark inputs (the reference ships no
# initializer; these fix the models, prompts and training ids).
SEED_MODEL = {"stories15M": 15, "stories42M": 42, "stories110M": 110}
SEED_PROMPT = 8
SEED_TRAIN = 256
N_PROMPT = 8
DECODE_POSITIONS = {"stories15M": 256, "stories42M": 1024, "stories110M": 1024}

STORIES = {
    # name: (dim, hidden, n_layers, n_heads, n_kv_heads, vocab, seq_len)
    "stories15M": (288, 768, 6, 6, 6, 32000, 256),
    "stories42M": (512, 1376, 8, 8, 8, 32000, 1024),
    "stories110M": (768, 2048, 12, 12, 12, 32000, 1024),
}
