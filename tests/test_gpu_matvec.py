"""GPU parity of the fp32 matvec (pt_matvec_fn drop-in) against the oracle.

Tolerances (north_star: per-output relative error <= 1e-5, fp32 with a
different reduction order):
  * integer-valued inputs (dev/tests/matvec/test_matvec.c:25-35 idea): every
    partial sum is exact in fp32, so GPU == oracle BIT FOR BIT;
  * U(-1,1) inputs: |y_gpu - y_oracle| <= 1e-5 * max(|y_oracle|, rms(y_oracle))
    per output (the rms floor keeps outputs that cancel to ~0 meaningful),
    and within the fp64 forward-error bound gamma_n * sum|W||x|.
"""
import numpy as np
import pytest

import pitorch_amd as pa
from tests._oracle import P, oracle
from tests.test_oracle import lcg_ints

pytestmark = pytest.mark.gpu

SWEEP = [(288, 288), (768, 288), (288, 768), (32000, 288), (2048, 768), (768, 2048), (32000, 768),
         (2304, 768), (4096, 768)]
EXTRA = [(48, 48), (512, 512), (1376, 512), (512, 1376), (1, 4), (3, 8), (37, 44), (16, 2304)]


def oracle_mv(W, x):
    y = np.zeros(W.shape[0], np.float32)
    oracle().po_smatvec(P(W), P(x), P(y), W.shape[0], W.shape[1])
    return y


def check_close(y, ref, W, x):
    scale = np.maximum(np.abs(ref), np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    rel = np.abs(y - ref) / scale
    assert rel.max() <= 1e-5, rel.max()
    exact = W.astype(np.float64) @ x.astype(np.float64)
    n = W.shape[1]
    gamma = n * 2.0 ** -24 / (1 - n * 2.0 ** -24)
    assert (np.abs(y - exact) <= gamma * (np.abs(W) @ np.abs(x)) + 1e-30).all()


@pytest.mark.parametrize("d,n", SWEEP + EXTRA)
def test_integer_inputs_bit_exact(d, n):
    W = lcg_ints(d * n, 42).reshape(d, n) if d * n <= 2_000_000 else \
        np.random.default_rng(d).integers(1, 9, (d, n)).astype(np.float32)
    x = lcg_ints(n, 137)
    y = pa.matvec(W, x)
    assert np.array_equal(y, oracle_mv(W, x))


@pytest.mark.parametrize("d,n", SWEEP + EXTRA)
def test_random_inputs_within_tolerance(d, n):
    W = pa.seed_uniform(1000 + d, d * n).reshape(d, n)
    x = pa.seed_uniform(2000 + n, n)
    y = pa.matvec(W, x)
    check_close(y, oracle_mv(W, x), W, x)


def test_long_rows_and_unaligned_views():
    rng = np.random.default_rng(3)
    W = rng.uniform(-1, 1, (288, 32000)).astype(np.float32)      # W_cls^T shape (dX path)
    x = rng.uniform(-1, 1, 32000).astype(np.float32)
    check_close(pa.matvec(W, x), oracle_mv(W, x), W, x)
    big = rng.uniform(-1, 1, 1 + 40 * 45).astype(np.float32)
    Wv = big[1:].reshape(40, 45)                                   # 4-byte aligned only, n%4 != 0
    x = rng.uniform(-1, 1, 45).astype(np.float32)
    check_close(pa.matvec(Wv, x), oracle_mv(np.ascontiguousarray(Wv), x), Wv, x)


def test_bad_arguments_are_errors():
    L = pa.load_ptmi()
    W = np.ones((4, 4), np.float32)
    y = np.zeros(4, np.float32)
    assert L.ptmi_matvec_checked(P(W), P(W[0]), P(y), 0, 4) == 1
    assert L.ptmi_matvec_checked(None, P(W[0]), P(y), 4, 4) == 1
    assert b"bad arguments" in L.ptmi_last_error()


def test_registered_weights_resolve_to_device_layout():
    """Host pointers into a registered blob hit the device copy, including the
    fused [wq;wk;wv] and row-interleaved [w1|w3] layouts."""
    cfg = pa.STORIES["stories15M"]
    D, H, Lyr, V = cfg[0], cfg[1], cfg[2], cfg[5]
    blob = pa.synth_model(cfg, 77)
    L = pa.load_ptmi()
    assert L.ptmi_register_weights(P(blob), blob.nbytes) == 0
    try:
        w = np.frombuffer(blob, np.float32, offset=28)
        o = {}
        off = 0
        for name, n in (("emb", V * D), ("rms_att", Lyr * D), ("wq", Lyr * D * D), ("wk", Lyr * D * D),
                        ("wv", Lyr * D * D), ("wo", Lyr * D * D), ("rms_ffn", Lyr * D), ("w1", Lyr * H * D),
                        ("w2", Lyr * D * H), ("w3", Lyr * H * D)):
            o[name] = off
            off += n
        rng = np.random.default_rng(9)
        views = [("wq", 2, D, D, 0), ("wk", 5, D, D, 0), ("wv", 0, D, D, 16), ("wo", 3, D, D, 0),
                 ("w1", 1, H, D, 0), ("w3", 4, H, D, 100), ("w2", 2, D, H, 0), ("emb", 0, V, D, 0)]
        for name, layer, rows, cols, r0 in views:
            start = o[name] + layer * rows * cols + r0 * cols
            nrow = rows - r0 if name != "w3" else 64
            W = w[start: start + nrow * cols].reshape(nrow, cols)
            x = rng.uniform(-1, 1, cols).astype(np.float32)
            y = np.zeros(nrow, np.float32)
            assert L.ptmi_matvec_checked(P(W), P(x), P(y), nrow, cols) == 0
            check_close(y, oracle_mv(np.ascontiguousarray(W), x), W, x)
        # invalidation: host writes become visible only after ptmi_invalidate
        start = o["wq"]
        W = w[start: start + D * D].reshape(D, D)
        x = rng.uniform(-1, 1, D).astype(np.float32)
        before = oracle_mv(np.ascontiguousarray(W), x)
        W *= 2.0
        y = np.zeros(D, np.float32)
        assert L.ptmi_matvec_checked(P(W), P(x), P(y), D, D) == 0
        check_close(y, before, W / 2, x)                 # stale device copy until invalidated
        assert L.ptmi_invalidate(P(W), W.nbytes) == 0
        assert L.ptmi_matvec_checked(P(W), P(x), P(y), D, D) == 0
        check_close(y, oracle_mv(np.ascontiguousarray(W), x), W, x)
    finally:
        L.ptmi_unregister_weights(P(blob))


def test_device_pointer_entry_with_row_stride():
    from pitorch_amd._hip import DeviceArray
    L = pa.load_ptmi()
    d, n = 4096, 768
    W = pa.seed_uniform(5, d * (n + 4)).reshape(d, n + 4)         # ld = n + 4
    x = pa.seed_uniform(6, n)
    dW, dx, dy = DeviceArray.from_host(W), DeviceArray.from_host(x), DeviceArray(d)
    assert L.ptmi_matvec_dev(dW.ptr, n + 4, dx.ptr, dy.ptr, d, n, None) == 0
    assert L.ptmi_sync() == 0
    Wc = np.ascontiguousarray(W[:, :n])
    check_close(dy.download(), oracle_mv(Wc, x), Wc, x)
    for a in (dW, dx, dy):
        a.free()


def dev_matvec(entry, W, x):
    """y = W x through a device-pointer entry (ptmi_matvec_dev or its x
    re-read ablation), on the library stream."""
    from pitorch_amd._hip import DeviceArray
    L = pa.load_ptmi()
    dW, dx = DeviceArray.from_host(np.ascontiguousarray(W)), DeviceArray.from_host(x)
    dy = DeviceArray.from_host(np.full(W.shape[0], np.nan, np.float32))
    assert getattr(L, entry)(dW.ptr, W.shape[1], dx.ptr, dy.ptr, W.shape[0], W.shape[1], None) == 0
    assert L.ptmi_sync() == 0
    y = dy.download()
    for a in (dW, dx, dy):
        a.free()
    return y


@pytest.mark.parametrize("d,n", SWEEP + [(48, 48), (37, 44), (16, 2304)])
def test_x_reread_ablation_matches(d, n):
    """The ablation kernel (x re-read per row pass, the counterpart of
    smatvec_tmu_no_packing, pitorch/ops/matvec/matvec_no_packing.c:25-85)
    is parity-held like the default: bit-exact on integer inputs, within
    the tolerance on U(-1,1), and equal to the default kernel bit for bit
    (same geometry, same per-row order)."""
    Wi = np.random.default_rng(d + n).integers(1, 9, (d, n)).astype(np.float32)
    xi = lcg_ints(n, 137)
    assert np.array_equal(dev_matvec("ptmi_matvec_dev_xreread", Wi, xi), oracle_mv(Wi, xi))
    W = pa.seed_uniform(1000 + d, d * n).reshape(d, n)
    x = pa.seed_uniform(2000 + n, n)
    y = dev_matvec("ptmi_matvec_dev_xreread", W, x)
    check_close(y, oracle_mv(W, x), W, x)
    assert np.array_equal(y, dev_matvec("ptmi_matvec_dev", W, x))


def test_x_reread_ablation_rejects_long_rows():
    from pitorch_amd._hip import DeviceArray
    L = pa.load_ptmi()
    a = DeviceArray(4 * 2400)
    assert L.ptmi_matvec_dev_xreread(a.ptr, 2400, a.ptr, a.ptr, 2, 2400, None) == 1
    a.free()


def test_registered_buffer_serves_w_until_invalidated():
    """ptmi_register_buffer: a host scratch matrix (the backward's
    host-transposed W, pitorch/train/pt_train.c:588-594, 662-679) is copied
    to HBM once and every W inside it is read from that copy; a host write
    is seen after ptmi_invalidate over the written part and not before;
    overlapping registrations are refused.  Integer inputs: exact."""
    L = pa.load_ptmi()
    D, V = 288, 4096
    buf = lcg_ints(D * V + 2 * D * D, 31, 16).astype(np.float32)     # [W_t (D x V) | two D x D blocks]
    x = lcg_ints(V, 32, 16).astype(np.float32)
    y = np.zeros(D, np.float32)
    assert L.ptmi_register_buffer(P(buf), buf.nbytes) == 0
    try:
        wt = buf[:D * V].reshape(D, V)
        for _ in range(3):                            # the T-1 calls of one backward
            assert L.ptmi_matvec_checked(P(wt), P(x), P(y), D, V) == 0
            assert np.array_equal(y, oracle_mv(wt, x))
        # a sub-matrix view at an offset (a layer's block of the packed transposes)
        blk = buf[D * V + D * D:].reshape(D, D)
        y2 = np.zeros(D, np.float32)
        assert L.ptmi_matvec_checked(P(blk), P(x[:D]), P(y2), D, D) == 0
        assert np.array_equal(y2, oracle_mv(blk, x[:D]))
        # host write without invalidate: the device copy still holds the old W
        old = oracle_mv(blk, x[:D])
        blk[:] = lcg_ints(D * D, 33, 16).astype(np.float32).reshape(D, D)
        assert L.ptmi_matvec_checked(P(blk), P(x[:D]), P(y2), D, D) == 0
        assert np.array_equal(y2, old)
        # invalidate the written part only: now the new W
        assert L.ptmi_invalidate(P(blk), blk.nbytes) == 0
        assert L.ptmi_matvec_checked(P(blk), P(x[:D]), P(y2), D, D) == 0
        assert np.array_equal(y2, oracle_mv(blk, x[:D]))
        assert L.ptmi_matvec_checked(P(wt), P(x), P(y), D, V) == 0    # the rest untouched
        assert np.array_equal(y, oracle_mv(wt, x))
        # overlaps are refused
        assert L.ptmi_register_buffer(P(blk), blk.nbytes) == 1
        assert "overlaps" in L.ptmi_last_error().decode()
    finally:
        assert L.ptmi_unregister_buffer(P(buf)) == 0
    assert L.ptmi_unregister_buffer(P(buf)) == 1
