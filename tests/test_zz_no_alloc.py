"""GPU: ptmi_gemm_dev_noalloc (the entry point that allocates nothing)
against ptmi_gemm_dev, through the C-ABI.

Both entries run the same kernels with the same K split, so they must agree
BIT FOR BIT; integer-valued inputs also make both exact (the oracle's closed
form).  Two calls in a row, the second smaller, show that the shared scratch
keeps nothing a later call depends on.  A GEMM whose split-K partials exceed
the fixed scratch is rejected before anything runs.
"""
import numpy as np
import pytest

import pitorch_amd as pa
from pitorch_amd._hip import DeviceArray

pytestmark = pytest.mark.gpu


def run(entry, op, A, B, M, N, K, acc, C0):
    L = pa.load_ptmi()
    dA, dB, dC = DeviceArray.from_host(A), DeviceArray.from_host(B), DeviceArray.from_host(C0)
    lda, ldb = A.shape[1], B.shape[1]
    st = getattr(L, entry)(op, dA.ptr, lda, dB.ptr, ldb, dC.ptr, N, M, N, K, acc, None)
    assert st == 0, L.ptmi_last_error()
    assert L.ptmi_sync() == 0
    out = dC.download().reshape(M, N)
    for a in (dA, dB, dC):
        a.free()
    return out


def operands(op, M, N, K, seed, integer):
    rng = np.random.default_rng(seed)
    shapes = {0: ((M, K), (K, N)), 1: ((K, M), (K, N)), 2: ((M, K), (N, K))}[op]
    if integer:
        return [rng.integers(1, 17, s).astype(np.float32) for s in shapes]
    return [rng.uniform(-1, 1, s).astype(np.float32) for s in shapes]


# (op, M, N, K): split K over 64x64 tiles (the 15M classifier's dX: 52
# splits), split K over 32x32 tiles, and unsplit; each followed by a
# smaller GEMM of the same form.  64x64x32768 is one tile whose split is
# bounded by ptmi_gemm_dev's workspace (64 partials of 64x64), not by the
# larger fixed scratch.
CASES = [((0, 255, 288, 32000), (0, 100, 96, 8192)),
         ((0, 64, 64, 32768), (0, 32, 48, 20000)),
         ((0, 100, 70, 3001), (0, 40, 33, 1500)),
         ((1, 288, 768, 255), (1, 64, 96, 100)),
         ((2, 256, 1536, 288), (2, 17, 50, 64))]


@pytest.mark.parametrize("first,second", CASES)
@pytest.mark.parametrize("integer", [True, False])
def test_noalloc_equals_gemm_dev(first, second, integer):
    pa.load_ptmi().ptmi_init(0)
    for k, (op, M, N, K) in enumerate((first, second)):
        A, B = operands(op, M, N, K, 10 * k + M, integer)
        C0 = np.full((M, N), 3.0 if integer else 0.5, np.float32)
        for acc in (0, 1):
            want = run("ptmi_gemm_dev", op, A, B, M, N, K, acc, C0)
            got = run("ptmi_gemm_dev_noalloc", op, A, B, M, N, K, acc, C0)
            assert np.array_equal(got, want), (op, M, N, K, acc)
            if integer:
                Aop = A.T if op == 1 else A
                Bop = B.T if op == 2 else B
                exact = Aop.astype(np.float64) @ Bop.astype(np.float64) + (C0 if acc else 0.0)
                assert np.array_equal(got, exact.astype(np.float32))


def test_noalloc_rejects_partials_beyond_the_scratch():
    L = pa.load_ptmi()
    L.ptmi_init(0)
    M, N, K = 1024, 1088, 4096          # 64x64 tiles, 272 blocks: 4 splits x 1024 x 1088 floats > 4 Mi
    a = DeviceArray(16)
    st = L.ptmi_gemm_dev_noalloc(0, a.ptr, K, a.ptr, N, a.ptr, N, M, N, K, 0, None)
    assert st == 1 and b"fixed scratch" in L.ptmi_last_error()
    a.free()
