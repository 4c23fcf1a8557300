"""GPU parity of the fp32 MFMA training GEMMs against the oracle.

* integer-valued inputs (1..16): every product and partial sum is exact in
  fp32 (|sum| < 2^24), so GPU == oracle BIT FOR BIT for any summation order —
  this also pins the MFMA operand/result lane layout;
* U(-1,1) inputs: |C - C_fp64| <= gamma_K * (|A||B|) elementwise (the fp32
  forward-error bound for a K-term dot product).
Shapes: the reference's GEMM unit-test sizes (dev/tests/gemm/test_gemm.c:
82-83) and every training GEMM of the 15M config at T=256 (R=255).
"""
import numpy as np
import pytest

import pitorch_amd as pa
from pitorch_amd._hip import DeviceArray
from tests._oracle import P, oracle
from tests.test_oracle import lcg_ints

pytestmark = pytest.mark.gpu
R = 255
DW = [(288, 288), (768, 288), (288, 768), (32000, 288)]      # dW[out,in] += dY^T X, K = R
DX = [(288, 288), (768, 288), (288, 768), (32000, 288)]      # dX[R,in] = dY[R,out] W[out,in], K = out


def ints(shape, seed):
    return np.random.default_rng(seed).integers(1, 17, shape).astype(np.float32)


def bound_ok(C, A64_B64_exact, absAB, K):
    gamma = K * 2.0 ** -24 / (1 - K * 2.0 ** -24)
    return np.all(np.abs(C - A64_B64_exact) <= gamma * absAB + 1e-30)


@pytest.mark.parametrize("n", [16, 32])
def test_sgemm_square_exact(n):
    A = lcg_ints(n * n, 42, 16).reshape(n, n)
    B = lcg_ints(n * n, 137, 16).reshape(n, n)
    C = np.zeros((n, n), np.float32)
    L = pa.load_ptmi()
    assert L.ptmi_sgemm_rect(P(A), P(B), P(C), n, n, n, 0) == 0
    ref = np.zeros((n, n), np.float32)
    oracle().po_sgemm(P(A), P(B), P(ref), n, n, n)
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("out_dim,in_dim", DW)
def test_backward_weight_batched_exact(out_dim, in_dim):
    dY, X = ints((R, out_dim), 1), ints((R, in_dim), 2)
    dW = ints((out_dim, in_dim), 3)
    ref = dW.copy()
    L = pa.load_ptmi()
    assert L.ptmi_matmul_backward_weight_batched_checked(P(dW), P(dY), P(X), out_dim, in_dim, R) == 0
    oracle().po_matmul_backward_weight_batched(P(ref), P(dY), P(X), out_dim, in_dim, R)
    assert np.array_equal(dW, ref)
    # the void entry with the reference's exact signature (pt_train.c:475-477)
    L.ptmi_matmul_backward_weight_batched(P(dW), P(dY), P(X), out_dim, in_dim, R)
    oracle().po_matmul_backward_weight_batched(P(ref), P(dY), P(X), out_dim, in_dim, R)
    assert np.array_equal(dW, ref)


# T = 1: the rank-1 matmul_backward_weight (pitorch/train/pt_backward_ops.c:
# 43-49), unit-tested by the reference at 32x16 (dev/tests/train/
# test_backward_ops.c:86-105); also the config-5 projection shapes.
@pytest.mark.parametrize("out_dim,in_dim", [(32, 16), (288, 288), (768, 288), (288, 768), (32000, 288), (5, 3)])
def test_backward_weight_rank1_exact(out_dim, in_dim):
    dy, x = ints(out_dim, 11), ints(in_dim, 12)
    dW = ints((out_dim, in_dim), 13)
    ref = dW.copy()
    L = pa.load_ptmi()
    L.ptmi_matmul_backward_weight_batched(P(dW), P(dy), P(x), out_dim, in_dim, 1)
    oracle().po_matmul_backward_weight(P(ref), P(dy), P(x), out_dim, in_dim)
    assert np.array_equal(dW, ref)


# sgemm_rect_tmu's own call site (matmul_backward_weight_gpu,
# pitorch/train/pt_train.c:536-543): C[V,D] += A[V,R] . X[R,D] with
# M = 32000, K = R = 255, N = D = 288, accumulate = 1, num_qpus = 12; and
# the rect shapes below, all integer-exact against the oracle's
# sgemm_rect_tmu restatement.
@pytest.mark.parametrize("M,K,N,acc", [(32000, 255, 288, 1), (255, 288, 288, 0), (255, 32000, 288, 1),
                                       (300, 77, 130, 1), (1, 5, 3, 0), (100, 3001, 70, 1), (1000, 301, 900, 0)])
def test_sgemm_rect_tmu_exact(M, K, N, acc):
    A, B = ints((M, K), M + 1), ints((K, N), K + 2)
    C = ints((M, N), N + 3) if acc else np.zeros((M, N), np.float32)
    ref = C.copy()
    L = pa.load_ptmi()
    L.ptmi_sgemm_rect_tmu(P(A), P(B), P(C), M, K, N, 12, acc)
    oracle().po_sgemm_rect(P(A), P(B), P(ref), M, K, N, acc)
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("n", [16, 32])
def test_sgemm_cpu_signature_exact(n):
    """ptmi_sgemm_cpu: sgemm_cpu's signature (pitorch/ops/gemm/gemm.h:19-20),
    at the reference's test sizes (dev/tests/gemm/test_gemm.c:82-83)."""
    A = lcg_ints(n * n, 7, 16).reshape(n, n)
    B = lcg_ints(n * n, 9, 16).reshape(n, n)
    C = np.full((n, n), np.nan, np.float32)
    L = pa.load_ptmi()
    L.ptmi_sgemm_cpu(P(A), P(B), P(C), n, n, n)
    ref = np.zeros((n, n), np.float32)
    oracle().po_sgemm(P(A), P(B), P(ref), n, n, n)
    assert np.array_equal(C, ref)


@pytest.mark.parametrize("out_dim,in_dim", DX)
def test_backward_input_batched_exact(out_dim, in_dim):
    dY, W = ints((R, out_dim), 4), ints((out_dim, in_dim), 5)
    dX = np.zeros((R, in_dim), np.float32)
    L = pa.load_ptmi()
    assert L.ptmi_matmul_backward_input_batched(P(dX), P(W), P(dY), out_dim, in_dim, R, 0) == 0
    ref = np.zeros((R, in_dim), np.float32)
    for t in range(R):
        oracle().po_matmul_backward_input(P(ref[t]), P(W), P(dY[t]), out_dim, in_dim)
    assert np.array_equal(dX, ref)


# Kernel paths: 32x32 tiles (255x288x288, 300x77x130, 1x5x3, 1000x301x900),
# 32x32 with split K (100x3001x70), 64x64 with split K (K = 32000); the
# 64x64 NT path for large outputs runs in the 15M training-step tests.
@pytest.mark.parametrize("M,K,N", [(255, 288, 288), (255, 32000, 288), (300, 77, 130), (1, 5, 3), (100, 3001, 70),
                                   (1000, 301, 900)])
def test_sgemm_rect_random_bounded(M, K, N):
    rng = np.random.default_rng(M + K + N)
    A = rng.uniform(-1, 1, (M, K)).astype(np.float32)
    B = rng.uniform(-1, 1, (K, N)).astype(np.float32)
    C0 = rng.uniform(-1, 1, (M, N)).astype(np.float32)
    C = C0.copy()
    L = pa.load_ptmi()
    assert L.ptmi_sgemm_rect(P(A), P(B), P(C), M, K, N, 1) == 0
    exact = C0.astype(np.float64) + A.astype(np.float64) @ B.astype(np.float64)
    assert bound_ok(C, exact, np.abs(C0) + np.abs(A) @ np.abs(B), K + 1)


@pytest.mark.parametrize("op", [0, 1, 2])
def test_gemm_dev_ops_with_strides(op):
    """Device-pointer entry: NN, TN, NT with padded leading dimensions."""
    rng = np.random.default_rng(op)
    M, N, K = 200, 96, 130
    pad = 4
    if op == 0:
        A = rng.uniform(-1, 1, (M, K + pad)); B = rng.uniform(-1, 1, (K, N + pad))
        Aop, Bop = A[:, :K], B[:, :N]
    elif op == 1:
        A = rng.uniform(-1, 1, (K, M + pad)); B = rng.uniform(-1, 1, (K, N + pad))
        Aop, Bop = A[:, :M].T, B[:, :N]
    else:
        A = rng.uniform(-1, 1, (M, K + pad)); B = rng.uniform(-1, 1, (N, K + pad))
        Aop, Bop = A[:, :K], B[:, :K].T
    A, B = A.astype(np.float32), B.astype(np.float32)
    C = np.zeros((M, N + pad), np.float32)
    dA, dB, dC = DeviceArray.from_host(A), DeviceArray.from_host(B), DeviceArray.from_host(C)
    L = pa.load_ptmi()
    assert L.ptmi_gemm_dev(op, dA.ptr, A.shape[1], dB.ptr, B.shape[1], dC.ptr, N + pad, M, N, K, 0, None) == 0
    assert L.ptmi_sync() == 0
    got = dC.download().reshape(M, N + pad)
    exact = Aop.astype(np.float32).astype(np.float64) @ Bop.astype(np.float32).astype(np.float64)
    absab = np.abs(Aop.astype(np.float32)) @ np.abs(Bop.astype(np.float32))
    assert bound_ok(got[:, :N], exact, absab, K)
    assert np.all(got[:, N:] == 0)          # padding columns untouched
    for a in (dA, dB, dC):
        a.free()


# Grids of 768 blocks and more take their tiles in XCD order (each XCD a
# contiguous tile range, ordered along the larger operand): ragged M, N and
# K on 64x64 and 32x32 tiles, split K for the NN forms; a NaN-filled C shows
# any tile left unwritten.
@pytest.mark.parametrize("op,M,N,K", [(2, 200, 20000, 300), (2, 260, 20000, 300), (0, 255, 320, 30000),
                                      (0, 130, 288, 30000), (1, 30004, 288, 130), (1, 32000, 256, 131)])
def test_gemm_dev_large_grids(op, M, N, K):
    rng = np.random.default_rng(M + N + K)
    if op == 0:
        A = rng.uniform(-1, 1, (M, K)); B = rng.uniform(-1, 1, (K, N))
        Aop, Bop = A, B
    elif op == 1:
        A = rng.uniform(-1, 1, (K, M)); B = rng.uniform(-1, 1, (K, N))
        Aop, Bop = A.T, B
    else:
        A = rng.uniform(-1, 1, (M, K)); B = rng.uniform(-1, 1, (N, K))
        Aop, Bop = A, B.T
    A, B = A.astype(np.float32), B.astype(np.float32)
    dA, dB = DeviceArray.from_host(A), DeviceArray.from_host(B)
    dC = DeviceArray.from_host(np.full((M, N), np.nan, np.float32))
    L = pa.load_ptmi()
    assert L.ptmi_gemm_dev(op, dA.ptr, A.shape[1], dB.ptr, B.shape[1], dC.ptr, N, M, N, K, 0, None) == 0
    assert L.ptmi_sync() == 0
    got = dC.download().reshape(M, N)
    Af, Bf = Aop.astype(np.float32).astype(np.float64), Bop.astype(np.float32).astype(np.float64)
    assert bound_ok(got, Af @ Bf, np.abs(Af) @ np.abs(Bf), K)
    for a in (dA, dB, dC):
        a.free()


# The direct-to-LDS tiles (NT with M >= 192 on 256x128 tiles, TN on 64x96;
# outputs of 4M elements and more, whole K, no fused epilogue):
# integer-exact at the classifier shapes of config 5, with and without
# accumulate, and on ragged M, N and K.
@pytest.mark.parametrize("op,M,N,K,acc", [(2, 256, 32000, 288, 0), (2, 256, 32000, 288, 1), (2, 193, 21845, 36, 1),
                                          (1, 32000, 288, 255, 0), (1, 32000, 288, 255, 1), (1, 16388, 260, 7, 0)])
def test_gemm_dev_direct_lds_exact(op, M, N, K, acc):
    if op == 1:
        A, B = ints((K, M), 21), ints((K, N), 22)
        ref = A.T.astype(np.float64) @ B.astype(np.float64)
    else:
        A, B = ints((M, K), 23), ints((N, K), 24)
        ref = A.astype(np.float64) @ B.T.astype(np.float64)
    C0 = ints((M, N), 25) if acc else np.full((M, N), np.nan, np.float32)
    if acc:
        ref = ref + C0
    dA, dB, dC = DeviceArray.from_host(A), DeviceArray.from_host(B), DeviceArray.from_host(C0)
    L = pa.load_ptmi()
    assert L.ptmi_gemm_dev(op, dA.ptr, A.shape[1], dB.ptr, B.shape[1], dC.ptr, N, M, N, K, acc, None) == 0
    assert L.ptmi_sync() == 0
    got = dC.download().reshape(M, N)
    assert np.array_equal(got, ref.astype(np.float32))
    for a in (dA, dB, dC):
        a.free()


# The per-layer NT GEMMs with at most 9 K steps per split take the panel
# kernel (every K tile of the split in flight): integer-exact at the
# config-5 forward shapes (K split 4 ways at K = 768, summed by the split-K
# reduction), with accumulate, and on ragged M, N and K.
@pytest.mark.parametrize("M,N,K,acc", [(256, 864, 288, 0), (256, 288, 288, 1), (256, 1536, 288, 0),
                                       (256, 288, 768, 1), (255, 100, 100, 0), (33, 31, 4, 1), (70, 2050, 284, 0)])
def test_gemm_dev_panel_nt_exact(M, N, K, acc):
    A, B = ints((M, K), 31), ints((N, K), 32)
    ref = A.astype(np.float64) @ B.T.astype(np.float64)
    C0 = ints((M, N), 33) if acc else np.full((M, N), np.nan, np.float32)
    if acc:
        ref = ref + C0
    dA, dB, dC = DeviceArray.from_host(A), DeviceArray.from_host(B), DeviceArray.from_host(C0)
    L = pa.load_ptmi()
    assert L.ptmi_gemm_dev(2, dA.ptr, K, dB.ptr, K, dC.ptr, N, M, N, K, acc, None) == 0
    assert L.ptmi_sync() == 0
    got = dC.download().reshape(M, N)
    assert np.array_equal(got, ref.astype(np.float32))
    for a in (dA, dB, dC):
        a.free()


def test_gemm_errors():
    L = pa.load_ptmi()
    A = np.ones((4, 4), np.float32)
    assert L.ptmi_sgemm_rect(P(A), P(A), P(A), 0, 4, 4, 0) == 1
    assert L.ptmi_gemm_dev(3, P(A), 4, P(A), 4, P(A), 4, 4, 4, 4, 0, None) == 1
