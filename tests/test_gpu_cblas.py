"""GPU parity of libjules_cblas.so's cblas_sgemm (include/jules_cblas.h), the
symbol the reference's LLVMBackend calls for every matmul it lowers
(lib/LLVMBackend.cpp:1242-1255) and its ORC JIT resolves from the process
(:1338-1356).

The emitted call, cblas_sgemm(101, 111, 111, M, N, K, 1, A, K, B, N, 0, C, N)
on host buffers, is bit-exact with the restated fma chain of the reference's
tiled kernel; alpha, beta, transposes, column-major storage and padded
leading dimensions are within 1e-5 of fp64, and the padding of C outside the
M x N elements is left as it was."""
import ctypes
import os
import subprocess

import numpy as np
import pytest
import torch

from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "jules_amd", "libjules_cblas.so")
RowMajor, ColMajor, NoTrans, Trans, ConjTrans = 101, 102, 111, 112, 113


@pytest.fixture(scope="module")
def cblas(dev):
    L = ctypes.CDLL(LIB, mode=ctypes.RTLD_GLOBAL)
    f = L.cblas_sgemm
    f.restype = None
    f.argtypes = [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_void_p, ctypes.c_int,
                                       ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
                                       ctypes.c_void_p, ctypes.c_int]
    L.jules_cblas_last_status.restype = ctypes.c_int
    return L


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (33, 48, 70), (512, 512, 512), (64, 256, 784),
                                   (300, 700, 2500)])
def test_emitted_call_bit_exact(cblas, M, N, K):
    """The call exactly as LLVMBackend emits it, on host buffers."""
    case(f"cblas_sgemm emitted call {M}x{N}x{K}")
    A = I.uniform(M + K, 0, (M, K), -1, 1)
    B = I.uniform(M + K, 1, (K, N), -1, 1)
    C = np.full((M, N), np.nan, np.float32)  # beta = 0: C is never read
    cblas.cblas_sgemm(RowMajor, NoTrans, NoTrans, M, N, K, 1.0, _p(A), K, _p(B), N, 0.0, _p(C), N)
    assert cblas.jules_cblas_last_status() == 0
    np.testing.assert_array_equal(C, po.tiled_matmul_act(A, B, "none"))


def _op(X, rows, cols, ld, trans):
    """The logical matrix of a row-major rows x ld buffer (rows x cols used),
    transposed when trans."""
    m = X[:, :cols].astype(np.float64)
    return m.T if trans else m


@pytest.mark.parametrize("order", [RowMajor, ColMajor])
@pytest.mark.parametrize("ta,tb", [(NoTrans, NoTrans), (Trans, NoTrans), (NoTrans, ConjTrans),
                                   (Trans, Trans)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.75, -1.25), (0.0, 2.0)])
@pytest.mark.parametrize("M,N,K", [(45, 37, 29), (64, 64, 4096)])
def test_general_forms(cblas, order, ta, tb, alpha, beta, M, N, K):
    """alpha/beta, transposes and both storage orders with padded leading
    dimensions, against fp64; C's padding is untouched.  64 x 64 x 4096 is
    one output tile, so the library splits K across workgroups and applies
    alpha, beta (reading C) and the transposes in its split-K reduction."""
    case(f"cblas_sgemm {M}x{N}x{K} order={order} ta={ta} tb={tb} alpha={alpha} beta={beta}")
    tA, tB = ta != NoTrans, tb != NoTrans
    if order == RowMajor:
        ar, ac = (K, M) if tA else (M, K)
        br, bc = (N, K) if tB else (K, N)
        cr, cc = M, N
    else:  # column-major: each matrix is stored as its transpose, row-major
        ar, ac = (M, K) if tA else (K, M)
        br, bc = (K, N) if tB else (N, K)
        cr, cc = N, M
    lda, ldb, ldc = ac + 3, bc + 5, cc + 2
    A = I.uniform(1, 0, (ar, lda), -1, 1)
    B = I.uniform(1, 1, (br, ldb), -1, 1)
    C = I.uniform(1, 2, (cr, ldc), -1, 1)
    C_in = C.copy()
    cblas.cblas_sgemm(order, ta, tb, M, N, K, alpha, _p(A), lda, _p(B), ldb, beta, _p(C), ldc)
    assert cblas.jules_cblas_last_status() == 0
    if order == RowMajor:
        opA = _op(A, ar, ac, lda, tA)
        opB = _op(B, br, bc, ldb, tB)
        ref = alpha * (opA @ opB) + beta * C_in[:, :cc].astype(np.float64)
        got = C[:, :cc]
    else:
        # column-major X stored row-major is X^T
        opA = A[:, :ac].astype(np.float64).T
        opA = opA.T if tA else opA
        opB = B[:, :bc].astype(np.float64).T
        opB = opB.T if tB else opB
        ref = (alpha * (opA @ opB)).T + beta * C_in[:, :cc].astype(np.float64)
        got = C[:, :cc]
    assert I.rel_err(got, ref) < I.TOL["f32"]
    np.testing.assert_array_equal(C[:, cc:], C_in[:, cc:])  # padding of C untouched


def test_device_pointers(cblas, dev):
    """Device buffers are used in place (no staging)."""
    case("cblas_sgemm on device pointers")
    M, N, K = 130, 96, 200
    A = I.uniform(2, 0, (M, K), -1, 1)
    B = I.uniform(2, 1, (K, N), -1, 1)
    tA = torch.from_numpy(A).to(dev)
    tB = torch.from_numpy(B).to(dev)
    tC = torch.empty((M, N), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    cblas.cblas_sgemm(RowMajor, NoTrans, NoTrans, M, N, K, 1.0, tA.data_ptr(), K, tB.data_ptr(),
                      N, 0.0, tC.data_ptr(), N)
    assert cblas.jules_cblas_last_status() == 0
    np.testing.assert_array_equal(tC.cpu().numpy(), po.tiled_matmul_act(A, B, "none"))


def test_dlopen_caller_on_gpu(cblas):
    """The plain C caller (dlopen + process-wide dlsym) runs the emitted call."""
    case("cblas_dlopen --gpu")
    exe = os.path.join(ROOT, "tests", "cpp", "cblas_dlopen")
    r = subprocess.run([exe, LIB, "--gpu"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "cblas dlopen ok" in r.stdout, r.stdout + r.stderr
