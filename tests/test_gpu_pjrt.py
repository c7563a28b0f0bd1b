"""GPU tests of the ROCm PJRT executor (jules_hip_pjrt_*, pjrt.cpp) against the
restated reference interpreter (oracle/pjrt_interp.py, lib/PJRT.cpp:169-858).

Built-in ops are compared with the oracle bit for bit where both compute one
IEEE fp32 operation per element (add, subtract, multiply, divide, maximum,
minimum, negate, relu, transpose, reshape, copy) or the same sequential sum
(reduce); exp, log, tanh and logistic within 2 ulp-ish (rtol 2e-6: the GPU's
libm is not the host's); dot_general at the fp32 bar (1e-5 normwise against
the fp64 product; the reference's cblas_sgemm bits are BLAS-specific).
custom_call targets are checked against the fp64 oracle of the kernel they
name, at the bar of that kernel's own tests.
"""
import ctypes

import numpy as np
import pytest
import torch

from jules_amd import _lib
from oracle import inputs as I
from oracle import pjrt_interp as pi
from oracle import pyoracle as po
from tests.helpers import case

pytestmark = pytest.mark.gpu

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.int8: _lib.I8, torch.int32: _lib.I32}
_NP = {_lib.F32: np.float32, _lib.BF16: np.uint16, _lib.I8: np.int8, _lib.I32: np.int32}
_hip = None


def _d2h(ptr, nbytes):
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        _hip.hipDeviceSynchronize.argtypes = []
    out = np.empty(nbytes, np.uint8)
    if nbytes:
        assert _hip.hipDeviceSynchronize() == 0
        assert _hip.hipMemcpy(out.ctypes.data, ptr, nbytes, 2) == 0   # device to host
    return out


def _desc(t):
    d = _lib.JhTensor()
    d.data = t.data_ptr()
    d.offset = 0
    d.rank = t.dim()
    d.dtype = _DT[t.dtype]
    for i in range(t.dim()):
        d.sizes[i] = t.shape[i]
        d.strides[i] = t.stride(i)
    return d


class Exe:
    def __init__(self, text):
        self.L = _lib.lib()
        self.h = ctypes.c_void_p()
        st = self.L.jules_hip_pjrt_compile(text.encode(), 0, ctypes.byref(self.h))
        assert st == 0, self.L.jules_hip_last_error()

    def run(self, *tensors, expect=0):
        ins = (_lib.JhTensor * max(1, len(tensors)))(*[_desc(t) for t in tensors])
        outs = (_lib.JhTensor * 64)()
        n = ctypes.c_int()
        st = self.L.jules_hip_pjrt_execute(self.h, len(tensors), ins, 64, outs, ctypes.byref(n))
        if expect:
            assert st == expect, (st, self.L.jules_hip_last_error())
            return None
        assert st == 0, self.L.jules_hip_last_error()
        res = []
        for i in range(n.value):
            o = outs[i]
            shape = [o.sizes[d] for d in range(o.rank)]
            cnt = int(np.prod(shape)) if shape else 1
            dt = _NP[o.dtype]
            a = _d2h(o.data, cnt * np.dtype(dt).itemsize).view(dt)
            if o.dtype == _lib.BF16:
                a = I.bf16_from_bits(a)
            res.append((a, shape))
        return res

    def close(self):
        if self.h:
            self.L.jules_hip_pjrt_destroy(self.h)
            self.h = ctypes.c_void_p()


def _to_dev(a, dev, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(device=dev, dtype=dtype)


def _oracle(text, arrays, cc=None):
    return pi.run(text, [(np.asarray(a, np.float32), list(np.shape(a))) for a in arrays], cc, multi_result=True)


def _check(got, want, exact_ops=True, rtol=0.0):
    assert len(got) == len(want)
    for (g, gs), (w, ws) in zip(got, want):
        assert gs == ws or int(np.prod(gs)) == int(np.prod(ws))
        if rtol == 0.0:
            np.testing.assert_array_equal(g.ravel(), w.ravel())
        else:
            np.testing.assert_allclose(g.ravel(), w.ravel(), rtol=rtol, atol=1e-30)


ELEMENTWISE = """func.func @main(%arg0: tensor<N>, %arg1: tensor<N>) {
  %0 = "stablehlo.add"(%arg0, %arg1) : () -> ()
  %1 = "stablehlo.subtract"(%arg0, %arg1) : () -> ()
  %2 = "stablehlo.multiply"(%arg0, %arg1) : () -> ()
  %3 = "stablehlo.divide"(%arg0, %arg1) : () -> ()
  %4 = "stablehlo.maximum"(%arg0, %arg1) : () -> ()
  %5 = "stablehlo.minimum"(%arg0, %arg1) : () -> ()
  %6 = "stablehlo.negate"(%3) : () -> ()
  %7 = "stablehlo.relu"(%1) : () -> ()
  %8 = "stablehlo.frobnicate"(%7) : () -> ()
}"""
TRANSCENDENTAL = """
  %0 = "stablehlo.exponential"(%arg0) : () -> ()
  %1 = "stablehlo.log"(%arg0) : () -> ()
  %2 = "stablehlo.tanh"(%arg0) : () -> ()
  %3 = "stablehlo.logistic"(%arg0) : () -> ()
"""


@pytest.mark.parametrize("shape", [(7,), (300, 257), (2, 3, 4, 5)])
def test_elementwise_bit_exact(dev, shape):
    case(f"pjrt elementwise {shape}")
    rng = np.random.default_rng(len(shape))
    a = rng.standard_normal(shape).astype(np.float32)
    b = rng.standard_normal(shape).astype(np.float32)
    b.ravel()[::5] = 0.0                    # division by zero -> 0
    a.ravel()[::7] = np.nan                 # std::max / std::min on NaN
    e = Exe(ELEMENTWISE)
    got = e.run(_to_dev(a, dev), _to_dev(b, dev))
    e.close()
    _check(got, _oracle(ELEMENTWISE, [a, b]))


def test_unequal_sizes_pad_with_zero(dev):
    case("pjrt binary with unequal sizes")
    a = np.arange(10, dtype=np.float32)
    b = np.arange(4, dtype=np.float32).reshape(2, 2) + 0.5
    e = Exe(ELEMENTWISE)
    got = e.run(_to_dev(a, dev), _to_dev(b, dev))
    e.close()
    want = _oracle(ELEMENTWISE, [a, b])
    for (g, _), (w, _) in zip(got, want):
        np.testing.assert_array_equal(g.ravel(), w.ravel())


@pytest.mark.parametrize("n", [5, 100003])
def test_transcendental(dev, n):
    case(f"pjrt exp/log/tanh/logistic n={n}")
    x = (np.random.default_rng(n).standard_normal(n) * 4).astype(np.float32)
    x[:3] = [0.0, -1.0, 1e-30]
    e = Exe(TRANSCENDENTAL)
    got = e.run(_to_dev(x, dev))
    e.close()
    want = _oracle(TRANSCENDENTAL, [x])
    for (g, _), (w, _) in zip(got, want):
        fin = np.isfinite(w)
        assert np.array_equal(np.isfinite(g), fin) and np.array_equal(g[~fin], w[~fin])
        np.testing.assert_allclose(g[fin], w[fin], rtol=2e-6, atol=1e-37)


LAYOUT = """
  %0 = "stablehlo.transpose"(%arg0) {permutation = dense<[2, 0, 1]> : tensor<3xi64>} : () -> ()
  %1 = "stablehlo.transpose"(%arg0) : () -> ()
  %2 = "stablehlo.reduce"(%arg0, %arg1) {dimensions = dense<[1]> : tensor<1xi64>} : () -> ()
  %3 = "stablehlo.reduce"(%0, %arg1) {dimensions = dense<[0, 2]> : tensor<2xi64>} : () -> ()
  %4 = "stablehlo.reduce"(%arg0, %arg1) : () -> ()
  %5 = "stablehlo.reshape"(%arg0) : tensor<6x4xf32>
  %6 = "stablehlo.constant"() {value = dense<1.5, -2.0, 0.25>} : () -> tensor<3xf32>
  %7 = "stablehlo.multiply"(%6, %4) : () -> ()
"""


@pytest.mark.parametrize("shape", [(2, 3, 4), (17, 33, 65)])
def test_transpose_reduce_reshape_constant(dev, shape):
    case(f"pjrt layout ops {shape}")
    x = np.random.default_rng(3).standard_normal(shape).astype(np.float32)
    text = LAYOUT.replace("6x4", f"{shape[0] * shape[1]}x{shape[2]}")
    e = Exe(text)
    got = e.run(_to_dev(x, dev), _to_dev(np.zeros(1, np.float32), dev))
    e.close()
    want = _oracle(text, [x, np.zeros(1, np.float32)])
    _check(got, want)


def test_rank2_transpose_and_dot_general(dev):
    case("pjrt dot_general and rank-2 transpose")
    rng = np.random.default_rng(5)
    A = rng.standard_normal((37, 50)).astype(np.float32)
    B = rng.standard_normal((50, 23)).astype(np.float32)
    text = """
  %0 = "stablehlo.dot_general"(%arg0, %arg1) : () -> ()
  %1 = "stablehlo.relu"(%0) : () -> ()
  %2 = "stablehlo.transpose"(%1) {permutation = dense<[0, 1]> : tensor<2xi64>} : () -> ()
  %3 = "stablehlo.reduce"(%2, %arg1) {dimensions = dense<[0]> : tensor<1xi64>} : () -> ()
"""
    e = Exe(text)
    got = e.run(_to_dev(A, dev), _to_dev(B, dev))
    e.close()
    want = _oracle(text, [A, B])
    (g0, s0), (w0, ws0) = got[0], want[0]
    assert s0 == ws0 == [37, 23]
    assert I.rel_err(g0.reshape(37, 23), (A.astype(np.float64) @ B)) < I.TOL["f32"]
    # downstream ops consume the GPU product: compare them on that product
    G = np.maximum(g0.reshape(37, 23), 0)
    np.testing.assert_array_equal(got[1][0], G.ravel())
    np.testing.assert_array_equal(got[2][0], G.T.ravel())
    want3 = pi.run('%0 = "stablehlo.reduce"(%arg0, %arg1) {dimensions = dense<[0]> : tensor<1xi64>} : () -> ()',
                   [(G.T.copy(), [37, 23]), (np.zeros(1, np.float32), [1])])
    np.testing.assert_array_equal(got[3][0], want3[0][0])


def _cc(target, config, args, types):
    """fp64 oracle of the registry kernels these tests name."""
    if target == "fusedMatmulBiasRelu":
        (A, sa), (B, sb), (bias, _) = args
        return [(po.gemm64(A.reshape(sa), B.reshape(sb), bias, "relu").ravel(), types[0][0])]
    if target == "fusedSoftmax":
        (x, s), = args
        return [(po.softmax64(x.reshape(s)).ravel(), types[0][0])]
    if target in ("gelu", "fusedGelu"):
        (x, s), = args
        return [(po.fused_gelu(x).ravel(), types[0][0])]
    if target == "fusedCrossEntropyLoss":
        (x, s), (t, _) = args
        loss, grad = po.cross_entropy64(x.reshape(s), t.astype(np.int32))
        return [(grad.ravel(), types[0][0]), (np.array([loss]), types[1][0])]
    raise KeyError(target)


CUSTOM = """
  %0 = "stablehlo.custom_call"(%arg0, %arg1, %arg2) {backend_config = "", call_target_name = "fusedMatmulBiasRelu", has_side_effect = false} : (tensor<64x96xf32>, tensor<96x48xf32>, tensor<48xf32>) -> tensor<64x48xf32>
  %1 = "stablehlo.custom_call"(%0) {call_target_name = "fusedSoftmax"} : (tensor<64x48xf32>) -> tensor<64x48xf32>
  %2 = "stablehlo.custom_call"(%arg0) {call_target_name = "gelu"} : (tensor<64x96xf32>) -> tensor<64x96xf32>
  %3 = "stablehlo.negate"(%1) : () -> ()
"""


def test_custom_call_runs_registry_kernels(dev):
    case("pjrt custom_call fusedMatmulBiasRelu / fusedSoftmax / gelu")
    rng = np.random.default_rng(11)
    A = rng.standard_normal((64, 96)).astype(np.float32)
    B = rng.standard_normal((96, 48)).astype(np.float32)
    bias = rng.standard_normal(48).astype(np.float32)
    e = Exe(CUSTOM)
    got = e.run(_to_dev(A, dev), _to_dev(B, dev), _to_dev(bias, dev))
    e.close()
    assert [s for _, s in got] == [[64, 48], [64, 48], [64, 96], [64, 48]]
    mm = po.gemm64(A, B, bias, "relu")
    assert I.rel_err(got[0][0].reshape(64, 48), mm) < I.TOL["f32"]
    # softmax of the GPU GEMM output, at the row kernels' bar
    assert I.rel_err(got[1][0].reshape(64, 48), po.softmax64(got[0][0].reshape(64, 48))) < I.TOL["f32"]
    np.testing.assert_array_equal(got[2][0], po.fused_gelu(A).ravel())   # bit-exact activation
    np.testing.assert_array_equal(got[3][0], -got[1][0])


def test_multi_result_custom_call(dev):
    case("pjrt custom_call fusedCrossEntropyLoss (two results)")
    text = """
  %0:2 = "stablehlo.custom_call"(%arg0, %arg1) {call_target_name = "fusedCrossEntropyLoss"} : (tensor<16x40xf32>, tensor<16xi32>) -> (tensor<16x40xf32>, tensor<1xf32>)
  %1 = "stablehlo.multiply"(%0#1, %0#1) : () -> ()
"""
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((16, 40)) * 2).astype(np.float32)
    t = rng.integers(0, 40, 16).astype(np.int32)
    e = Exe(text)
    got = e.run(_to_dev(x, dev), _to_dev(t, dev, torch.int32))
    e.close()
    loss64, grad64 = po.cross_entropy64(x, t)
    assert [s for _, s in got] == [[16, 40], [1], [1]]
    assert I.rel_err(got[0][0].reshape(16, 40), grad64) < I.TOL["f32"]
    assert abs(got[1][0][0] - loss64) < 1e-5 * max(1.0, abs(loss64))
    assert got[2][0][0] == np.float32(got[1][0][0] * got[1][0][0])


def test_bf16_custom_call_flash_attention(dev):
    case("pjrt custom_call flashAttention bf16")
    B, H, S, D = 1, 2, 100, 64
    rng = np.random.default_rng(9)
    q, k, v = (I.bf16_round(rng.standard_normal((B, H, S, D)).astype(np.float32)) for _ in range(3))
    text = ('%0 = "stablehlo.custom_call"(%arg0, %arg1, %arg2) {call_target_name = "flashAttentionCausal"} : '
            f'(tensor<{B}x{H}x{S}x{D}xbf16>, tensor<{B}x{H}x{S}x{D}xbf16>, tensor<{B}x{H}x{S}x{D}xbf16>) '
            f'-> tensor<{B}x{H}x{S}x{D}xbf16>')
    e = Exe(text)
    got = e.run(*[_to_dev(a, dev, torch.bfloat16) for a in (q, k, v)])
    e.close()
    (o, s), = got
    assert s == [B, H, S, D]
    ref = po.attention64(q, k, v, True, 1.0 / np.sqrt(D))
    assert I.rel_err(o.reshape(B, H, S, D), ref) < I.TOL["bf16"]


def test_errors_and_reuse(dev):
    case("pjrt error paths and handle reuse")
    x = _to_dev(np.arange(6, dtype=np.float32).reshape(2, 3), dev)
    e = Exe('%0 = "stablehlo.custom_call"(%arg0) {call_target_name = "noSuchKernel"} : (tensor<2x3xf32>) -> tensor<2x3xf32>')
    e.run(x, expect=9)                       # JH_ERR_NOT_FOUND
    e.close()
    # a transpose whose data is not its shape's size (the reference would read
    # past the end): the binary op gives 6 values under the rank-2 shape [1, 2]
    text = ('%0 = "stablehlo.add"(%arg1, %arg0) : () -> ()\n'
            '%1 = "stablehlo.transpose"(%0) : () -> ()')
    e = Exe(text)
    e.run(x.reshape(6), _to_dev(np.zeros((1, 2), np.float32), dev), expect=2)   # JH_ERR_SHAPE
    e.close()
    # one handle, several calls, different input counts (parsed per count)
    e = Exe('%0 = "stablehlo.add"(%arg0, %arg1) : () -> ()\n%1 = "stablehlo.negate"(%arg0) : () -> ()')
    for i in range(3):
        got = e.run(x, x)
        np.testing.assert_array_equal(got[0][0], 2 * np.arange(6, dtype=np.float32))
    got = e.run(x)                           # %arg1 undefined: the add is skipped
    assert len(got) == 1
    np.testing.assert_array_equal(got[0][0], -np.arange(6, dtype=np.float32))
    e.close()


def test_cxx_api_selftest(dev):
    """The C++ API (jules_hip_pjrt.hpp): client, device, buffers, executeAsync,
    executePipeline, custom_call and error statuses, from a C++ program."""
    import os
    import subprocess
    case("pjrt C++ API selftest")
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "cpp",
                       "pjrt_selftest")
    assert os.path.exists(exe), "tests/cpp/pjrt_selftest is built by __graft_entry__.build()"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "pjrt selftest ok" in r.stdout, r.stdout + r.stderr
