"""GPU parity of the jules::kernel C++ entry points (include/jules_hip_kernel.hpp),
driven the way the reference's caller drives them (benchmarks/bench_kernel.cpp:
141,148,155,242,545): synchronous calls on host buffers, on device buffers,
and in place where the reference allows it.

tests/cpp/shim_selftest reads the seeded inputs this module writes, calls
every hot-path shim and writes the results back; they are compared here with
the oracle: bit-exact where the C ABI is bit-exact (the fp32 GEMM's fma chain
and its activations, fusedGelu's vector part, matmulInt8), within the fp32
bar (1e-5 against fp64) otherwise.  The planner, arena and
shouldUseFlashAttention checks run inside the program."""
import os
import subprocess

import numpy as np
import pytest

from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "cpp", "shim_selftest")

# shapes of tests/cpp/shim_selftest.cpp
GM, GN, GK = 67, 80, 45
GELU_N = 1000
RM, RN = 37, 100
AB, AH, AS, AD = 2, 3, 100, 64
I1, I2 = (8, 96, 256), (40, 70, 200)
ACTS = ["none", "relu", "sigmoid", "tanh", "gelu", "silu"]


def _inputs():
    x = {
        "gemm_A": I.uniform(0, 0, (GM, GK), -1, 1),
        "gemm_B": I.uniform(0, 1, (GK, GN), -1, 1),
        "gemm_bias": I.uniform(0, 2, (GN,), -1, 1),
        "gemm_C0": I.uniform(0, 3, (GM, GN), -1, 1),
        "gelu_x": I.uniform(1, 0, (GELU_N,), -6, 6),
        "row_x": I.normal(2, 0, (RM, RN), 3.0),
        "ln_gamma": I.normal(2, 1, (RN,)),
        "ln_beta": I.normal(2, 2, (RN,)),
        "ce_t": (np.arange(RM, dtype=np.int64) * 7 % RN).astype(np.int32),
        "attn_q": I.normal(3, 0, (AB, AH, AS, AD)),
        "attn_k": I.normal(3, 1, (AB, AH, AS, AD)),
        "attn_v": I.normal(3, 2, (AB, AH, AS, AD)),
        "i8_A1": I.int8_uniform(4, 0, (I1[0], I1[2])),
        "i8_B1": I.int8_uniform(4, 1, (I1[2], I1[1])),
        "i8_bias1": I.uniform(4, 2, (I1[1],), -1, 1),
        "i8_A2": I.int8_uniform(5, 0, (I2[0], I2[2])),
        "i8_B2": I.int8_uniform(5, 1, (I2[2], I2[1])),
        "i8_bias2": I.uniform(5, 2, (I2[1],), -1, 1),
    }
    return {k: np.ascontiguousarray(v) for k, v in x.items()}


@pytest.fixture(scope="module")
def run(dev, tmp_path_factory):
    """Write the inputs, run the selftest once, return (inputs, load)."""
    d = tmp_path_factory.mktemp("shims")
    x = _inputs()
    for k, v in x.items():
        v.tofile(str(d / f"{k}.bin"))
    case("shim_selftest (jules::kernel entry points on host and device buffers)")
    r = subprocess.run([EXE, str(d)], capture_output=True, text=True, timeout=120)
    print(r.stdout[-4000:], r.stderr[-2000:])
    assert r.returncode == 0 and "shim selftest ok" in r.stdout, r.stdout[-2000:]

    def load(name, shape, dtype=np.float32):
        return np.fromfile(str(d / f"{name}.bin"), dtype=dtype).reshape(shape)

    return x, load


def test_gemm_shims_bit_exact(run):
    """tiledMatmulWithActivation (every ActivationType), fusedMatmulRelu and
    fusedMatmulBiasRelu equal the restated fma chain bit for bit, on host and
    device buffers and with every kernel of the tile table."""
    x, load = run
    A, B, bias = x["gemm_A"], x["gemm_B"], x["gemm_bias"]
    for i, act in enumerate(ACTS):
        ref = po.tiled_matmul_act(A, B, act)
        for mode in "HD":
            np.testing.assert_array_equal(load(f"gemm_act{i}_{mode}", (GM, GN)), ref, err_msg=act)
    gelu = po.tiled_matmul_act(A, B, "gelu")
    for v in range(4):
        np.testing.assert_array_equal(load(f"gemm_var{v}", (GM, GN)), gelu, err_msg=f"variant {v}")
    for mode in "HD":
        np.testing.assert_array_equal(load(f"gemm_relu_{mode}", (GM, GN)),
                                      po.tiled_matmul_act(A, B, "relu"))
        np.testing.assert_array_equal(load(f"gemm_bias_relu_{mode}", (GM, GN)),
                                      po.matmul_bias_act(A, B, bias, "relu"))


def test_blas_matmul(run):
    """blasMatmul (FusedKernels.h:633-644): the plain product is the fma chain
    bit for bit; alpha, beta and transposes are within 1e-5 of fp64."""
    x, load = run
    A64, B64 = x["gemm_A"].astype(np.float64), x["gemm_B"].astype(np.float64)
    C0 = x["gemm_C0"].astype(np.float64)
    opA = {False: A64, True: A64.reshape(GK, GM).T}
    opB = {False: B64, True: B64.reshape(GN, GK).T}
    cases = {"blas_nn": (1.0, 0.0, False, False), "blas_ab": (0.5, 2.0, False, False),
             "blas_tn": (1.0, 0.0, True, False), "blas_nt": (-1.5, 0.0, False, True),
             "blas_tt": (2.0, -1.0, True, True)}
    for name, (alpha, beta, ta, tb) in cases.items():
        ref = alpha * (opA[ta] @ opB[tb]) + beta * C0
        for mode in "HD":
            y = load(f"{name}_{mode}", (GM, GN))
            assert I.rel_err(y, ref) < I.TOL["f32"], (name, mode)
    for mode in "HD":
        np.testing.assert_array_equal(load(f"blas_nn_{mode}", (GM, GN)),
                                      po.tiled_matmul_act(x["gemm_A"], x["gemm_B"], "none"))


def test_fused_gelu_with_tail(run):
    """fusedGelu at N = 1000: the first 992 elements (full groups of 16) are
    the vector path bit for bit; the 8-element tail follows the reference's
    tanhf formula (within 4 ulp of the restatement, which uses the host libm;
    the vector form would be ~1e-5 off there).  Host, device, in place, and
    in ExecutionArena memory."""
    x, load = run
    g = x["gelu_x"]
    ref = po.fused_gelu(g)
    nv = GELU_N & ~15
    x64 = g.astype(np.float64)
    ref64 = 0.5 * x64 * (1 + np.tanh(0.7978845608 * (x64 + 0.044715 * x64 ** 3)))
    for name in ("gelu_H", "gelu_I", "gelu_D", "gelu_DI", "gelu_arena"):
        y = load(name, (GELU_N,))
        np.testing.assert_array_equal(y[:nv], ref[:nv], err_msg=name)
        ulp = np.spacing(np.abs(ref[nv:]).astype(np.float32))
        assert np.all(np.abs(y[nv:] - ref[nv:]) <= 4 * ulp), name
        assert I.rel_err(y, ref64) < I.TOL["f32"], name


def test_row_kernel_shims(run):
    """fusedSoftmax, fusedLayerNorm, fusedCrossEntropyLoss through the shims:
    within the fp32 bar of fp64 and within rounding of the restated reference;
    in place on host and device buffers."""
    x, load = run
    rx, t = x["row_x"], x["ce_t"]
    for name in ("softmax_H", "softmax_I", "softmax_DI"):
        y = load(name, (RM, RN))
        assert I.rel_err(y, po.softmax64(rx)) < I.TOL["f32"], name
        assert I.rel_err(y, po.softmax(rx)) < 2e-6, name
    for name in ("layernorm_H", "layernorm_DI"):
        y = load(name, (RM, RN))
        assert I.rel_err(y, po.layernorm64(rx, x["ln_gamma"], x["ln_beta"])) < I.TOL["f32"], name
    loss64, grad64 = po.cross_entropy64(rx, t)
    for mode in ("H", "I", "DI"):
        g = load(f"ce_grad_{mode}", (RM, RN))
        loss = load(f"ce_loss_{mode}", (1,))[0]
        assert I.rel_err(g, grad64) < I.TOL["f32"], mode
        assert abs(loss - loss64) <= I.TOL["f32"] * abs(loss64), mode


def test_attention_shims(run):
    """flashAttention, attention and standardAttention (non-causal, scale
    1/sqrtf(D), FlashAttention.h:130-135) against fp64."""
    x, load = run
    q, k, v = x["attn_q"], x["attn_k"], x["attn_v"]
    scale = float(np.float32(1.0) / np.sqrt(np.float32(AD)))
    ref = po.attention64(q, k, v, False, scale)
    for name in ("flash_H", "flash_D", "attention_H", "standard_H"):
        y = load(name, q.shape)
        assert I.rel_err(y, ref) < I.TOL["f32"], name


def test_matmul_int8_shim(run):
    """matmulInt8 (scalar-path semantics, FusedKernels.h:1046-1066), bit for
    bit: the decode path with bias on host and device buffers, the general
    path without."""
    x, load = run
    ref1 = po.matmul_int8(x["i8_A1"], x["i8_B1"], 0.013, 0.021, x["i8_bias1"])
    for mode in "HD":
        np.testing.assert_array_equal(load(f"i8_1_{mode}", (I1[0], I1[1])), ref1)
    np.testing.assert_array_equal(load("i8_2_H", (I2[0], I2[1])),
                                  po.matmul_int8(x["i8_A2"], x["i8_B2"], 0.5, 0.25))
