"""Pins the CPU oracle (oracle/) before it is trusted as the GPU's checker.

The reference ships no golden vectors and cannot be compiled here (its kernel
headers include <cblas.h>, absent from the image), so every function is pinned
by what the mathematics fixes: fp64 evaluations of the textbook definitions,
closed forms (B = I, K = 1, A = 0, one-hot activations), invariants (V = 1,
Q = 0, causal row 0, permutation and tiling invariance) and exact brute force
(rational arithmetic) on tiny shapes.  Each check is chosen so that a
plausible slip in the restatement (dropped term, wrong coefficient, transposed
operand, wrong mask) fails it.
"""
import ctypes
import os
import shutil
import subprocess
from fractions import Fraction

import numpy as np
import pytest

from oracle import inputs as I
from oracle import pyoracle as po

ACTS = ["none", "relu", "sigmoid", "tanh", "gelu", "silu"]


# ---- exact fp32 arithmetic for brute force ---------------------------------
def _round_f32(x: Fraction) -> np.float32:
    """Correctly rounded (ties to even) Fraction -> float32."""
    f = np.float32(float(x))
    best = None
    for c in (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))):
        if not np.isfinite(c):
            continue
        d = abs(Fraction(float(c)) - x)
        if best is None or d < best[0] or (d == best[0] and (int(c.view(np.uint32)) & 1) == 0):
            best = (d, c)
    return best[1]


def fma32(a, b, c):
    return _round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def add32(a, b):
    return _round_f32(Fraction(float(a)) + Fraction(float(b)))


# ---- activations -----------------------------------------------------------
def _sweep():
    top = np.float32(88.0).view(np.uint32)
    pos = np.arange(0, top, 613, dtype=np.uint32).view(np.float32)
    return np.concatenate([pos, -pos])


def test_fast_exp_against_fp64():
    """Reference fast_exp_zmm (FusedKernels.h:90-133): degree-6 polynomial.
    Measured bound 1.74e-5 relative over [-87, 88]; a dropped Horner term or a
    wrong coefficient moves it past 1e-4, a wrong exponent bias past 0.5."""
    x = _sweep()
    y = po.fast_exp(x).astype(np.float64)
    e = np.exp(x.astype(np.float64))
    m = x > -87.0
    rel = np.abs(y[m] - e[m]) / e[m]
    assert rel.max() < 2.0e-5
    assert rel.max() > 1.0e-6  # it is a polynomial, not a libm call
    # exact points: 2^0 * p(0) = 1; clamp at -88 gives 2^-127 -> exponent bits 0 -> 0.0
    assert po.fast_exp(np.float32([0.0]))[0] == 1.0
    assert po.fast_exp(np.float32([-88.0, -1000.0]))[0] == 0.0
    assert po.fast_exp(np.float32([-1000.0]))[0] == 0.0
    assert po.fast_exp(np.float32([1000.0]))[0] == po.fast_exp(np.float32([88.0]))[0]


def test_fast_exp_planted_mistake_is_caught():
    """The bound above is tight enough to see the smallest plausible slip: the
    same polynomial with its last coefficient dropped, evaluated in numpy."""
    x = _sweep()
    x = x[(x > -80) & (x < 80)]
    r = (x * np.float32(1.4426950408889634)).astype(np.float32)
    ri = np.floor(r)
    rf = (r - ri).astype(np.float64)
    c = [1.0, 0.693147180, 0.240226507, 0.055495506, 0.009614425, 0.001333356]  # c6 dropped
    p = sum(ci * rf ** i for i, ci in enumerate(c))
    y = np.ldexp(p, ri.astype(np.int64))
    rel = np.abs(y - np.exp(x.astype(np.float64))) / np.exp(x.astype(np.float64))
    assert rel.max() > 2.0e-5


@pytest.mark.parametrize("act", ["sigmoid", "tanh", "gelu", "silu"])
def test_activation_against_fp64(act):
    x = np.linspace(-12, 12, 200001, dtype=np.float32)
    y = po.act_array(act, x).astype(np.float64)
    o = np.array([po.lib().jo64_act(po.ACT[act], float(v)) for v in x[::97]])
    yo = y[::97]
    # pointwise: |y - o| <= 1e-5 * max(|o|, |x| * 1e-3, 1e-3); normwise well under 1e-5
    assert np.max(np.abs(yo - o)) / np.max(np.abs(o)) < 1e-5
    # GELU(x) at large |x|: x for x >> 0, 0 for x << 0
    if act == "gelu":
        g = po.act_array("gelu", np.float32([-20.0, 20.0]))
        assert g[1] == np.float32(20.0) and abs(g[0]) < 1e-6


# ---- the reference's bits as g++ compiles them ------------------------------
_PROBE_SRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "gxx_activation_probe.cpp")
_PROBE_LIB = os.path.join(os.path.dirname(_PROBE_SRC), "libgxx_activation_probe.so")
# benchmarks/bench_kernel.cpp:15-19, plus -mavx512bw (GCC 11's headers need
# it); no -ffp-contract option, so C++'s default (fast) applies
_REF_FLAGS = ["-O3", "-mavx512f", "-mavx512dq", "-mavx512vl", "-mfma", "-mavx512bw"]


@pytest.fixture(scope="module")
def gxx_probe():
    """tests/cpp/gxx_activation_probe.cpp built with the reference's flags:
    the reference's intrinsic sequences as g++ compiles them."""
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    if (not os.path.exists(_PROBE_LIB)
            or os.path.getmtime(_PROBE_LIB) < os.path.getmtime(_PROBE_SRC)):
        tmp = _PROBE_LIB + ".tmp"
        subprocess.run(["g++", *_REF_FLAGS, "-fPIC", "-shared", _PROBE_SRC, "-o", tmp], check=True)
        os.replace(tmp, _PROBE_LIB)
    lib = ctypes.CDLL(_PROBE_LIB)
    if not lib.probe_has_avx512f():
        pytest.skip("host CPU has no AVX-512F")
    f = ctypes.POINTER(ctypes.c_float)
    lib.probe_act.argtypes = [ctypes.c_int, f, f, ctypes.c_int64]
    lib.probe_fused_gelu.argtypes = [f, f, ctypes.c_int]
    lib.probe_tiled.argtypes = [f, f, f] + [ctypes.c_int] * 7
    return lib


def _fp(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _act_inputs():
    """Every 97th fp32 bit pattern below |x| = 30, plus edge values."""
    top = np.float32(30.0).view(np.uint32)
    pos = np.arange(0, top, 97, dtype=np.uint32).view(np.float32)
    x = np.concatenate([pos, -pos, np.float32([88.0, -88.0, 1e30, -1e30, np.inf, -np.inf])])
    return np.ascontiguousarray(x[: x.size // 16 * 16])


@pytest.mark.parametrize("act", ["relu", "sigmoid", "tanh", "gelu"])
def test_vector_activation_matches_gxx_build(gxx_probe, act):
    """The restated vector-path activation equals the reference's intrinsic
    sequence compiled by g++ with the reference's flags, bit for bit, over
    ~21M inputs.  g++ fuses x + d*x^3 (gelu) and the add/subtract of
    exp = scale*poly (tanh, sigmoid) into fmas; a restatement that rounds
    those products separately fails (checked below for gelu)."""
    x = _act_inputs()
    want = np.empty_like(x)
    gxx_probe.probe_act(po.ACT[act], _fp(want), _fp(x), x.size)
    got = po.act_array(act, x)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gxx_contraction_is_visible():
    """Planted mistake: gelu with x + d*x^3 and exp's product each rounded
    on their own (no contraction) differs from the restatement on many
    inputs, so the bitwise check above can tell the two apart."""
    x = I.uniform(11, 0, (1 << 16,), -6, 6)
    y = po.act_array("gelu", x)
    f = np.float32
    x3 = x * (x * x)
    inner = f(0.7978845608) * (x + f(0.044715) * x3)
    two = (f(2.0) * inner).astype(np.float32)
    two = np.minimum(np.maximum(two, f(-88.0)), f(88.0))
    r = two * f(1.4426950408889634)
    ri = np.floor(r)
    rf = (r - ri).astype(np.float32)
    p = np.full_like(rf, f(0.000154040))
    for c in (0.001333356, 0.009614425, 0.055495506, 0.240226507, 0.693147180, 1.0):
        p = (p.astype(np.float64) * rf + f(c)).astype(np.float32)  # fma: one rounding
    e = (np.ldexp(np.float32(1.0), ri.astype(np.int32)).astype(np.float32) * p).astype(np.float32)
    t = ((e - f(1.0)) / (e + f(1.0))).astype(np.float32)
    twice_rounded = (f(0.5) * (x * (f(1.0) + t))).astype(np.float32)
    assert np.count_nonzero(twice_rounded != y) > 100


def test_fused_gelu_matches_gxx_build(gxx_probe):
    """fusedGelu (FusedKernels.h:606-627): the vector groups and the tanhf
    tail (where g++ fuses x + (0.044715*x*x)*x), bit for bit; both sides call
    the same libm tanhf."""
    for n in (5, 16, 37, 1000, 4099):
        x = I.uniform(12, n, (n,), -6, 6)
        want = np.empty_like(x)
        gxx_probe.probe_fused_gelu(_fp(want), _fp(x), n)
        np.testing.assert_array_equal(po.fused_gelu(x).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("act", ["none", "relu", "sigmoid", "tanh", "gelu"])
def test_tiled_gemm_matches_gxx_build(gxx_probe, act):
    """tiledMatmulWithActivation (FusedKernels.h:378-458) restated, against
    the g++ build of the same loops, bit for bit: the fmadd chains reloaded
    between K slices, the scalar columns past each tile's last 16-wide block
    (an fma chain after g++'s contraction of `sum += a*b`) and both
    epilogues, at ragged shapes and tiles with tails in every dimension."""
    for (M, N, K, tiles) in ((37, 53, 71, (16, 32, 16)), (64, 48, 96, (32, 32, 128)),
                             (8, 21, 7, (16, 16, 4)), (33, 100, 300, (16, 48, 64))):
        A = I.uniform(13, M, (M, K), -1, 1)
        B = I.uniform(13, N, (K, N), -1, 1)
        want = np.empty((M, N), np.float32)
        gxx_probe.probe_tiled(_fp(A), _fp(B), _fp(want), M, N, K, *tiles, po.ACT[act])
        got = po.tiled_matmul_act(A, B, act, tiles=tiles)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=str((M, N, K, tiles)))


def test_activation_closed_forms():
    x = np.float32([0.0, 1.0, -1.0, 3.0])
    assert list(po.act_array("relu", np.float32([-1.0, -0.0, 2.0, np.nan]))) == [0.0, 0.0, 2.0, 0.0]
    assert np.signbit(po.act_array("relu", np.float32([-0.0]))[0]) == np.False_  # maxps(-0, +0) = +0
    assert po.act_array("sigmoid", np.float32([0.0]))[0] == 0.5
    assert po.act_array("tanh", np.float32([0.0]))[0] == 0.0
    assert po.act_array("gelu", np.float32([0.0]))[0] == 0.0
    assert po.act_array("silu", np.float32([0.0]))[0] == 0.0
    np.testing.assert_array_equal(po.act_array("none", x), x)


def test_fused_gelu_matches_vector_path_and_tail():
    x = I.uniform(1, 0, (37,), -4, 4)
    y = po.fused_gelu(x)
    np.testing.assert_array_equal(y[:32], po.act_array("gelu", x[:32]))
    # the last 5 elements take the tanhf tail (FusedKernels.h:614-617): within
    # fp32 rounding of the fp64 formula
    t = x[32:].astype(np.float64)
    tail = 0.5 * t * (1.0 + np.tanh(0.7978845608 * (t + 0.044715 * t ** 3)))
    np.testing.assert_allclose(y[32:], tail, rtol=2e-6, atol=1e-7)


# ---- GEMM ----------------------------------------------------------------
@pytest.mark.parametrize("act", ACTS)
def test_gemm_against_fp64(act):
    A, B, bias = I.gemm_inputs(96, 80, 130, "f32", seed=3)
    y = po.matmul_bias_act(A, B, bias, act)
    o = po.gemm64(A, B, bias, act)
    assert I.rel_err(y, o) < 1e-5
    # the fp64 oracle agrees with an independent numpy evaluation
    z = A.astype(np.float64) @ B.astype(np.float64) + bias
    ref = np.array([[po.lib().jo64_act(po.ACT[act], float(v)) for v in row] for row in z[:4]])
    np.testing.assert_allclose(o[:4], ref, rtol=1e-12, atol=1e-12)


def test_gemm_identity_is_exact():
    """B = I: every fma adds an exact zero except one a*1, so C = act(A + bias)
    bit for bit; a transposed operand or dropped bias fails."""
    A = I.uniform(5, 0, (48, 64), -3, 3)
    bias = I.uniform(5, 2, (64,), -1, 1)
    for act in ACTS:
        y = po.matmul_bias_act(A, np.eye(64, dtype=np.float32), bias, act)
        np.testing.assert_array_equal(y, po.act_array(act, A + bias))


def test_gemm_k1_and_zero_a():
    A = I.uniform(6, 0, (32, 1), -2, 2)
    B = I.uniform(6, 1, (1, 48), -2, 2)
    bias = I.uniform(6, 2, (48,), -1, 1)
    y = po.matmul_bias_act(A, B, bias, "gelu")
    np.testing.assert_array_equal(y, po.act_array("gelu", (A * B) + bias))
    z = po.matmul_bias_act(np.zeros((16, 40), np.float32), I.uniform(6, 3, (40, 32), -1, 1),
                           bias[:32], "sigmoid")
    np.testing.assert_array_equal(z, np.broadcast_to(po.act_array("sigmoid", bias[:32] + 0.0), (16, 32)))


def test_gemm_bruteforce_fma_chain():
    """Exact rational fma chain on a ragged shape: every element is the
    sequential fma over k from 0, then one rounded add of bias.  Columns past
    the last 16-wide vector of a tile go through the scalar tail, which also
    chains in fma."""
    M, N, K = 3, 21, 7
    A = I.uniform(7, 0, (M, K), -1, 1)
    B = I.uniform(7, 1, (K, N), -1, 1)
    bias = I.uniform(7, 2, (N,), -1, 1)
    y = po.matmul_bias_act(A, B, bias, "none", tiles=(16, 16, 4))
    for i in range(M):
        for j in range(N):
            acc = np.float32(0.0)
            for k in range(K):
                acc = fma32(A[i, k], B[k, j], acc)
            assert y[i, j] == add32(acc, bias[j]), (i, j)


def test_gemm_tile_invariance():
    A, B, bias = I.gemm_inputs(64, 96, 200, "f32", seed=8)
    ys = [po.matmul_bias_act(A, B, bias, "gelu", tiles=t)
          for t in [(16, 16, 16), (32, 32, 128), (64, 96, 200), (48, 32, 24)]]
    for y in ys[1:]:
        np.testing.assert_array_equal(ys[0], y)


def test_tile_planner_restatement():
    """TilePlanner::computeAnalytical (TilePlanner.h:97-136) with this
    container's cache sizes as the reference reads them (index0 = 48K L1d,
    index1 = 32K L1i taken as L2): the tiles the reference's planner picks
    on that machine."""
    assert po.tile_analytical(512, 512, 512) == (32, 32, 128)
    assert po.tile_analytical(8, 8, 8) == (16, 16, 8)
    # K*N*4 fits 3/4 of L2 -> tile_k = K
    assert po.tile_analytical(64, 16, 64, l2=1 << 20) == (32, 16, 64)
    assert po.flash_tiles(1024, 64) == (4, 16)
    assert po.flash_tiles(4096, 128) == (4, 8)
    assert po.flash_tiles(1024, 64, l2=2 << 20) == (32, 64)


# ---- attention ---------------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("S,tiles", [(1, (32, 64)), (37, (32, 64)), (128, (4, 16)), (200, (32, 64))])
def test_flash_against_fp64(causal, S, tiles):
    Q, K, V = I.attn_inputs(2, 2, S, 64, "f32", seed=S)
    scale = 1.0 / np.sqrt(64.0)
    y = po.flash_attention(Q, K, V, causal, np.float32(scale), tiles)
    o = po.attention64(Q, K, V, causal, float(np.float32(scale)))
    assert I.rel_err(y, o) < 1e-5


def test_attention64_against_numpy():
    Q, K, V = I.attn_inputs(1, 1, 19, 64, "f32", seed=2)
    for causal in (False, True):
        o = po.attention64_head(Q[0, 0], K[0, 0], V[0, 0], causal, 0.125)
        s = Q[0, 0].astype(np.float64) @ K[0, 0].astype(np.float64).T * 0.125
        if causal:
            s[np.triu_indices(19, 1)] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        ref = (p / p.sum(1, keepdims=True)) @ V[0, 0].astype(np.float64)
        np.testing.assert_allclose(o, ref, rtol=1e-12, atol=1e-13)


def test_flash_invariants():
    B, H, S, D = 1, 2, 70, 64
    Q, K, V = I.attn_inputs(B, H, S, D, "f32", seed=11)
    ones = np.ones_like(V)
    for causal in (False, True):
        y = po.flash_attention(Q, K, ones, causal)
        np.testing.assert_allclose(y, 1.0, rtol=0, atol=4e-7)
        # Q = 0: uniform weights -> mean of visible V rows (prefix means if causal)
        z = po.flash_attention(np.zeros_like(Q), K, V, causal)
        if causal:
            ref = np.cumsum(V.astype(np.float64), axis=2) / np.arange(1, S + 1)[None, None, :, None]
        else:
            ref = np.broadcast_to(V.astype(np.float64).mean(axis=2, keepdims=True), V.shape)
        np.testing.assert_allclose(z, ref, rtol=0, atol=2e-6)
        # causal row 0 sees only key 0: O[0] = V[0] exactly
        if causal:
            c = po.flash_attention(Q, K, V, True)
            np.testing.assert_array_equal(c[:, :, 0], V[:, :, 0])
    # non-causal: permuting keys and values together changes nothing
    perm = np.random.default_rng(0).permutation(S)
    a = po.flash_attention(Q, K, V, False)
    b = po.flash_attention(Q, K[:, :, perm], V[:, :, perm], False)
    # the weights pass through fast_exp (1.7e-5 relative), so the order of
    # keys moves results at that level: compare at the fp32 normwise bar
    assert I.rel_err(b, a) < 1e-5
    # causal: changing keys/values after position i leaves rows <= i unchanged
    K2, V2 = K.copy(), V.copy()
    K2[:, :, 40:] += 1.0
    V2[:, :, 40:] -= 1.0
    c1 = po.flash_attention(Q, K, V, True)
    c2 = po.flash_attention(Q, K2, V2, True)
    np.testing.assert_array_equal(c1[:, :, :40], c2[:, :, :40])
    assert not np.array_equal(c1[:, :, 40:], c2[:, :, 40:])


def test_flash_tiling_invariance():
    Q, K, V = I.attn_inputs(1, 1, 96, 64, "f32", seed=5)
    ref = po.flash_attention(Q, K, V, True, tiles=(32, 64))
    for t in [(4, 8), (4, 16), (96, 96), (16, 32)]:
        assert I.rel_err(po.flash_attention(Q, K, V, True, tiles=t), ref) < 1e-5


# ---- int8 / W8A16 ------------------------------------------------------------
def test_w8a8_oracle_pinned():
    """The per-token / per-channel W8A8 restatement: with constant scale vectors
    it is matmulInt8's scalar path bit for bit; a one-hot A selects row k of B
    times its scales exactly; fp64 agrees to fp32 rounding."""
    A = I.int8_uniform(3, 0, (9, 70))
    B = I.int8_uniform(3, 1, (70, 33))
    bias = I.uniform(3, 2, (33,), -0.1, 0.1)
    y = po.w8a8(A, B, np.full(9, 0.013, np.float32), np.full(33, 0.021, np.float32), bias)
    assert np.array_equal(y, po.matmul_int8(A, B, 0.013, 0.021, bias))
    sa = I.uniform(3, 3, (9,), 1e-3, 1e-2)
    sb = I.uniform(3, 4, (33,), 1e-3, 1e-2)
    e = np.zeros((9, 70), np.int8)
    e[np.arange(9), np.arange(9) * 7] = 1
    y1 = po.w8a8(e, B, sa, sb)
    for i in range(9):
        want = B[7 * i].astype(np.float32) * (np.float32(sa[i]) * sb)
        assert np.array_equal(y1[i], want.astype(np.float32))
    y2 = po.w8a8(A, B, sa, sb, bias)
    ref = (A.astype(np.float64) @ B) * (sa.astype(np.float64)[:, None] * sb[None, :]) + bias
    assert I.rel_err(y2, ref) < 1e-6
    assert np.array_equal(po.w8a8(A, B, None, sb), po.w8a8(A, B, np.ones(9, np.float32), sb))


def test_matmul_int8_exact():
    A = I.int8_uniform(1, 0, (9, 70))
    B = I.int8_uniform(1, 1, (70, 33))
    bias = I.uniform(1, 2, (33,), -1, 1)
    sa, sb = np.float32(0.013), np.float32(0.021)
    y = po.matmul_int8(A, B, sa, sb, bias)
    acc = A.astype(np.int64) @ B.astype(np.int64)
    ref = (acc.astype(np.float32) * np.float32(sa * sb)) + bias
    np.testing.assert_array_equal(y, ref)
    # one-hot KAT: A = e_k picks row k of B (B indexed B[k*N+j], FusedKernels.h:1053)
    e = np.zeros((1, 70), np.int8)
    e[0, 17] = 1
    y1 = po.matmul_int8(e, B, 1.0, 1.0, None)
    np.testing.assert_array_equal(y1[0], B[17].astype(np.float32))


def test_w8a16_against_fp64_and_kat():
    x, W, scale, bias = I.w8a16_inputs(8, 64, 256, seed=4)
    y = po.w8a16(x, W, scale, bias, "silu")
    o = po.w8a16_64(x, W, scale, bias, "silu")
    assert I.rel_err(y, o) < 1e-5
    ref = x.astype(np.float64) @ W.astype(np.float64) * scale + bias
    ref = ref / (1 + np.exp(-ref))
    np.testing.assert_allclose(o, ref, rtol=1e-12, atol=1e-14)
    # one-hot x: acc = W[k0, j] exactly, y = act(W*scale + bias) bit for bit
    xh = np.zeros((2, 256), np.float32)
    xh[0, 5] = 1.0
    xh[1, 200] = 1.0
    yh = po.w8a16(xh, W, scale, bias, "silu")
    for r, k0 in ((0, 5), (1, 200)):
        pre = W[k0].astype(np.float32) * scale + bias
        np.testing.assert_array_equal(yh[r], po.act_array("silu", pre))


# ---- inputs / metric ------------------------------------------------------
def test_inputs_deterministic_and_distributed():
    a = I.normal(0, 1, (1 << 16,))
    np.testing.assert_array_equal(a, I.normal(0, 1, (1 << 16,)))
    assert not np.array_equal(a, I.normal(0, 2, (1 << 16,)))
    assert abs(a.mean()) < 0.02 and abs(a.std() - 1) < 0.02
    u = I.uniform(0, 0, (1 << 16,), -1, 1)
    assert u.min() >= -1 and u.max() < 1 and abs(u.mean()) < 0.02
    w = I.int8_uniform(0, 0, (1 << 16,))
    assert w.min() == -127 and w.max() == 127
    # sub-ranges are prefix independent
    np.testing.assert_array_equal(I.bits(3, 4, 10, offset=5), I.bits(3, 4, 15)[5:])


def test_bf16_round_matches_torch():
    torch = pytest.importorskip("torch")
    x = I.normal(1, 1, (100000,)) * np.float32(7.3)
    x[:4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 65504.0]  # ties both ways
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(I.bf16_round(x), ref)


def test_rel_err_metric():
    o = np.array([1.0, -4.0, 2.0])
    assert I.rel_err(o, o) == 0.0
    assert I.rel_err(o + np.array([0, 0.4, 0]), o) == pytest.approx(0.1)


# ---- row kernels (reference FusedKernels.h:464-526, :532-600, :766-854) ----
ROW_SHAPES = [(3, 1), (4, 10), (5, 15), (5, 16), (5, 17), (4, 31), (4, 33), (8, 256), (3, 1000)]


def _rows(M, N, seed, scale=3.0):
    return (np.random.default_rng(seed).standard_normal((M, N)) * scale).astype(np.float32)


@pytest.mark.parametrize("M,N", ROW_SHAPES)
def test_softmax_against_fp64_and_invariants(M, N):
    x = _rows(M, N, M * 100 + N)
    y = po.softmax(x)
    y64 = po.softmax64(x)
    assert I.rel_err(y, y64) < 2e-6
    assert np.abs(y.astype(np.float64).sum(1) - 1.0).max() < 2e-6
    # shift invariance: the row max is subtracted first
    y2 = po.softmax(x + np.float32(7.0))
    assert I.rel_err(y2, y64) < 5e-6
    # a uniform row gives exactly 1/N's rounding: every entry equal
    u = po.softmax(np.full((2, N), 0.25, np.float32))
    assert np.all(u == u[0, 0]) and abs(float(u[0, 0]) - 1.0 / N) < 1e-6 / N * 4


def test_softmax_split_between_fast_exp_and_expf():
    """Elements j < N & ~15 use fast_exp, the tail libm expf (reference :484-497)."""
    N = 20
    x = _rows(1, N, 7)
    y = po.softmax(x)
    mx = x.max()
    fe = po.fast_exp(x[0, :16] - mx)
    tail = np.exp((x[0, 16:] - mx).astype(np.float32))
    e = np.concatenate([fe, tail.astype(np.float32)])
    np.testing.assert_allclose(y[0], e / e.astype(np.float64).sum(), rtol=2e-6)
    # fast_exp is not libm exp: the restatement must be using it on the vector part
    assert np.any(fe != np.exp(x[0, :16] - mx).astype(np.float32))


@pytest.mark.parametrize("M,N", ROW_SHAPES)
def test_layernorm_against_fp64_and_closed_forms(M, N):
    x = _rows(M, N, M * 7 + N, scale=2.0) + np.float32(1.5)
    rng = np.random.default_rng(N)
    g = rng.standard_normal(N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    y = po.layernorm(x, g, b)
    assert I.rel_err(y, po.layernorm64(x, g, b)) < 2e-6
    # gamma = 1, beta = 0: zero mean, variance var / (var + eps)
    ones, zeros = np.ones(N, np.float32), np.zeros(N, np.float32)
    z = po.layernorm(x, ones, zeros).astype(np.float64)
    var = x.astype(np.float64).var(1)
    if N > 1:
        assert np.abs(z.mean(1)).max() < 1e-5
        np.testing.assert_allclose(z.var(1), var / (var + 1e-5), rtol=1e-5)
    # a constant row normalises to beta exactly
    c = po.layernorm(np.full((2, N), 3.25, np.float32), g, b)
    assert np.array_equal(c, np.broadcast_to(b, (2, N)))


def test_layernorm_planted_mistake_is_caught():
    """A slip that forgets the epsilon or uses the sample variance fails the fp64 check."""
    x = _rows(4, 33, 3)
    g, b = np.ones(33, np.float32), np.zeros(33, np.float32)
    y = po.layernorm(x, g, b)
    m = x.mean(1, keepdims=True)
    wrong = (x - m) / np.sqrt(x.var(1, ddof=1, keepdims=True) + 1e-5)
    assert I.rel_err(wrong.astype(np.float32), po.layernorm64(x, g, b)) > 1e-3
    assert I.rel_err(y, po.layernorm64(x, g, b)) < 2e-6


@pytest.mark.parametrize("M,N", [(1, 1), (4, 10), (5, 17), (8, 256), (3, 1000)])
def test_cross_entropy_against_fp64_and_invariants(M, N):
    x = _rows(M, N, 11 * M + N)
    t = np.random.default_rng(N).integers(0, N, M).astype(np.int32)
    t[0] = N - 1
    loss, g = po.cross_entropy(x, t)
    loss64, g64 = po.cross_entropy64(x, t)
    assert abs(loss - loss64) <= 2e-6 * max(1.0, abs(loss64))
    assert I.rel_err(g, g64) < 2e-6
    # gradient rows sum to 0; grad[target] = (p - 1) / M
    assert np.abs(g.astype(np.float64).sum(1)).max() < 1e-6
    p = po.softmax(x)
    np.testing.assert_allclose(g[np.arange(M), t], (p[np.arange(M), t] - 1.0) / M, rtol=1e-6,
                               atol=1e-9)
    # uniform logits: loss = log N (up to the 1e-10 guard)
    lu, _ = po.cross_entropy(np.zeros((M, N), np.float32), t)
    assert abs(lu - np.log(N)) < 1e-5 * max(1.0, np.log(N)) + 1e-6


# ---- 2-layer MLP forward + backward (interleavedMLPForwardBackward) --------
def _mlp_loss64(X, W1, b1, W2, b2, t):
    return po.mlp_forward_backward64(X, W1, b1, W2, b2, t)["loss"]


def test_mlp_oracle_gradients_match_finite_differences():
    """Central differences of the oracle's own loss, in fp64, on a tiny MLP:
    a dropped term, a transposed product or a wrong mask in any gradient
    fails.  (The analytic gradient is (p - onehot)/M, the derivative of
    -log p; the +1e-10 inside the log moves it by ~1e-10/p.)"""
    X, W1, b1, W2, b2, t = I.mlp_inputs(5, 4, 6, 3, seed=3, scaled=True)
    X, W1, b1, W2, b2 = (np.asarray(a, np.float64) for a in (X, W1, b1, W2, b2))
    g = po.mlp_forward_backward64(X, W1, b1, W2, b2, t)
    params = {"dX": X, "dW1": W1, "db1": b1, "dW2": W2, "db2": b2}
    eps = 1e-6
    for name, arr in params.items():
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            old = arr[idx]
            arr[idx] = old + eps
            lp = _mlp_loss64(X, W1, b1, W2, b2, t)
            arr[idx] = old - eps
            lm = _mlp_loss64(X, W1, b1, W2, b2, t)
            arr[idx] = old
            num[idx] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(g[name], num, rtol=1e-6, atol=1e-8, err_msg=name)
    # an explicit relu mask equal to h > 0 changes nothing; the opposite mask
    # changes the layer-1 gradients
    h = X @ W1 + b1
    same = po.mlp_forward_backward64(X, W1, b1, W2, b2, t, relu_mask=h > 0)
    flip = po.mlp_forward_backward64(X, W1, b1, W2, b2, t, relu_mask=h <= 0)
    for name in g:
        np.testing.assert_array_equal(np.asarray(same[name]), np.asarray(g[name]), err_msg=name)
    assert not np.allclose(flip["dW1"], g["dW1"]) and np.array_equal(flip["dW2"], g["dW2"])


def test_mlp_oracle_against_torch_autograd():
    """An independent implementation: torch autograd (CPU, fp64) of the same
    graph, with the loss written as in the reference (:188-194)."""
    torch = pytest.importorskip("torch")
    X, W1, b1, W2, b2, t = I.mlp_inputs(37, 20, 33, 10, seed=4, scaled=True)
    ts = [torch.tensor(np.asarray(a, np.float64), requires_grad=True) for a in (X, W1, b1, W2, b2)]
    Xt, W1t, b1t, W2t, b2t = ts
    h = Xt @ W1t + b1t
    o = torch.relu(h) @ W2t + b2t
    p = torch.softmax(o, dim=1)
    loss = -torch.log(p[torch.arange(37), torch.tensor(t, dtype=torch.long)] + 1e-10).sum() / 37
    loss.backward()
    g = po.mlp_forward_backward64(X, W1, b1, W2, b2, t)
    assert abs(g["loss"] - loss.item()) <= 1e-12 * abs(loss.item())
    np.testing.assert_allclose(g["output"], o.detach().numpy(), rtol=1e-12, atol=1e-12)
    for name, tt in zip(("dX", "dW1", "db1", "dW2", "db2"), ts):
        # autograd differentiates the +1e-10 too: relative effect <= 1e-10 / min p
        np.testing.assert_allclose(g[name], tt.grad.numpy(), rtol=1e-6, atol=1e-9, err_msg=name)


def test_mlp_oracle_closed_forms():
    """W2 = 0: the output is b2 in every row, so dO = (softmax(b2) -
    onehot(t))/M, db2 is its column sum, and nothing reaches layer 1 (dW1 =
    db1 = dX = 0).  The loss and dO part must also agree with the C
    restatement of fusedCrossEntropyLoss on the oracle's output."""
    X, W1, b1, W2, b2, t = I.mlp_inputs(9, 7, 5, 4, seed=5)
    W2 = np.zeros_like(W2)
    g = po.mlp_forward_backward64(X, W1, b1, W2, b2, t)
    np.testing.assert_allclose(g["output"], np.tile(b2.astype(np.float64), (9, 1)), atol=0)
    e = np.exp(b2.astype(np.float64) - b2.max())
    sm = e / e.sum()
    dO = np.tile(sm, (9, 1))
    dO[np.arange(9), t] -= 1
    dO /= 9
    np.testing.assert_allclose(g["db2"], dO.sum(0), rtol=1e-12, atol=1e-15)
    for name in ("dW1", "db1", "dX"):
        assert not np.any(g[name]), name
    # loss/dO against the C cross-entropy restatement at generic weights
    X, W1, b1, W2, b2, t = I.mlp_inputs(16, 8, 12, 6, seed=6, scaled=True)
    g = po.mlp_forward_backward64(X, W1, b1, W2, b2, t)
    loss_c, grad_c = po.cross_entropy64(g["output"].astype(np.float32), t)
    assert abs(loss_c - g["loss"]) <= 1e-6 * abs(g["loss"])
    a = np.maximum(np.asarray(X, np.float64) @ W1 + b1, 0)
    np.testing.assert_allclose(g["dW2"], a.T @ grad_c, rtol=1e-5, atol=1e-7)


def test_mlp_oracle_planted_mistake_is_caught():
    """A mask taken from the wrong sign (h < 0), planted in a copy of the
    oracle's backward, gives a db1 that the oracle's (finite-difference
    checked) db1 rejects."""
    X, W1, b1, W2, b2, t = I.mlp_inputs(5, 4, 6, 3, seed=3, scaled=True)
    X, W1, b1, W2, b2 = (np.asarray(a, np.float64) for a in (X, W1, b1, W2, b2))
    g = po.mlp_forward_backward64(X, W1, b1, W2, b2, t)
    h = X @ W1 + b1
    # rebuild dH with the planted sign error and compare db1
    a = np.where(h > 0, h, 0)
    o = a @ W2 + b2
    p = np.exp(o - o.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    p[np.arange(5), t] -= 1
    p /= 5
    wrong = np.where(h < 0, p @ W2.T, 0).sum(0)
    assert not np.allclose(wrong, g["db1"], rtol=1e-3)


# ---- attention backward ------------------------------------------------------
@pytest.mark.parametrize("causal", [False, True])
def test_attention_bwd_oracle_finite_differences(causal):
    """Central differences of L = sum(O * dO) with respect to Q, K and V, in
    fp64, on a tiny head: a wrong sign, a missing rowsum term, a transposed
    product or the scale on the wrong gradient fails."""
    rng = np.random.default_rng(7)
    Q, K, V, dO = (rng.standard_normal((1, 2, 5, 3)) for _ in range(4))
    scale = 0.7
    dQ, dK, dV, _ = po.attention_bwd64(Q, K, V, dO, causal, scale)

    def loss():
        return float(np.sum(po.attention_bwd64(Q, K, V, dO, causal, scale)[3] * dO))

    eps = 1e-6
    for name, arr, grad in (("dQ", Q, dQ), ("dK", K, dK), ("dV", V, dV)):
        num = np.zeros_like(arr)
        for idx in np.ndindex(arr.shape):
            old = arr[idx]
            arr[idx] = old + eps
            lp = loss()
            arr[idx] = old - eps
            lm = loss()
            arr[idx] = old
            num[idx] = (lp - lm) / (2 * eps)
        np.testing.assert_allclose(grad, num, rtol=1e-6, atol=1e-9, err_msg=name)


def test_attention_bwd_oracle_against_torch_autograd():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(8)
    Q, K, V, dO = (rng.standard_normal((2, 2, 9, 4)) for _ in range(4))
    for causal in (False, True):
        ts = [torch.tensor(a, requires_grad=True) for a in (Q, K, V)]
        s = ts[0] @ ts[1].transpose(-1, -2) * 0.5
        if causal:
            s = s.masked_fill(torch.triu(torch.ones(9, 9, dtype=torch.bool), 1), float("-inf"))
        O = torch.softmax(s, dim=-1) @ ts[2]
        (O * torch.tensor(dO)).sum().backward()
        got = po.attention_bwd64(Q, K, V, dO, causal, 0.5)
        np.testing.assert_allclose(got[3], O.detach().numpy(), rtol=1e-12, atol=1e-12)
        for g, t in zip(got[:3], ts):
            np.testing.assert_allclose(g, t.grad.numpy(), rtol=1e-10, atol=1e-12)
