"""GPU parity of the row kernels: jules_hip_softmax, jules_hip_layernorm and
jules_hip_cross_entropy (reference FusedKernels.h:464-526, :532-600,
:766-854), fp32.

Each is compared with the fp64 oracle at the fp32 bar (1e-5, normwise) and
with the restated reference path to rounding (the GPU sums in a fixed tree
order instead of the reference's 16 lane partials).  Shapes cover the
reference's own benchmark shapes (softmax [64,256], [64,10], [2048,2048];
layernorm [64,256], [2048,256]), the 16-element vector/tail split (N = 15,
16, 17, 33), N = 1, ragged M, rows held in registers at every cache size,
rows of 4097-65536 held by one 1024-thread block (16-byte and 4-byte
accesses, with and without a tail), rows longer than 65536 (the streaming
passes, 16-byte and 4-byte accesses, up to 131073), rows that are not
16-byte aligned (the 4-byte path) and in-place softmax and cross entropy.
Up to 64 rows longer than 65536 are split over 4096-element segments (three
launches); the shapes with 65 rows keep the one-workgroup-per-row streaming
path covered."""
import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case, registry_call, to_dev, to_np

pytestmark = pytest.mark.gpu

SHAPES = [(64, 256), (64, 10), (2048, 2048), (2048, 256), (1, 1), (3, 15), (5, 16), (7, 17),
          (9, 33), (13, 100), (6, 600), (5, 1500), (3, 4000), (3, 4096), (2, 4097), (2, 10000),
          (3, 16386), (2, 20001), (2, 32768), (2, 32769), (2, 40000), (2, 50257), (2, 65536),
          (2, 65537), (1, 131073),
          # the most rows the split path takes (64), and one more: one streaming
          # workgroup per row
          (64, 65537), (65, 70001)]


def _x(M, N, seed, scale=3.0):
    return (np.random.default_rng(seed).standard_normal((M, N)) * scale).astype(np.float32)


# The restated reference sums each row as 16 sequential fp32 lane partials,
# whose rounding grows with N (its outputs differ from their own fp64
# renormalisation by up to 5e-7 at N <= 32768, 2.7e-6 at N = 40000, 3e-6 at
# N = 131073); the kernels sum in a tree and land within 3e-7 of the exact
# sum.  Up to RAW_N the kernels are held to the reference's own outputs at
# 2e-6; at every N they are held, element by element, to the reference's
# per-element arithmetic (fast_exp on whole 16-float vectors, expf on the
# tail) with the row sum taken exactly: the reference's output renormalised
# in fp64.  A per-element mistake (expf on the vector part, fast_exp on the
# tail) moves elements by 9e-6 to 1.4e-5 of their value, so the 1e-6 bar
# catches it.
RAW_N = 32768


def _exact_sum(r):
    r = np.asarray(r, np.float64)
    return r / r.sum(axis=-1, keepdims=True)


def _ratio_err(y, ref):
    m = np.abs(ref) > 1e-30
    return float(np.max(np.abs(np.asarray(y, np.float64)[m] / ref[m] - 1.0))) if m.any() else 0.0


def _check_softmax(y, x):
    r = po.softmax(x)
    assert _ratio_err(y, _exact_sum(r)) < 1e-6
    if x.shape[1] <= RAW_N:
        assert I.rel_err(y, r) < 2e-6


def _check_cross_entropy(loss, g, x, t):
    M, N = x.shape
    rows = np.arange(M)
    p = _exact_sum(po.softmax(x))
    gx = p / M
    gx[rows, t] -= 1.0 / M
    off = np.ones_like(gx, bool)
    off[rows, t] = False
    assert _ratio_err(np.where(off, g, 0.0), np.where(off, gx, 0.0)) < 1e-6
    assert np.max(np.abs(g[rows, t] - gx[rows, t])) <= 1e-6 / M
    lx = float(np.mean(-np.log(p[rows, t] + 1e-10)))
    assert abs(loss - lx) <= 2e-6 * max(1.0, abs(lx))
    if N <= RAW_N:
        lr, gr = po.cross_entropy(x, t)
        assert I.rel_err(g, gr) < 2e-6
        assert abs(loss - lr) <= 2e-6 * max(1.0, abs(lr))


@pytest.mark.parametrize("M,N", SHAPES)
def test_softmax(dev, M, N):
    case(f"softmax [{M},{N}]")
    x = _x(M, N, M * 31 + N)
    y = to_np(ops.softmax(to_dev(x, torch.float32, dev)))
    assert I.rel_err(y, po.softmax64(x)) < I.TOL["f32"]
    _check_softmax(y, x)
    assert np.abs(y.astype(np.float64).sum(1) - 1.0).max() < 1e-5


@pytest.mark.parametrize("N", [300, 40000, 70001])
def test_softmax_in_place_and_extremes(dev, N):
    case(f"softmax in place, large and -inf logits N={N}")
    x = _x(16, N, 5, scale=40.0)
    x[3, :] = -np.inf
    x[3, 7] = 0.0                      # one finite logit: that entry is 1
    x[4, :] = 1e30                     # all equal, huge: uniform
    t = to_dev(x, torch.float32, dev)
    ops.softmax(t, out=t)
    y = to_np(t)
    _check_softmax(y, x)
    assert y[3, 7] == 1.0 and np.all(np.delete(y[3], 7) == 0.0)
    np.testing.assert_allclose(y[4], 1.0 / N, rtol=1e-6)


@pytest.mark.parametrize("M,N", SHAPES)
def test_layernorm(dev, M, N):
    case(f"layernorm [{M},{N}]")
    x = _x(M, N, M * 17 + N, scale=2.0) + np.float32(0.75)
    rng = np.random.default_rng(N)
    g = rng.standard_normal(N).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    y = to_np(ops.layernorm(to_dev(x, torch.float32, dev), to_dev(g, torch.float32, dev),
                            to_dev(b, torch.float32, dev)))
    assert I.rel_err(y, po.layernorm64(x, g, b)) < I.TOL["f32"]
    assert I.rel_err(y, po.layernorm(x, g, b)) < 2e-6


def test_layernorm_epsilon_and_constant_rows(dev):
    case("layernorm epsilon, constant rows")
    N = 96
    x = _x(8, N, 9)
    x[2, :] = 5.0                      # constant row -> beta exactly
    g = np.full(N, 1.5, np.float32)
    b = np.linspace(-1, 1, N).astype(np.float32)
    for eps in (1e-5, 0.1, 0.0):
        y = to_np(ops.layernorm(to_dev(x, torch.float32, dev), to_dev(g, torch.float32, dev),
                                to_dev(b, torch.float32, dev), eps=eps))
        ok = np.arange(8) != 2 if eps == 0.0 else np.ones(8, bool)
        assert I.rel_err(y[ok], po.layernorm64(x, g, b, eps)[ok]) < I.TOL["f32"]
        if eps > 0:
            assert np.array_equal(y[2], b)


@pytest.mark.parametrize("M,N", [(64, 10), (128, 1000), (7, 17), (1, 1), (5, 4096), (3, 7000),
                                 (2048, 512), (3, 32000), (2, 20001), (2, 40000), (2, 50257),
                                 (2, 65537), (2, 131072), (64, 65540), (65, 131072)])
def test_cross_entropy(dev, M, N):
    case(f"cross entropy [{M},{N}]")
    x = _x(M, N, 3 * M + N)
    t = np.random.default_rng(M + N).integers(0, N, M).astype(np.int32)
    t[0] = N - 1
    loss, g = ops.cross_entropy(to_dev(x, torch.float32, dev), to_dev(t, torch.int32, dev))
    loss, g = float(to_np(loss)[0]), to_np(g)
    loss64, g64 = po.cross_entropy64(x, t)
    assert abs(loss - loss64) <= I.TOL["f32"] * max(1.0, abs(loss64))
    assert I.rel_err(g, g64) < I.TOL["f32"]
    _check_cross_entropy(loss, g, x, t)


@pytest.mark.parametrize("M,N", [(40000, 8), (16384, 16), (20001, 12)])
def test_cross_entropy_many_rows(dev, M, N):
    """More rows than the loss reduction's 1024 threads x 16 loads (a second
    round), at a power-of-two M (gradient by the product with 1/M) and two
    others (the division)."""
    case(f"cross entropy many rows [{M},{N}]")
    x = _x(M, N, M + N)
    t = np.random.default_rng(M).integers(0, N, M).astype(np.int32)
    loss, g = ops.cross_entropy(to_dev(x, torch.float32, dev), to_dev(t, torch.int32, dev))
    loss, g = float(to_np(loss)[0]), to_np(g)
    loss64, g64 = po.cross_entropy64(x, t)
    assert abs(loss - loss64) <= I.TOL["f32"] * max(1.0, abs(loss64))
    assert I.rel_err(g, g64) < I.TOL["f32"]
    # the gradient is (p - onehot) / M with the reference's rounding: exactly
    # the restatement's division of the kernel's own p - onehot
    xt = to_dev(x, torch.float32, dev)
    p = ops.softmax(xt).cpu().numpy()
    p[np.arange(M), t] -= np.float32(1.0)
    np.testing.assert_array_equal(g, (p / np.float32(M)).astype(np.float32))


def test_cross_entropy_bad_target_and_repeat(dev):
    """An out-of-range target gives a NaN loss (the reference reads out of
    bounds); the workspace is reused across calls without stale data."""
    case("cross entropy bad target, repeated calls")
    x = _x(6, 50, 1)
    t = np.array([0, 49, 3, 3, 10, 20], np.int32)
    xt, ws = to_dev(x, torch.float32, dev), ops.cross_entropy_workspace(6, dev)
    l1, _ = ops.cross_entropy(xt, to_dev(t, torch.int32, dev), workspace=ws)
    bad = t.copy()
    bad[2] = 50
    l2, g2 = ops.cross_entropy(xt, to_dev(bad, torch.int32, dev), workspace=ws)
    l3, _ = ops.cross_entropy(xt, to_dev(t, torch.int32, dev), workspace=ws)
    assert np.isfinite(float(to_np(l1)[0])) and np.isnan(float(to_np(l2)[0]))
    assert float(to_np(l1)[0]) == float(to_np(l3)[0])
    # the bad row's gradient is the plain softmax / M (no onehot subtraction)
    np.testing.assert_allclose(to_np(g2)[2], po.softmax(x)[2] / 6, rtol=2e-6)


@pytest.mark.parametrize("M,N", [(5, 256), (5, 2048), (5, 8192), (5, 40000), (5, 70000),
                                 (65, 40000), (65, 70000)])
def test_unaligned_rows_and_in_place(dev, M, N):
    """Rows whose start is only 4-byte aligned take the 4-byte path (same
    results); cross entropy with grad written over the logits.  Five rows of
    70000 take the split path, 65 the streaming one."""
    case(f"row kernels unaligned, in place [{M},{N}]")
    x = _x(M, N, N + 1)
    flat = torch.empty((M * N + 1,), dtype=torch.float32, device=dev)
    xs = flat[1:].view(M, N)
    xs.copy_(to_dev(x, torch.float32, dev))
    assert xs.data_ptr() % 16 != 0
    y = to_np(ops.softmax(xs, out=torch.empty_like(xs)))
    _check_softmax(y, x)
    g = np.linspace(-1, 1, N).astype(np.float32)
    b = np.linspace(2, 0, N).astype(np.float32)
    gf = torch.empty((N + 1,), dtype=torch.float32, device=dev)
    gs = gf[1:]
    gs.copy_(to_dev(g, torch.float32, dev))
    y = to_np(ops.layernorm(xs, gs, to_dev(b, torch.float32, dev), eps=1e-5))
    assert I.rel_err(y, po.layernorm64(x, g, b, 1e-5)) < I.TOL["f32"]
    t = np.random.default_rng(N).integers(0, N, M).astype(np.int32)
    loss, gg = ops.cross_entropy(xs, to_dev(t, torch.int32, dev), grad=xs)  # in place, unaligned
    _check_cross_entropy(float(to_np(loss)[0]), to_np(gg), x, t)
    xa = to_dev(x, torch.float32, dev)
    loss, gg = ops.cross_entropy(xa, to_dev(t, torch.int32, dev), grad=xa)  # in place, aligned
    _check_cross_entropy(float(to_np(loss)[0]), to_np(gg), x, t)


@pytest.mark.parametrize("N", [70000, 70003])
def test_split_rows_segment_edges(dev, N):
    """Few long rows are split over workgroups of 4096-element segments
    (16-byte accesses at N = 70000, 4-byte with a tail at 70003): the targets
    sit on both sides of a segment edge and at the row's end, one row has an
    invalid target (NaN loss, no onehot subtraction), and the cross entropy
    runs in place."""
    case(f"split rows, segment edges N={N}")
    M = 4
    x = _x(M, N, 77)
    t = np.array([4095, 4096, N - 1, N], np.int32)  # the last one is invalid
    xt = to_dev(x, torch.float32, dev)
    _check_softmax(to_np(ops.softmax(xt)), x)
    gam = np.linspace(-1, 1, N).astype(np.float32)
    bet = np.linspace(2, 0, N).astype(np.float32)
    y = to_np(ops.layernorm(xt, to_dev(gam, torch.float32, dev), to_dev(bet, torch.float32, dev)))
    assert I.rel_err(y, po.layernorm64(x, gam, bet)) < I.TOL["f32"]
    assert I.rel_err(y, po.layernorm(x, gam, bet)) < 2e-6
    loss, g = ops.cross_entropy(xt, to_dev(t, torch.int32, dev), grad=xt)  # in place
    assert np.isnan(float(to_np(loss)[0]))
    g = to_np(g)
    # (p - onehot) / M, the invalid row without the onehot
    p = _exact_sum(po.softmax(x))
    gx = p / M
    rows = np.arange(3)
    gx[rows, t[:3]] -= 1.0 / M
    off = np.ones_like(gx, bool)
    off[rows, t[:3]] = False
    assert _ratio_err(np.where(off, g, 0.0), np.where(off, gx, 0.0)) < 1e-6
    assert np.max(np.abs(g[rows, t[:3]] - gx[rows, t[:3]])) <= 1e-6 / M


def test_registry_row_kernels(dev):
    """fusedSoftmax / fusedLayerNorm / fusedCrossEntropyLoss through jules_hip_lookup."""
    case("registry row kernels")
    x = _x(12, 80, 2)
    xt = to_dev(x, torch.float32, dev)
    y = torch.empty_like(xt)
    st = registry_call("fusedSoftmax", [xt], [y])
    assert st == 0, _lib.lib().jules_hip_last_error()
    assert I.rel_err(to_np(y), po.softmax64(x)) < I.TOL["f32"]
    g = to_dev(np.full(80, 2.0, np.float32), torch.float32, dev)
    b = to_dev(np.full(80, -1.0, np.float32), torch.float32, dev)
    st = registry_call("fusedLayerNorm", [xt, g, b], [y], b"epsilon=0.5")
    assert st == 0, _lib.lib().jules_hip_last_error()
    assert I.rel_err(to_np(y), po.layernorm64(x, np.full(80, 2.0), np.full(80, -1.0), 0.5)) < I.TOL["f32"]
    t = to_dev(np.arange(12, dtype=np.int32) * 5, torch.int32, dev)
    loss = torch.empty((1,), dtype=torch.float32, device=dev)
    st = registry_call("fusedCrossEntropyLoss", [xt, t], [y, loss])
    assert st == 0, _lib.lib().jules_hip_last_error()
    l64, g64 = po.cross_entropy64(x, np.arange(12, dtype=np.int32) * 5)
    assert abs(float(to_np(loss)[0]) - l64) < 1e-5 * max(1, abs(l64))
    assert I.rel_err(to_np(y), g64) < I.TOL["f32"]
