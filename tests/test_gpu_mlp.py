"""GPU parity of the 2-layer MLP forward + loss + backward
(jules_hip_mlp_forward_backward; reference interleavedMLPForwardBackward,
InterleavedAutodiff.h:55-441) against the fp64 oracle
(po.mlp_forward_backward64, pinned in tests/test_oracle.py by finite
differences, torch autograd and closed forms).

fp32 bar: every output within 1e-5 of the oracle, as max |y - ref| / max |ref|
per tensor (the reference's products are BLAS calls, so only a tolerance is
defined: parity of the exact bits is unpinned).  The loss within 1e-5
relative.  relu'(h) for the few h within fp32 rounding of 0 is decided by
rounding, so the backward is checked against the oracle run with the GPU's
own mask (a > 0, read from the workspace), after checking that the GPU's
activations match the oracle's and that every mask disagreement sits at
|h| < 1e-4."""
import os
import subprocess

import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case, registry_call, to_dev, to_np

pytestmark = pytest.mark.gpu
TOL = 1e-5
NAMES = ("output", "dW1", "db1", "dW2", "db2", "dX")


def _run(dev, ins, with_dX=True, workspace=None):
    X, W1, b1, W2, b2, t = ins
    args = [to_dev(a, torch.float32, dev) for a in (X, W1, b1, W2, b2)]
    return ops.mlp_forward_backward(*args, to_dev(t, torch.int32, dev), with_dX=with_dX,
                                    workspace=workspace)


def _check(got, ins, with_dX=True, act=None):
    """act: the GPU's activations relu(X W1 + b1) (first M*N1 floats of the
    workspace), or None to use the oracle's mask."""
    mask = None
    if act is not None:
        X, W1, b1 = (np.asarray(a, np.float64) for a in ins[:3])
        h = X @ W1 + b1
        assert I.rel_err(act, np.maximum(h, 0)) < TOL, "activations"
        mask = act > 0
        flips = mask != (h > 0)
        assert flips.sum() <= max(2, flips.size // 100000), int(flips.sum())
        assert np.all(np.abs(h[flips]) < 1e-4 * np.abs(h).max())
    ref = po.mlp_forward_backward64(*ins, relu_mask=mask)
    for n in NAMES:
        if n == "dX" and not with_dX:
            assert got[n] is None
            continue
        err = I.rel_err(to_np(got[n]), ref[n])
        assert err < TOL, f"{n}: rel err {err:.3g}"
    loss = float(to_np(got["loss"])[0])
    assert abs(loss - ref["loss"]) <= TOL * abs(ref["loss"]), (loss, ref["loss"])


def _run_check(dev, ins, with_dX=True):
    M, N1 = ins[0].shape[0], ins[1].shape[1]
    ws = ops.mlp_workspace(M, ins[0].shape[1], N1, ins[3].shape[1], dev)
    got = _run(dev, ins, with_dX, ws)
    act = ws[:M * N1 * 4].view(torch.float32).reshape(M, N1).cpu().numpy()
    _check(got, ins, with_dX, act)


def test_reference_benchmark_shape(dev):
    """bench_kernel.cpp:268-290: MLP [64, 784] -> 256 -> 10, all operands
    U[-1, 1] (the softmax saturates), with dX."""
    case("mlp 64x784x256x10 unscaled")
    ins = I.mlp_inputs(64, 784, 256, 10, seed=0)
    _run_check(dev, ins)


@pytest.mark.parametrize("M,K1,N1,N2", [(1, 1, 1, 2), (37, 50, 33, 10), (130, 200, 129, 17),
                                        (257, 64, 300, 1000), (1000, 96, 160, 33),
                                        (128, 128, 128, 128), (2048, 512, 384, 100)])
def test_shapes_against_fp64(dev, M, K1, N1, N2):
    case(f"mlp {M}x{K1}x{N1}x{N2}")
    ins = I.mlp_inputs(M, K1, N1, N2, seed=M + K1 + N1 + N2, scaled=True)
    _run_check(dev, ins)
    _run_check(dev, ins, with_dX=False)


def test_deterministic(dev):
    case("mlp determinism")
    ins = I.mlp_inputs(300, 130, 250, 40, seed=9, scaled=True)
    a, b = _run(dev, ins), _run(dev, ins)
    for n in NAMES + ("loss",):
        assert torch.equal(a[n], b[n]), n


def test_zero_rows_and_bad_target(dev):
    """M = 0: gradients zeroed, loss NaN (the reference's 0/0).  A target
    outside [0, N2): NaN loss, as jules_hip_cross_entropy."""
    case("mlp M=0 and out-of-range target")
    X, W1, b1, W2, b2, t = I.mlp_inputs(8, 6, 5, 4, seed=2, scaled=True)
    args = [to_dev(a, torch.float32, dev) for a in (X[:0], W1, b1, W2, b2)]
    g = ops.mlp_forward_backward(*args, to_dev(t[:0], torch.int32, dev))
    assert torch.isnan(g["loss"]).all()
    for n in ("dW1", "db1", "dW2", "db2"):
        assert not torch.any(g[n]), n
    t = t.copy()
    t[3] = 4
    g = _run(dev, (X, W1, b1, W2, b2, t))
    assert torch.isnan(g["loss"]).all()


def test_registry_path(dev):
    case("registry interleavedMLPForwardBackward")
    X, W1, b1, W2, b2, t = ins = I.mlp_inputs(33, 40, 24, 7, seed=12, scaled=True)
    tin = [to_dev(a, torch.float32, dev) for a in (X, W1, b1, W2, b2)] + [to_dev(t, torch.int32, dev)]
    outs = [torch.empty(s, dtype=torch.float32, device=dev)
            for s in ((33, 7), (40, 24), (24,), (24, 7), (7,), (1,), (33, 40))]
    st = registry_call("interleavedMLPForwardBackward", tin, outs)
    assert st == 0, _lib.lib().jules_hip_last_error()
    got = dict(zip(("output", "dW1", "db1", "dW2", "db2", "loss", "dX"), outs))
    _check(got, ins)


@pytest.mark.parametrize("M,K1,N1,N2", [(64, 784, 256, 10), (1, 1, 1, 1), (37, 50, 33, 10),
                                        (257, 64, 300, 1000), (2048, 512, 384, 100), (8, 4096, 4096, 8)])
def test_forward_against_fp64(dev, M, K1, N1, N2):
    """fusedMLPForward (FusedKernels.h:659-760): relu(X W1 + b1) W2 + b2,
    within 1e-5 of the oracle's forward; two calls in a row agree bit for
    bit, and the forward agrees with the forward half of the training step
    bit for bit (same GEMMs, same split plan)."""
    case(f"mlp forward {M}x{K1}x{N1}x{N2}")
    ins = I.mlp_inputs(M, K1, N1, N2, seed=M * 3 + K1 + N1 + N2, scaled=True)
    X, W1, b1, W2, b2 = (to_dev(a, torch.float32, dev) for a in ins[:5])
    y = ops.mlp_forward(X, W1, b1, W2, b2)
    ref = po.mlp_forward_backward64(*ins)["output"]
    err = I.rel_err(to_np(y), ref)
    assert err < TOL, f"rel err {err:.3g}"
    assert torch.equal(y, ops.mlp_forward(X, W1, b1, W2, b2))
    if N2 > 1:
        step = ops.mlp_forward_backward(X, W1, b1, W2, b2, to_dev(ins[5], torch.int32, dev))
        assert torch.equal(y, step["output"])


def test_forward_zero_rows_and_registry(dev):
    case("mlp forward M=0 and registry fusedMLPForward")
    X, W1, b1, W2, b2, _ = ins = I.mlp_inputs(21, 40, 24, 7, seed=5, scaled=True)
    d = [to_dev(a, torch.float32, dev) for a in (X, W1, b1, W2, b2)]
    assert ops.mlp_forward(d[0][:0], *d[1:]).shape == (0, 7)
    out = torch.full((21, 7), float("nan"), dtype=torch.float32, device=dev)
    st = registry_call("fusedMLPForward", d, [out])
    assert st == 0, _lib.lib().jules_hip_last_error()
    assert I.rel_err(to_np(out), po.mlp_forward_backward64(*ins)["output"]) < TOL
    st = registry_call("fusedMLPForward", d[:4], [out])
    assert st != 0


def test_cxx_kernel_selftest(dev):
    """jules::kernel::interleavedMLPForwardBackward and fusedMLPForward with
    host buffers, from a C++ program, against its own double-precision
    loops."""
    case("kernel C++ selftest")
    exe = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "tests", "cpp",
                       "kernel_selftest")
    assert os.path.exists(exe), "tests/cpp/kernel_selftest is built by __graft_entry__.build()"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "kernel selftest ok" in r.stdout, r.stdout + r.stderr
