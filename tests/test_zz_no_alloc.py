"""GPU check of the W8A16 entry point that allocates nothing
(jules_hip_w8a16_gemm_bias_act_noalloc; no counterpart in the reference, for
callers that cannot allocate): through the C ABI its output equals the bits of
jules_hip_w8a16_gemm_bias_act with a caller workspace (same kernels, fixed
reduction order) on consecutive calls whose sizes shrink, so the second call
runs on the scratch the first one left behind; the largest shape that fits the
static scratch works, and one column tile more is rejected before any launch;
captured once in a HIP graph, the call replays correctly with new inputs;
after every pattern of calls (different split counts back to back, graph
replays) the per-tile arrival counters in the static array are back at 0."""
import ctypes

import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from jules_amd._lib import ACT
from oracle import inputs as I
from tests.helpers import case, to_dev

pytestmark = pytest.mark.gpu

OK, WORKSPACE = 0, 6


def _operands(dev, M, N, K, seed):
    x, W, scale, bias = I.w8a16_inputs(M, N, K, seed=seed)
    return (to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
            to_dev(scale, torch.float32, dev), to_dev(bias, torch.float32, dev))


def _noalloc(x, W, scale, bias, act, y):
    M, K = x.shape
    N = W.shape[1]
    return _lib.lib().jules_hip_w8a16_gemm_bias_act_noalloc(
        ACT[act], x.data_ptr(), W.data_ptr(), scale.data_ptr(),
        None if bias is None else bias.data_ptr(), y.data_ptr(), M, N, K,
        torch.cuda.current_stream().cuda_stream)


@pytest.mark.parametrize("act,with_bias", [("silu", True), ("gelu", False)])
def test_noalloc_equals_workspace_entry_point(dev, act, with_bias):
    """C5 (8 x 8192 x 8192), then a smaller ragged shape on the same scratch:
    bit-identical to the entry point with a caller workspace."""
    for M, N, K, seed in ((8, 8192, 8192, 0), (3, 1040, 2056, 1)):
        case(f"w8a16 noalloc {M}x{N}x{K} act={act} bias={with_bias}")
        x, W, scale, bias = _operands(dev, M, N, K, seed)
        b = bias if with_bias else None
        ref = ops.w8a16_gemm(x, W, scale, b, act)
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        st = _noalloc(x, W, scale, b, act, y)
        assert st == OK, _lib.lib().jules_hip_last_error()
        torch.cuda.synchronize()
        assert torch.equal(y, ref)


def _counters():
    out = (ctypes.c_uint32 * 1024)()
    st = _lib.lib().jules_hip_w8a16_noalloc_counters(ctypes.cast(out, ctypes.c_void_p), 1024)
    assert st == OK, _lib.lib().jules_hip_last_error()
    return np.frombuffer(out, dtype=np.uint32).copy()


def test_noalloc_counters_return_to_zero(dev):
    """Calls whose split-K plans differ (K = 64, 1024, 8192, 2056: from one
    split to eight) back to back on one stream, with no synchronisation in
    between: every call's results equal the workspace entry point's, and the
    counter words of all 1024 column tiles read 0 afterwards (each tile's
    last arrival wraps its counter back to 0 in the same atomic)."""
    assert not _counters().any()
    shapes = ((8, 8192, 8192, 20), (4, 3072, 64, 21), (8, 8192, 1024, 22), (1, 16384, 2056, 23),
              (8, 8192, 8192, 24))
    outs, refs = [], []
    for M, N, K, seed in shapes:
        case(f"w8a16 noalloc counters {M}x{N}x{K}")
        x, W, scale, bias = _operands(dev, M, N, K, seed)
        y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=dev)
        assert _noalloc(x, W, scale, bias, "silu", y) == OK, _lib.lib().jules_hip_last_error()
        outs.append(y)
        refs.append(ops.w8a16_gemm(x, W, scale, bias, "silu"))
    torch.cuda.synchronize()
    for (M, N, K, _), y, ref in zip(shapes, outs, refs):
        assert torch.equal(y, ref), (M, N, K)
    assert not _counters().any()


def test_noalloc_size_limit(dev):
    """N = 16384 (64 column tiles x 8 splits: the whole scratch) works; one
    column tile more is rejected with JH_ERR_WORKSPACE before any launch."""
    L = _lib.lib()
    assert L.jules_hip_w8a16_noalloc_max_bytes() == (8 << 20) + 4096
    M, N, K = 2, 16384, 8192
    case(f"w8a16 noalloc at the scratch limit {M}x{N}x{K}")
    x, W, scale, bias = _operands(dev, M, N, K, 2)
    ref = ops.w8a16_gemm(x, W, scale, bias, "silu")
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    assert _noalloc(x, W, scale, bias, "silu", y) == OK, L.jules_hip_last_error()
    torch.cuda.synchronize()
    assert torch.equal(y, ref)
    W2 = torch.zeros((K, N + 256), dtype=torch.int8, device=dev)
    s2 = torch.ones((N + 256,), dtype=torch.float32, device=dev)
    y2 = torch.empty((M, N + 256), dtype=torch.bfloat16, device=dev)
    assert _noalloc(x, W2, s2, None, "silu", y2) == WORKSPACE
    assert b"static scratch" in L.jules_hip_last_error()


def test_noalloc_graph_replay(dev):
    """Callers under graph capture: the launch is captured once and replayed
    with new activations copied in between (eager work and a synchronisation
    between replays); every replay equals the eager workspace entry point on
    the same inputs.  The kernel's launch arguments carry no per-call value
    (its tiles' arrival counters are reset by their last workgroup), so a
    replay cannot mistake an earlier replay's partial tiles for its own."""
    M, N, K = 8, 4096, 4096
    case(f"w8a16 noalloc captured in a graph {M}x{N}x{K}")
    x, W, scale, bias = _operands(dev, M, N, K, 3)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
    assert _noalloc(x, W, scale, bias, "silu", y) == OK  # eager first call
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = _noalloc(x, W, scale, bias, "silu", y)
    assert st == OK, _lib.lib().jules_hip_last_error()
    for i in range(4):
        xi, _, _, _ = _operands(dev, M, N, K, 10 + i)
        x.copy_(xi)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        ref = ops.w8a16_gemm(x, W, scale, bias, "silu")
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"
    assert not _counters().any()
