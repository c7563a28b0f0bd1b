"""GPU parity of the flash-attention forward (C ABI jules_hip_flash_attn_fwd).

Bars (normwise, against the fp64 oracle): 1e-5 for fp32, 1e-2 for bf16.
Full-size configs are checked on sampled heads/rows against the fp64 oracle
and on every head against a torch fp32 evaluation on the GPU.  Head dims
other than 64 and 128 (zero-padded to the next of the two) are checked at
the same bars."""
import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case, to_dev, to_np

pytestmark = pytest.mark.gpu
DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _run(dev, Q, K, V, dt, causal, scale=None, lse=None):
    return ops.flash_attention(to_dev(Q, DT[dt], dev), to_dev(K, DT[dt], dev),
                               to_dev(V, DT[dt], dev), causal, scale, lse=lse)


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,S,D", [(1, 1, 1, 64), (1, 2, 37, 64), (2, 1, 128, 128),
                                     (1, 3, 200, 128), (1, 1, 129, 64), (2, 2, 300, 64),
                                     # head dims zero-padded to 64 / 128
                                     (1, 2, 70, 8), (2, 1, 100, 32), (1, 2, 130, 48),
                                     (1, 1, 257, 80), (2, 2, 96, 96), (1, 2, 65, 100),
                                     (1, 1, 64, 127)])
def test_small_against_fp64(dev, dt, causal, B, H, S, D):
    case(f"flash {dt} causal={causal} [{B},{H},{S},{D}]")
    Q, K, V = I.attn_inputs(B, H, S, D, dt, seed=S + D)
    scale = ops.default_scale(D)
    lse = torch.empty((B, H, S), device=dev)
    y = to_np(_run(dev, Q, K, V, dt, causal, lse=lse))
    o = po.attention64(Q, K, V, causal, scale)
    assert I.rel_err(y, o) < I.TOL[dt]
    # log-sum-exp of the scaled scores, fp64
    ref = np.empty((B, H, S))
    for b in range(B):
        for h in range(H):
            s = Q[b, h].astype(np.float64) @ K[b, h].astype(np.float64).T * scale
            if causal:
                s[np.triu_indices(S, 1)] = -np.inf
            m = s.max(1)
            ref[b, h] = m + np.log(np.exp(s - m[:, None]).sum(1))
    np.testing.assert_allclose(lse.cpu().numpy(), ref, rtol=0, atol=1e-4)


def test_c2_full_size_f32(dev):
    """fp32 [4,8,1024,64], causal, scale 1/8, N(0,1)."""
    case("flash f32 C2 [4,8,1024,64] causal")
    Q, K, V = I.attn_inputs(4, 8, 1024, 64, "f32", seed=0)
    y = to_np(_run(dev, Q, K, V, "f32", True))
    o = po.attention64(Q, K, V, True, ops.default_scale(64))
    assert I.rel_err(y, o) < I.TOL["f32"]
    # the restated reference kernel (tiles as its cache probe picks them) agrees
    r = po.flash_attention(Q, K, V, True, ops.default_scale(64), po.flash_tiles(1024, 64))
    assert I.rel_err(y, r) < 2 * I.TOL["f32"]


def test_c4_full_size_bf16(dev):
    """bf16 [8,32,4096,128], causal.  Sampled rows of 6
    heads against the fp64 oracle; every head against torch fp32 on the GPU."""
    case("flash bf16 C4 [8,32,4096,128] causal")
    B, H, S, D = 8, 32, 4096, 128
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    Qt = torch.randn((B, H, S, D), generator=g, device=dev).bfloat16()
    Kt = torch.randn((B, H, S, D), generator=g, device=dev).bfloat16()
    Vt = torch.randn((B, H, S, D), generator=g, device=dev).bfloat16()
    scale = ops.default_scale(D)
    Ot = ops.flash_attention(Qt, Kt, Vt, True, scale)
    torch.cuda.synchronize()
    rows = np.unique(np.concatenate([[0, 1, 2, 63, 64, 127, 128, 2047, 4095],
                                     np.arange(5, S, 197)])).astype(np.int32)
    for b, h in [(0, 0), (0, 31), (3, 7), (5, 16), (7, 0), (7, 31)]:
        q, k, v = (t[b, h].float().cpu().numpy() for t in (Qt, Kt, Vt))
        o = po.attention64_head(q, k, v, True, scale, rows=rows)
        assert I.rel_err(Ot[b, h].float().cpu().numpy()[rows], o) < I.TOL["bf16"], (b, h)
    mask = torch.ones((S, S), device=dev, dtype=torch.bool).triu(1)
    worst = 0.0
    for b in range(B):
        for h0 in range(0, H, 8):
            q = Qt[b, h0:h0 + 8].float()
            k = Kt[b, h0:h0 + 8].float().transpose(1, 2).contiguous()
            s = torch.matmul(q, k) * scale
            s.masked_fill_(mask, float("-inf"))
            ref = torch.matmul(torch.softmax(s, -1), Vt[b, h0:h0 + 8].float())
            err = ((Ot[b, h0:h0 + 8].float() - ref).abs().max() / ref.abs().max()).item()
            worst = max(worst, err)
    assert worst < I.TOL["bf16"], worst


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,S,D", [(3, 8, 300, 128), (1, 24, 257, 64), (5, 8, 300, 128),
                                     (3, 16, 130, 128), (1, 56, 257, 64)])
def test_odd_heads_per_xcd_against_fp64(dev, dt, causal, B, H, S, D):
    """B*H = 24, 40, 48, 56: 3, 5, 6 and 7 heads per XCD, so the workgroup
    order's groups of four interleaved heads end with an incomplete group of
    3, 1, 2 and 3 heads."""
    case(f"flash {dt} odd J causal={causal} [{B},{H},{S},{D}]")
    Q, K, V = I.attn_inputs(B, H, S, D, dt, seed=B * H + S)
    y = to_np(_run(dev, Q, K, V, dt, causal))
    assert I.rel_err(y, po.attention64(Q, K, V, causal, ops.default_scale(D))) < I.TOL[dt]


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_invariants(dev, dt):
    case(f"flash {dt} invariants")
    B, H, S, D = 1, 2, 160, 128
    Q, K, V = I.attn_inputs(B, H, S, D, dt, seed=3)
    ones = np.ones_like(V)
    for causal in (False, True):
        y = to_np(_run(dev, Q, K, ones, dt, causal))
        np.testing.assert_allclose(y, 1.0, rtol=0, atol=1e-6 if dt == "f32" else 4e-3)
        z = to_np(_run(dev, np.zeros_like(Q), K, V, dt, causal))
        if causal:
            ref = np.cumsum(V.astype(np.float64), axis=2) / np.arange(1, S + 1)[None, None, :, None]
        else:
            ref = np.broadcast_to(V.astype(np.float64).mean(axis=2, keepdims=True), V.shape)
        assert I.rel_err(z, ref) < I.TOL[dt]
    c = to_np(_run(dev, Q, K, V, dt, True))
    np.testing.assert_allclose(c[:, :, 0], V[:, :, 0], rtol=0, atol=1e-6 if dt == "f32" else 1e-2)
    # causal: later keys never influence earlier rows
    K2, V2 = K.copy(), V.copy()
    K2[:, :, 100:] = 0.5
    V2[:, :, 100:] = -2.0
    c2 = to_np(_run(dev, Q, K2, V2, dt, True))
    np.testing.assert_array_equal(c[:, :, :100], c2[:, :, :100])


def test_deterministic_and_scale(dev):
    case("flash determinism and explicit scale")
    Q, K, V = I.attn_inputs(2, 2, 256, 64, "bf16", seed=4)
    a = _run(dev, Q, K, V, "bf16", True)
    b = _run(dev, Q, K, V, "bf16", True)
    assert torch.equal(a, b)
    y = to_np(_run(dev, Q, K, V, "bf16", False, scale=0.3))
    assert I.rel_err(y, po.attention64(Q, K, V, False, float(np.float32(0.3)))) < I.TOL["bf16"]


def test_registry_path(dev):
    """extern_kernel 'flashAttention' / 'flashAttentionCausal' through the
    descriptor ABI, default scale 1/sqrtf(D) (FlashAttention.h:135)."""
    case("flash registry")
    Q, K, V = I.attn_inputs(1, 2, 96, 64, "f32", seed=6)
    tq, tk, tv = (to_dev(x, torch.float32, dev) for x in (Q, K, V))
    for name, causal in (("flashAttention", False), ("flashAttentionCausal", True)):
        out = torch.empty_like(tq)
        ins = (_lib.JhTensor * 3)()
        for d, t in zip(ins, (tq, tk, tv)):
            _fill(d, t)
        o = (_lib.JhTensor * 1)()
        _fill(o[0], out)
        fn = _lib.lookup(name)
        assert fn(3, ins, 1, o, None, torch.cuda.current_stream().cuda_stream) == 0
        ref = po.attention64(Q, K, V, causal, ops.default_scale(64))
        assert I.rel_err(to_np(out), ref) < I.TOL["f32"]


def _fill(d, t):
    d.data = t.data_ptr()
    d.offset = 0
    d.rank = t.dim()
    for i in range(t.dim()):
        d.sizes[i] = t.shape[i]
        d.strides[i] = t.stride(i)
    d.dtype = {torch.float32: 0, torch.bfloat16: 1, torch.int8: 2}[t.dtype]
