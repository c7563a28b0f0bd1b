"""GPU parity of the flash-attention backward (jules_hip_flash_attn_bwd; the
reference has no backward) against the fp64 oracle po.attention_bwd64
(pinned in tests/test_oracle.py by finite differences and torch autograd).

Inputs: Q, K, V, dO ~ N(0,1) rounded to bf16; O and lse come from this
library's forward.  Bar: bf16, every gradient within 1e-2 of fp64 as
max |y - ref| / max |ref| per tensor (P and dS are rounded to bf16 before
their products, as the forward rounds P)."""
import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case, to_dev, to_np

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _grads(dev, Q, K, V, dO, causal, scale=None):
    tq, tk, tv, tdo = (to_dev(a, torch.bfloat16, dev) for a in (Q, K, V, dO))
    B, H, S, D = Q.shape
    lse = torch.empty((B, H, S), dtype=torch.float32, device=dev)
    O = ops.flash_attention(tq, tk, tv, causal, scale, lse=lse)
    return ops.flash_attention_bwd(tq, tk, tv, O, tdo, lse, causal, scale)


def _inputs(B, H, S, D, seed):
    Q, K, V = I.attn_inputs(B, H, S, D, "bf16", seed=seed)
    dO = I.bf16_round(I.normal(seed, 3, (B, H, S, D)))
    return Q, K, V, dO


@pytest.mark.parametrize("B,H,S,D", [(1, 1, 1, 64), (1, 2, 37, 64), (2, 2, 128, 128),
                                     (1, 3, 200, 128), (2, 4, 256, 64), (1, 2, 333, 128),
                                     # head dims zero-padded to 64 / 128
                                     (1, 2, 70, 32), (2, 1, 100, 96), (1, 1, 129, 80),
                                     (1, 2, 37, 100)])
@pytest.mark.parametrize("causal", [False, True])
def test_against_fp64(dev, B, H, S, D, causal):
    case(f"flash bwd B{B} H{H} S{S} D{D} causal={causal}")
    Q, K, V, dO = _inputs(B, H, S, D, seed=S + D)
    scale = 1.0 / np.sqrt(D)
    got = _grads(dev, Q, K, V, dO, causal, scale)
    ref = po.attention_bwd64(Q, K, V, dO, causal, scale)
    for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
        err = I.rel_err(to_np(g), r)
        assert err < TOL, f"{name}: rel err {err:.3g}"


def test_large_causal_against_torch_fp32(dev):
    """[1, 8, 1024, 128] causal: every head against torch fp32 autograd on
    the GPU (fp32 math; the same bf16 inputs)."""
    case("flash bwd 1x8x1024x128 causal vs torch fp32")
    B, H, S, D = 1, 8, 1024, 128
    Q, K, V, dO = _inputs(B, H, S, D, seed=5)
    scale = 1.0 / np.sqrt(D)
    got = _grads(dev, Q, K, V, dO, True, scale)
    ts = [torch.from_numpy(np.ascontiguousarray(a)).to(dev).float().requires_grad_(True)
          for a in (Q, K, V)]
    s = torch.matmul(ts[0], ts[1].transpose(-1, -2).contiguous()) * scale
    s = s.masked_fill(torch.triu(torch.ones(S, S, dtype=torch.bool, device=dev), 1), float("-inf"))
    O = torch.matmul(torch.softmax(s, dim=-1), ts[2])
    (O * torch.from_numpy(dO).to(dev).float()).sum().backward()
    for name, g, t in zip(("dQ", "dK", "dV"), got, ts):
        err = I.rel_err(to_np(g), t.grad.detach().cpu().numpy())
        assert err < TOL, f"{name}: rel err {err:.3g}"


@pytest.mark.parametrize("B,H,S,D", [(3, 8, 256, 128), (1, 24, 130, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_odd_heads_per_xcd_against_fp64(dev, B, H, S, D, causal):
    """B*H = 24: three heads per XCD in the head-pair workgroup order, so one
    pair is incomplete (the mapping's odd case)."""
    case(f"flash bwd odd J B{B} H{H} S{S} D{D} causal={causal}")
    Q, K, V, dO = _inputs(B, H, S, D, seed=B * H + S)
    scale = 1.0 / np.sqrt(D)
    got = _grads(dev, Q, K, V, dO, causal, scale)
    ref = po.attention_bwd64(Q, K, V, dO, causal, scale)
    for name, g, r in zip(("dQ", "dK", "dV"), got, ref):
        err = I.rel_err(to_np(g), r)
        assert err < TOL, f"{name}: rel err {err:.3g}"


def test_c4_length_causal_against_torch_fp32(dev):
    """[2, 8, 4096, 128] causal: the sequence length and head-pair mapping of
    the timed C4-shape backward (16 heads, two per XCD).  Four heads spread
    over both batches and both members of a pair, against torch fp32 autograd
    on the GPU, per head (fp32 math; the same bf16 inputs)."""
    B, H, S, D = 2, 8, 4096, 128
    case(f"flash bwd [{B},{H},{S},{D}] causal vs torch fp32")
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    tq, tk, tv, tdo = (torch.randn((B, H, S, D), generator=g, device=dev).bfloat16()
                       for _ in range(4))
    scale = 1.0 / np.sqrt(D)
    lse = torch.empty((B, H, S), dtype=torch.float32, device=dev)
    O = ops.flash_attention(tq, tk, tv, True, scale, lse=lse)
    dQ, dK, dV = ops.flash_attention_bwd(tq, tk, tv, O, tdo, lse, True, scale)
    torch.cuda.synchronize()
    mask = torch.ones((S, S), dtype=torch.bool, device=dev).triu(1)
    for b, h in ((0, 0), (0, 5), (1, 2), (1, 7)):
        q, k, v = (t[b, h].float().requires_grad_(True) for t in (tq, tk, tv))
        s = torch.matmul(q, k.t().contiguous()) * scale
        s = s.masked_fill(mask, float("-inf"))
        o = torch.matmul(torch.softmax(s, dim=-1), v)
        (o * tdo[b, h].float()).sum().backward()
        for name, got, ref in (("dQ", dQ, q.grad), ("dK", dK, k.grad), ("dV", dV, v.grad)):
            err = ((got[b, h].float() - ref).abs().max() / ref.abs().max()).item()
            assert err < TOL, f"({b},{h}) {name}: rel err {err:.3g}"
        del q, k, v, s, o


def test_deterministic(dev):
    case("flash bwd determinism")
    Q, K, V, dO = _inputs(2, 2, 300, 128, seed=11)
    a = _grads(dev, Q, K, V, dO, True)
    b = _grads(dev, Q, K, V, dO, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
