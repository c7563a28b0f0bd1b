"""GPU parity of the packed-weight W8A16 path (jules_hip_w8a16_pack +
jules_hip_w8a16_packed_gemm_bias_act).

- The pack is a permutation with zero padding: unpacking it with the inverse
  map written here gives W back, and every padding byte is zero.
- The GEMM is within 1e-2 of the fp64 oracle at the C5 size and at ragged
  shapes (N % 32 == 16, K not a multiple of 32, M from 1 to 16), for every
  activation; on one-hot activations it is bit-exact (the product of one
  weight and one scale, then bias and activation) and bit-identical to the
  row-major entry point."""
import numpy as np
import pytest
import torch

from jules_amd import ops
from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case, to_dev, to_np

pytestmark = pytest.mark.gpu
ACTS = ["none", "relu", "sigmoid", "tanh", "gelu", "silu"]


def _packed(dev, x, W, scale, bias, act):
    Wp = ops.w8a16_pack(to_dev(W, torch.int8, dev))
    return ops.w8a16_gemm_packed(to_dev(x, torch.bfloat16, dev), Wp,
                                 to_dev(scale, torch.float32, dev),
                                 None if bias is None else to_dev(bias, torch.float32, dev), act)


def _unpack(buf, K, N):
    """Inverse of the packed layout: block (tile c, k-step s) at
    (s*tiles + c)*1024, lane l = 16*kg + j holds W[32s + 8kg + i][32c + j]
    (bytes 0-7) and W[32s + 8kg + i][32c + 16 + j] (bytes 8-15).  Returns the
    padded [32*ksteps, 32*tiles] matrix."""
    ks, tiles = -(-K // 32), -(-N // 32)
    b = buf.reshape(ks, tiles, 4, 16, 2, 8)  # s, c, kg, j, half, i
    # -> [s, kg, i, c, half, j]
    return b.transpose(0, 2, 5, 1, 4, 3).reshape(ks * 32, tiles * 32)


@pytest.mark.parametrize("K,N", [(8, 16), (40, 272), (1000, 512), (4096, 8192), (2056, 1040)])
def test_pack_is_a_permutation(dev, K, N):
    case(f"w8a16 pack K={K} N={N}")
    W = I.int8_uniform(K + N, 0, (K, N))
    Wp = ops.w8a16_pack(to_dev(W, torch.int8, dev))
    buf = Wp.data.cpu().numpy().view(np.int8)
    assert buf.size == -(-K // 32) * -(-N // 32) * 1024
    full = _unpack(buf, K, N)
    np.testing.assert_array_equal(full[:K, :N], W)
    assert not full[K:, :].any() and not full[:, N:].any()


def test_c5_full_size(dev):
    """BASELINE config 5 on the packed path: M=8, N=K=8192, SiLU."""
    case("w8a16 packed C5 8x8192x8192 silu")
    x, W, scale, bias = I.w8a16_inputs(8, 8192, 8192, seed=0)
    y = to_np(_packed(dev, x, W, scale, bias, "silu"))
    assert I.rel_err(y, po.w8a16_64(x, W, scale, bias, "silu")) < I.TOL["bf16"]
    # the same outputs as the row-major entry point to within one bf16 step,
    # plus the fp32 rounding of 8192-term sums near zero (the two paths add
    # the products in different orders: ~1e-4 absolute at these magnitudes)
    r = ops.w8a16_gemm(to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
                       to_dev(scale, torch.float32, dev), to_dev(bias, torch.float32, dev), "silu")
    d = np.abs(y.astype(np.float64) - to_np(r).astype(np.float64))
    assert (d <= 2.0 ** -7 * np.abs(y) + 2e-5 * np.abs(y).max()).all()


# k-steps of 32 are dealt to the 4 waves in adjacent pairs (8 per round):
# the shapes cover every remainder of ksteps % 8 (K = 352: 11 steps, 480: 15,
# 192: 6 steps, no full round) and M on both sides of the paired-x path
@pytest.mark.parametrize("M,N,K", [(1, 16, 8), (3, 272, 40), (8, 512, 1000), (9, 256, 4096),
                                   (16, 1040, 2056), (8, 8192, 64), (5, 4096, 33000),
                                   (2, 48, 264), (3, 160, 352), (7, 96, 480), (1, 16, 192),
                                   (12, 64, 480), (8, 32, 136), (4, 48, 384)])
def test_shapes_against_fp64(dev, M, N, K):
    case(f"w8a16 packed {M}x{N}x{K}")
    x, W, scale, bias = I.w8a16_inputs(M, N, K, seed=M + N + K)
    y = to_np(_packed(dev, x, W, scale, bias, "silu"))
    assert I.rel_err(y, po.w8a16_64(x, W, scale, bias, "silu")) < I.TOL["bf16"]


@pytest.mark.parametrize("act", ACTS)
def test_activations(dev, act):
    case(f"w8a16 packed act={act}")
    x, W, scale, bias = I.w8a16_inputs(8, 768, 1024, seed=2)
    y = to_np(_packed(dev, x, W, scale, bias, act))
    assert I.rel_err(y, po.w8a16_64(x, W, scale, bias, act)) < I.TOL["bf16"]


def test_one_hot_kat_bit_exact(dev):
    """x = one-hot rows picks W[k0, :]: y = bf16(act(W[k0,j]*scale[j] + bias[j]))
    exactly, and bit-identical to the row-major entry point."""
    case("w8a16 packed one-hot KAT")
    M, N, K = 8, 1040, 4104
    _, W, scale, bias = I.w8a16_inputs(M, N, K, seed=5)
    ks = [0, 1, 31, 32, 1000, 2047, 4090, 4103]
    x = np.zeros((M, K), np.float32)
    for m, k0 in enumerate(ks):
        x[m, k0] = 1.0
    for act in ("silu", "none", "gelu"):
        y = _packed(dev, x, W, scale, bias, act).view(torch.int16).cpu().numpy().view(np.uint16)
        for m, k0 in enumerate(ks):
            pre = W[k0].astype(np.float32) * scale + bias
            ref = I.bf16_bits(po.act_array(act, pre))
            np.testing.assert_array_equal(y[m], ref, err_msg=f"act={act} row {m} k0={k0}")
        r = ops.w8a16_gemm(to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
                           to_dev(scale, torch.float32, dev), to_dev(bias, torch.float32, dev),
                           act).view(torch.int16).cpu().numpy().view(np.uint16)
        np.testing.assert_array_equal(y, r)
    y = _packed(dev, x, W, scale, None, "none").float().cpu().numpy()
    for m, k0 in enumerate(ks):
        np.testing.assert_array_equal(y[m], I.bf16_round(W[k0].astype(np.float32) * scale))


def test_extreme_weights(dev):
    """Every weight -128 or 127 and x = +-1: the int8 -> bf16 conversion of the
    extreme bytes (sign extension) and long sums (K = 8192)."""
    case("w8a16 packed extreme weights")
    M, N, K = 4, 256, 8192
    rng = np.random.default_rng(11)
    W = np.where(rng.random((K, N)) < 0.5, -128, 127).astype(np.int8)
    x = np.where(rng.random((M, K)) < 0.5, -1.0, 1.0).astype(np.float32)
    scale = np.full(N, 1e-3, np.float32)
    y = to_np(_packed(dev, x, W, scale, None, "none"))
    ref = po.w8a16_64(x, W, scale, None, "none")
    assert I.rel_err(y, ref) < I.TOL["bf16"]
