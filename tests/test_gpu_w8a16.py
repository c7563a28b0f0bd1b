"""GPU parity of the W8A16 decode GEMM (jules_hip_w8a16_gemm_bias_act) and of
matmulInt8 (jules_hip_matmul_int8).

W8A16: within 1e-2 of the fp64 oracle; bit-exact on one-hot activations (the
int8 index W[k*N+j] and the dequantising multiply by scale[j]).
matmulInt8: bit-exact against the scalar path of the reference
(FusedKernels.h:1046-1066)."""
import numpy as np
import pytest
import torch

from jules_amd import _lib, ops
from oracle import inputs as I
from oracle import pyoracle as po
from tests.helpers import case, registry_call, to_dev, to_np

pytestmark = pytest.mark.gpu
ACTS = ["none", "relu", "sigmoid", "tanh", "gelu", "silu"]


def _w8(dev, x, W, scale, bias, act, ws=None):
    return ops.w8a16_gemm(to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
                          to_dev(scale, torch.float32, dev),
                          None if bias is None else to_dev(bias, torch.float32, dev), act,
                          workspace=ws)


def test_c5_full_size(dev):
    """M=8, N=K=8192, W int8 U[-127,127], per-channel scale
    U[1e-3,1e-2], x N(0,1) bf16, bias U[-0.1,0.1], SiLU."""
    case("w8a16 C5 8x8192x8192 silu")
    x, W, scale, bias = I.w8a16_inputs(8, 8192, 8192, seed=0)
    y = to_np(_w8(dev, x, W, scale, bias, "silu"))
    o = po.w8a16_64(x, W, scale, bias, "silu")
    assert I.rel_err(y, o) < I.TOL["bf16"]
    # and against the restated fp32 path
    r = po.w8a16(x, W, scale, bias, "silu")
    assert I.rel_err(y, r) < I.TOL["bf16"]


@pytest.mark.parametrize("M,N,K", [(1, 16, 8), (3, 272, 40), (8, 512, 1000), (9, 256, 4096),
                                   (16, 1040, 2056), (8, 8192, 64), (5, 4096, 33000)])
def test_shapes_against_fp64(dev, M, N, K):
    case(f"w8a16 {M}x{N}x{K}")
    x, W, scale, bias = I.w8a16_inputs(M, N, K, seed=M + N + K)
    y = to_np(_w8(dev, x, W, scale, bias, "silu"))
    assert I.rel_err(y, po.w8a16_64(x, W, scale, bias, "silu")) < I.TOL["bf16"]


@pytest.mark.parametrize("act", ACTS)
def test_activations(dev, act):
    case(f"w8a16 act={act}")
    x, W, scale, bias = I.w8a16_inputs(8, 768, 1024, seed=2)
    y = to_np(_w8(dev, x, W, scale, bias, act))
    assert I.rel_err(y, po.w8a16_64(x, W, scale, bias, act)) < I.TOL["bf16"]


def test_one_hot_kat_bit_exact(dev):
    """x = one-hot rows picks W[k0, :]; then y = bf16(act(W[k0,j]*scale[j] +
    bias[j])) exactly: pins the W[k*N+j] indexing and the one fp32 multiply
    of the dequantisation."""
    case("w8a16 one-hot KAT")
    M, N, K = 8, 1024, 4096
    _, W, scale, bias = I.w8a16_inputs(M, N, K, seed=5)
    ks = [0, 1, 31, 32, 1000, 2047, 4090, 4095]
    x = np.zeros((M, K), np.float32)
    for m, k0 in enumerate(ks):
        x[m, k0] = 1.0
    for act in ("silu", "none", "gelu"):
        y = _w8(dev, x, W, scale, bias, act).view(torch.int16).cpu().numpy().view(np.uint16)
        for m, k0 in enumerate(ks):
            pre = W[k0].astype(np.float32) * scale + bias
            ref = I.bf16_bits(po.act_array(act, pre))
            np.testing.assert_array_equal(y[m], ref, err_msg=f"act={act} row {m} k0={k0}")
    # no bias: y = W*scale exactly (bf16-rounded)
    y = _w8(dev, x, W, scale, None, "none").float().cpu().numpy()
    for m, k0 in enumerate(ks):
        np.testing.assert_array_equal(y[m], I.bf16_round(W[k0].astype(np.float32) * scale))


def test_deterministic_and_workspace_reuse(dev):
    case("w8a16 determinism, workspace reuse")
    ws = ops.w8a16_workspace(16, 8192, 8192, dev)
    x, W, scale, bias = I.w8a16_inputs(8, 8192, 8192, seed=7)
    a = _w8(dev, x, W, scale, bias, "silu", ws)
    b = _w8(dev, x, W, scale, bias, "silu", ws)
    assert torch.equal(a, b)
    # a different shape through the same workspace, then the first again
    x2, W2, s2, b2 = I.w8a16_inputs(3, 512, 256, seed=8)
    c = to_np(_w8(dev, x2, W2, s2, b2, "gelu", ws))
    assert I.rel_err(c, po.w8a16_64(x2, W2, s2, b2, "gelu")) < I.TOL["bf16"]
    assert torch.equal(a, _w8(dev, x, W, scale, bias, "silu", ws))
    # stale partials in the workspace do not leak into the next result
    ws.fill_(0x7F)
    assert torch.equal(a, _w8(dev, x, W, scale, bias, "silu", ws))


def test_split_reduction_bit_exact_from_partials(dev):
    """The split-K reduction, checked bit for bit: after a call the workspace
    still holds the KS fp32 partial tiles, and y must equal
    bf16(act(((p0 + p1) + ... + p_{KS-1}) * scale + bias)) computed from them
    in fp32 on the host, in split order."""
    case("w8a16 split reduction from workspace partials")
    M, N, K = 8, 8192, 8192
    x, W, scale, bias = I.w8a16_inputs(M, N, K, seed=11)
    ws = ops.w8a16_workspace(M, N, K, dev)
    # workspace = [KS][tiles] partial tiles of 16 KiB, each in the MFMA
    # accumulator layout [j 16][lane 64][row-in-group 4] fp32 (lane = 16*lg +
    # lc holds rows 4*lg.., column 16*lc + j of the 256-column tile), then one
    # 8-byte flag per (tile, split)
    tiles = N // 256
    KS = ws.numel() // (tiles * (16384 + 8))
    assert ws.numel() == KS * tiles * (16384 + 8) and 1 <= KS <= 16

    def partials():
        a = ws[:KS * tiles * 16384].view(torch.float32).cpu().numpy()
        a = a.reshape(KS, tiles, 16, 4, 16, 4).transpose(0, 3, 5, 1, 4, 2)
        return a.reshape(KS, 16, tiles * 256)[:, :M, :N]

    for act, b in (("silu", bias), ("gelu", None)):
        y = _w8(dev, x, W, scale, b, act, ws).view(torch.int16).cpu().numpy().view(np.uint16)
        parts = partials()
        s = parts[0].copy()
        for p in range(1, KS):
            s = s + parts[p]
        pre = s * scale
        if b is not None:
            pre = pre + b
        np.testing.assert_array_equal(y, I.bf16_bits(po.act_array(act, pre)), err_msg=act)
        # and the partials are those of the product
        assert I.rel_err(parts.sum(0, dtype=np.float64), po.w8a16_64(x, W, np.ones_like(scale),
                                                                     None, "none")) < 1e-5


def test_alternating_calls_same_workspace(dev):
    """Back-to-back calls with different inputs on one workspace: every result
    equals that input's first result, so no call reads another call's
    partials or flags.  Every fifth call first overwrites the workspace."""
    case("w8a16 alternating calls, one workspace")
    M, N, K = 8, 8192, 8192
    ws = ops.w8a16_workspace(M, N, K, dev)
    ins = [I.w8a16_inputs(M, N, K, seed=s) for s in (21, 22)]
    dev_ins = [(to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
                to_dev(sc, torch.float32, dev), to_dev(b, torch.float32, dev))
               for x, W, sc, b in ins]
    first = [ops.w8a16_gemm(*t, "silu", workspace=ws) for t in dev_ins]
    for (x, W, sc, b), y in zip(ins, first):
        assert I.rel_err(to_np(y), po.w8a16_64(x, W, sc, b, "silu")) < I.TOL["bf16"]
    outs = []
    for i in range(60):
        if i % 5 == 4:
            ws.fill_(i)
        outs.append(ops.w8a16_gemm(*dev_ins[i % 2], "silu", workspace=ws))
    for i, y in enumerate(outs):
        assert torch.equal(y, first[i % 2]), f"call {i}"


def test_registry_path(dev):
    case("w8a16 registry matmulW8A16BiasSilu")
    x, W, scale, bias = I.w8a16_inputs(4, 512, 512, seed=9)
    tx, tw, ts, tb = (to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
                      to_dev(scale, torch.float32, dev), to_dev(bias, torch.float32, dev))
    out = torch.empty((4, 512), dtype=torch.bfloat16, device=dev)
    ins = (_lib.JhTensor * 4)()
    for d, t in zip(ins, (tx, tw, ts, tb)):
        _fill(d, t)
    o = (_lib.JhTensor * 1)()
    _fill(o[0], out)
    fn = _lib.lookup("matmulW8A16BiasSilu")
    assert fn(4, ins, 1, o, None, torch.cuda.current_stream().cuda_stream) == 0
    assert I.rel_err(to_np(out), po.w8a16_64(x, W, scale, bias, "silu")) < I.TOL["bf16"]


# ---- matmulInt8 ---------------------------------------------------------------
# Paths: rows not 16-byte aligned (K or N % 16 != 0) take the SIMT kernel;
# M <= 16 the streaming split-K kernel; M, N multiples of 256 and K of 64 the
# LDS-DMA ring (1, 2, 3 and 32 slices); other larger M the 128x128 MFMA tiles
# (ragged M/N edges, K tails of a 64-row slice).
@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (8, 33, 70), (64, 64, 64), (130, 200, 515),
                                   (1, 256, 64), (5, 48, 16), (8, 8192, 8192), (16, 4096, 1040),
                                   (17, 144, 80), (200, 272, 144), (512, 768, 1024),
                                   (256, 256, 64), (256, 512, 128), (512, 256, 192),
                                   (1024, 1024, 2048)])
def test_int8_bit_exact(dev, M, N, K):
    case(f"matmulInt8 {M}x{N}x{K}")
    A = I.int8_uniform(1, 0, (M, K))
    B = I.int8_uniform(1, 1, (K, N))
    bias = I.uniform(1, 2, (N,), -1, 1)
    for b in (bias, None):
        y = ops.matmul_int8(to_dev(A, torch.int8, dev), to_dev(B, torch.int8, dev), 0.013, 0.021,
                            None if b is None else to_dev(b, torch.float32, dev))
        np.testing.assert_array_equal(to_np(y), po.matmul_int8(A, B, 0.013, 0.021, b))


@pytest.mark.parametrize("M", [2, 40])
def test_int8_extreme_sums(dev, M):
    """The largest |sum| the entry point can meet: every product (-128)*(-128)
    = 2^14 at K = 131056 (the largest multiple of 16 within the K <= 131071
    limit) sums to 2,147,221,504, just inside int32, and a column of
    127 * -128 products to -2,130,444,288; the split-K partials and their
    combination stay exact."""
    case(f"matmulInt8 extreme sums M={M}")
    K, N = 131056, 16
    A = np.full((M, K), -128, np.int8)
    B = np.full((K, N), -128, np.int8)
    B[:, 3] = 127
    y = to_np(ops.matmul_int8(to_dev(A, torch.int8, dev), to_dev(B, torch.int8, dev), 1.0, 1.0))
    np.testing.assert_array_equal(y, po.matmul_int8(A, B, 1.0, 1.0))
    assert y[0, 0] == np.float32(128 * 128 * K) and y[0, 3] == np.float32(-128 * 127 * K)
    assert 128 * 128 * K < 2**31 and 128 * 128 * (K + 16) >= 2**31


def test_int8_decode_two_streams(dev):
    """The decode path's workspace is per (device, stream): calls alternating
    on two streams, with inputs of two sizes (the workspace grows once), all
    give the exact result."""
    case("matmulInt8 decode on two streams")
    ins = []
    for i, (M, N, K) in enumerate([(8, 2048, 4096), (16, 4096, 8192)]):
        A = I.int8_uniform(20 + i, 0, (M, K))
        B = I.int8_uniform(20 + i, 1, (K, N))
        ins.append((A, B, po.matmul_int8(A, B, 0.5, 0.25), to_dev(A, torch.int8, dev),
                    to_dev(B, torch.int8, dev)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    outs = []
    for rep in range(6):
        for si, st in enumerate(streams):
            A, B, ref, tA, tB = ins[(rep + si) % 2]
            with torch.cuda.stream(st):
                outs.append((ops.matmul_int8(tA, tB, 0.5, 0.25), ref))
    torch.cuda.synchronize()
    for y, ref in outs:
        np.testing.assert_array_equal(to_np(y), ref)


def test_int8_one_hot_kat(dev):
    case("matmulInt8 one-hot KAT")
    B = I.int8_uniform(2, 1, (70, 40))
    A = np.zeros((3, 70), np.int8)
    A[0, 0], A[1, 17], A[2, 69] = 1, 1, -1
    y = to_np(ops.matmul_int8(to_dev(A, torch.int8, dev), to_dev(B, torch.int8, dev), 1.0, 1.0))
    np.testing.assert_array_equal(y[0], B[0].astype(np.float32))
    np.testing.assert_array_equal(y[1], B[17].astype(np.float32))
    np.testing.assert_array_equal(y[2], -B[69].astype(np.float32))


def _fill(d, t):
    d.data = t.data_ptr()
    d.offset = 0
    d.rank = t.dim()
    for i in range(t.dim()):
        d.sizes[i] = t.shape[i]
        d.strides[i] = t.stride(i)
    d.dtype = {torch.float32: 0, torch.bfloat16: 1, torch.int8: 2}[t.dtype]



@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (8, 8192, 1024), (37, 129, 300), (256, 96, 4096),
                                   (256, 512, 2048)])
def test_w8a8_bit_exact(dev, M, N, K):
    """Per-token / per-channel W8A8 (jules_hip_matmul_w8a8) against the numpy
    restatement, bit for bit, with and without bias and per-token scales."""
    case(f"w8a8 M={M} N={N} K={K}")
    A = I.int8_uniform(5, 0, (M, K))
    B = I.int8_uniform(5, 1, (K, N))
    sa = I.uniform(5, 2, (M,), 1e-3, 1e-2)
    sb = I.uniform(5, 3, (N,), 1e-3, 1e-2)
    bias = I.uniform(5, 4, (N,), -0.1, 0.1)
    tA, tB = to_dev(A, torch.int8, dev), to_dev(B, torch.int8, dev)
    for use_sa in (True, False):
        for b in (None, bias):
            y = ops.matmul_w8a8(tA, tB, to_dev(sa, torch.float32, dev) if use_sa else None,
                                to_dev(sb, torch.float32, dev),
                                None if b is None else to_dev(b, torch.float32, dev))
            np.testing.assert_array_equal(to_np(y), po.w8a8(A, B, sa if use_sa else None, sb, b))


def test_w8a8_constant_scales_equal_matmul_int8(dev):
    case("w8a8 with constant scales == matmulInt8")
    A = I.int8_uniform(6, 0, (33, 200))
    B = I.int8_uniform(6, 1, (200, 70))
    tA, tB = to_dev(A, torch.int8, dev), to_dev(B, torch.int8, dev)
    y1 = ops.matmul_w8a8(tA, tB, to_dev(np.full(33, 0.013, np.float32), torch.float32, dev),
                         to_dev(np.full(70, 0.021, np.float32), torch.float32, dev))
    y2 = ops.matmul_int8(tA, tB, 0.013, 0.021)
    assert torch.equal(y1, y2)


def test_w8a8_registry(dev):
    case("registry matmulW8A8")
    A = I.int8_uniform(7, 0, (16, 64))
    B = I.int8_uniform(7, 1, (64, 48))
    sa = I.uniform(7, 2, (16,), 1e-3, 1e-2)
    sb = I.uniform(7, 3, (48,), 1e-3, 1e-2)
    bias = I.uniform(7, 4, (48,), -0.1, 0.1)
    c = torch.empty((16, 48), dtype=torch.float32, device=dev)
    st = registry_call("matmulW8A8", [to_dev(A, torch.int8, dev), to_dev(B, torch.int8, dev),
                                      to_dev(sa, torch.float32, dev), to_dev(sb, torch.float32, dev),
                                      to_dev(bias, torch.float32, dev)], [c])
    assert st == 0, _lib.lib().jules_hip_last_error()
    np.testing.assert_array_equal(to_np(c), po.w8a8(A, B, sa, sb, bias))


def test_w8a16_registry_two_streams(dev):
    """The registry's W8A16 entry holds its split-K workspace per (device,
    stream): calls alternating on two streams, with inputs of two sizes (each
    stream's workspace grows once), give the bits of the typed entry point
    with a caller workspace."""
    case("registry matmulW8A16BiasSilu on two streams")
    ins = []
    for i, (M, N, K) in enumerate([(8, 2048, 4096), (16, 4096, 8192)]):
        x, W, scale, bias = I.w8a16_inputs(M, N, K, seed=30 + i)
        t = [to_dev(x, torch.bfloat16, dev), to_dev(W, torch.int8, dev),
             to_dev(scale, torch.float32, dev), to_dev(bias, torch.float32, dev)]
        ref = ops.w8a16_gemm(*t[:3], bias=t[3], act="silu")
        ins.append((t, ref, (M, N)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    outs = []
    for rep in range(6):
        for si, st in enumerate(streams):
            t, ref, (M, N) = ins[(rep + si) % 2]
            with torch.cuda.stream(st):
                y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)
                assert registry_call("matmulW8A16BiasSilu", t, [y]) == 0, \
                    _lib.lib().jules_hip_last_error()
                outs.append((y, ref))
    torch.cuda.synchronize()
    for y, ref in outs:
        assert torch.equal(y, ref)
