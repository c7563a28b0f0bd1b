"""Seeded synthetic inputs and the error metric -- TEST INFRASTRUCTURE ONLY.

The generator is counter based (SplitMix64 of (seed, tensor id, index)), so
the same (seed, tensor id) gives the same tensor on any machine and any numpy
version, and any sub-range can be produced without generating the prefix.

  uniform(a, b):  a + (b - a) * u,  u = (bits >> 40) * 2^-24        (float32)
  normal(0, s):   Box-Muller on two 53-bit uniforms, computed in float64,
                  rounded once to float32, then multiplied by s in float32
  int8 in [lo,hi]: lo + ((bits >> 32) * (hi - lo + 1) >> 32)   (multiply-shift)

Tensor ids used by the configs: A=0, B=1, bias=2; Q,K,V = 0,1,2;
W=0, scale=1, x=2, bias=3.

Error metric (fixed for every kernel and config):
  rel_err(y, o) = max_i |y_i - o_i| / max_i |o_i|
with o the fp64 oracle.  Bars: 1e-5 for fp32, 1e-2 for bf16 outputs.
"""
import numpy as np

_M64 = np.uint64(0xFFFFFFFFFFFFFFFF)


def _sm64(x):
    x = x + np.uint64(0x9E3779B97F4A7C15)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def bits(seed, tid, n, offset=0):
    """n uint64 draws for (seed, tensor id), starting at counter `offset`."""
    with np.errstate(over="ignore"):
        key = _sm64(np.uint64(seed) ^ (np.uint64(tid) * np.uint64(0xD1B54A32D192ED03)))
        ctr = np.arange(offset, offset + n, dtype=np.uint64)
        return _sm64(ctr + key)


def uniform(seed, tid, shape, lo, hi):
    n = int(np.prod(shape))
    u = (bits(seed, tid, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    return (np.float32(lo) + np.float32(hi - lo) * u).astype(np.float32).reshape(shape)


def normal(seed, tid, shape, std=1.0):
    n = int(np.prod(shape))
    b = bits(seed, tid, 2 * n)
    u1 = ((b[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0 ** -53  # (0, 1]
    u2 = (b[1::2] >> np.uint64(11)).astype(np.float64) * 2.0 ** -53           # [0, 1)
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (z.astype(np.float32) * np.float32(std)).reshape(shape)


def int8_uniform(seed, tid, shape, lo=-127, hi=127):
    n = int(np.prod(shape))
    b = bits(seed, tid, n) >> np.uint64(32)
    span = np.uint64(hi - lo + 1)
    with np.errstate(over="ignore"):
        v = (b * span) >> np.uint64(32)
    return (v.astype(np.int64) + lo).astype(np.int8).reshape(shape)


def bf16_round(x):
    """Round float32 to the nearest bfloat16 (ties to even); returns float32
    holding the bf16 value (exact widening)."""
    x = np.ascontiguousarray(x, np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u >> np.uint64(16)) & np.uint64(1)) + np.uint64(0x7FFF)
    hi = ((u + r) >> np.uint64(16)).astype(np.uint32)
    nan = np.isnan(x)
    hi = np.where(nan, (u >> np.uint64(16)).astype(np.uint32) | np.uint32(0x40), hi)
    return (hi << np.uint32(16)).view(np.float32).reshape(x.shape)


def bf16_bits(x):
    """uint16 bit patterns of bf16_round(x)."""
    return (bf16_round(x).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


def bf16_from_bits(b):
    return (np.ascontiguousarray(b, np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def rel_err(y, o):
    y = np.asarray(y, np.float64)
    o = np.asarray(o, np.float64)
    den = np.max(np.abs(o)) if o.size else 0.0
    num = np.max(np.abs(y - o)) if o.size else 0.0
    if den == 0.0:
        return float(num)
    return float(num / den)


TOL = {"f32": 1e-5, "bf16": 1e-2}


# ---- the five BASELINE configs, generated with the conventions above -------
def gemm_inputs(M, N, K, dtype, seed=0):
    """C1 (fp32): A, B, bias ~ U[-1,1].  C3 (bf16): A, B ~ N(0, std=1/sqrt(K))
    rounded to bf16, bias ~ U[-0.1, 0.1] kept in fp32."""
    if dtype == "f32":
        A = uniform(seed, 0, (M, K), -1.0, 1.0)
        B = uniform(seed, 1, (K, N), -1.0, 1.0)
        bias = uniform(seed, 2, (N,), -1.0, 1.0)
    else:
        std = 1.0 / np.sqrt(K)
        A = bf16_round(normal(seed, 0, (M, K), std))
        B = bf16_round(normal(seed, 1, (K, N), std))
        bias = uniform(seed, 2, (N,), -0.1, 0.1)
    return A, B, bias


def attn_inputs(B, H, S, D, dtype, seed=0):
    Q = normal(seed, 0, (B, H, S, D))
    K = normal(seed, 1, (B, H, S, D))
    V = normal(seed, 2, (B, H, S, D))
    if dtype == "bf16":
        Q, K, V = bf16_round(Q), bf16_round(K), bf16_round(V)
    return Q, K, V


def w8a16_inputs(M, N, K, seed=0):
    W = int8_uniform(seed, 0, (K, N))
    scale = uniform(seed, 1, (N,), 1e-3, 1e-2)
    x = bf16_round(normal(seed, 2, (M, K)))
    bias = uniform(seed, 3, (N,), -0.1, 0.1)
    return x, W, scale, bias


def mlp_inputs(M, K1, N1, N2, seed=0, scaled=False):
    """interleavedMLPForwardBackward operands.  The reference benchmark
    (benchmarks/bench_kernel.cpp:285-290) draws X, W1, b1, W2, b2 ~ U[-1, 1]
    and targets ~ U{0..N2-1}; `scaled` divides each weight by sqrt(fan_in) so
    the logits stay O(1) and the softmax does not saturate."""
    X = uniform(seed, 0, (M, K1), -1.0, 1.0)
    W1 = uniform(seed, 1, (K1, N1), -1.0, 1.0)
    b1 = uniform(seed, 2, (N1,), -1.0, 1.0)
    W2 = uniform(seed, 3, (N1, N2), -1.0, 1.0)
    b2 = uniform(seed, 4, (N2,), -1.0, 1.0)
    if scaled:
        W1 = (W1 / np.float32(np.sqrt(K1))).astype(np.float32)
        W2 = (W2 / np.float32(np.sqrt(N1))).astype(np.float32)
    b = bits(seed, 5, M) >> np.uint64(32)
    with np.errstate(over="ignore"):
        t = ((b * np.uint64(N2)) >> np.uint64(32)).astype(np.int32)
    return X, W1, b1, W2, b2, t
