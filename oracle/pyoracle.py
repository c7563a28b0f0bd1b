"""ctypes wrapper around oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg,
never by the product package.  Every function takes and returns numpy arrays;
bf16 tensors are passed widened to float32 (exact).
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ACT = {"none": 0, "relu": 1, "sigmoid": 2, "tanh": 3, "gelu": 4, "silu": 5}

_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} missing: run oracle/build_oracle.py")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "jo_fast_exp": (ctypes.c_float, [ctypes.c_float]),
            "jo_gelu": (ctypes.c_float, [ctypes.c_float]),
            "jo_sigmoid": (ctypes.c_float, [ctypes.c_float]),
            "jo_fast_tanh": (ctypes.c_float, [ctypes.c_float]),
            "jo_silu": (ctypes.c_float, [ctypes.c_float]),
            "jo_act": (ctypes.c_float, [_c_int, ctypes.c_float]),
            "jo_act_array": (None, [_c_int, _f32p, _f32p, _c_i64]),
            "jo_fast_exp_array": (None, [_f32p, _f32p, _c_i64]),
            "jo_fused_gelu": (None, [_f32p, _f32p, _c_int]),
            "jo_tiled_matmul_act": (None, [_f32p, _f32p, _f32p] + [_c_int] * 7),
            "jo_matmul_bias_act": (None, [_f32p, _f32p, _f32p, _f32p] + [_c_int] * 7),
            "jo_tile_analytical": (None, [_c_int] * 3 + [_c_i64, _c_i64, _c_int,
                                                          ctypes.POINTER(_c_int),
                                                          ctypes.POINTER(_c_int),
                                                          ctypes.POINTER(_c_int)]),
            "jo_flash_attention": (None, [_f32p] * 4 + [_c_int] * 7 + [ctypes.c_float]),
            "jo_flash_tiles": (None, [_c_int, _c_int, _c_i64, ctypes.POINTER(_c_int),
                                      ctypes.POINTER(_c_int)]),
            "jo_matmul_int8": (None, [_i8p, _i8p, _f32p, _c_int, _c_int, _c_int,
                                      ctypes.c_float, ctypes.c_float, _f32p]),
            "jo_w8a16": (None, [_f32p, _i8p, _f32p, _f32p, _f32p] + [_c_int] * 4),
            "jo64_act": (ctypes.c_double, [_c_int, ctypes.c_double]),
            "jo64_gemm_bias_act": (None, [_f32p, _f32p, _f32p, _f64p] + [_c_int] * 4
                                   + [_i32p, _c_int]),
            "jo64_attention_head": (None, [_f32p, _f32p, _f32p, _f64p, _c_int, _c_int,
                                           _c_int, ctypes.c_double, _i32p, _c_int]),
            "jo64_w8a16": (None, [_f32p, _i8p, _f32p, _f32p, _f64p] + [_c_int] * 4),
            "jo_softmax": (None, [_f32p, _f32p, _c_int, _c_int]),
            "jo_layernorm": (None, [_f32p, _f32p, _f32p, _f32p, _c_int, _c_int, ctypes.c_float]),
            "jo_cross_entropy": (ctypes.c_float, [_f32p, _i32p, _f32p, _c_int, _c_int]),
            "jo64_softmax": (None, [_f64p, _f32p, _c_int, _c_int]),
            "jo64_layernorm": (None, [_f64p, _f32p, _f32p, _f32p, _c_int, _c_int,
                                      ctypes.c_double]),
            "jo64_cross_entropy": (ctypes.c_double, [_f32p, _i32p, _f64p, _c_int, _c_int]),
            "jo_max_threads": (_c_int, []),
            "jo_set_threads": (None, [_c_int]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a, ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctype))


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def act_code(act):
    return ACT[act] if isinstance(act, str) else int(act)


# ---- scalar / elementwise -------------------------------------------------
def fast_exp(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().jo_fast_exp_array(_p(out, ctypes.c_float), _p(x, ctypes.c_float), x.size)
    return out


def act_array(act, x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().jo_act_array(act_code(act), _p(out, ctypes.c_float), _p(x, ctypes.c_float), x.size)
    return out


def fused_gelu(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().jo_fused_gelu(_p(out, ctypes.c_float), _p(x, ctypes.c_float), x.size)
    return out


# ---- GEMM ----------------------------------------------------------------
def tile_analytical(M, N, K, l1d=48 * 1024, l2=32 * 1024, avx512=True):
    """TilePlanner::computeAnalytical.  The l2 default reproduces the
    reference's reading of sysfs cache/index1 (the L1 instruction cache on
    x86) as "L2" (reference ExecutionArena.h:74-76)."""
    tm, tn, tk = _c_int(), _c_int(), _c_int()
    lib().jo_tile_analytical(M, N, K, l1d, l2, int(avx512), ctypes.byref(tm),
                             ctypes.byref(tn), ctypes.byref(tk))
    return tm.value, tn.value, tk.value


def matmul_bias_act(A, B, bias, act, tiles=None):
    """act(A.B + bias) via the restated tiled AVX-512 kernel (fp32)."""
    A = _f32(A)
    B = _f32(B)
    M, K = A.shape
    K2, N = B.shape
    assert K == K2
    bias = None if bias is None else _f32(bias)
    tm, tn, tk = tiles if tiles is not None else tile_analytical(M, N, K)
    out = np.empty((M, N), np.float32)
    lib().jo_matmul_bias_act(_p(A, ctypes.c_float), _p(B, ctypes.c_float),
                             _p(bias, ctypes.c_float), _p(out, ctypes.c_float),
                             M, K, N, tm, tn, tk, act_code(act))
    return out


def tiled_matmul_act(A, B, act, tiles=None):
    A = _f32(A)
    B = _f32(B)
    M, K = A.shape
    _, N = B.shape
    tm, tn, tk = tiles if tiles is not None else tile_analytical(M, N, K)
    out = np.empty((M, N), np.float32)
    lib().jo_tiled_matmul_act(_p(A, ctypes.c_float), _p(B, ctypes.c_float),
                              _p(out, ctypes.c_float), M, N, K, tm, tn, tk, act_code(act))
    return out


def gemm64(A, B, bias, act, rows=None):
    A = _f32(A)
    B = _f32(B)
    M, K = A.shape
    _, N = B.shape
    bias = None if bias is None else _f32(bias)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    R = M if r is None else len(r)
    out = np.empty((R, N), np.float64)
    lib().jo64_gemm_bias_act(_p(A, ctypes.c_float), _p(B, ctypes.c_float),
                             _p(bias, ctypes.c_float), _p(out, ctypes.c_double),
                             M, N, K, act_code(act), _p(r, ctypes.c_int32), R)
    return out


# ---- attention -------------------------------------------------------------
def flash_tiles(S, D, l2=32 * 1024):
    tq, tk = _c_int(), _c_int()
    lib().jo_flash_tiles(S, D, l2, ctypes.byref(tq), ctypes.byref(tk))
    return tq.value, tk.value


def flash_attention(Q, K, V, causal, scale=None, tiles=(32, 64)):
    Q = _f32(Q)
    K = _f32(K)
    V = _f32(V)
    B, H, S, D = Q.shape
    if scale is None:
        scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.empty_like(Q)
    lib().jo_flash_attention(_p(out, ctypes.c_float), _p(Q, ctypes.c_float),
                             _p(K, ctypes.c_float), _p(V, ctypes.c_float),
                             B, H, S, D, tiles[0], tiles[1], int(causal), scale)
    return out


def attention64_head(q, k, v, causal, scale, rows=None):
    """fp64 softmax attention for one head; q,k,v [S,D]."""
    q = _f32(q)
    k = _f32(k)
    v = _f32(v)
    S, D = q.shape
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    R = S if r is None else len(r)
    out = np.empty((R, D), np.float64)
    lib().jo64_attention_head(_p(q, ctypes.c_float), _p(k, ctypes.c_float),
                              _p(v, ctypes.c_float), _p(out, ctypes.c_double),
                              S, D, int(causal), float(scale), _p(r, ctypes.c_int32), R)
    return out


def attention64(Q, K, V, causal, scale):
    B, H, S, D = Q.shape
    out = np.empty((B, H, S, D), np.float64)
    for b in range(B):
        for h in range(H):
            out[b, h] = attention64_head(Q[b, h], K[b, h], V[b, h], causal, scale)
    return out


# ---- int8 ------------------------------------------------------------------
def matmul_int8(A, B, scale_a, scale_b, bias=None):
    A = np.ascontiguousarray(A, np.int8)
    B = np.ascontiguousarray(B, np.int8)
    M, K = A.shape
    _, N = B.shape
    bias = None if bias is None else _f32(bias)
    out = np.empty((M, N), np.float32)
    lib().jo_matmul_int8(_p(A, ctypes.c_int8), _p(B, ctypes.c_int8), _p(out, ctypes.c_float),
                         M, N, K, float(scale_a), float(scale_b), _p(bias, ctypes.c_float))
    return out


def w8a8(A, B, scale_a, scale_b, bias=None):
    """W8A8 with per-token scales scale_a [M] (None: 1) and per-channel scales
    scale_b [N]: the per-element form of matmulInt8's scalar path
    (FusedKernels.h:1046-1066).  Exact integer accumulation, the product
    scale_a[i] * scale_b[j] rounded to fp32, one fp32 multiply of the
    fp32-rounded integer, one fp32 add of bias.  numpy, bit-exact."""
    A = np.asarray(A, np.int8)
    B = np.asarray(B, np.int8)
    M, N = A.shape[0], B.shape[1]
    acc = A.astype(np.int64) @ B.astype(np.int64)
    sa = np.ones(M, np.float32) if scale_a is None else np.asarray(scale_a, np.float32)
    sb = np.asarray(scale_b, np.float32)
    prod = (sa[:, None] * sb[None, :]).astype(np.float32)
    c = acc.astype(np.float32) * prod
    if bias is not None:
        c = c + np.asarray(bias, np.float32)[None, :]
    return c.astype(np.float32)


def w8a16(x, W, scale, bias, act):
    x = _f32(x)
    W = np.ascontiguousarray(W, np.int8)
    scale = _f32(scale)
    bias = None if bias is None else _f32(bias)
    M, K = x.shape
    _, N = W.shape
    out = np.empty((M, N), np.float32)
    lib().jo_w8a16(_p(x, ctypes.c_float), _p(W, ctypes.c_int8), _p(scale, ctypes.c_float),
                   _p(bias, ctypes.c_float), _p(out, ctypes.c_float), M, N, K, act_code(act))
    return out


def w8a16_64(x, W, scale, bias, act):
    x = _f32(x)
    W = np.ascontiguousarray(W, np.int8)
    scale = _f32(scale)
    bias = None if bias is None else _f32(bias)
    M, K = x.shape
    _, N = W.shape
    out = np.empty((M, N), np.float64)
    lib().jo64_w8a16(_p(x, ctypes.c_float), _p(W, ctypes.c_int8), _p(scale, ctypes.c_float),
                     _p(bias, ctypes.c_float), _p(out, ctypes.c_double), M, N, K, act_code(act))
    return out


# ---- row kernels (reference FusedKernels.h:464-526, :532-600, :766-854) ----
def softmax(x):
    """fusedSoftmax restated (AVX-512 path) over the rows of a 2-D array."""
    x = _f32(x)
    M, N = x.shape
    out = np.empty_like(x)
    lib().jo_softmax(_p(out, ctypes.c_float), _p(x, ctypes.c_float), M, N)
    return out


def softmax64(x):
    x = _f32(x)
    M, N = x.shape
    out = np.empty((M, N), np.float64)
    lib().jo64_softmax(_p(out, ctypes.c_double), _p(x, ctypes.c_float), M, N)
    return out


def layernorm(x, gamma, beta, eps=1e-5):
    """fusedLayerNorm restated (AVX-512 path)."""
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    M, N = x.shape
    out = np.empty_like(x)
    lib().jo_layernorm(_p(out, ctypes.c_float), _p(x, ctypes.c_float), _p(gamma, ctypes.c_float),
                       _p(beta, ctypes.c_float), M, N, float(eps))
    return out


def layernorm64(x, gamma, beta, eps=1e-5):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    M, N = x.shape
    out = np.empty((M, N), np.float64)
    lib().jo64_layernorm(_p(out, ctypes.c_double), _p(x, ctypes.c_float),
                         _p(gamma, ctypes.c_float), _p(beta, ctypes.c_float), M, N, float(eps))
    return out


def cross_entropy(logits, targets):
    """fusedCrossEntropyLoss restated (AVX-512 path): (mean loss, grad)."""
    x = _f32(logits)
    t = np.ascontiguousarray(targets, np.int32)
    M, N = x.shape
    grad = np.empty_like(x)
    loss = lib().jo_cross_entropy(_p(x, ctypes.c_float), _p(t, ctypes.c_int32),
                                  _p(grad, ctypes.c_float), M, N)
    return float(loss), grad


def cross_entropy64(logits, targets):
    x = _f32(logits)
    t = np.ascontiguousarray(targets, np.int32)
    M, N = x.shape
    grad = np.empty((M, N), np.float64)
    loss = lib().jo64_cross_entropy(_p(x, ctypes.c_float), _p(t, ctypes.c_int32),
                                    _p(grad, ctypes.c_double), M, N)
    return float(loss), grad


def attention_bwd64(Q, K, V, dO, causal, scale):
    """Attention backward in fp64 numpy, per (b, h), from the textbook
    definitions (the reference has no backward; its forward is
    FlashAttention.h:130-309):
      S = scale Q K^T (causal: key j > query i masked), P = softmax(S),
      O = P V, dP = dO V^T, dS = P * (dP - rowsum(dO * O)),
      dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO.
    Q, K, V, dO: [B, H, S, D].  Returns (dQ, dK, dV, O) as float64."""
    Q, K, V, dO = (np.asarray(a, np.float64) for a in (Q, K, V, dO))
    Sq = Q.shape[2]
    s = np.einsum("bhid,bhjd->bhij", Q, K) * scale
    if causal:
        s = np.where(np.tril(np.ones((Sq, Sq), bool)), s, -np.inf)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    O = np.einsum("bhij,bhjd->bhid", p, V)
    dP = np.einsum("bhid,bhjd->bhij", dO, V)
    dS = p * (dP - np.sum(dO * O, axis=-1, keepdims=True))
    dQ = scale * np.einsum("bhij,bhjd->bhid", dS, K)
    dK = scale * np.einsum("bhij,bhid->bhjd", dS, Q)
    dV = np.einsum("bhij,bhid->bhjd", p, dO)
    return dQ, dK, dV, O


def mlp_forward_backward64(X, W1, b1, W2, b2, targets, relu_mask=None):
    """interleavedMLPForwardBackward (include/jules/Kernel/InterleavedAutodiff.h
    :55-441) restated in fp64 numpy, whole-matrix instead of per tile (the
    reference's tiles only change the summation order of its BLAS calls):
      h = X W1 + b1, a = relu(h)                       :144-166
      o = a W2 + b2 (the output)                       :168-176
      p = exp(o - rowmax) / rowsum, loss_i = -log(p[t_i] + 1e-10),
      dO = (p - onehot(t)) / M                         :178-197
      dW2 = a^T dO, db2 = colsum(dO)                   :207-221
      dH = (dO W2^T) * (h > 0)                         :223-247
      dW1 = X^T dH, db1 = colsum(dH), dX = dH W1^T     :249-267
      loss = sum_i loss_i / M                          :435
    Returns a dict of float64 arrays (loss a float).  M = 0 gives zero
    gradients and a NaN loss (0/0).  relu_mask, if given, replaces h > 0 in
    the backward (relu'(h) for |h| within rounding of 0 is decided by the
    rounding of whoever computed h; a checker passes the mask the checked
    code used)."""
    X = np.asarray(X, np.float64)
    W1, b1 = np.asarray(W1, np.float64), np.asarray(b1, np.float64)
    W2, b2 = np.asarray(W2, np.float64), np.asarray(b2, np.float64)
    t = np.asarray(targets, np.int64)
    M = X.shape[0]
    h = X @ W1 + b1
    a = np.where(h > 0, h, 0.0)
    o = a @ W2 + b2
    if M == 0:
        z = np.zeros
        return {"output": o, "loss": float("nan"), "dW1": z(W1.shape), "db1": z(b1.shape),
                "dW2": z(W2.shape), "db2": z(b2.shape), "dX": z(X.shape)}
    e = np.exp(o - o.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    rows = np.arange(M)
    loss = float(np.sum(-np.log(p[rows, t] + 1e-10)) / M)
    dO = p.copy()
    dO[rows, t] -= 1.0
    dO /= M
    dH = np.where(h > 0 if relu_mask is None else relu_mask, dO @ W2.T, 0.0)
    return {"output": o, "loss": loss, "dW1": X.T @ dH, "db1": dH.sum(axis=0), "dW2": a.T @ dO,
            "db2": dO.sum(axis=0), "dX": dH @ W1.T}


def max_threads():
    return lib().jo_max_threads()


def set_threads(n):
    lib().jo_set_threads(int(n))
