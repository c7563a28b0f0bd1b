"""torch-tensor front end of the C ABI.

Each function checks every tensor it is given (inputs, outputs, workspaces):
first dtype, contiguity and shape, then, for all of them together, that they
are GPU tensors on one device; only then does it call the corresponding
jules_hip_* entry point on torch's current HIP stream.  The C ABI sees raw
pointers only, so these checks are what keep a wrongly shaped tensor from
becoming an out-of-bounds GPU access.  torch provides device memory and the
stream only; all arithmetic happens in libjules_hip.so.  Names follow the
reference's jules::kernel functions (include/jules/Kernel/FusedKernels.h,
FlashAttention.h).
"""
import numpy as np

import torch

from ._lib import ACT, BF16, F32, check, lib

_DT = {torch.float32: F32, torch.bfloat16: BF16}


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t):
    return None if t is None else t.data_ptr()


def _need(t, name, dtypes, shape=None, numel=None):
    """Structural check of one tensor argument: dtype, contiguity and shape
    (or element count).  Raises ValueError."""
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.dtype not in dtypes:
        raise ValueError(f"{name}: dtype {t.dtype} not in {dtypes}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{name}: {t.numel()} elements, expected {numel}")


def _rank(t, name, rank):
    if not isinstance(t, torch.Tensor):
        raise ValueError(f"{name} must be a torch.Tensor")
    if t.dim() != rank:
        raise ValueError(f"{name} must have {rank} dimensions, got {t.dim()}")


def _workspace(ws, name):
    """A caller-supplied workspace: any dtype, contiguous; returns its size
    in bytes (the C ABI checks it against what the call needs)."""
    if not isinstance(ws, torch.Tensor) or not ws.is_contiguous():
        raise ValueError(f"{name} must be a contiguous tensor")
    return ws.numel() * ws.element_size()


def _on_device(**tensors):
    """Every given tensor (None entries skipped) is a GPU tensor on the device
    of the first one; returns that device."""
    dev = None
    for name, t in tensors.items():
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{name} must be a GPU tensor")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")
    return dev


def _act(act):
    return ACT[act] if isinstance(act, str) else int(act)


def gemm_bias_act(A, B, bias=None, act="none", out=None):
    """C = act(A @ B + bias).  fp32 (bit-exact with the reference's fma chain) or
    bf16 (MFMA, fp32 accumulate).  Mirrors tiledMatmulWithActivation /
    fusedMatmulBiasRelu (FusedKernels.h:378, :265)."""
    _rank(A, "A", 2)
    _rank(B, "B", 2)
    _need(A, "A", (torch.float32, torch.bfloat16))
    _need(B, "B", (A.dtype,))
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    if bias is not None:
        _need(bias, "bias", (torch.float32,), numel=N)
    if out is not None:
        _need(out, "out", (A.dtype,), shape=(M, N))
    _on_device(A=A, B=B, bias=bias, out=out)
    if out is None:
        out = torch.empty((M, N), dtype=A.dtype, device=A.device)
    check(lib().jules_hip_gemm_bias_act(_DT[A.dtype], _act(act), _ptr(A), _ptr(B), _ptr(bias),
                                        _ptr(out), M, N, K, _stream(A)))
    return out


def activation(x, act="gelu", out=None):
    """out = act(x), fp32; act='gelu' is fusedGelu (FusedKernels.h:606)."""
    _need(x, "x", (torch.float32,))
    if out is not None:
        _need(out, "out", (torch.float32,), numel=x.numel())
    _on_device(x=x, out=out)
    if out is None:
        out = torch.empty_like(x)
    check(lib().jules_hip_activation(_act(act), _ptr(out), _ptr(x), x.numel(), _stream(x)))
    return out


def default_scale(D):
    """1.0f / sqrtf((float)D) evaluated in fp32, as FlashAttention.h:135 does."""
    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


def flash_attention(Q, K, V, causal=False, scale=None, out=None, lse=None):
    """Flash-attention forward, [B,H,S,D]; scale defaults to 1/sqrtf(D) as in
    flashAttention (FlashAttention.h:135)."""
    _rank(Q, "Q", 4)
    _need(Q, "Q", (torch.float32, torch.bfloat16))
    _need(K, "K", (Q.dtype,), shape=Q.shape)
    _need(V, "V", (Q.dtype,), shape=Q.shape)
    B, H, S, D = Q.shape
    if out is not None:
        _need(out, "out", (Q.dtype,), shape=Q.shape)
    if lse is not None:
        _need(lse, "lse", (torch.float32,), numel=B * H * S)
    _on_device(Q=Q, K=K, V=V, out=out, lse=lse)
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty_like(Q)
    check(lib().jules_hip_flash_attn_fwd(_DT[Q.dtype], int(bool(causal)), float(scale), _ptr(Q),
                                         _ptr(K), _ptr(V), _ptr(out), _ptr(lse), B, H, S, D,
                                         _stream(Q)))
    return out


def flash_attention_bwd(Q, K, V, O, dO, lse, causal=False, scale=None, dQ=None, dK=None, dV=None,
                        workspace=None):
    """Flash-attention backward (jules_hip_flash_attn_bwd; no reference
    counterpart): (dQ, dK, dV) for the forward O = flash_attention(Q, K, V,
    causal, scale, lse=lse).  bf16 [B,H,S,D]; lse fp32 [B,H,S]."""
    _rank(Q, "Q", 4)
    _need(Q, "Q", (torch.bfloat16,))
    for t, n in ((K, "K"), (V, "V"), (O, "O"), (dO, "dO")):
        _need(t, n, (Q.dtype,), shape=Q.shape)
    B, H, S, D = Q.shape
    _need(lse, "lse", (torch.float32,), numel=B * H * S)
    for t, n in ((dQ, "dQ"), (dK, "dK"), (dV, "dV")):
        if t is not None:
            _need(t, n, (Q.dtype,), shape=Q.shape)
    ws_bytes = None if workspace is None else _workspace(workspace, "workspace")
    _on_device(Q=Q, K=K, V=V, O=O, dO=dO, lse=lse, dQ=dQ, dK=dK, dV=dV, workspace=workspace)
    if scale is None:
        scale = default_scale(D)
    dQ = torch.empty_like(Q) if dQ is None else dQ
    dK = torch.empty_like(Q) if dK is None else dK
    dV = torch.empty_like(Q) if dV is None else dV
    if workspace is None:
        nbytes = lib().jules_hip_flash_attn_bwd_workspace_size(B, H, S)
        workspace = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=Q.device)
        ws_bytes = workspace.numel()
    check(lib().jules_hip_flash_attn_bwd(_DT[Q.dtype], int(bool(causal)), float(scale), _ptr(Q),
                                         _ptr(K), _ptr(V), _ptr(O), _ptr(dO), _ptr(lse), _ptr(dQ),
                                         _ptr(dK), _ptr(dV), B, H, S, D, _ptr(workspace),
                                         ws_bytes, _stream(Q)))
    return dQ, dK, dV


def w8a16_workspace(M, N, K, device):
    n = lib().jules_hip_w8a16_workspace_size(M, N, K)
    return torch.zeros(max(n, 16), dtype=torch.uint8, device=device)


def w8a16_gemm(x, W, scale, bias=None, act="silu", out=None, workspace=None):
    """y = act(scale * (x @ W) + bias); x bf16 [M,K], W int8 [K,N]."""
    _rank(x, "x", 2)
    _rank(W, "W", 2)
    _need(x, "x", (torch.bfloat16,))
    _need(W, "W", (torch.int8,))
    M, K = x.shape
    K2, N = W.shape
    if K != K2:
        raise ValueError("inner dimensions differ")
    _need(scale, "scale", (torch.float32,), numel=N)
    if bias is not None:
        _need(bias, "bias", (torch.float32,), numel=N)
    if out is not None:
        _need(out, "out", (torch.bfloat16,), shape=(M, N))
    ws_bytes = None if workspace is None else _workspace(workspace, "workspace")
    _on_device(x=x, W=W, scale=scale, bias=bias, out=out, workspace=workspace)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    if workspace is None:
        workspace = w8a16_workspace(M, N, K, x.device)
        ws_bytes = workspace.numel()
    check(lib().jules_hip_w8a16_gemm_bias_act(_act(act), _ptr(x), _ptr(W), _ptr(scale),
                                              _ptr(bias), _ptr(out), M, N, K, _ptr(workspace),
                                              ws_bytes, _stream(x)))
    return out


class PackedW8:
    """int8 weights [K,N] repacked for jules_hip_w8a16_packed_gemm_bias_act:
    `data` is the packed uint8 array, K and N the logical shape."""

    def __init__(self, data, K, N):
        self.data, self.K, self.N = data, K, N


def w8a16_pack(W):
    """Repack int8 W [K,N] (row-major) into the packed W8A16 layout (done
    once, at weight-load time)."""
    _rank(W, "W", 2)
    _need(W, "W", (torch.int8,))
    _on_device(W=W)
    K, N = W.shape
    n = lib().jules_hip_w8a16_packed_size(K, N)
    if n == 0:
        raise ValueError(f"w8a16_pack: unsupported shape {tuple(W.shape)}")
    Wp = torch.empty((n,), dtype=torch.uint8, device=W.device)
    check(lib().jules_hip_w8a16_pack(_ptr(W), K, N, _ptr(Wp), n, _stream(W)))
    return PackedW8(Wp, K, N)


def w8a16_gemm_packed(x, Wp, scale, bias=None, act="silu", out=None):
    """y = act(scale * (x @ W) + bias) with W given packed (w8a16_pack);
    x bf16 [M,K]."""
    if not isinstance(Wp, PackedW8):
        raise TypeError("Wp must come from w8a16_pack")
    _rank(x, "x", 2)
    _need(x, "x", (torch.bfloat16,))
    M, K = x.shape
    N = Wp.N
    if K != Wp.K:
        raise ValueError("inner dimensions differ")
    _need(Wp.data, "Wp", (torch.uint8,), numel=lib().jules_hip_w8a16_packed_size(K, N))
    _need(scale, "scale", (torch.float32,), numel=N)
    if bias is not None:
        _need(bias, "bias", (torch.float32,), numel=N)
    if out is not None:
        _need(out, "out", (torch.bfloat16,), shape=(M, N))
    _on_device(x=x, Wp=Wp.data, scale=scale, bias=bias, out=out)
    if out is None:
        out = torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    check(lib().jules_hip_w8a16_packed_gemm_bias_act(_act(act), _ptr(x), _ptr(Wp.data), _ptr(scale),
                                                     _ptr(bias), _ptr(out), M, N, K, _stream(x)))
    return out


def _int8_operands(A, B, bias, out):
    _rank(A, "A", 2)
    _rank(B, "B", 2)
    _need(A, "A", (torch.int8,))
    _need(B, "B", (torch.int8,))
    M, K = A.shape
    K2, N = B.shape
    if K != K2:
        raise ValueError(f"inner dimensions differ: {K} vs {K2}")
    if bias is not None:
        _need(bias, "bias", (torch.float32,), numel=N)
    if out is not None:
        _need(out, "out", (torch.float32,), shape=(M, N))
    return M, N, K


def matmul_int8(A, B, scale_a, scale_b, bias=None, out=None):
    """matmulInt8 (FusedKernels.h:867) with the scalar path's semantics."""
    M, N, K = _int8_operands(A, B, bias, out)
    _on_device(A=A, B=B, bias=bias, out=out)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=A.device)
    check(lib().jules_hip_matmul_int8(_ptr(A), _ptr(B), _ptr(out), M, N, K, float(scale_a),
                                      float(scale_b), _ptr(bias), _stream(A)))
    return out


def matmul_w8a8(A, B, scale_a, scale_b, bias=None, out=None):
    """C = float(A @ B) * (scale_a[i] * scale_b[j]) [+ bias] with exact int32
    accumulation (jules_hip_matmul_w8a8): int8 A [M,K], B [K,N], fp32
    per-token scale_a [M] (or None) and per-channel scale_b [N]."""
    M, N, K = _int8_operands(A, B, bias, out)
    if scale_a is not None:
        _need(scale_a, "scale_a", (torch.float32,), numel=M)
    _need(scale_b, "scale_b", (torch.float32,), numel=N)
    _on_device(A=A, B=B, scale_a=scale_a, scale_b=scale_b, bias=bias, out=out)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=A.device)
    check(lib().jules_hip_matmul_w8a8(_ptr(A), _ptr(B), _ptr(out), M, N, K, _ptr(scale_a),
                                      _ptr(scale_b), _ptr(bias), _stream(A)))
    return out


def _rows(x):
    N = x.shape[-1] if x.dim() > 0 else 1
    return x.numel() // max(N, 1) if N else 0, N


def softmax(x, out=None):
    """fusedSoftmax (FusedKernels.h:464) over the last dimension of fp32 x."""
    _need(x, "x", (torch.float32,))
    if out is not None:
        _need(out, "out", (torch.float32,), shape=x.shape)
    _on_device(x=x, out=out)
    if out is None:
        out = torch.empty_like(x)
    M, N = _rows(x)
    check(lib().jules_hip_softmax(_ptr(out), _ptr(x), M, N, _stream(x)))
    return out


def layernorm(x, gamma, beta, eps=1e-5, out=None):
    """fusedLayerNorm (FusedKernels.h:532) over the last dimension of fp32 x."""
    _need(x, "x", (torch.float32,))
    M, N = _rows(x)
    _need(gamma, "gamma", (torch.float32,), numel=N)
    _need(beta, "beta", (torch.float32,), numel=N)
    if out is not None:
        _need(out, "out", (torch.float32,), shape=x.shape)
    _on_device(x=x, gamma=gamma, beta=beta, out=out)
    if out is None:
        out = torch.empty_like(x)
    check(lib().jules_hip_layernorm(_ptr(out), _ptr(x), _ptr(gamma), _ptr(beta), M, N,
                                    float(eps), _stream(x)))
    return out


def cross_entropy_workspace(M, device):
    nbytes = lib().jules_hip_cross_entropy_workspace_size(int(M))
    return torch.empty(((nbytes + 3) // 4,), dtype=torch.float32, device=device)


def cross_entropy(logits, targets, grad=None, loss=None, workspace=None):
    """fusedCrossEntropyLoss (FusedKernels.h:766): returns (loss[1], grad) on the device."""
    _need(logits, "logits", (torch.float32,))
    M, N = _rows(logits)
    _need(targets, "targets", (torch.int32,), numel=M)
    if grad is not None:
        _need(grad, "grad", (torch.float32,), shape=logits.shape)
    if loss is not None:
        _need(loss, "loss", (torch.float32,), numel=1)
    ws_bytes = None if workspace is None else _workspace(workspace, "workspace")
    _on_device(logits=logits, targets=targets, grad=grad, loss=loss, workspace=workspace)
    if grad is None:
        grad = torch.empty_like(logits)
    if loss is None:
        loss = torch.empty((1,), dtype=torch.float32, device=logits.device)
    if workspace is None:
        workspace = cross_entropy_workspace(M, logits.device)
        ws_bytes = workspace.numel() * 4
    check(lib().jules_hip_cross_entropy(_ptr(logits), _ptr(targets), _ptr(grad), _ptr(loss), M, N,
                                        _ptr(workspace), ws_bytes, _stream(logits)))
    return loss, grad


def _mlp_operands(X, W1, b1, W2, b2):
    for t, n in ((X, "X"), (W1, "W1"), (W2, "W2")):
        _rank(t, n, 2)
    for t, n in ((X, "X"), (W1, "W1"), (b1, "b1"), (W2, "W2"), (b2, "b2")):
        _need(t, n, (torch.float32,))
    M, K1 = X.shape
    K1b, N1 = W1.shape
    N1b, N2 = W2.shape
    if K1b != K1 or N1b != N1 or b1.numel() != N1 or b2.numel() != N2:
        raise ValueError("mlp: operand shapes disagree")
    return M, K1, N1, N2


def mlp_forward(X, W1, b1, W2, b2, out=None, workspace=None):
    """fusedMLPForward (FusedKernels.h:659): relu(X W1 + b1) W2 + b2, fp32."""
    M, K1, N1, N2 = _mlp_operands(X, W1, b1, W2, b2)
    if out is not None:
        _need(out, "out", (torch.float32,), shape=(M, N2))
    ws_bytes = None if workspace is None else _workspace(workspace, "workspace")
    _on_device(X=X, W1=W1, b1=b1, W2=W2, b2=b2, out=out, workspace=workspace)
    if out is None:
        out = torch.empty((M, N2), dtype=torch.float32, device=X.device)
    if workspace is None:
        nbytes = lib().jules_hip_mlp_forward_workspace_size(M, K1, N1, N2)
        workspace = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=X.device)
        ws_bytes = workspace.numel()
    check(lib().jules_hip_mlp_forward(_ptr(X), _ptr(W1), _ptr(b1), _ptr(W2), _ptr(b2), _ptr(out),
                                      M, K1, N1, N2, _ptr(workspace), ws_bytes, _stream(X)))
    return out


def mlp_workspace(M, K1, N1, N2, device):
    nbytes = lib().jules_hip_mlp_workspace_size(int(M), int(K1), int(N1), int(N2))
    return torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=device)


def mlp_forward_backward(X, W1, b1, W2, b2, targets, with_dX=False, workspace=None, out=None):
    """interleavedMLPForwardBackward (InterleavedAutodiff.h:55): fp32 2-layer
    MLP, softmax cross entropy against int32 targets, and the gradients.
    Returns a dict with output, loss (1 element), dW1, db1, dW2, db2 and
    dX (None unless with_dX), all on X's device; `out`, a dict returned by an
    earlier call with the same shapes, is reused instead of allocating."""
    M, K1, N1, N2 = _mlp_operands(X, W1, b1, W2, b2)
    _need(targets, "targets", (torch.int32,), numel=M)
    shapes = {"output": (M, N2), "loss": (1,), "dW1": (K1, N1), "db1": (N1,), "dW2": (N1, N2),
              "db2": (N2,), "dX": (M, K1)}
    if out is not None:
        with_dX = out["dX"] is not None
        for k, shp in shapes.items():
            if out[k] is not None:
                _need(out[k], f"out[{k!r}]", (torch.float32,), shape=shp)
    ws_bytes = None if workspace is None else _workspace(workspace, "workspace")
    outs = {} if out is None else {f"out[{k!r}]": v for k, v in out.items()}
    dev = _on_device(X=X, W1=W1, b1=b1, W2=W2, b2=b2, targets=targets, workspace=workspace, **outs)
    if out is None:
        out = {k: torch.empty(shp, dtype=torch.float32, device=dev)
               if k != "dX" or with_dX else None for k, shp in shapes.items()}
    if workspace is None:
        workspace = mlp_workspace(M, K1, N1, N2, dev)
        ws_bytes = workspace.numel()
    check(lib().jules_hip_mlp_forward_backward(
        _ptr(X), _ptr(W1), _ptr(b1), _ptr(W2), _ptr(b2), _ptr(targets), _ptr(out["output"]),
        _ptr(out["dW1"]), _ptr(out["db1"]), _ptr(out["dW2"]), _ptr(out["db2"]), _ptr(out["dX"]),
        M, K1, N1, N2, _ptr(out["loss"]), _ptr(workspace), ws_bytes, _stream(X)))
    return out


def mfma_ceiling(out, workgroups, iters):
    """Launch the MFMA calibration kernel (jules_hip_mfma_ceiling; no
    counterpart in the reference) on torch's current stream: `workgroups` x 4
    waves, each issuing 16 * iters v_mfma_f32_32x32x16_bf16 on random
    operands.  out: fp32 GPU tensor of workgroups * 256 elements.  Returns
    the FLOP count of the launch."""
    _need(out, "out", (torch.float32,))
    if out.numel() < workgroups * 256:
        raise ValueError("out must hold workgroups * 256 floats")
    _on_device(out=out)
    check(lib().jules_hip_mfma_ceiling(_ptr(out), int(workgroups), int(iters), _stream(out)))
    return 32768.0 * 16 * iters * 4 * workgroups


def hbm_read_floor(buf, out, workgroups=256):
    """Launch the HBM read calibration (jules_hip_hbm_read_floor; no
    counterpart in the reference) on torch's current stream: one streaming
    read of `buf` (contiguous, a multiple of 16 bytes).  out: int32 GPU tensor
    of workgroups * 256 elements.  Returns the bytes read."""
    if not isinstance(buf, torch.Tensor) or not buf.is_contiguous():
        raise ValueError("buf must be a contiguous tensor")
    _need(out, "out", (torch.int32,))
    if out.numel() < workgroups * 256:
        raise ValueError("out must hold workgroups * 256 int32")
    _on_device(buf=buf, out=out)
    nbytes = buf.numel() * buf.element_size()
    check(lib().jules_hip_hbm_read_floor(_ptr(buf), nbytes, _ptr(out), int(workgroups), _stream(buf)))
    return nbytes
