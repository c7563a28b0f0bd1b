"""CPU tests of the torch front end's argument checks (jules_amd/ops.py).

The C ABI sees raw pointers only, so a tensor of the wrong shape handed to it
would become an out-of-bounds GPU access.  The front end checks dtype,
contiguity and shape of every input, output and workspace before the device,
so these cases raise ValueError on CPU tensors without reaching the library.
"""
import pytest
import torch

from jules_amd import ops

f32, bf16, i8, i32 = torch.float32, torch.bfloat16, torch.int8, torch.int32


def _t(shape, dtype=f32):
    return torch.zeros(shape, dtype=dtype)


def _raises(fn, *args, match, **kw):
    with pytest.raises(ValueError, match=match):
        fn(*args, **kw)


def test_need_rejects_cpu_tensor_last():
    # a well-formed CPU tensor gets the device message, not a shape message
    _raises(ops.gemm_bias_act, _t((4, 8)), _t((8, 16)), match="GPU tensor")


@pytest.mark.parametrize("kw,match", [
    (dict(B=_t((9, 16))), "inner dimensions"),
    (dict(bias=_t((15,))), "elements"),
    (dict(out=_t((4, 15))), "shape"),
    (dict(out=_t((4, 16), bf16)), "dtype"),
    (dict(A=_t((4, 8, 1))), "dimensions"),
])
def test_gemm_checks(kw, match):
    args = dict(A=_t((4, 8)), B=_t((8, 16)), bias=None, out=None)
    args.update(kw)
    _raises(ops.gemm_bias_act, args["A"], args["B"], bias=args["bias"], out=args["out"], match=match)


def test_activation_out_size():
    _raises(ops.activation, _t((4, 8)), out=_t((31,)), match="elements")


@pytest.mark.parametrize("kw,match", [
    (dict(K=_t((1, 2, 9, 64), bf16)), "shape"),
    (dict(out=_t((1, 2, 8, 32), bf16)), "shape"),
    (dict(lse=_t((1, 2, 7))), "elements"),
    (dict(Q=_t((2, 8, 64), bf16)), "dimensions"),
])
def test_flash_checks(kw, match):
    a = dict(Q=_t((1, 2, 8, 64), bf16), K=_t((1, 2, 8, 64), bf16), V=_t((1, 2, 8, 64), bf16),
             out=None, lse=None)
    a.update(kw)
    _raises(ops.flash_attention, a["Q"], a["K"], a["V"], out=a["out"], lse=a["lse"], match=match)


def test_flash_bwd_checks():
    q = _t((1, 2, 8, 64), bf16)
    _raises(ops.flash_attention_bwd, q, q, q, _t((1, 2, 8, 32), bf16), q, _t((16,)), match="shape")
    _raises(ops.flash_attention_bwd, q, q, q, q, q, _t((15,)), match="elements")
    _raises(ops.flash_attention_bwd, q, q, q, q, q, _t((16,)), dK=_t((1, 2, 8, 63), bf16),
            match="shape")


@pytest.mark.parametrize("kw,match", [
    (dict(W=_t((64, 32), i8)), "inner dimensions"),
    (dict(scale=_t((31,))), "elements"),
    (dict(bias=_t((33,))), "elements"),
    (dict(out=_t((8, 32), f32)), "dtype"),
    (dict(out=_t((8, 16), bf16)), "shape"),
])
def test_w8a16_checks(kw, match):
    a = dict(x=_t((8, 32), bf16), W=_t((32, 32), i8), scale=_t((32,)), bias=None, out=None)
    a.update(kw)
    _raises(ops.w8a16_gemm, a["x"], a["W"], a["scale"], bias=a["bias"], out=a["out"], match=match)


@pytest.mark.parametrize("kw,match", [
    (dict(B=_t((31, 16), i8)), "inner dimensions"),
    (dict(bias=_t((17,))), "elements"),
    (dict(out=_t((4, 17))), "shape"),
])
def test_int8_checks(kw, match):
    a = dict(A=_t((4, 32), i8), B=_t((32, 16), i8), bias=None, out=None)
    a.update(kw)
    _raises(ops.matmul_int8, a["A"], a["B"], 1.0, 1.0, bias=a["bias"], out=a["out"], match=match)


def test_w8a8_checks():
    A, B = _t((4, 32), i8), _t((32, 16), i8)
    _raises(ops.matmul_w8a8, A, B, _t((3,)), _t((16,)), match="elements")
    _raises(ops.matmul_w8a8, A, B, None, _t((15,)), match="elements")
    _raises(ops.matmul_w8a8, A, B, None, _t((16,)), bias=_t((8,)), match="elements")
    _raises(ops.matmul_w8a8, A, B, None, _t((16,)), out=_t((16, 4)), match="shape")


def test_row_kernel_checks():
    x = _t((4, 10))
    _raises(ops.softmax, x, out=_t((4, 9)), match="shape")
    _raises(ops.softmax, x, out=_t((4, 10), bf16), match="dtype")
    _raises(ops.layernorm, x, _t((9,)), _t((10,)), match="elements")
    _raises(ops.layernorm, x, _t((10,)), _t((11,)), match="elements")
    _raises(ops.layernorm, x, _t((10,)), _t((10,)), out=_t((40,)), match="shape")
    _raises(ops.cross_entropy, x, _t((3,), i32), match="elements")
    _raises(ops.cross_entropy, x, _t((4,), i32), grad=_t((4, 11)), match="shape")
    _raises(ops.cross_entropy, x, _t((4,), i32), loss=_t((2,)), match="elements")


def test_mlp_checks():
    X, W1, b1, W2, b2 = _t((4, 3)), _t((3, 5)), _t((5,)), _t((5, 2)), _t((2,))
    _raises(ops.mlp_forward, _t((4, 3, 1)), W1, b1, W2, b2, match="dimensions")
    _raises(ops.mlp_forward_backward, X, W1, b1, W2, b2, _t((4,), i32), match="GPU tensor")
