"""CPU tests of the C ABI boundary: the library loads, exports every function
include/*.h declares, the registry resolves the extern_kernel names, and every
argument error is reported as a status before any device work is done."""
import ctypes
import os
import re
import subprocess

import pytest

from jules_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "jules_hip.h")
CXX_HEADER = os.path.join(ROOT, "include", "jules_hip_kernel.hpp")


def _declared_c_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(jules_hip_\w+)\s*\(", text)))


def _exported():
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if " T " in line}


def test_every_declared_c_function_is_exported():
    decl = _declared_c_functions()
    assert len(decl) >= 11
    exported = _exported()
    missing = [f for f in decl if f not in exported]
    assert not missing, missing
    # the Python binding covers exactly the declared set
    assert sorted(_lib.SIGNATURES) == decl


def test_cxx_shim_symbols_exported():
    """The jules::kernel entry points of include/jules_hip_kernel.hpp."""
    exported = _exported()
    text = open(CXX_HEADER).read()
    names = ["fusedMatmulRelu", "fusedMatmulBiasRelu", "tiledMatmulWithActivation", "fusedGelu",
             "matmulInt8", "flashAttention", "attention", "standardAttention", "lastStatus",
             "fusedSoftmax", "fusedLayerNorm", "fusedCrossEntropyLoss",
             "fusedMLPForward", "interleavedMLPForwardBackward"]
    for n in names:
        assert re.search(rf"\b{n}\s*\(", text), n
        mangled = f"_ZN5jules6kernel{len(n)}{n}E"
        assert any(s.startswith(mangled) for s in exported), n


def test_abi_version_and_status_strings():
    L = _lib.lib()
    assert L.jules_hip_abi_version() == 1
    assert L.jules_hip_status_string(0) == b"ok"
    for code in range(1, 11):
        assert L.jules_hip_status_string(code) not in (b"ok", b"unknown status")
    assert L.jules_hip_status_string(99) == b"unknown status"


def test_registry_names():
    names = _lib.kernel_names()
    routed = ["fusedMatmulRelu", "fusedMatmulSigmoid", "fusedMatmulTanh", "fusedMatmulGelu",
              "fusedMatmulBiasRelu", "fusedMatmulBiasSigmoid", "fusedMatmulBiasTanh",
              "fusedGelu", "matmulInt8", "flashAttention", "fusedSoftmax", "fusedLayerNorm",
              "fusedCrossEntropyLoss", "fusedMLPForward", "interleavedMLPForwardBackward"]
    added = ["fusedMatmulBiasGelu", "flashAttentionCausal", "matmulW8A16BiasSilu"]
    for n in routed + added:
        assert n in names
        assert _lib.lookup(n) is not None
    assert _lib.lookup("noSuchKernel") is None
    assert b"noSuchKernel" in _lib.lib().jules_hip_last_error()
    assert len(set(names)) == len(names)


def test_tensor_descriptor_layout():
    # data, offset, sizes[6], strides[6], rank, dtype (LLVMBackend.h:60-66 + dtype)
    assert ctypes.sizeof(_lib.JhTensor) == 8 + 8 + 48 + 48 + 4 + 4


# ---- validation: these return before touching the device ------------------
OK, NULL, SHAPE, DTYPE, ALIGN, ACT, WS, HIP, UNSUP, NOTFOUND, ARG = range(11)
P = 0x10000  # a non-null, 64 KiB aligned address that is never dereferenced


@pytest.mark.parametrize("args,status", [
    ((0, 9, P, P, None, P, 4, 4, 4, None), ACT),
    ((0, 0, P, P, None, P, -1, 4, 4, None), SHAPE),
    ((0, 0, P, P, None, P, 4, 4, -4, None), SHAPE),
    ((7, 0, P, P, None, P, 4, 4, 4, None), DTYPE),
    ((0, 0, None, P, None, P, 4, 4, 4, None), NULL),
    ((0, 0, P, P, None, None, 4, 4, 4, None), NULL),
    ((1, 0, P, P, None, P, 12, 16, 16, None), UNSUP),
    ((1, 0, P + 2, P, None, P, 16, 16, 16, None), ALIGN),
    ((0, 0, P + 1, P, None, P, 4, 4, 4, None), ALIGN),
    ((0, 0, None, None, None, None, 0, 4, 4, None), OK),    # M = 0: nothing to do
    ((1, 4, None, None, None, None, 8, 0, 8, None), OK),    # N = 0
    ((0, 0, P, P, None, P, 1 << 21, 1 << 21, 1 << 21, None), SHAPE),
])
def test_gemm_validation(args, status):
    assert _lib.lib().jules_hip_gemm_bias_act(*args) == status


@pytest.mark.parametrize("args,status", [
    ((7, 0, 0.125, P, P, P, P, None, 1, 1, 8, 64, None), DTYPE),
    ((0, 0, 0.125, P, P, P, P, None, 1, 1, 8, 160, None), UNSUP),   # head_dim > 128
    ((0, 0, 0.125, P, P, P, P, None, 1, 1, 8, 0, None), SHAPE),
    ((0, 0, float("nan"), P, P, P, P, None, 1, 1, 8, 64, None), ARG),
    ((0, 0, -1.0, P, P, P, P, None, 1, 1, 8, 64, None), ARG),
    ((0, 2, 0.125, P, P, P, P, None, 1, 1, 8, 64, None), ARG),
    ((0, 0, 0.125, None, P, P, P, None, 1, 1, 8, 64, None), NULL),
    ((1, 1, 0.125, P + 8, P, P, P, None, 1, 1, 8, 128, None), ALIGN),
    ((0, 0, 0.125, P, P, P, P, None, -1, 1, 8, 64, None), SHAPE),
    ((0, 1, 0.125, None, None, None, None, None, 0, 4, 8, 64, None), OK),
    ((0, 1, 0.125, None, None, None, None, None, 2, 4, 0, 128, None), OK),
])
def test_flash_validation(args, status):
    assert _lib.lib().jules_hip_flash_attn_fwd(*args) == status


def test_w8a16_validation():
    L = _lib.lib()
    ws = L.jules_hip_w8a16_workspace_size(8, 8192, 8192)
    assert L.jules_hip_w8a16_workspace_size(17, 64, 64) == 0
    assert L.jules_hip_w8a16_workspace_size(8, 40, 64) == 0
    f = L.jules_hip_w8a16_gemm_bias_act
    assert f(9, P, P, P, None, P, 8, 64, 64, P, 1 << 20, None) == ACT
    assert f(5, P, P, P, None, P, 17, 64, 64, P, 1 << 20, None) == UNSUP
    assert f(5, P, P, P, None, P, 8, 40, 64, P, 1 << 20, None) == UNSUP
    assert f(5, P, P, P, None, P, 8, 64, 63, P, 1 << 20, None) == UNSUP
    assert f(5, P, P, P, None, P, 8, 64, 60, P, 1 << 20, None) == UNSUP
    assert f(5, None, P, P, None, P, 8, 64, 64, P, 1 << 20, None) == NULL
    assert f(5, P, P + 4, P, None, P, 8, 64, 64, P, 1 << 20, None) == ALIGN
    if ws > 0:
        assert f(5, P, P, P, None, P, 8, 8192, 8192, None, 0, None) == WS
        assert f(5, P, P, P, None, P, 8, 8192, 8192, P, ws - 1, None) == WS
    assert f(5, None, None, None, None, None, 0, 64, 64, None, 0, None) == OK


def test_int8_and_activation_validation():
    L = _lib.lib()
    assert L.jules_hip_matmul_int8(P, P, P, 4, 4, 200000, 1.0, 1.0, None, None) == SHAPE
    assert L.jules_hip_matmul_int8(None, P, P, 4, 4, 4, 1.0, 1.0, None, None) == NULL
    assert L.jules_hip_matmul_int8(None, None, None, 0, 4, 4, 1.0, 1.0, None, None) == OK
    assert L.jules_hip_activation(11, P, P, 16, None) == ACT
    assert L.jules_hip_activation(4, None, P, 16, None) == NULL
    assert L.jules_hip_activation(4, P, P, -1, None) == SHAPE
    assert L.jules_hip_activation(4, None, None, 0, None) == OK


def test_registry_descriptor_validation():
    """Descriptor errors are caught before launch."""
    fn = _lib.lookup("fusedMatmulBiasRelu")
    t = (_lib.JhTensor * 3)()
    o = (_lib.JhTensor * 1)()
    # wrong operand count
    assert fn(2, t, 1, o, None, None) == ARG
    # rank mismatch
    for x in list(t) + list(o):
        x.rank = 3
    assert fn(3, t, 1, o, None, None) == SHAPE


def test_rowops_validation():
    """Row kernels reject bad arguments before touching the device."""
    L = _lib.lib()
    assert L.jules_hip_softmax(None, None, -1, 4, None) == 2        # shape
    assert L.jules_hip_softmax(None, None, 0, 4, None) == 0         # empty: no work
    assert L.jules_hip_softmax(None, None, 4, 4, None) == 1         # null
    assert L.jules_hip_softmax(2, 2, 4, 4, None) == 4               # misaligned (rejected before any launch)
    assert L.jules_hip_layernorm(None, None, None, None, 2, 3, float("nan"), None) == 10
    assert L.jules_hip_layernorm(None, None, None, None, 2, 3, -1.0, None) == 10
    assert L.jules_hip_layernorm(None, None, None, None, 2, 3, 1e-5, None) == 1
    assert L.jules_hip_cross_entropy_workspace_size(10) == 40
    assert L.jules_hip_cross_entropy_workspace_size(0) == 4
    assert L.jules_hip_cross_entropy(None, None, None, None, 3, 0, None, 0, None) == 2
    assert L.jules_hip_cross_entropy(None, None, None, None, 3, 5, None, 0, None) == 1
    assert L.jules_hip_cross_entropy(16, 16, 16, 16, 3, 5, None, 0, None) == 6   # workspace
    assert L.jules_hip_cross_entropy(16, 16, 16, 16, 3, 5, 16, 8, None) == 6


def test_mfma_ceiling_validation():
    """The calibration entry point rejects bad arguments before any launch."""
    L = _lib.lib()
    assert L.jules_hip_mfma_ceiling(None, 4, 16, None) == 1            # null
    assert L.jules_hip_mfma_ceiling(2, 4, 16, None) == 4               # misaligned
    assert L.jules_hip_mfma_ceiling(16, 0, 16, None) == 2              # no workgroups
    assert L.jules_hip_mfma_ceiling(16, 65536, 16, None) == 2
    assert L.jules_hip_mfma_ceiling(16, 4, 0, None) == 2               # no iterations
    assert L.jules_hip_mfma_ceiling(16, 4, (1 << 20) + 1, None) == 2


def test_w8a8_validation():
    """matmulW8A8 rejects bad arguments before touching the device."""
    L = _lib.lib()
    assert L.jules_hip_matmul_w8a8(None, None, None, -1, 4, 4, None, None, None, None) == 2
    assert L.jules_hip_matmul_w8a8(None, None, None, 4, 4, 131073, None, None, None, None) == 2
    assert L.jules_hip_matmul_w8a8(None, None, None, 0, 4, 4, None, None, None, None) == 0
    assert L.jules_hip_matmul_w8a8(16, 16, 16, 4, 4, 4, None, None, None, None) == 1   # scale_B
    assert L.jules_hip_matmul_w8a8(16, 16, 16, 4, 4, 4, 2, 16, None, None) == 4        # scale_A
    assert L.jules_hip_matmul_w8a8(16, 16, 18, 4, 4, 4, None, 16, None, None) == 4      # C


def test_mlp_validation():
    L = _lib.lib()
    f = L.jules_hip_mlp_forward_backward
    assert L.jules_hip_mlp_workspace_size(4, 3, 0, 2) == 0
    assert L.jules_hip_mlp_workspace_size(4, 3, 5, 2) > 0
    args = [P] * 12 + [4, 3, 5, 2, P, P, 1 << 20, None]
    bad = list(args)
    bad[13] = 0  # K1 = 0
    assert f(*bad) == SHAPE
    bad = list(args)
    bad[1] = None  # W1
    assert f(*bad) == NULL
    bad = list(args)
    bad[17] = 0  # workspace bytes
    assert f(*bad) == WS


def test_mlp_forward_validation():
    L = _lib.lib()
    f = L.jules_hip_mlp_forward
    assert L.jules_hip_mlp_forward_workspace_size(4, 3, 0, 2) == 0
    assert L.jules_hip_mlp_forward_workspace_size(4, 3, 5, 2) >= 4 * 5 * 4
    args = [P] * 6 + [4, 3, 5, 2, P, 1 << 20, None]
    for i, code in ((7, SHAPE), (2, NULL), (11, WS)):
        bad = list(args)
        bad[i] = 0 if i != 2 else None
        assert f(*bad) == code, i
    bad = list(args)
    bad[0] = P + 2  # X misaligned
    assert f(*bad) == ALIGN
    assert f(*([P] * 6 + [0, 3, 5, 2, None, 0, None])) == 0  # M = 0: nothing to do
