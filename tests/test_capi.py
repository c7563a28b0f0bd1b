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


def test_reference_header_callers_compile_and_link(tmp_path):
    """A caller that uses every public member of the reference's kernel
    headers (ExecutionArena.h, TilePlanner.h incl. ShapeSignature and
    setBenchmarkKernel, FusedKernels.h, FlashAttention.h,
    InterleavedAutodiff.h) compiles against include/jules_hip_kernel.hpp and
    links against libjules_hip.so.  Nothing is run (no GPU here)."""
    src = os.path.join(ROOT, "tests", "cpp", "header_api_compile.cpp")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    lib_dir = os.path.join(ROOT, "jules_amd")
    exe = str(tmp_path / "header_api_compile")
    cmd = ["g++", "-std=c++17", "-Wall", "-Werror", f"-I{os.path.join(ROOT, 'include')}", src,
           f"-L{lib_dir}", "-ljules_hip", f"-L{rocm}/lib", "-lamdhip64",
           f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath,{rocm}/lib", "-o", exe]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    # without arguments the program touches no GPU and exits 0
    assert subprocess.run([exe], capture_output=True).returncode == 0


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


def test_flash_bwd_validation():
    """Every case fails validation, so the placeholder addresses are never
    dereferenced (this runs without a GPU)."""
    f = _lib.lib().jules_hip_flash_attn_bwd
    args = [1, 1, 0.125] + [P] * 9 + [1, 1, 16, 128, P, 1 << 20, None]
    for idx, val, status in ((0, 0, UNSUP),        # fp32: not implemented
                             (15, 160, UNSUP),     # head_dim > 128
                             (15, 0, SHAPE),
                             (17, 0, WS),          # workspace bytes
                             (8, None, NULL),      # lse
                             (3, P + 8, ALIGN),    # Q 16-byte alignment
                             (1, 2, ARG),          # causal not 0/1
                             (2, float("nan"), ARG)):
        bad = list(args)
        bad[idx] = val
        assert f(*bad) == status, (idx, val)


def test_int8_depth_limit():
    """K <= 131071 keeps every int32 sum exact ((-128)^2 * 131071 < 2^31);
    K = 131072 could reach 2^31 and is rejected before any launch."""
    L = _lib.lib()
    assert L.jules_hip_matmul_int8(P, P, P, 4, 16, 131072, 1.0, 1.0, None, None) == SHAPE
    assert L.jules_hip_matmul_w8a8(P, P, P, 4, 16, 131072, None, P, None, None) == SHAPE
    assert L.jules_hip_matmul_int8(None, P, P, 4, 16, 131071, 1.0, 1.0, None, None) == NULL


def test_registry_softmax_rank0_output():
    """A rank-0 output descriptor is rejected before its sizes are read."""
    fn = _lib.lookup("fusedSoftmax")
    x = (_lib.JhTensor * 1)()
    y = (_lib.JhTensor * 1)()
    x[0].data, x[0].rank, x[0].dtype = P, 1, 0
    x[0].sizes[0], x[0].strides[0] = 1, 1
    y[0].data, y[0].rank, y[0].dtype = P, 0, 0
    assert fn(1, x, 1, y, None, None) == SHAPE


CBLAS_LIB = os.path.join(ROOT, "jules_amd", "libjules_cblas.so")


def test_cblas_symbols_in_their_own_library():
    """cblas_sgemm lives in libjules_cblas.so only: loading libjules_hip.so
    never interposes a BLAS for other callers."""
    assert not any(s.startswith("cblas_") for s in _exported())
    out = subprocess.run(["nm", "-D", "--defined-only", CBLAS_LIB], capture_output=True, text=True,
                         check=True).stdout
    syms = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert {"cblas_sgemm", "jules_cblas_last_status"} <= syms


def test_cblas_dlopen_validation():
    """A plain C caller binds cblas_sgemm through dlopen + a process-wide dlsym
    (as the reference's ORC JIT resolves it) and gets every argument error as
    a status, with C untouched and no device work."""
    exe = os.path.join(ROOT, "tests", "cpp", "cblas_dlopen")
    r = subprocess.run([exe, CBLAS_LIB], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "cblas dlopen ok" in r.stdout, r.stdout + r.stderr


def _tile(dtype, M, N, K):
    out = (ctypes.c_int * 4)()
    assert _lib.lib().jules_hip_gemm_tile(dtype, M, N, K, out) == OK
    return tuple(out)


def test_gemm_tile_table():
    """The launch table: C1 runs the row kernel with 2 rows per wave, the
    reference's published shape [64,784]x[784,256] 1 row per wave, large fp32
    GEMMs 64x64 tiles, C3 the bf16 LDS-DMA kernel, ragged bf16 the
    register-staged one."""
    assert _tile(0, 512, 512, 512) == (1, 8, 64, 512)
    assert _tile(0, 64, 256, 784) == (0, 4, 64, 784)
    assert _tile(0, 67, 80, 45) == (0, 4, 64, 48)
    assert _tile(0, 512, 512, 4096) == (2, 32, 32, 32)        # K beyond the row kernel's LDS
    assert _tile(0, 4096, 4096, 4096) == (3, 64, 64, 32)
    assert _tile(0, 1024, 2048, 64) == (3, 64, 64, 32)        # 512 tiles of 64x64
    assert _tile(0, 1024, 1040, 64) == (2, 32, 32, 32)        # 272 tiles of 64x64
    assert _tile(1, 4096, 4096, 4096) == (4, 256, 256, 32)
    assert _tile(1, 4104, 4096, 4096) == (5, 256, 256, 64)
    out = (ctypes.c_int * 4)()
    assert _lib.lib().jules_hip_gemm_tile(2, 4, 4, 4, out) == DTYPE
    assert _lib.lib().jules_hip_gemm_tile(0, -1, 4, 4, out) == SHAPE
    assert _lib.lib().jules_hip_gemm_tile(0, 4, 4, 4, None) == NULL


@pytest.mark.parametrize("args,status", [
    ((2, 0, 4, 4, 4, 1.0, P, 4, P, 4, 0.0, P, 4, None), ARG),      # transA not 0/1
    ((0, 0, -1, 4, 4, 1.0, P, 4, P, 4, 0.0, P, 4, None), SHAPE),
    ((0, 0, 4, 4, 4, 1.0, P, 3, P, 4, 0.0, P, 4, None), SHAPE),    # lda < K
    ((1, 0, 5, 4, 4, 1.0, P, 4, P, 4, 0.0, P, 4, None), SHAPE),    # transA: lda < M
    ((0, 1, 4, 5, 4, 1.0, P, 4, P, 3, 0.0, P, 5, None), SHAPE),    # transB: ldb < K
    ((0, 0, 4, 4, 4, 1.0, P, 4, P, 4, 0.0, P, 3, None), SHAPE),    # ldc < N
    ((0, 0, 4, 4, 4, 1.0, None, 4, P, 4, 0.0, P, 4, None), NULL),
    ((0, 0, 4, 4, 4, 1.0, P, 4, P, 4, 0.0, None, 4, None), NULL),
    ((0, 0, 4, 4, 4, 1.0, P + 2, 4, P, 4, 0.0, P, 4, None), ALIGN),
    ((0, 0, 0, 4, 4, 1.0, None, 4, None, 4, 0.0, None, 4, None), OK),   # M = 0
])
def test_sgemm_validation(args, status):
    assert _lib.lib().jules_hip_sgemm(*args) == status


def test_w8a16_noalloc_validation():
    """The no-allocation W8A16 entry point checks its arguments like the
    workspace one and rejects shapes whose workspace exceeds the static
    scratch (65 column tiles x 8 splits here) before touching the device."""
    L = _lib.lib()
    f = L.jules_hip_w8a16_gemm_bias_act_noalloc
    assert L.jules_hip_w8a16_noalloc_max_bytes() == (8 << 20) + 4096
    assert f(9, P, P, P, None, P, 8, 64, 64, None) == ACT
    assert f(5, P, P, P, None, P, 17, 64, 64, None) == UNSUP
    assert f(5, None, P, P, None, P, 8, 64, 64, None) == NULL
    assert f(5, P, P + 4, P, None, P, 8, 64, 64, None) == ALIGN
    assert f(5, P, P, P, None, P, 8, 16640, 8192, None) == WS
    assert b"static scratch" in L.jules_hip_last_error()
    assert f(5, None, None, None, None, None, 0, 64, 64, None) == OK


def test_hbm_read_floor_validation():
    L = _lib.lib()
    f = L.jules_hip_hbm_read_floor
    assert f(None, 1 << 20, P, 256, None) == NULL
    assert f(P, 1 << 20, None, 256, None) == NULL
    assert f(P + 8, 1 << 20, P, 256, None) == ALIGN
    assert f(P, (1 << 20) + 8, P, 256, None) == SHAPE
    assert f(P, 0, P, 256, None) == SHAPE
    assert f(P, 1 << 20, P, 0, None) == SHAPE


def test_w8a16_packed_validation():
    """Packed W8A16: the packed size, the pack's argument checks and the GEMM's
    (the same as the row-major entry point's), all before any device work."""
    L = _lib.lib()
    assert L.jules_hip_w8a16_packed_size(8192, 8192) == 8192 * 8192
    assert L.jules_hip_w8a16_packed_size(40, 272) == 9 * 2 * 1024
    assert L.jules_hip_w8a16_packed_size(0, 64) == 0
    assert L.jules_hip_w8a16_packed_size(64, -16) == 0
    pack = L.jules_hip_w8a16_pack
    assert pack(P, -1, 64, P, 1 << 20, None) == SHAPE
    assert pack(None, 0, 64, None, 0, None) == OK
    assert pack(P, 64, 40, P, 1 << 20, None) == UNSUP
    assert pack(P, 60, 64, P, 1 << 20, None) == UNSUP
    assert pack(None, 64, 64, P, 1 << 20, None) == NULL
    assert pack(P, 64, 64, None, 1 << 20, None) == NULL
    assert pack(P, 64, 64, P + 8, 1 << 20, None) == ALIGN
    assert pack(P, 64, 64, P, 64 * 64 - 1, None) == WS
    f = L.jules_hip_w8a16_packed_gemm_bias_act
    assert f(9, P, P, P, None, P, 8, 64, 64, None) == ACT
    assert f(5, P, P, P, None, P, 17, 64, 64, None) == UNSUP
    assert f(5, P, P, P, None, P, 8, 40, 64, None) == UNSUP
    assert f(5, P, P, P, None, P, 8, 64, 60, None) == UNSUP
    assert f(5, None, P, P, None, P, 8, 64, 64, None) == NULL
    assert f(5, P, P + 4, P, None, P, 8, 64, 64, None) == ALIGN
    assert f(5, None, None, None, None, None, 0, 64, 64, None) == OK
