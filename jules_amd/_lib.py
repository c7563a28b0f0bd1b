"""ctypes binding of libjules_hip.so's C ABI (include/jules_hip.h).

Loading fails loudly when the library is missing: there is no CPU fallback
anywhere in the product path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libjules_hip.so")

# jh_dtype / jh_act / jh_status values of include/jules_hip.h
F32, BF16, I8, I32 = 0, 1, 2, 3
ACT = {"none": 0, "relu": 1, "sigmoid": 2, "tanh": 3, "gelu": 4, "silu": 5}
STATUS = {0: "JH_OK", 1: "JH_ERR_NULL", 2: "JH_ERR_SHAPE", 3: "JH_ERR_DTYPE",
          4: "JH_ERR_ALIGN", 5: "JH_ERR_ACT", 6: "JH_ERR_WORKSPACE", 7: "JH_ERR_HIP",
          8: "JH_ERR_UNSUPPORTED", 9: "JH_ERR_NOT_FOUND", 10: "JH_ERR_ARG"}

_vp = ctypes.c_void_p
_int = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_size = ctypes.c_size_t


class JhTensor(ctypes.Structure):
    _fields_ = [("data", _vp), ("offset", _i64), ("sizes", _i64 * 6), ("strides", _i64 * 6),
                ("rank", ctypes.c_int32), ("dtype", ctypes.c_int32)]


KERNEL_FN = ctypes.CFUNCTYPE(_int, _int, ctypes.POINTER(JhTensor), _int, ctypes.POINTER(JhTensor),
                             ctypes.c_char_p, _vp)

# name -> (restype, argtypes); every function declared in include/jules_hip.h
SIGNATURES = {
    "jules_hip_abi_version": (_int, []),
    "jules_hip_status_string": (ctypes.c_char_p, [_int]),
    "jules_hip_last_error": (ctypes.c_char_p, []),
    "jules_hip_gemm_bias_act": (_int, [_int, _int, _vp, _vp, _vp, _vp, _int, _int, _int, _vp]),
    "jules_hip_gemm_tile": (_int, [_int, _int, _int, _int, ctypes.POINTER(_int)]),
    "jules_hip_sgemm": (_int, [_int, _int, _int, _int, _int, _f32, _vp, _int, _vp, _int, _f32, _vp,
                               _int, _vp]),
    "jules_hip_activation": (_int, [_int, _vp, _vp, _i64, _vp]),
    "jules_hip_flash_attn_fwd": (_int, [_int, _int, _f32, _vp, _vp, _vp, _vp, _vp, _int, _int,
                                        _int, _int, _vp]),
    "jules_hip_flash_attn_bwd_workspace_size": (_size, [_int, _int, _int]),
    "jules_hip_flash_attn_bwd": (_int, [_int, _int, _f32] + [_vp] * 9 + [_int] * 4 + [_vp, _size,
                                                                                  _vp]),
    "jules_hip_w8a16_workspace_size": (_size, [_int, _int, _int]),
    "jules_hip_w8a16_gemm_bias_act": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _int, _int, _int,
                                             _vp, _size, _vp]),
    "jules_hip_w8a16_packed_size": (_size, [_int, _int]),
    "jules_hip_w8a16_pack": (_int, [_vp, _int, _int, _vp, _size, _vp]),
    "jules_hip_w8a16_packed_gemm_bias_act": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _int, _int,
                                                    _int, _vp]),
    "jules_hip_w8a16_noalloc_max_bytes": (_size, []),
    "jules_hip_w8a16_noalloc_counters": (_int, [_vp, _int]),
    "jules_hip_w8a16_gemm_bias_act_noalloc": (_int, [_int, _vp, _vp, _vp, _vp, _vp, _int, _int,
                                                     _int, _vp]),
    "jules_hip_matmul_int8": (_int, [_vp, _vp, _vp, _int, _int, _int, _f32, _f32, _vp, _vp]),
    "jules_hip_matmul_w8a8": (_int, [_vp, _vp, _vp, _int, _int, _int, _vp, _vp, _vp, _vp]),
    "jules_hip_softmax": (_int, [_vp, _vp, _int, _int, _vp]),
    "jules_hip_mfma_ceiling": (_int, [_vp, _int, _int, _vp]),
    "jules_hip_hbm_read_floor": (_int, [_vp, _i64, _vp, _int, _vp]),
    "jules_hip_layernorm": (_int, [_vp, _vp, _vp, _vp, _int, _int, _f32, _vp]),
    "jules_hip_cross_entropy_workspace_size": (_size, [_int]),
    "jules_hip_cross_entropy": (_int, [_vp, _vp, _vp, _vp, _int, _int, _vp, _size, _vp]),
    "jules_hip_mlp_forward_workspace_size": (_size, [_int, _int, _int, _int]),
    "jules_hip_mlp_forward": (_int, [_vp] * 6 + [_int] * 4 + [_vp, _size, _vp]),
    "jules_hip_mlp_workspace_size": (_size, [_int, _int, _int, _int]),
    "jules_hip_mlp_forward_backward": (_int, [_vp] * 12 + [_int, _int, _int, _int, _vp, _vp, _size,
                                                           _vp]),
    "jules_hip_lookup": (_vp, [ctypes.c_char_p]),
    "jules_hip_kernel_count": (_int, []),
    "jules_hip_kernel_name": (ctypes.c_char_p, [_int]),
    "jules_hip_pjrt_compile": (_int, [ctypes.c_char_p, _int, ctypes.POINTER(_vp)]),
    "jules_hip_pjrt_execute": (_int, [_vp, _int, ctypes.POINTER(JhTensor), _int,
                                      ctypes.POINTER(JhTensor), ctypes.POINTER(_int)]),
    "jules_hip_pjrt_destroy": (_int, [_vp]),
    "jules_hip_pjrt_describe": (_int, [ctypes.c_char_p, _int, ctypes.c_char_p, _size]),
}

_lib = None


class JulesHipError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


def lib():
    """Load libjules_hip.so (built by jules_amd/build.py); raise if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing; build it with `python -c 'import __graft_entry__ as g; "
                f"g.build()'` (hipcc, gfx950).  There is no fallback implementation.")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status):
    if status != 0:
        raise JulesHipError(status, lib().jules_hip_last_error().decode())
    return status


def lookup(name):
    """Resolve an extern_kernel name to a callable, or None."""
    p = lib().jules_hip_lookup(name.encode())
    return KERNEL_FN(p) if p else None


def kernel_names():
    L = lib()
    return [L.jules_hip_kernel_name(i).decode() for i in range(L.jules_hip_kernel_count())]
