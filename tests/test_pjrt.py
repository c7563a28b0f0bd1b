"""CPU tests of the ROCm PJRT executor's program handling (no GPU).

1. The oracle (oracle/pjrt_interp.py, restating the reference's CPU
   interpreter, lib/PJRT.cpp:169-858) is pinned op by op against closed forms
   and against the parse rules it restates, one text per quirk.
2. The library's parser (jules_hip_pjrt_describe, pjrt.cpp) gives the same op
   list as the oracle for every test program.
3. The C ABI rejects bad arguments before touching a device.
"""
import ctypes
import math

import numpy as np
import pytest

from jules_amd import _lib
from oracle import pjrt_interp as pi


def _in(a):
    a = np.asarray(a, np.float32)
    return (a, list(a.shape))


def _run(text, *arrays, **kw):
    return pi.run(text, [_in(a) for a in arrays], **kw)


BIN = '%0 = "stablehlo.{op}"(%arg0, %arg1) : (tensor<4xf32>, tensor<4xf32>) -> tensor<4xf32>'
UN = '%0 = "stablehlo.{op}"(%arg0) : (tensor<5xf32>) -> tensor<5xf32>'


# ---- 1. oracle pinning ------------------------------------------------------

def test_binary_closed_forms_and_padding():
    a = np.array([1.5, -2.0, 3.0, 0.0], np.float32)
    b = np.array([0.5, 4.0, 0.0, -1.0], np.float32)
    cases = {"add": a + b, "subtract": a - b, "multiply": a * b,
             "divide": np.array([3.0, -0.5, 0.0, -0.0], np.float32),   # x/0 -> 0 (PJRT.cpp:234-236)
             "maximum": np.maximum(a, b), "minimum": np.minimum(a, b)}
    for op, want in cases.items():
        (y, s), = _run(BIN.format(op=op), a, b)
        assert np.array_equal(y, want), op
        assert s == [4]
    # unequal sizes: the shorter operand reads as 0 past its end; shape of the
    # larger-rank operand (PJRT.cpp:617-627)
    (y, s), = _run(BIN.format(op="add"), np.ones((2, 3), np.float32), np.array([5.0, 6.0], np.float32))
    assert np.array_equal(y, [6, 7, 1, 1, 1, 1]) and s == [2, 3]
    # equal ranks: the left operand's shape, even when the right one has more
    # data (the result then holds 3 values under shape [1])
    (y, s), = _run(BIN.format(op="subtract"), np.array([1.0], np.float32), np.arange(3, dtype=np.float32))
    assert np.array_equal(y, [1, -1, -2]) and s == [1]


def test_max_min_follow_std_max_min_on_nan():
    nan = np.float32("nan")
    a = np.array([nan, 1.0], np.float32)
    b = np.array([1.0, nan], np.float32)
    (mx, _), = _run(BIN.format(op="maximum"), a, b)
    (mn, _), = _run(BIN.format(op="minimum"), a, b)
    # std::max(a, b) = a < b ? b : a ; std::min(a, b) = b < a ? b : a
    assert math.isnan(mx[0]) and mx[1] == 1.0
    assert math.isnan(mn[0]) and mn[1] == 1.0


def test_unary_closed_forms():
    x = np.array([-2.0, -0.5, 0.0, 0.5, 3.0], np.float32)
    x64 = x.astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        want = {"negate": -x64, "relu": np.maximum(x64, 0), "logistic": 1 / (1 + np.exp(-x64)),
                "tanh": np.tanh(x64), "exponential": np.exp(x64),
                "log": np.array([-np.inf, -np.inf, -np.inf, math.log(0.5), math.log(3.0)])}
    for op, w in want.items():
        (y, s), = _run(UN.format(op=op), x)
        assert s == [5]
        np.testing.assert_array_equal(y, w.astype(np.float32), err_msg=op)


def test_matmul_rule_and_transpose():
    A = np.arange(6, dtype=np.float32).reshape(2, 3)
    B = np.arange(12, dtype=np.float32).reshape(3, 4) - 5
    (y, s), = _run('%0 = "stablehlo.dot_general"(%arg0, %arg1) : (tensor<2x3xf32>, tensor<3x4xf32>) -> tensor<2x4xf32>', A, B)
    assert s == [2, 4] and np.array_equal(y.reshape(2, 4), A @ B)
    # rank-1 rhs: N = 1, rhs read as K x 1 (PJRT.cpp:677-682)
    (y, s), = _run('%0 = "stablehlo.dot_general"(%arg0, %arg1) : () -> ()', A, np.array([1, 2, 3], np.float32))
    assert s == [2, 1] and np.array_equal(y, A @ [1, 2, 3])
    # N-D transpose with a parsed permutation equals numpy's
    X = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    (y, s), = _run('%0 = "stablehlo.transpose"(%arg0) {permutation = dense<[2, 0, 1]> : tensor<3xi64>} : () -> ()', X)
    assert s == [4, 2, 3] and np.array_equal(y, np.transpose(X, (2, 0, 1)).ravel())
    # no permutation attribute: reversed dimensions
    (y, s), = _run('%0 = "stablehlo.transpose"(%arg0) : () -> ()', X)
    assert s == [4, 3, 2] and np.array_equal(y, np.transpose(X).ravel())
    # rank 2 always swaps, whatever the permutation (PJRT.cpp:768-777)
    (y, s), = _run('%0 = "stablehlo.transpose"(%arg0) {permutation = dense<[0, 1]> : tensor<2xi64>} : () -> ()', A)
    assert s == [2, 3] and np.array_equal(y, A.T.ravel())


def test_reduce_sequential_sum():
    X = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    (y, s), = _run('%0 = "stablehlo.reduce"(%arg0, %arg1) {dimensions = dense<[1]> : tensor<1xi64>} : () -> ()', X, np.zeros(1))
    assert s == [2, 4] and np.array_equal(y, X.sum(1).ravel())
    (y, s), = _run('%0 = "stablehlo.reduce"(%arg0, %arg1) {dimensions = dense<[0, 2]> : tensor<2xi64>} : () -> ()', X, np.zeros(1))
    assert s == [3] and np.array_equal(y, X.sum((0, 2)))
    (y, s), = _run('%0 = "stablehlo.reduce"(%arg0, %arg1) : () -> ()', X, np.zeros(1))
    assert s == [1] and y[0] == X.sum()
    # the order is sequential in input order: 1e8 + 1 ... in fp32
    v = np.array([1e8, 1.0, 1.0, 1.0, 1.0, -1e8], np.float32)
    (y, _), = _run('%0 = "stablehlo.reduce"(%arg0, %arg1) : () -> ()', v, np.zeros(1))
    want = np.float32(0)
    for t in v:
        want = np.float32(want + t)
    assert y[0] == want == 0.0   # each +1 is lost at 1e8 (pairwise summation would keep 4)


def test_constants_and_shapes_parse_like_the_reference():
    # dense<a, b> parses; dense<[a, b]> does not (istringstream stops at '[')
    (c, s), = _run('%0 = "stablehlo.constant"() {value = dense<1.5, -2.0>} : () -> tensor<2xf32>')
    assert np.array_equal(c, [1.5, -2.0]) and s == [2]
    (c, s), = _run('%0 = "stablehlo.constant"() {value = dense<[1.5, -2.0]>} : () -> tensor<2xf32>')
    assert np.array_equal(c, [0.0]) and s == [1]
    # a reshape's shape is read only from `: tensor<...>` right after the operands
    X = np.arange(6, dtype=np.float32)
    (y, s), = _run('%0 = "stablehlo.reshape"(%arg0) : tensor<2x3xf32>', X)
    assert s == [2, 3] and np.array_equal(y, X)
    (y, s), = _run('%0 = "stablehlo.reshape"(%arg0) : (tensor<6xf32>) -> tensor<2x3xf32>', X)
    assert s == [6]


def test_outputs_copies_skips_and_forward_references():
    x = np.array([1.0, 2.0], np.float32)
    text = ('%0 = "stablehlo.negate"(%arg0) : () -> ()\n'
            '%1 = "stablehlo.frobnicate"(%0) : () -> ()\n'      # unknown op: copy of operand 0
            '%2 = "stablehlo.add"(%0, %later) : () -> ()\n'     # %later not written: skipped
            '%later = "stablehlo.exponential"(%arg0) : () -> ()\n')
    outs = _run(text, x)
    # every written buffer past the inputs, in index order: %0, %1, %later
    assert [list(o[0]) for o in outs] == [[-1, -2], [-1, -2], list(np.exp(x.astype(np.float64)).astype(np.float32))]
    # an empty program copies buffer 0
    (y, _), = _run("func.func @main() {}", x)
    assert np.array_equal(y, x)


# ---- 2. the library parses as the oracle does -------------------------------

PROGRAMS = [
    (BIN.format(op="add"), 2),
    ('%0 = "stablehlo.dot_general"(%arg0, %arg1) : () -> ()\n%1 = "stablehlo.relu"(%0) : () -> ()', 2),
    ('%0 = "stablehlo.transpose"(%arg0) {permutation = dense<[2, 0, 1]> : tensor<3xi64>} : () -> ()\n'
     '%1 = "stablehlo.reduce"(%0, %arg1) {dimensions = dense<[0, 2]> : tensor<2xi64>} : () -> ()', 2),
    ('%0 = "stablehlo.constant"() {value = dense<1.5, -2.0>} : () -> tensor<2xf32>\n'
     '%1 = "stablehlo.reshape"(%arg0) : tensor<2x3xf32>\n%2 = "stablehlo.multiply"(%0, %1) : () -> ()', 1),
    ('%0 = "stablehlo.negate"(%arg0) : () -> ()\n%1 = "stablehlo.frobnicate"(%0) : () -> ()\n'
     '%2 = "stablehlo.add"(%0, %later) : () -> ()\n%later = "stablehlo.exponential"(%arg0) : () -> ()', 1),
    ('%0 = "stablehlo.custom_call"(%arg0, %arg1) {backend_config = "", call_target_name = "fusedMatmulBiasRelu", '
     'has_side_effect = false} : (tensor<4x8xf32>, tensor<8x16xf32>) -> tensor<4x16xf32>', 2),
    ('%0:2 = "stablehlo.custom_call"(%arg0, %arg1) {call_target_name = "fusedCrossEntropyLoss"} : '
     '(tensor<2x3xf32>, tensor<2xi32>) -> (tensor<2x3xf32>, tensor<1xf32>)\n'
     '%1 = "stablehlo.negate"(%0#1) : () -> ()', 2),
    ("func.func @main() {}", 1),
]


def _describe(text, n):
    L = _lib.lib()
    buf = ctypes.create_string_buffer(1 << 16)
    st = L.jules_hip_pjrt_describe(text.encode(), n, buf, len(buf))
    assert st == 0, L.jules_hip_last_error()
    return buf.value.decode()


def _oracle_lines(text, n):
    P = pi.Program(text, n, multi_result=True)
    lines = []
    for op in P.ops:
        lines.append((tuple(op["outs"]), op["kind"], tuple(op["ins"])))
    return lines, P.next


KIND = {"add": "binary", "sub": "binary", "mul": "binary", "div": "binary", "max": "binary",
        "min": "binary", "neg": "unary", "relu": "unary", "sigmoid": "unary", "tanh": "unary",
        "exp": "unary", "log": "unary"}


@pytest.mark.parametrize("text,n", PROGRAMS)
def test_library_parse_matches_oracle(text, n):
    got = _describe(text, n).strip().splitlines()
    assert got[-1] == f"buffers {_oracle_lines(text, n)[1]}"
    want, _ = _oracle_lines(text, n)
    assert len(got) - 1 == len(want)
    for line, (outs, kind, ins) in zip(got, want):
        lhs, rhs = line.split(" = ", 1)
        toks = rhs.split()
        assert tuple(int(x) for x in lhs.split(",")) == outs
        assert toks[0] == KIND.get(kind, kind)
        assert tuple(int(t) for t in toks[2:2 + len(ins)]) == ins
    P = pi.Program(text, n, multi_result=True)
    for line, op in zip(got, P.ops):
        if op["kind"] == "transpose":
            assert f"perm=[{','.join(map(str, op['perm']))}]" in line
        if op["kind"] == "reduce":
            assert f"dims=[{','.join(map(str, op['dims']))}]" in line
        if op["kind"] == "reshape":
            assert f"shape=[{','.join(map(str, op['shape']))}]" in line
        if op["kind"] == "custom_call":
            assert f"target={op['target']}" in line


# ---- 3. C ABI validation ------------------------------------------------------

def test_pjrt_abi_validation():
    L = _lib.lib()
    buf = ctypes.create_string_buffer(16)
    assert L.jules_hip_pjrt_describe(None, 1, buf, 16) == 1
    assert L.jules_hip_pjrt_describe(b"x", -1, buf, 16) == 10
    assert L.jules_hip_pjrt_describe(BIN.format(op="add").encode(), 2, buf, 16) == 6   # too small
    assert L.jules_hip_pjrt_describe(b'%0 = "stablehlo.custom_call"(%arg0) : () -> tensor<2xf32>', 1,
                                     buf, 16) == 10                                   # no target
    assert L.jules_hip_pjrt_describe(b'%0 = "stablehlo.custom_call"(%arg0) {call_target_name = "x"} : () -> tensor<2xf64>',
                                     1, buf, 16) == 3                                 # result dtype
    out = ctypes.c_void_p()
    assert L.jules_hip_pjrt_compile(None, 0, ctypes.byref(out)) == 1
    n = ctypes.c_int()
    assert L.jules_hip_pjrt_execute(None, 0, None, 0, None, ctypes.byref(n)) == 1
    assert L.jules_hip_pjrt_destroy(None) == 0


def test_cxx_header_is_self_contained(tmp_path):
    """include/jules_hip_pjrt.hpp compiles on its own with the host compiler."""
    import os
    import subprocess
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    src = tmp_path / "inc.cpp"
    src.write_text('#include "jules_hip_pjrt.hpp"\nint main() { return 0; }\n')
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Werror",
                        f"-I{os.path.join(root, 'include')}", str(src)], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
