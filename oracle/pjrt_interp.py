"""CPU restatement of the reference's StableHLO text interpreter -- TEST
INFRASTRUCTURE ONLY (imported by tests/, never by the product package).

It follows CPUTensorInterpreter in lib/PJRT.cpp (the CPU PJRT executable of
the reference) and is the checker for the ROCm PJRT executor
(jules_amd/csrc/pjrt.cpp):

  - parse          PJRT.cpp:177-205 (arguments %arg0..%arg{n-1} take buffers
                   0..n-1; an empty program becomes one copy of buffer 0) and
                   :348-500 (one regex pass over the text; every matched op
                   takes the next buffer index in text order; an operand name
                   not seen yet takes a fresh index that is never written)
  - shapes         :505-541 (result type `: tensor<AxBx..>` directly after the
                   operand list, no attribute dict in between; otherwise none)
  - transpose perm :545-564, reduce dims :567-594, constants :454-484
  - execute        :208-324, binary :606-630, unary :632-648, constant
                   :650-657, matmul :662-700, reshape :704-722, transpose
                   :726-801, reduce :805-857
  - outputs        :300-323: every buffer written during execution whose
                   index is >= the number of inputs, in index order; with none,
                   copies of the inputs.

One deliberate difference: the reference turns "stablehlo.custom_call" (and
every op it does not know) into a copy of operand 0 (:491-499).  Here an op
whose name is "stablehlo.custom_call" is evaluated by `custom_call_fn`, the
caller's restatement of the named kernel (the ROCm executor dispatches it
through the kernel registry); other unknown ops stay copies.  Multi-result
custom calls (`%r:2 = ...`, used as `%r#0`, `%r#1`) are an extension the
reference regex does not match; they are parsed here only when
`multi_result=True`.

Values are float32 numpy arrays (the reference converts every buffer to
float, PJRT.cpp:935-946).  Pinning: tests/test_pjrt.py checks each op against
its closed form on small inputs (numpy), and the parse rules on texts written
for each quirk above.
"""
import math
import re

import numpy as np

# PJRT.cpp:357-358 and :369
_OP = re.compile(r'%(\w+)\s*=\s*"([\w.]+)"\(([^)]*)\)')
_OP_MULTI = re.compile(r'%(\w+)(?::(\d+))?\s*=\s*"([\w.]+)"\(([^)]*)\)')
_OPERAND = re.compile(r'%(\w+)(?:#(\d+))?')

_BINARY = {"stablehlo.add": "add", "stablehlo.subtract": "sub", "stablehlo.multiply": "mul",
           "stablehlo.divide": "div", "stablehlo.maximum": "max", "stablehlo.minimum": "min"}
_UNARY = {"stablehlo.negate": "neg", "stablehlo.relu": "relu", "stablehlo.logistic": "sigmoid",
          "stablehlo.tanh": "tanh", "stablehlo.exponential": "exp", "stablehlo.log": "log"}
_TYPES = ("f32", "f64", "f16", "bf16", "i1", "i8", "i32", "i64")


def _floats(s):
    """istringstream >> float, skipping one ',' after each value (PJRT.cpp:472-477)."""
    out = []
    pos, n = 0, len(s)
    num = re.compile(r'\s*([+-]?(?:\d+\.?\d*|\.\d+)(?:[eE][+-]?\d+)?|[+-]?(?:inf|nan))', re.I)
    while pos < n:
        m = num.match(s, pos)
        if not m:
            break
        out.append(np.float32(float(m.group(1))))
        pos = m.end()
        if pos < n and s[pos] == ",":
            pos += 1
    return out


def _ints(s):
    out = []
    for tok in re.split(r"\s*,\s*", s.strip()):
        m = re.match(r"[+-]?\d+", tok)
        if not m:
            break
        out.append(int(m.group(0)))
    return out


def parse_shape(text, name):
    """PJRT.cpp:505-541."""
    pat = re.compile("%" + name + r'\s*=\s*"[^"]*"\([^)]*\)[^{]*:\s*tensor<([^>]+)>')
    for m in pat.finditer(text):
        dims = []
        for tok in m.group(1).split("x"):
            if tok in _TYPES:
                break
            try:
                dims.append(int(tok))
            except ValueError:
                break
        if dims:
            return dims
    return []


def parse_perm(text, name):
    """PJRT.cpp:545-564."""
    pat = re.compile("%" + name +
                     r'\s*=\s*"stablehlo\.transpose"\([^)]*\)\s*\{permutation\s*=\s*dense<\[([^\]]*)\]>')
    for m in pat.finditer(text):
        p = _ints(m.group(1))
        if p:
            return p
    return []


def parse_reduce_dims(text, name):
    """PJRT.cpp:567-594."""
    pat = re.compile("%" + name + r'\s*=\s*"stablehlo\.reduce"[^}]*\}')
    for m in pat.finditer(text):
        d = re.search(r'dimensions\s*=\s*dense<\[([^\]]*)\]>', m.group(0))
        if d:
            v = _ints(d.group(1))
            if v:
                return v
    return []


def parse_const(text, name):
    """PJRT.cpp:462-484."""
    pat = re.compile(r'%(\w+)\s*=\s*"stablehlo\.constant"\(\)\s*\{value\s*=\s*dense<([^>]*)>\}')
    for m in pat.finditer(text):
        if m.group(1) == name:
            return _floats(m.group(2))
    return []


def _attr(text, start, key):
    """Value of `key = "..."` in the attribute dict that follows position
    `start` on the op's line (custom_call target and backend_config)."""
    end = text.find("\n", start)
    line = text[start:end if end >= 0 else len(text)]
    m = re.search(key + r'\s*=\s*"([^"]*)"', line)
    return m.group(1) if m else None


def _result_types(text, start):
    end = text.find("\n", start)
    line = text[start:end if end >= 0 else len(text)]
    arrow = line.rfind("->")
    if arrow < 0:
        return []
    types = []
    for t in re.finditer(r"tensor<([^>]*)>", line[arrow:]):
        dims, dt = [], "f32"
        for tok in t.group(1).split("x"):
            if tok in _TYPES:
                dt = tok
                break
            dims.append(int(tok))
        types.append((dims, dt))
    return types


class Program:
    def __init__(self, text, n_inputs, multi_result=False):
        self.text = text
        self.n_inputs = n_inputs
        self.ops = []
        self.names = {f"arg{i}": i for i in range(n_inputs)}
        self.next = n_inputs
        rx = _OP_MULTI if multi_result else _OP
        for m in rx.finditer(text):
            if multi_result:
                name, count, opname, operands = m.group(1), int(m.group(2) or 1), m.group(3), m.group(4)
            else:
                name, count, opname, operands = m.group(1), 1, m.group(2), m.group(3)
            ins = [self._ref(o.group(1), o.group(2), multi_result) for o in _OPERAND.finditer(operands)]
            outs = []
            for r in range(count):
                idx = self.next
                self.next += 1
                outs.append(idx)
                self.names[name if count == 1 else f"{name}#{r}"] = idx
            if count > 1:
                self.names[name] = outs[0]
            op = {"name": opname, "ins": ins, "outs": outs, "result": name}
            if opname in _BINARY:
                op["kind"] = _BINARY[opname]
            elif opname in _UNARY:
                op["kind"] = _UNARY[opname]
            elif opname == "stablehlo.dot_general":
                op["kind"] = "matmul"
            elif opname == "stablehlo.reshape":
                op["kind"] = "reshape"
                op["shape"] = parse_shape(text, name)
            elif opname == "stablehlo.transpose":
                op["kind"] = "transpose"
                op["perm"] = parse_perm(text, name)
            elif opname == "stablehlo.reduce":
                op["kind"] = "reduce"
                op["dims"] = parse_reduce_dims(text, name)
            elif opname == "stablehlo.constant":
                op["kind"] = "constant"
                op["data"] = parse_const(text, name)
            elif opname == "stablehlo.custom_call":
                op["kind"] = "custom_call"
                op["target"] = _attr(text, m.end(), "call_target_name")
                op["config"] = _attr(text, m.end(), "backend_config") or ""
                op["types"] = _result_types(text, m.end())
            else:
                op["kind"] = "copy"
            if op["kind"] == "copy" and not ins:
                op["ins"] = [0]
            self.ops.append(op)
        if not self.ops:
            self.ops.append({"kind": "copy", "ins": [0], "outs": [self._fresh()], "name": "copy"})

    def _fresh(self):
        idx = self.next
        self.next += 1
        return idx

    def _ref(self, name, sub, multi_result):
        key = f"{name}#{sub}" if (multi_result and sub is not None) else name
        if key not in self.names:
            self.names[key] = self._fresh()
        return self.names[key]


def _binary(kind, a, b):
    n = max(a.size, b.size, 1)
    x = np.zeros(n, np.float32)
    y = np.zeros(n, np.float32)
    x[:a.size] = a.ravel()
    y[:b.size] = b.ravel()
    with np.errstate(all="ignore"):
        if kind == "add":
            r = x + y
        elif kind == "sub":
            r = x - y
        elif kind == "mul":
            r = x * y
        elif kind == "div":
            r = np.where(y != 0, x / np.where(y != 0, y, 1), np.float32(0))
        elif kind == "max":
            r = np.where(x < y, y, x)   # std::max(a, b)
        else:
            r = np.where(y < x, y, x)   # std::min(a, b)
    return r.astype(np.float32)


def _unary(kind, a):
    a = a.astype(np.float64)
    with np.errstate(all="ignore"):
        if kind == "neg":
            r = -a
        elif kind == "relu":
            r = np.where(a > 0, a, 0.0)
        elif kind == "sigmoid":
            r = 1.0 / (1.0 + np.exp(-a))
        elif kind == "tanh":
            r = np.tanh(a)
        elif kind == "exp":
            r = np.exp(a)
        else:
            r = np.where(a > 0, np.log(np.where(a > 0, a, 1.0)), -np.inf)
    return r.astype(np.float32)


def _transpose(a, shape, perm):
    rank = len(shape)
    if rank == 0:
        return a.copy(), list(shape)
    if not perm:
        perm = list(range(rank - 1, -1, -1))
    out_shape = [shape[p] for p in perm]
    if rank == 2:   # PJRT.cpp:768-777: always [1, 0], whatever perm says
        M, N = shape
        return a.ravel()[:M * N].reshape(M, N).T.ravel().copy(), out_shape
    return np.transpose(a.ravel().reshape(shape), perm).ravel().copy(), out_shape


def _reduce(a, shape, dims):
    rank = len(shape)
    if rank == 0:
        return a.copy(), list(shape)
    if not dims:
        dims = list(range(rank))
    red = [False] * rank
    for d in dims:
        if 0 <= d < rank:
            red[d] = True
    out_shape = [shape[d] for d in range(rank) if not red[d]] or [1]
    out = np.zeros(int(np.prod(out_shape)), np.float32)
    idx = np.indices(shape).reshape(rank, -1)
    ostr = [1] * len(out_shape)
    for i in range(len(out_shape) - 2, -1, -1):
        ostr[i] = ostr[i + 1] * out_shape[i + 1]
    flat_out = np.zeros(idx.shape[1], np.int64)
    k = 0
    for d in range(rank):
        if not red[d]:
            flat_out += idx[d] * ostr[k]
            k += 1
    data = a.ravel()
    for i in range(data.size):   # sequential fp32 accumulation in input order
        out[flat_out[i]] = np.float32(out[flat_out[i]] + data[i])
    return out, out_shape


def execute(prog, inputs, custom_call_fn=None):
    """inputs: list of (numpy array, shape).  Returns [(array, shape), ...]."""
    buf = {}
    for i, (a, s) in enumerate(inputs[:prog.n_inputs]):
        buf[i] = (np.asarray(a, np.float32).ravel().copy(), list(s))
    for op in prog.ops:
        k = op["kind"]
        ins = op["ins"]
        have = all(i in buf for i in ins[:2]) if k in _BINARY.values() or k == "matmul" else \
            (ins[0] in buf if ins else True)
        if k in _BINARY.values():
            if len(ins) < 2 or not have:
                continue
            (a, sa), (b, sb) = buf[ins[0]], buf[ins[1]]
            buf[op["outs"][0]] = (_binary(k, a, b), list(sa if len(sa) >= len(sb) else sb))
        elif k in _UNARY.values():
            if not ins or ins[0] not in buf:
                continue
            a, sa = buf[ins[0]]
            buf[op["outs"][0]] = (_unary(k, a), list(sa))
        elif k == "constant":
            d = op["data"]
            buf[op["outs"][0]] = (np.array(d, np.float32), [len(d)]) if d else (np.zeros(1, np.float32), [1])
        elif k == "matmul":
            if len(ins) < 2 or not have:
                continue
            (a, sa), (b, sb) = buf[ins[0]], buf[ins[1]]
            M = sa[-2] if len(sa) >= 2 else 1
            K = sa[-1] if len(sa) >= 1 else 1
            N = sb[-1] if len(sb) >= 2 else 1
            out = np.zeros(M * N, np.float32)
            if M > 0 and N > 0 and K > 0:
                out = (a[:M * K].astype(np.float64).reshape(M, K) @
                       b[:K * N].astype(np.float64).reshape(K, N)).astype(np.float32).ravel()
            buf[op["outs"][0]] = (out, [M, N])
        elif k == "reshape":
            if not ins or ins[0] not in buf:
                continue
            a, sa = buf[ins[0]]
            buf[op["outs"][0]] = (a.copy(), list(op["shape"]) if op["shape"] else list(sa))
        elif k == "transpose":
            if not ins or ins[0] not in buf:
                continue
            a, sa = buf[ins[0]]
            buf[op["outs"][0]] = _transpose(a, sa, op["perm"])
        elif k == "reduce":
            if not ins or ins[0] not in buf:
                continue
            a, sa = buf[ins[0]]
            buf[op["outs"][0]] = _reduce(a, sa, op["dims"])
        elif k == "custom_call":
            args = [buf[i] for i in ins]
            outs = custom_call_fn(op["target"], op["config"], args, op["types"])
            for idx, o in zip(op["outs"], outs):
                buf[idx] = o
        else:  # copy
            if ins[0] not in buf:
                continue
            a, sa = buf[ins[0]]
            buf[op["outs"][0]] = (a.copy(), list(sa))
    outs = [buf[i] for i in sorted(buf) if i >= prog.n_inputs]
    if not outs:
        outs = [(np.asarray(a, np.float32).ravel().copy(), list(s)) for a, s in inputs]
    return outs


def run(text, inputs, custom_call_fn=None, multi_result=False):
    prog = Program(text, len(inputs), multi_result)
    return execute(prog, inputs, custom_call_fn)
