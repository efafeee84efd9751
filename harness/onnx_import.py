"""ONNX model files -> this harness's graphs: the counterpart of MIRA's ONNX front end
(mira/frontends/onnx_import.py) for the operators of the W8A8 CNN and MLP path, so that
exported ResNet / MobileNet / MLP models run on the rocm target.

The `onnx` package is not needed: the model is decoded straight from the protobuf wire
format, using the field numbers of onnx.proto (they are part of the file format).  The
graph an ONNX model turns into is the one MIRA's importer builds for it, because the
target and the W8A8 rewrite see those op patterns:

    Conv                -> conv2d (+ add of an (O,1,1) bias); asymmetric pads -> pad first
    BatchNormalization  -> mul + add of per-channel constants, folded in f64
                           (mira/frontends/onnx_import.py:423-431)
    Relu / Clip         -> relu / maximum, minimum with scalars
    MaxPool             -> pad with -inf (and the ceil_mode remainder) + maxpool2d
    GlobalAveragePool   -> reduce_mean over (2, 3), keepdims
    Gemm / MatMul       -> matmul (a transposed constant weight folded in) + add
    Flatten / Reshape   -> reshape;  Add / Sub / Mul / Div -> the binary ops
    Identity / Dropout  -> nothing (inference)
    Constant, Shape, and Gather / Unsqueeze / Concat / Cast / arithmetic on constants
                        -> folded at import

Anything else raises OnnxImportError naming the operator.
"""
from __future__ import annotations

import struct
from typing import Optional

import numpy as np

from harness.graph import Graph, Value

# ---------------------------------------------------------------- protobuf wire format

VARINT, FIXED64, LEN, FIXED32 = 0, 1, 2, 5


class OnnxImportError(ValueError):
    """The model uses something this importer does not take."""


def _varint(buf: bytes, i: int) -> tuple[int, int]:
    value, shift = 0, 0
    while True:
        b = buf[i]
        i += 1
        value |= (b & 0x7F) << shift
        if b < 0x80:
            return value, i
        shift += 7
        if shift > 63:
            raise OnnxImportError("malformed varint")


def _fields(buf: bytes):
    """(field number, wire type, value) of each field of one message: an int for VARINT,
    FIXED32 and FIXED64 (raw little-endian bits), the bytes of a LEN field."""
    i, n = 0, len(buf)
    while i < n:
        key, i = _varint(buf, i)
        field, wire = key >> 3, key & 7
        if wire == VARINT:
            value, i = _varint(buf, i)
        elif wire == FIXED64:
            value, i = int.from_bytes(buf[i:i + 8], "little"), i + 8
        elif wire == FIXED32:
            value, i = int.from_bytes(buf[i:i + 4], "little"), i + 4
        elif wire == LEN:
            size, i = _varint(buf, i)
            value, i = buf[i:i + size], i + size
        else:
            raise OnnxImportError(f"unsupported protobuf wire type {wire}")
        yield field, wire, value


def _signed(v: int) -> int:
    """int64 fields are encoded as their two's-complement varint."""
    return v - (1 << 64) if v >= 1 << 63 else v


def _repeated_ints(wire: int, value) -> list[int]:
    """A repeated int64 field: packed (one LEN field) or one VARINT per element."""
    if wire == VARINT:
        return [_signed(value)]
    out, i = [], 0
    while i < len(value):
        v, i = _varint(value, i)
        out.append(_signed(v))
    return out


def _repeated_f32(wire: int, value) -> list[float]:
    if wire == FIXED32:
        return [struct.unpack("<f", value.to_bytes(4, "little"))[0]]
    return list(np.frombuffer(value, "<f4"))


# TensorProto.DataType -> NumPy dtype
_TENSOR_DTYPES = {1: np.float32, 2: np.uint8, 3: np.int8, 5: np.int16, 6: np.int32, 7: np.int64, 9: np.bool_,
                  10: np.float16, 11: np.float64}


def _tensor(buf: bytes) -> tuple[str, np.ndarray]:
    """TensorProto: dims 1, data_type 2, float_data 4, int32_data 5, int64_data 7, name 8,
    raw_data 9, double_data 10."""
    dims, dtype, name, raw = [], 1, "", None
    floats, ints32, ints64, doubles = [], [], [], []
    for f, w, v in _fields(buf):
        if f == 1:
            dims += _repeated_ints(w, v)
        elif f == 2:
            dtype = v
        elif f == 4:
            floats += _repeated_f32(w, v)
        elif f == 5:
            ints32 += _repeated_ints(w, v)
        elif f == 7:
            ints64 += _repeated_ints(w, v)
        elif f == 8:
            name = v.decode()
        elif f == 9:
            raw = v
        elif f == 10:
            doubles += list(np.frombuffer(v, "<f8")) if w == LEN else [struct.unpack("<d", v.to_bytes(8, "little"))[0]]
        elif f in (12, 13, 14):
            raise OnnxImportError(f"tensor '{name}': external data is not supported")
    if dtype not in _TENSOR_DTYPES:
        raise OnnxImportError(f"tensor '{name}': unsupported data type {dtype}")
    np_dtype = np.dtype(_TENSOR_DTYPES[dtype]).newbyteorder("<")
    if raw is not None:
        arr = np.frombuffer(raw, np_dtype).astype(np_dtype.newbyteorder("="))
    elif dtype == 1:
        arr = np.array(floats, np.float32)
    elif dtype == 11:
        arr = np.array(doubles, np.float64)
    elif dtype == 7:
        arr = np.array(ints64, np.int64)
    elif dtype == 10:      # float16 payloads travel as the bit patterns in int32_data
        arr = np.array(ints32, np.uint16).view(np.float16)
    else:
        arr = np.array(ints32, np_dtype)
    return name, arr.reshape(dims)


def _attribute(buf: bytes) -> tuple[str, object]:
    """AttributeProto: name 1, f 2, i 3, s 4, t 5, floats 7, ints 8, strings 9."""
    name, value, ints, floats, strings = "", None, None, None, None
    for f, w, v in _fields(buf):
        if f == 1:
            name = v.decode()
        elif f == 2:
            value = struct.unpack("<f", v.to_bytes(4, "little"))[0]
        elif f == 3:
            value = _signed(v)
        elif f == 4:
            value = bytes(v)
        elif f == 5:
            value = _tensor(v)[1]
        elif f == 6:
            raise OnnxImportError(f"attribute '{name}': subgraphs (control flow) are not supported")
        elif f == 7:
            floats = (floats or []) + _repeated_f32(w, v)
        elif f == 8:
            ints = (ints or []) + _repeated_ints(w, v)
        elif f == 9:
            strings = (strings or []) + [bytes(v)]
    for rep in (ints, floats, strings):
        if rep is not None:
            value = rep
    return name, value


def _node(buf: bytes) -> dict:
    """NodeProto: input 1, output 2, name 3, op_type 4, attribute 5, domain 7."""
    n = {"input": [], "output": [], "name": "", "op_type": "", "attrs": {}, "domain": ""}
    for f, _, v in _fields(buf):
        if f == 1:
            n["input"].append(v.decode())
        elif f == 2:
            n["output"].append(v.decode())
        elif f == 3:
            n["name"] = v.decode()
        elif f == 4:
            n["op_type"] = v.decode()
        elif f == 5:
            k, a = _attribute(v)
            n["attrs"][k] = a
        elif f == 7:
            n["domain"] = v.decode()
    return n


def _value_info(buf: bytes) -> tuple[str, int, list]:
    """ValueInfoProto name 1, type 2 -> TypeProto.tensor_type 1 -> elem_type 1, shape 2 ->
    dim 1 -> dim_value 1 | dim_param 2 (None for a symbolic extent)."""
    name, elem, dims = "", 0, []
    for f, _, v in _fields(buf):
        if f == 1:
            name = v.decode()
        elif f == 2:
            for f2, _, v2 in _fields(v):
                if f2 != 1:
                    raise OnnxImportError(f"value '{name}': only tensor types are supported")
                for f3, _, v3 in _fields(v2):
                    if f3 == 1:
                        elem = v3
                    elif f3 == 2:
                        for f4, _, v4 in _fields(v3):
                            if f4 == 1:
                                d = None
                                for f5, _, v5 in _fields(v4):
                                    if f5 == 1:
                                        d = _signed(v5)
                                dims.append(d)
    return name, elem, dims


def read_model(data: bytes) -> dict:
    """The parts of a ModelProto the importer uses: {"opset": default-domain version,
    "nodes", "initializers" (name -> array), "inputs", "outputs" ((name, elem, dims))}.
    ModelProto: graph 7, opset_import 8 (domain 1, version 2); GraphProto: node 1,
    initializer 5, input 11, output 12."""
    opset, graph = None, None
    for f, _, v in _fields(data):
        if f == 7:
            graph = v
        elif f == 8:
            domain, version = "", 0
            for f2, _, v2 in _fields(v):
                if f2 == 1:
                    domain = v2.decode()
                elif f2 == 2:
                    version = v2
            if domain in ("", "ai.onnx"):
                opset = version
    if graph is None:
        raise OnnxImportError("no graph in the model")
    m = {"opset": opset or 1, "nodes": [], "initializers": {}, "inputs": [], "outputs": []}
    for f, _, v in _fields(graph):
        if f == 1:
            m["nodes"].append(_node(v))
        elif f == 5:
            name, arr = _tensor(v)
            m["initializers"][name] = arr
        elif f == 11:
            m["inputs"].append(_value_info(v))
        elif f == 12:
            m["outputs"].append(_value_info(v))
    return m


# ---------------------------------------------------------------- graph building

_ELEM_DTYPES = {1: "f32", 10: "f16"}


class _Importer:
    def __init__(self, model: dict, input_shapes: Optional[dict], name: str):
        self.m = model
        self.g = Graph(name)
        self.env: dict[str, object] = {}       # ONNX name -> Value, or np.ndarray for a constant
        self.input_shapes = input_shapes or {}

    # values and constants
    def const(self, name: str) -> Optional[np.ndarray]:
        v = self.env.get(name)
        return v if isinstance(v, np.ndarray) else None

    def need_const(self, name: str, what: str) -> np.ndarray:
        a = self.const(name)
        if a is None:
            raise OnnxImportError(f"{what}: '{name}' must be a constant")
        return a

    def value(self, name: str, dtype=np.float32) -> Value:
        """A graph value for `name` (a constant becomes a const op in the graph's float type)."""
        v = self.env[name]
        if isinstance(v, np.ndarray):
            v = self.g.const(np.asarray(v, dtype))
            self.env[name] = v
        return v

    def scalar(self, x: float, like: Value) -> Value:
        return self.g.const(np.array(x, like.type.np_dtype))

    def run(self) -> Graph:
        m = self.m
        for k, a in m["initializers"].items():
            self.env[k] = a
        for name, elem, dims in m["inputs"]:
            if name in self.env:
                continue
            given = self.input_shapes.get(name)
            if given is not None:
                if len(given) != len(dims) or any(d is not None and d != e for d, e in zip(dims, given)):
                    raise OnnxImportError(f"input '{name}' has shape {dims} in the model; got {list(given)}")
                dims = list(given)
            if any(d is None for d in dims):
                raise OnnxImportError(f"input '{name}' has symbolic extents {dims}; give input_shapes")
            if elem not in _ELEM_DTYPES:
                raise OnnxImportError(f"input '{name}': element type {elem} is not float32/float16")
            self.env[name] = self.g.input(name, tuple(dims), _ELEM_DTYPES[elem])
        for node in m["nodes"]:
            self.node(node)
        self.g.outputs = [self.value(name) for name, _, _ in m["outputs"]]
        return self.g

    def node(self, n: dict) -> None:
        op, ins, a = n["op_type"], n["input"], n["attrs"]
        if n["domain"] not in ("", "ai.onnx"):
            raise OnnxImportError(f"custom operator {n['domain']}.{op} is not supported")
        present = [x for x in ins if x]
        if op == "Constant":
            outs = [self._constant(a)]
        elif op in _FOLD and all(self.const(x) is not None for x in present):
            outs = [np.asarray(_FOLD[op](self, [self.const(x) if x else None for x in ins], a))]
        elif op in _HANDLERS:
            outs = [_HANDLERS[op](self, ins, a)]
        else:
            raise OnnxImportError(f"ONNX operator '{op}' is not supported (node '{n['name']}')")
        for name, v in zip(n["output"], outs):
            if name:
                self.env[name] = v

    @staticmethod
    def _constant(a: dict) -> np.ndarray:
        if "value" in a:
            return np.asarray(a["value"])
        for k in ("value_float", "value_int", "value_floats", "value_ints"):
            if k in a:
                return np.array(a[k])
        raise OnnxImportError(f"Constant with attributes {sorted(a)} is not supported")


def _pads(a: dict, hw, kernel, dilation=(1, 1)) -> tuple:
    """(top, left, bottom, right) from auto_pad / pads."""
    auto = a.get("auto_pad", b"NOTSET")
    auto = auto.decode() if isinstance(auto, bytes) else auto
    strides = a.get("strides", [1, 1])
    if auto in ("SAME_UPPER", "SAME_LOWER"):
        lo_hi = []
        for size, k, s, d in zip(hw, kernel, strides, dilation):
            total = max((-(-size // s) - 1) * s + d * (k - 1) + 1 - size, 0)
            lo = total // 2 if auto == "SAME_UPPER" else total - total // 2
            lo_hi.append((lo, total - lo))
        return lo_hi[0][0], lo_hi[1][0], lo_hi[0][1], lo_hi[1][1]
    if auto == "VALID":
        return 0, 0, 0, 0
    p = list(a.get("pads", [0, 0, 0, 0]))
    return p[0], p[1], p[2], p[3]


def _conv(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    if x.type.rank != 4:
        raise OnnxImportError("Conv: only 2-D convolutions of NCHW tensors are supported")
    w = imp.value(ins[1])
    dil = tuple(a.get("dilations", [1, 1]))
    top, left, bottom, right = _pads(a, x.type.shape[2:], w.type.shape[2:], dil)
    if (top, left) != (bottom, right):
        x = imp.g.op("pad", [x], {"pads": ((0, 0), (0, 0), (top, bottom), (left, right))})
        top = left = 0
    s = a.get("strides", [1, 1])
    attrs = {"stride": (s[0], s[1]), "padding": (top, left)}
    if dil != (1, 1):
        attrs["dilation"] = dil
    if a.get("group", 1) != 1:
        attrs["groups"] = int(a["group"])
    y = imp.g.op("conv2d", [x, w], attrs)
    if len(ins) > 2 and ins[2]:
        b = imp.const(ins[2])
        bias = imp.g.const(b.reshape(-1, 1, 1).astype(np.float32)) if b is not None else \
            imp.g.op("reshape", [imp.value(ins[2])], {"shape": (w.type.shape[0], 1, 1)})
        y = imp.g.op("add", [y, bias])
    return y


def _batchnorm(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    gamma, beta, mean, var = (imp.need_const(n, "BatchNormalization").astype(np.float64) for n in ins[1:5])
    scale = gamma / np.sqrt(var + a.get("epsilon", 1e-5))
    shift = beta - mean * scale
    shape = (x.type.shape[1],) + (1,) * (x.type.rank - 2)
    y = imp.g.op("mul", [x, imp.g.const(scale.reshape(shape).astype(x.type.np_dtype))])
    return imp.g.op("add", [y, imp.g.const(shift.reshape(shape).astype(x.type.np_dtype))])


def _clip(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    if imp.m["opset"] < 11:
        lo, hi = a.get("min"), a.get("max")
    else:
        lo = float(imp.need_const(ins[1], "Clip").item()) if len(ins) > 1 and ins[1] else None
        hi = float(imp.need_const(ins[2], "Clip").item()) if len(ins) > 2 and ins[2] else None
    if lo is not None:
        x = imp.g.op("maximum", [x, imp.scalar(lo, x)])
    if hi is not None:
        x = imp.g.op("minimum", [x, imp.scalar(hi, x)])
    return x


def _maxpool(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    k, s = list(a["kernel_shape"]), list(a.get("strides", [1, 1]))
    if k[0] != k[1] or s[0] != s[1] or any(d != 1 for d in a.get("dilations", [1, 1])):
        raise OnnxImportError("MaxPool: only square windows, equal strides and no dilation are supported")
    h, w = x.type.shape[2:]
    top, left, bottom, right = _pads(a, (h, w), k)
    extra = [0, 0]
    if a.get("ceil_mode", 0):      # the last window may start in the padding only if it starts inside
        for ax, (size, lo, hi) in enumerate(((h, top, bottom), (w, left, right))):
            n_out = -(-(size + lo + hi - k[ax]) // s[ax]) + 1
            if (n_out - 1) * s[ax] >= size + lo:
                n_out -= 1
            extra[ax] = max(0, (n_out - 1) * s[ax] + k[ax] - (size + lo + hi))
    pads = ((0, 0), (0, 0), (top, bottom + extra[0]), (left, right + extra[1]))
    if any(lo or hi for lo, hi in pads):
        x = imp.g.op("pad", [x], {"pads": pads, "value": -np.inf})
    return imp.g.op("maxpool2d", [x], {"size": k[0], "stride": s[0]})


def _global_avg(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    return imp.g.op("reduce_mean", [x], {"axes": tuple(range(2, x.type.rank)), "keepdims": True})


def _gemm(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    if a.get("transA", 0):
        x = imp.g.op("transpose", [x], {"perm": (1, 0)})
    wc = imp.const(ins[1])
    if wc is not None:
        w = imp.g.const(np.ascontiguousarray(wc.T if a.get("transB", 0) else wc).astype(x.type.np_dtype))
    else:
        w = imp.value(ins[1])
        if a.get("transB", 0):
            w = imp.g.op("transpose", [w], {"perm": (1, 0)})
    y = imp.g.op("matmul", [x, w])
    if a.get("alpha", 1.0) != 1.0:
        y = imp.g.op("mul", [y, imp.scalar(a["alpha"], y)])
    if len(ins) > 2 and ins[2]:
        beta = a.get("beta", 1.0)
        cc = imp.const(ins[2])
        if cc is not None:       # a constant C: beta * C folded in f32
            c = imp.g.const(_f32(cc) * np.float32(beta) if beta != 1.0 else _f32(cc))
        else:
            c = imp.value(ins[2])
            if beta != 1.0:
                c = imp.g.op("mul", [c, imp.scalar(beta, c)])
        y = imp.g.op("add", [y, c])
    return y


def _matmul(imp: _Importer, ins, a):
    x, w = imp.value(ins[0]), imp.value(ins[1])
    if x.type.rank < 2 or w.type.rank < 2:
        raise OnnxImportError("MatMul: 1-D operands are not supported")
    return imp.g.op("matmul", [x, w])


def _binary(kind):
    def h(imp: _Importer, ins, a):
        x = imp.env[ins[0]]
        like = x if isinstance(x, Value) else imp.env[ins[1]]
        dtype = like.type.np_dtype if isinstance(like, Value) else np.float32
        return imp.g.op(kind, [imp.value(ins[0], dtype), imp.value(ins[1], dtype)])
    return h


def _reshape(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    target = [int(d) for d in imp.need_const(ins[1], "Reshape shape").ravel()]
    shape = [x.type.shape[i] if d == 0 and not a.get("allowzero", 0) else d for i, d in enumerate(target)]
    if -1 in shape:
        shape[shape.index(-1)] = x.type.numel // int(np.prod([d for d in shape if d != -1]))
    return imp.g.op("reshape", [x], {"shape": tuple(shape)})


def _flatten(imp: _Importer, ins, a):
    x = imp.value(ins[0])
    ax = a.get("axis", 1) % (x.type.rank + 1)
    lead = int(np.prod(x.type.shape[:ax], dtype=np.int64))
    return imp.g.op("reshape", [x], {"shape": (lead, x.type.numel // max(lead, 1))})


def _identity(imp: _Importer, ins, a):
    return imp.env[ins[0]]


def _shape(imp: _Importer, ins, a):
    """Shape of a graph value: its static extents, a constant (start / end slice it)."""
    v = imp.env[ins[0]]
    dims = np.array(v.type.shape if isinstance(v, Value) else v.shape, np.int64)
    return dims[a.get("start", 0):a.get("end", len(dims))]


_HANDLERS = {
    "Conv": _conv, "BatchNormalization": _batchnorm, "Relu": lambda imp, ins, a: imp.g.op("relu", [imp.value(ins[0])]),
    "Clip": _clip, "MaxPool": _maxpool, "GlobalAveragePool": _global_avg, "Gemm": _gemm, "MatMul": _matmul,
    "Add": _binary("add"), "Sub": _binary("sub"), "Mul": _binary("mul"), "Div": _binary("div"),
    "Reshape": _reshape, "Flatten": _flatten, "Identity": _identity, "Dropout": _identity, "Shape": _shape,
}

# shape arithmetic on constants (what exporters emit around Reshape), evaluated at import
_FOLD = {
    "Gather": lambda imp, xs, a: np.take(xs[0], xs[1], axis=a.get("axis", 0)),
    "Unsqueeze": lambda imp, xs, a: np.expand_dims(
        xs[0], tuple(int(i) for i in (a["axes"] if "axes" in a else xs[1].ravel()))),
    "Concat": lambda imp, xs, a: np.concatenate([x for x in xs if x is not None], axis=a["axis"]),
    "Cast": lambda imp, xs, a: xs[0].astype(_TENSOR_DTYPES[a["to"]]),
    "Identity": lambda imp, xs, a: xs[0],
    # arithmetic on constants only (a Gemm's beta * C, say), in the graph's f32 arithmetic
    "Add": lambda imp, xs, a: _f32(xs[0]) + _f32(xs[1]),
    "Sub": lambda imp, xs, a: _f32(xs[0]) - _f32(xs[1]),
    "Mul": lambda imp, xs, a: _f32(xs[0]) * _f32(xs[1]),
    "Div": lambda imp, xs, a: _f32(xs[0]) / _f32(xs[1]),
}


def _f32(a: np.ndarray) -> np.ndarray:
    return np.asarray(a, np.float32)


def import_model(data: bytes, input_shapes: Optional[dict] = None, name: str = "main") -> Graph:
    """An ONNX model (the bytes of a .onnx file) as a harness Graph; input_shapes fixes
    symbolic input extents (the batch size, say)."""
    return _Importer(read_model(data), input_shapes, name).run()


def load(path: str, input_shapes: Optional[dict] = None) -> Graph:
    with open(path, "rb") as f:
        return import_model(f.read(), input_shapes, name=str(path).rsplit("/", 1)[-1].rsplit(".", 1)[0])
