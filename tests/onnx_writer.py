"""Test infrastructure: ONNX model bytes from plain node lists and NumPy arrays, encoded
with the protobuf wire format and onnx.proto's field numbers (the `onnx` package and
torch's exporter, which needs it, are not installed).  It writes the forms exporters
use: packed repeated fields, raw_data tensors, typed attributes."""
import struct

import numpy as np

_DTYPE_CODES = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3, np.dtype(np.int32): 6,
                np.dtype(np.int64): 7, np.dtype(np.float16): 10, np.dtype(np.float64): 11}
# AttributeProto.AttributeType
_FLOAT, _INT, _STRING, _TENSOR, _FLOATS, _INTS = 1, 2, 3, 4, 6, 7


def _varint(v: int) -> bytes:
    v &= (1 << 64) - 1           # negative int64 as two's complement
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field: int, wire: int) -> bytes:
    return _varint((field << 3) | wire)


def _len(field: int, payload: bytes) -> bytes:
    return _key(field, 2) + _varint(len(payload)) + payload


def _int(field: int, v: int) -> bytes:
    return _key(field, 0) + _varint(int(v))


def _f32(field: int, v: float) -> bytes:
    return _key(field, 5) + struct.pack("<f", v)


def _packed_ints(field: int, vs) -> bytes:
    return _len(field, b"".join(_varint(int(v)) for v in vs))


def tensor(name: str, a: np.ndarray, raw: bool = True) -> bytes:
    """TensorProto: dims 1, data_type 2, name 8, raw_data 9 (or float_data 4 / int64_data 7)."""
    a = np.asarray(a)
    out = (_packed_ints(1, a.shape) if a.ndim else b"") + _int(2, _DTYPE_CODES[a.dtype]) + _len(8, name.encode())
    if raw or a.dtype not in (np.float32, np.int64):
        return out + _len(9, np.ascontiguousarray(a).astype(a.dtype.newbyteorder("<")).tobytes())
    if a.dtype == np.float32:
        return out + _len(4, a.astype("<f4").tobytes())
    return out + _packed_ints(7, a.ravel())


def attribute(name: str, v) -> bytes:
    out = _len(1, name.encode())
    if isinstance(v, (bool, int, np.integer)):
        return out + _int(20, _INT) + _int(3, int(v))
    if isinstance(v, (float, np.floating)):
        return out + _int(20, _FLOAT) + _f32(2, float(v))
    if isinstance(v, (bytes, str)):
        return out + _int(20, _STRING) + _len(4, v.encode() if isinstance(v, str) else v)
    if isinstance(v, np.ndarray):
        return out + _int(20, _TENSOR) + _len(5, tensor("", v))
    v = list(v)
    if all(isinstance(x, (int, np.integer)) for x in v):
        return out + _int(20, _INTS) + _packed_ints(8, v)
    return out + _int(20, _FLOATS) + _len(7, struct.pack(f"<{len(v)}f", *v))


def _value_info(name: str, shape, elem: int = 1) -> bytes:
    dims = b"".join(_len(1, _len(2, str(d).encode()) if isinstance(d, str) else _int(1, d)) for d in shape)
    tensor_type = _int(1, elem) + _len(2, dims)
    return _len(1, name.encode()) + _len(2, _len(1, tensor_type))


class Model:
    """nodes, initializers, graph inputs/outputs -> ModelProto bytes (ir_version 7)."""

    def __init__(self, opset: int = 13):
        self.opset = opset
        self.nodes, self.inits, self.ins, self.outs = [], [], [], []
        self._n = 0

    def init(self, a: np.ndarray, name: str = None) -> str:
        name = name or f"c{len(self.inits)}"
        self.inits.append(tensor(name, np.asarray(a)))
        return name

    def node(self, op_type: str, inputs, n_out: int = 1, **attrs) -> str:
        self._n += 1
        outs = [f"{op_type.lower()}{self._n}_{i}" for i in range(n_out)]
        body = b"".join(_len(1, i.encode()) for i in inputs) + b"".join(_len(2, o.encode()) for o in outs)
        body += _len(3, f"n{self._n}".encode()) + _len(4, op_type.encode())
        body += b"".join(_len(5, attribute(k, v)) for k, v in attrs.items())
        self.nodes.append(body)
        return outs[0] if n_out == 1 else outs

    def input(self, name: str, shape, elem: int = 1) -> str:
        self.ins.append(_value_info(name, shape, elem))
        return name

    def output(self, name: str, shape) -> None:
        self.outs.append(_value_info(name, shape))

    def bytes(self) -> bytes:
        graph = b"".join(_len(1, n) for n in self.nodes) + _len(2, b"g")
        graph += b"".join(_len(5, t) for t in self.inits)
        graph += b"".join(_len(11, i) for i in self.ins) + b"".join(_len(12, o) for o in self.outs)
        opset = _len(1, b"") + _int(2, self.opset)
        return _int(1, 7) + _len(2, b"tests") + _len(7, graph) + _len(8, opset)
