"""A reader for the subset of the ONNX protobuf schema an inference graph uses.

The ``onnx`` package is not part of this stack, so ``.onnx`` files are read
straight from the protobuf wire format: a message is a sequence of
``(field number << 3 | wire type)`` keys, each followed by a varint (type 0),
a 64-bit word (1), a length-prefixed byte run (2) or a 32-bit word (5).
Field numbers are the published ones of onnx/onnx.proto (ModelProto,
GraphProto, NodeProto, AttributeProto, TensorProto, ValueInfoProto,
TypeProto, TensorShapeProto, OperatorSetIdProto). Unknown fields are skipped,
as protobuf readers do, and repeated scalars are accepted packed or unpacked.

What the reference takes from ``onnx`` (mdlc/frontend/onnx_importer.py:12-13,
``onnx.load`` and ``numpy_helper.to_array``) is the decoded model below:
plain dataclasses and NumPy arrays, nothing that refers back to the bytes.
"""

from __future__ import annotations

import os
import struct
from dataclasses import dataclass, field
from typing import Any, Iterator, Optional, Union

import numpy as np

__all__ = ["OnnxDecodeError", "ModelProto", "GraphProto", "NodeProto", "AttributeProto",
           "TensorProto", "ValueInfoProto", "load_model", "parse_model", "tensor_to_array",
           "TENSOR_DTYPES"]


class OnnxDecodeError(ValueError):
    """The bytes are not a well-formed ONNX model, or use a feature this
    reader does not decode (external tensor data, sparse initializers)."""


# TensorProto.DataType -> NumPy dtype (onnx.proto's enum values)
TENSOR_DTYPES = {
    1: np.float32, 2: np.uint8, 3: np.int8, 4: np.uint16, 5: np.int16, 6: np.int32,
    7: np.int64, 9: np.bool_, 10: np.float16, 11: np.float64, 12: np.uint32, 13: np.uint64,
}

# AttributeProto.AttributeType values
ATTR_FLOAT, ATTR_INT, ATTR_STRING, ATTR_TENSOR, ATTR_GRAPH = 1, 2, 3, 4, 5
ATTR_FLOATS, ATTR_INTS, ATTR_STRINGS, ATTR_TENSORS, ATTR_GRAPHS = 6, 7, 8, 9, 10


# -- wire format -------------------------------------------------------------

def _varint(buf: memoryview, pos: int) -> tuple:
    value = shift = 0
    while True:
        if pos >= len(buf):
            raise OnnxDecodeError("truncated varint")
        b = buf[pos]
        pos += 1
        value |= (b & 0x7F) << shift
        if b < 0x80:
            return value, pos
        shift += 7
        if shift > 63:
            raise OnnxDecodeError("varint longer than 10 bytes")


def _signed(v: int) -> int:
    """int32/int64 fields are sent as the 64-bit two's complement."""
    return v - (1 << 64) if v >= 1 << 63 else v


def _fields(buf: memoryview) -> Iterator[tuple]:
    """Yield (field number, wire type, value) of one message: an int for
    wire types 0, 1 and 5 (the raw word), a memoryview for type 2."""
    pos, end = 0, len(buf)
    while pos < end:
        key, pos = _varint(buf, pos)
        num, wt = key >> 3, key & 7
        if wt == 0:
            v, pos = _varint(buf, pos)
        elif wt == 1:
            if pos + 8 > end:
                raise OnnxDecodeError("truncated 64-bit field")
            v = int.from_bytes(buf[pos:pos + 8], "little")
            pos += 8
        elif wt == 2:
            n, pos = _varint(buf, pos)
            if pos + n > end:
                raise OnnxDecodeError(f"field {num}: length {n} runs past the message")
            v = buf[pos:pos + n]
            pos += n
        elif wt == 5:
            if pos + 4 > end:
                raise OnnxDecodeError("truncated 32-bit field")
            v = int.from_bytes(buf[pos:pos + 4], "little")
            pos += 4
        else:
            raise OnnxDecodeError(f"field {num}: wire type {wt} is not used by onnx.proto")
        if num == 0:
            raise OnnxDecodeError("field number 0")
        yield num, wt, v


def _str(v) -> str:
    return bytes(v).decode("utf-8")


def _ints(out: list, wt: int, v, signed: bool = True) -> None:
    """Append a repeated varint field's values, packed (type 2) or not."""
    if wt == 2:
        pos = 0
        while pos < len(v):
            x, pos = _varint(v, pos)
            out.append(_signed(x) if signed else x)
    elif wt == 0:
        out.append(_signed(v) if signed else v)
    else:
        raise OnnxDecodeError(f"integer field sent with wire type {wt}")


def _fixed(out: list, wt: int, v, fmt: str) -> None:
    """Append a repeated float ('f', wire type 5) or double ('d', type 1)."""
    size = struct.calcsize("<" + fmt)
    if wt == 2:
        if len(v) % size:
            raise OnnxDecodeError("packed fixed-width field of ragged length")
        out.extend(np.frombuffer(bytes(v), dtype="<" + fmt).tolist())
    elif wt in (1, 5):
        out.append(struct.unpack("<" + fmt, v.to_bytes(size, "little"))[0])
    else:
        raise OnnxDecodeError(f"floating field sent with wire type {wt}")


# -- messages ----------------------------------------------------------------

@dataclass
class TensorProto:
    name: str = ""
    dims: list = field(default_factory=list)
    data_type: int = 0
    raw_data: Optional[bytes] = None
    float_data: list = field(default_factory=list)
    int32_data: list = field(default_factory=list)
    int64_data: list = field(default_factory=list)
    double_data: list = field(default_factory=list)
    uint64_data: list = field(default_factory=list)
    external: bool = False


@dataclass
class AttributeProto:
    name: str = ""
    type: int = 0
    f: float = 0.0
    i: int = 0
    s: bytes = b""
    t: Optional[TensorProto] = None
    has_graph: bool = False
    floats: list = field(default_factory=list)
    ints: list = field(default_factory=list)
    strings: list = field(default_factory=list)
    tensors: list = field(default_factory=list)
    present: set = field(default_factory=set)


@dataclass
class NodeProto:
    op_type: str = ""
    name: str = ""
    domain: str = ""
    input: list = field(default_factory=list)
    output: list = field(default_factory=list)
    attribute: list = field(default_factory=list)


@dataclass
class ValueInfoProto:
    name: str = ""
    elem_type: int = 0
    has_shape: bool = False
    dims: list = field(default_factory=list)     # int, str (dim_param) or None


@dataclass
class GraphProto:
    name: str = ""
    node: list = field(default_factory=list)
    initializer: list = field(default_factory=list)
    input: list = field(default_factory=list)
    output: list = field(default_factory=list)
    value_info: list = field(default_factory=list)


@dataclass
class ModelProto:
    ir_version: int = 0
    producer_name: str = ""
    producer_version: str = ""
    opset_import: dict = field(default_factory=dict)   # domain -> version
    graph: GraphProto = field(default_factory=GraphProto)


def _tensor(buf) -> TensorProto:
    t = TensorProto()
    for num, wt, v in _fields(buf):
        if num == 1:
            _ints(t.dims, wt, v)
        elif num == 2:
            t.data_type = _signed(v)
        elif num == 4:
            _fixed(t.float_data, wt, v, "f")
        elif num == 5:
            _ints(t.int32_data, wt, v)
        elif num == 7:
            _ints(t.int64_data, wt, v)
        elif num == 8:
            t.name = _str(v)
        elif num == 9:
            t.raw_data = bytes(v)
        elif num == 10:
            _fixed(t.double_data, wt, v, "d")
        elif num == 11:
            _ints(t.uint64_data, wt, v, signed=False)
        elif num == 13:
            t.external = True
        elif num == 14:
            t.external = t.external or v == 1
        elif num == 3:
            raise OnnxDecodeError(f"tensor {t.name!r}: segmented tensors are not supported")
    return t


def _attribute(buf) -> AttributeProto:
    a = AttributeProto()
    for num, wt, v in _fields(buf):
        a.present.add(num)
        if num == 1:
            a.name = _str(v)
        elif num == 20:
            a.type = _signed(v)
        elif num == 2:
            a.f = struct.unpack("<f", v.to_bytes(4, "little"))[0]
        elif num == 3:
            a.i = _signed(v)
        elif num == 4:
            a.s = bytes(v)
        elif num == 5:
            a.t = _tensor(v)
        elif num == 6:
            a.has_graph = True
        elif num == 7:
            _fixed(a.floats, wt, v, "f")
        elif num == 8:
            _ints(a.ints, wt, v)
        elif num == 9:
            a.strings.append(bytes(v))
        elif num == 10:
            a.tensors.append(_tensor(v))
    if a.type == 0:                       # writers before IR version 3 left it unset
        for num, typ in ((5, ATTR_TENSOR), (6, ATTR_GRAPH), (4, ATTR_STRING), (2, ATTR_FLOAT),
                         (3, ATTR_INT), (7, ATTR_FLOATS), (8, ATTR_INTS), (9, ATTR_STRINGS),
                         (10, ATTR_TENSORS)):
            if num in a.present:
                a.type = typ
                break
    return a


def _node(buf) -> NodeProto:
    n = NodeProto()
    for num, _wt, v in _fields(buf):
        if num == 1:
            n.input.append(_str(v))
        elif num == 2:
            n.output.append(_str(v))
        elif num == 3:
            n.name = _str(v)
        elif num == 4:
            n.op_type = _str(v)
        elif num == 5:
            n.attribute.append(_attribute(v))
        elif num == 7:
            n.domain = _str(v)
    return n


def _value_info(buf) -> ValueInfoProto:
    vi = ValueInfoProto()
    for num, _wt, v in _fields(buf):
        if num == 1:
            vi.name = _str(v)
        elif num == 2:                                    # TypeProto
            for tn, _tw, tv in _fields(v):
                if tn != 1:                               # only tensor_type
                    continue
                for en, _ew, ev in _fields(tv):
                    if en == 1:
                        vi.elem_type = _signed(ev)
                    elif en == 2:                         # TensorShapeProto
                        vi.has_shape = True
                        for sn, _sw, sv in _fields(ev):
                            if sn != 1:
                                continue
                            dim: Union[int, str, None] = None
                            for dn, _dw, dv in _fields(sv):
                                if dn == 1:
                                    dim = _signed(dv)
                                elif dn == 2:
                                    dim = _str(dv) or None
                            vi.dims.append(dim)
    return vi


def _graph(buf) -> GraphProto:
    g = GraphProto()
    for num, _wt, v in _fields(buf):
        if num == 1:
            g.node.append(_node(v))
        elif num == 2:
            g.name = _str(v)
        elif num == 5:
            g.initializer.append(_tensor(v))
        elif num == 11:
            g.input.append(_value_info(v))
        elif num == 12:
            g.output.append(_value_info(v))
        elif num == 13:
            g.value_info.append(_value_info(v))
        elif num == 15:
            raise OnnxDecodeError("sparse initializers are not supported")
    return g


def parse_model(data: Union[bytes, bytearray, memoryview]) -> ModelProto:
    """Decode a serialized ModelProto."""
    m = ModelProto()
    seen_graph = False
    for num, _wt, v in _fields(memoryview(bytes(data))):
        if num == 1:
            m.ir_version = _signed(v)
        elif num == 2:
            m.producer_name = _str(v)
        elif num == 3:
            m.producer_version = _str(v)
        elif num == 7:
            m.graph = _graph(v)
            seen_graph = True
        elif num == 8:
            domain, version = "", 0
            for on, _ow, ov in _fields(v):
                if on == 1:
                    domain = _str(ov)
                elif on == 2:
                    version = _signed(ov)
            m.opset_import[domain] = version
    if not seen_graph:
        raise OnnxDecodeError("no graph in the model (is this an ONNX file?)")
    return m


def load_model(path: Union[str, os.PathLike]) -> ModelProto:
    with open(path, "rb") as f:
        return parse_model(f.read())


def tensor_to_array(t: TensorProto) -> np.ndarray:
    """NumPy value of a TensorProto: raw little-endian bytes, or the typed
    repeated field the type is stored in (float_data for float, int32_data
    for every type of 32 bits or fewer, float16 as its bit patterns,
    int64_data, double_data, uint64_data for uint32/uint64)."""
    if t.external:
        raise OnnxDecodeError(f"tensor {t.name!r}: external data is not supported")
    if t.data_type not in TENSOR_DTYPES:
        raise OnnxDecodeError(f"tensor {t.name!r}: data type {t.data_type} is not supported")
    dt = np.dtype(TENSOR_DTYPES[t.data_type])
    shape = tuple(int(d) for d in t.dims)
    count = int(np.prod(shape, dtype=np.int64)) if shape else 1
    if t.raw_data is not None:
        if len(t.raw_data) != count * dt.itemsize:
            raise OnnxDecodeError(f"tensor {t.name!r}: {len(t.raw_data)} raw bytes for "
                                  f"{count} x {dt.name}")
        return np.frombuffer(t.raw_data, dtype=dt.newbyteorder("<")).astype(dt).reshape(shape)
    if dt == np.float32:
        vals = np.asarray(t.float_data, np.float32)
    elif dt == np.float64:
        vals = np.asarray(t.double_data, np.float64)
    elif dt == np.int64:
        vals = np.asarray(t.int64_data, np.int64)
    elif dt in (np.uint32, np.uint64):
        vals = np.asarray(t.uint64_data, np.uint64).astype(dt)
    elif dt == np.float16:
        vals = np.asarray(t.int32_data, np.int64).astype(np.uint16).view(np.float16)
    elif dt == np.bool_:
        vals = np.asarray(t.int32_data, np.int64) != 0
    else:
        vals = np.asarray(t.int32_data, np.int64).astype(dt)
    if vals.size != count:
        raise OnnxDecodeError(f"tensor {t.name!r}: {vals.size} values for shape {shape}")
    return vals.reshape(shape)


def attribute_value(a: AttributeProto) -> Any:
    """Plain Python value of an attribute (the reference's _decode_attr,
    mdlc/frontend/onnx_importer.py:28-47): int, float, str, lists of those,
    or a NumPy array for a tensor."""
    if a.type == ATTR_INT:
        return int(a.i)
    if a.type == ATTR_FLOAT:
        return float(a.f)
    if a.type == ATTR_STRING:
        return a.s.decode("utf-8")
    if a.type == ATTR_INTS:
        return [int(v) for v in a.ints]
    if a.type == ATTR_FLOATS:
        return [float(v) for v in a.floats]
    if a.type == ATTR_STRINGS:
        return [s.decode("utf-8") for s in a.strings]
    if a.type == ATTR_TENSOR and a.t is not None:
        return tensor_to_array(a.t)
    raise NotImplementedError(f"unsupported attribute type {a.type} on {a.name!r}")


# -- writer ------------------------------------------------------------------

class _Writer:
    """Builds one message's bytes; nested messages are written separately and
    added as length-delimited fields."""

    def __init__(self) -> None:
        self.buf = bytearray()

    def _varint(self, v: int) -> None:
        v &= (1 << 64) - 1                   # negatives as 64-bit two's complement
        while v >= 0x80:
            self.buf.append((v & 0x7F) | 0x80)
            v >>= 7
        self.buf.append(v)

    def int(self, num: int, v: int) -> "_Writer":
        self._varint(num << 3)
        self._varint(int(v))
        return self

    def bytes(self, num: int, b) -> "_Writer":
        self._varint(num << 3 | 2)
        self._varint(len(b))
        self.buf += b
        return self

    def str(self, num: int, s: str) -> "_Writer":
        return self.bytes(num, s.encode("utf-8"))

    def float(self, num: int, f: float) -> "_Writer":
        self._varint(num << 3 | 5)
        self.buf += struct.pack("<f", f)
        return self

    def packed_ints(self, num: int, vals) -> "_Writer":
        inner = _Writer()
        for v in vals:
            inner._varint(int(v))
        return self.bytes(num, inner.buf)

    def packed_floats(self, num: int, vals) -> "_Writer":
        return self.bytes(num, np.asarray(vals, "<f4").tobytes())


def _write_tensor(t: TensorProto) -> bytes:
    w = _Writer()
    if t.dims:
        w.packed_ints(1, t.dims)
    w.int(2, t.data_type)
    if t.float_data:
        w.packed_floats(4, t.float_data)
    if t.int32_data:
        w.packed_ints(5, t.int32_data)
    if t.int64_data:
        w.packed_ints(7, t.int64_data)
    w.str(8, t.name)
    if t.raw_data is not None:
        w.bytes(9, t.raw_data)
    return bytes(w.buf)


def array_to_tensor(name: str, arr) -> TensorProto:
    """A TensorProto holding ``arr`` as little-endian raw bytes."""
    arr = np.asarray(arr)
    codes = {np.dtype(v): k for k, v in TENSOR_DTYPES.items()}
    if arr.dtype not in codes:
        raise OnnxDecodeError(f"tensor {name!r}: NumPy dtype {arr.dtype} has no ONNX type here")
    return TensorProto(name=name, dims=[int(d) for d in arr.shape], data_type=codes[arr.dtype],
                       raw_data=np.ascontiguousarray(arr).astype(arr.dtype.newbyteorder("<"))
                       .tobytes())


def _write_attribute(a: AttributeProto) -> bytes:
    w = _Writer().str(1, a.name)
    if a.type == ATTR_FLOAT:
        w.float(2, a.f)
    elif a.type == ATTR_INT:
        w.int(3, a.i)
    elif a.type == ATTR_STRING:
        w.bytes(4, a.s)
    elif a.type == ATTR_TENSOR:
        w.bytes(5, _write_tensor(a.t))
    elif a.type == ATTR_FLOATS:
        w.packed_floats(7, a.floats)
    elif a.type == ATTR_INTS:
        w.packed_ints(8, a.ints)
    elif a.type == ATTR_STRINGS:
        for s in a.strings:
            w.bytes(9, s)
    else:
        raise OnnxDecodeError(f"attribute {a.name!r}: type {a.type} is not written")
    w.int(20, a.type)
    return bytes(w.buf)


def _write_value_info(vi: ValueInfoProto) -> bytes:
    shape = _Writer()
    for d in vi.dims:
        dim = _Writer()
        if isinstance(d, str):
            dim.str(2, d)
        elif d is not None:
            dim.int(1, d)
        shape.bytes(1, dim.buf)
    tensor = _Writer().int(1, vi.elem_type)
    if vi.has_shape or vi.dims:
        tensor.bytes(2, shape.buf)
    return bytes(_Writer().str(1, vi.name).bytes(2, _Writer().bytes(1, tensor.buf).buf).buf)


def serialize_model(m: ModelProto) -> bytes:
    """The wire bytes of ``m``, with fields in onnx.proto's numbering, so
    that ``parse_model(serialize_model(m))`` gives ``m`` back."""
    g = _Writer()
    for n in m.graph.node:
        nw = _Writer()
        for e in n.input:
            nw.str(1, e)
        for e in n.output:
            nw.str(2, e)
        nw.str(3, n.name).str(4, n.op_type)
        for a in n.attribute:
            nw.bytes(5, _write_attribute(a))
        if n.domain:
            nw.str(7, n.domain)
        g.bytes(1, nw.buf)
    g.str(2, m.graph.name)
    for t in m.graph.initializer:
        g.bytes(5, _write_tensor(t))
    for num, vis in ((11, m.graph.input), (12, m.graph.output), (13, m.graph.value_info)):
        for vi in vis:
            g.bytes(num, _write_value_info(vi))
    w = _Writer().int(1, m.ir_version).str(2, m.producer_name)
    if m.producer_version:
        w.str(3, m.producer_version)
    w.bytes(7, g.buf)
    for domain, version in m.opset_import.items():
        w.bytes(8, _Writer().str(1, domain).int(2, version).buf)
    return bytes(w.buf)
