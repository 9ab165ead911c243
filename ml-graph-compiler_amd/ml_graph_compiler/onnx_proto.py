"""ONNX model files, read and written without the onnx package.

An ``.onnx`` file is one serialized ``onnx.ModelProto``: a protocol-buffers message (proto2
syntax) holding a GraphProto of NodeProtos, TensorProto initializers and ValueInfoProto
inputs/outputs. The reference compiler parses it with the onnx package
(src/ml_graph_compiler/onnx_import.py:8-9, ``onnx.load`` at :112 and ``numpy_helper.to_array``
at :121); that package is not part of this build, so this module holds a small wire-format
codec and plain dataclasses for the messages a model file uses. The dataclass attribute names
are those of the generated onnx classes (``graph.node``, ``node.op_type``, ``tensor.raw_data``,
``attr.ints`` ...), so the importer reads like code written against onnx.

Field numbers and enum values are those of the published schema (onnx/onnx.proto, IR version
10): ModelProto ir_version=1 producer_name=2 producer_version=3 domain=4 model_version=5
doc_string=6 graph=7 opset_import=8; OperatorSetIdProto domain=1 version=2; GraphProto node=1
name=2 initializer=5 doc_string=10 input=11 output=12 value_info=13; NodeProto input=1
output=2 name=3 op_type=4 attribute=5 doc_string=6 domain=7; AttributeProto name=1 f=2 i=3
s=4 t=5 g=6 floats=7 ints=8 strings=9 tensors=10 graphs=11 doc_string=13 type=20
sparse_tensor=22 sparse_tensors=23 (tp=14 type_protos=15 are kept opaque); ValueInfoProto
name=1 type=2; TypeProto tensor_type=1; TypeProto.Tensor elem_type=1 shape=2;
TensorShapeProto dim=1; Dimension dim_value=1 dim_param=2; TensorProto dims=1 data_type=2
float_data=4 int32_data=5 string_data=6 int64_data=7 name=8 raw_data=9 double_data=10
uint64_data=11 external_data=13 data_location=14; StringStringEntryProto key=1 value=2.

Decoding accepts repeated numeric fields both packed and unpacked (a proto2 parser must);
encoding writes them the way onnx's own serializer does (tensor payloads as raw_data,
attribute lists unpacked). Unknown fields are skipped, so files from newer IR versions load.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass, field
from numbers import Integral, Real
from pathlib import Path
from typing import Any, Iterator, Sequence

import numpy as np

from .errors import ModelImportError

# TensorProto.DataType
UNDEFINED, FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64, STRING, BOOL = range(10)
FLOAT16, DOUBLE, UINT32, UINT64, COMPLEX64, COMPLEX128, BFLOAT16 = range(10, 17)

# AttributeProto.AttributeType
A_UNDEFINED, A_FLOAT, A_INT, A_STRING, A_TENSOR, A_GRAPH = 0, 1, 2, 3, 4, 5
A_FLOATS, A_INTS, A_STRINGS, A_TENSORS, A_GRAPHS = 6, 7, 8, 9, 10
A_SPARSE_TENSOR, A_SPARSE_TENSORS, A_TYPE_PROTO, A_TYPE_PROTOS = 11, 12, 13, 14

# TensorProto.DataLocation
DEFAULT, EXTERNAL = 0, 1

# numpy dtype of each data type a tensor payload can be converted to
NP_TYPES: dict[int, np.dtype] = {
    FLOAT: np.dtype("<f4"),
    UINT8: np.dtype("u1"),
    INT8: np.dtype("i1"),
    UINT16: np.dtype("<u2"),
    INT16: np.dtype("<i2"),
    INT32: np.dtype("<i4"),
    INT64: np.dtype("<i8"),
    BOOL: np.dtype("?"),
    FLOAT16: np.dtype("<f2"),
    DOUBLE: np.dtype("<f8"),
    UINT32: np.dtype("<u4"),
    UINT64: np.dtype("<u8"),
}
_DATA_TYPE_OF = {dt.newbyteorder("="): code for code, dt in NP_TYPES.items()}

_VARINT, _I64, _LEN, _I32 = 0, 1, 2, 5
_U64 = (1 << 64) - 1


class DecodeError(ModelImportError):
    """A byte string that is not a well-formed message of the expected type."""


# ---------------------------------------------------------------------------------------------
# wire format


def _varint_at(buf: memoryview, pos: int) -> tuple[int, int]:
    value = shift = 0
    end = len(buf)
    while True:
        if pos >= end:
            raise DecodeError("truncated varint")
        b = buf[pos]
        pos += 1
        value |= (b & 0x7F) << shift
        if b < 0x80:
            return value & _U64, pos
        shift += 7
        if shift >= 70:
            raise DecodeError("varint longer than 10 bytes")


def _fields(buf: memoryview) -> Iterator[tuple[int, int, Any]]:
    """(field number, wire type, value) of each field of one message body: an int for varints,
    a memoryview for the other wire types."""
    pos, end = 0, len(buf)
    while pos < end:
        key, pos = _varint_at(buf, pos)
        number, wire = key >> 3, key & 7
        if number == 0:
            raise DecodeError("field number 0")
        if wire == _VARINT:
            value, pos = _varint_at(buf, pos)
        elif wire == _LEN:
            n, pos = _varint_at(buf, pos)
            if pos + n > end:
                raise DecodeError(f"field {number} runs past the end of its message")
            value = buf[pos : pos + n]
            pos += n
        elif wire in (_I64, _I32):
            n = 8 if wire == _I64 else 4
            if pos + n > end:
                raise DecodeError(f"field {number} runs past the end of its message")
            value = buf[pos : pos + n]
            pos += n
        else:
            raise DecodeError(f"unsupported wire type {wire} (field {number})")
        yield number, wire, value


def _signed(v: int) -> int:
    return v - (1 << 64) if v >= 1 << 63 else v


def _text(v: Any, wire: int) -> str:
    if wire != _LEN:
        raise DecodeError("string field with a non length-delimited wire type")
    try:
        return bytes(v).decode("utf-8")
    except UnicodeDecodeError as exc:
        raise DecodeError(f"string field is not UTF-8: {exc}") from exc


def _bytes(v: Any, wire: int) -> bytes:
    if wire != _LEN:
        raise DecodeError("bytes field with a non length-delimited wire type")
    return bytes(v)


def _message(v: Any, wire: int) -> memoryview:
    if wire != _LEN:
        raise DecodeError("message field with a non length-delimited wire type")
    return v


def _packed_varints(data: memoryview) -> np.ndarray:
    """All varints of a packed field at once (uint64): byte j of a varint holds bits
    7j..7j+6; a byte below 0x80 ends the varint."""
    b = np.frombuffer(data, np.uint8)
    if b.size == 0:
        return np.zeros(0, np.uint64)
    if b[-1] & 0x80:
        raise DecodeError("truncated packed varint field")
    ends = b < 0x80
    starts = np.flatnonzero(np.concatenate(([True], ends[:-1])))
    lengths = np.diff(np.append(starts, b.size))
    if lengths.max() > 10:
        raise DecodeError("varint longer than 10 bytes")
    within = np.arange(b.size) - np.repeat(starts, lengths)
    parts = (b & 0x7F).astype(np.uint64) << (7 * within).astype(np.uint64)
    return np.bitwise_or.reduceat(parts, starts)


class _Numbers:
    """Accumulates a repeated numeric field that may arrive packed, unpacked or both."""

    def __init__(self, kind: str):
        self.kind = kind  # "varint", "f4" or "f8"
        self.chunks: list[np.ndarray] = []

    def add(self, wire: int, v: Any) -> None:
        if self.kind == "varint":
            if wire == _VARINT:
                self.chunks.append(np.array([v], np.uint64))
            elif wire == _LEN:
                self.chunks.append(_packed_varints(v))
            else:
                raise DecodeError("integer list with a fixed-width wire type")
            return
        size = 4 if self.kind == "f4" else 8
        if wire == _LEN:
            if len(v) % size:
                raise DecodeError("packed floating-point field of a ragged length")
        elif wire != (_I32 if size == 4 else _I64):
            raise DecodeError("floating-point list with the wrong wire type")
        self.chunks.append(np.frombuffer(bytes(v), "<" + self.kind))

    def array(self, dtype: Any) -> np.ndarray | None:
        if not self.chunks:
            return None
        joined = np.concatenate(self.chunks) if len(self.chunks) > 1 else self.chunks[0]
        if self.kind == "varint" and np.dtype(dtype).kind == "i":
            return joined.view(np.int64).astype(dtype, copy=False)
        return joined.astype(dtype, copy=False)


class _Writer:
    """Serializes fields in the order they are added (callers add them by field number)."""

    def __init__(self) -> None:
        self.parts: list[bytes] = []

    @staticmethod
    def varint(n: int) -> bytes:
        n &= _U64
        out = bytearray()
        while n >= 0x80:
            out.append((n & 0x7F) | 0x80)
            n >>= 7
        out.append(n)
        return bytes(out)

    def tag(self, number: int, wire: int) -> None:
        self.parts.append(self.varint(number << 3 | wire))

    def int(self, number: int, n: int) -> None:
        self.tag(number, _VARINT)
        self.parts.append(self.varint(int(n)))

    def bytes(self, number: int, data: bytes) -> None:
        self.tag(number, _LEN)
        self.parts.append(self.varint(len(data)))
        self.parts.append(data)

    def str(self, number: int, s: str) -> None:
        self.bytes(number, s.encode("utf-8"))

    def float(self, number: int, x: float) -> None:
        self.tag(number, _I32)
        self.parts.append(struct.pack("<f", x))

    def packed_varints(self, number: int, values: Sequence[int]) -> None:
        self.bytes(number, b"".join(self.varint(int(v)) for v in values))

    def packed(self, number: int, array: np.ndarray) -> None:
        self.bytes(number, np.ascontiguousarray(array).tobytes())

    def done(self) -> bytes:
        return b"".join(self.parts)


# ---------------------------------------------------------------------------------------------
# messages


@dataclass
class OperatorSetIdProto:
    domain: str = ""
    version: int = 0

    @classmethod
    def decode(cls, buf: memoryview) -> OperatorSetIdProto:
        out = cls()
        for num, wire, v in _fields(buf):
            if num == 1:
                out.domain = _text(v, wire)
            elif num == 2 and wire == _VARINT:
                out.version = _signed(v)
        return out

    def encode(self) -> bytes:
        w = _Writer()
        w.str(1, self.domain)
        w.int(2, self.version)
        return w.done()


@dataclass
class Dimension:
    """One TensorShapeProto.Dimension: ``dim_value`` is None when the field is absent
    (``HasField("dim_value")`` of the onnx class)."""

    dim_value: int | None = None
    dim_param: str = ""

    @classmethod
    def decode(cls, buf: memoryview) -> Dimension:
        out = cls()
        for num, wire, v in _fields(buf):
            if num == 1 and wire == _VARINT:
                out.dim_value, out.dim_param = _signed(v), ""
            elif num == 2:
                out.dim_param, out.dim_value = _text(v, wire), None
        return out

    def encode(self) -> bytes:
        w = _Writer()
        if self.dim_value is not None:
            w.int(1, self.dim_value)
        elif self.dim_param:
            w.str(2, self.dim_param)
        return w.done()


@dataclass
class ValueInfoProto:
    """A named value with its TypeProto flattened: elem_type stays 0 when the type is not a
    tensor type (or absent); ``shape`` is None when the tensor type carries no shape."""

    name: str = ""
    elem_type: int = 0
    shape: list[Dimension] | None = None

    @classmethod
    def decode(cls, buf: memoryview) -> ValueInfoProto:
        out = cls()
        for num, wire, v in _fields(buf):
            if num == 1:
                out.name = _text(v, wire)
            elif num == 2:
                for tnum, twire, tv in _fields(_message(v, wire)):
                    if tnum != 1:  # sequence, map, optional and sparse types stay untyped
                        continue
                    for fnum, fwire, fv in _fields(_message(tv, twire)):
                        if fnum == 1 and fwire == _VARINT:
                            out.elem_type = _signed(fv)
                        elif fnum == 2:
                            dims = out.shape if out.shape is not None else []
                            for snum, swire, sv in _fields(_message(fv, fwire)):
                                if snum == 1:
                                    dims.append(Dimension.decode(_message(sv, swire)))
                            out.shape = dims
        return out

    def encode(self) -> bytes:
        tensor = _Writer()
        tensor.int(1, self.elem_type)
        if self.shape is not None:
            shape = _Writer()
            for d in self.shape:
                shape.bytes(1, d.encode())
            tensor.bytes(2, shape.done())
        typ = _Writer()
        typ.bytes(1, tensor.done())
        w = _Writer()
        w.str(1, self.name)
        w.bytes(2, typ.done())
        return w.done()


@dataclass
class TensorProto:
    name: str = ""
    dims: list[int] = field(default_factory=list)
    data_type: int = UNDEFINED
    raw_data: bytes | None = None
    float_data: np.ndarray | None = None
    int32_data: np.ndarray | None = None
    int64_data: np.ndarray | None = None
    double_data: np.ndarray | None = None
    uint64_data: np.ndarray | None = None
    string_data: list[bytes] = field(default_factory=list)
    data_location: int = DEFAULT
    external_data: dict[str, str] = field(default_factory=dict)

    @classmethod
    def decode(cls, buf: memoryview) -> TensorProto:
        out = cls()
        dims = _Numbers("varint")
        lists = {4: _Numbers("f4"), 5: _Numbers("varint"), 7: _Numbers("varint"),
                 10: _Numbers("f8"), 11: _Numbers("varint")}
        for num, wire, v in _fields(buf):
            if num == 1:
                dims.add(wire, v)
            elif num == 2 and wire == _VARINT:
                out.data_type = _signed(v)
            elif num in lists:
                lists[num].add(wire, v)
            elif num == 6:
                out.string_data.append(_bytes(v, wire))
            elif num == 8:
                out.name = _text(v, wire)
            elif num == 9:
                out.raw_data = _bytes(v, wire)
            elif num == 13:
                key = value = ""
                for enum, ewire, ev in _fields(_message(v, wire)):
                    if enum == 1:
                        key = _text(ev, ewire)
                    elif enum == 2:
                        value = _text(ev, ewire)
                out.external_data[key] = value
            elif num == 14 and wire == _VARINT:
                out.data_location = _signed(v)
        d = dims.array(np.int64)
        out.dims = [] if d is None else [int(x) for x in d]
        out.float_data = lists[4].array(np.float32)
        out.int32_data = lists[5].array(np.int64)
        out.int64_data = lists[7].array(np.int64)
        out.double_data = lists[10].array(np.float64)
        out.uint64_data = lists[11].array(np.uint64)
        return out

    def encode(self) -> bytes:
        w = _Writer()
        for d in self.dims:
            w.int(1, d)
        w.int(2, self.data_type)
        if self.float_data is not None:
            w.packed(4, np.asarray(self.float_data, "<f4"))
        if self.int32_data is not None:
            w.packed_varints(5, np.asarray(self.int32_data, np.int64).tolist())
        for s in self.string_data:
            w.bytes(6, s)
        if self.int64_data is not None:
            w.packed_varints(7, np.asarray(self.int64_data, np.int64).tolist())
        if self.name:
            w.str(8, self.name)
        if self.raw_data is not None:
            w.bytes(9, self.raw_data)
        if self.double_data is not None:
            w.packed(10, np.asarray(self.double_data, "<f8"))
        if self.uint64_data is not None:
            w.packed_varints(11, np.asarray(self.uint64_data, np.uint64).tolist())
        for key, value in self.external_data.items():
            entry = _Writer()
            entry.str(1, key)
            entry.str(2, value)
            w.bytes(13, entry.done())
        if self.data_location != DEFAULT:
            w.int(14, self.data_location)
        return w.done()


@dataclass
class OpaqueProto:
    """A sub-message the compiler does not interpret (sparse tensors, type protos): kept as
    bytes so that a file round-trips and error messages can name the attribute."""

    kind: str
    payload: bytes = b""


@dataclass
class AttributeProto:
    name: str = ""
    type: int = A_UNDEFINED
    f: float = 0.0
    i: int = 0
    s: bytes = b""
    t: TensorProto | None = None
    g: GraphProto | None = None
    floats: list[float] = field(default_factory=list)
    ints: list[int] = field(default_factory=list)
    strings: list[bytes] = field(default_factory=list)
    tensors: list[TensorProto] = field(default_factory=list)
    graphs: list[GraphProto] = field(default_factory=list)
    opaque: list[OpaqueProto] = field(default_factory=list)

    @classmethod
    def decode(cls, buf: memoryview) -> AttributeProto:
        out = cls()
        floats, ints = _Numbers("f4"), _Numbers("varint")
        present: list[int] = []
        for num, wire, v in _fields(buf):
            present.append(num)
            if num == 1:
                out.name = _text(v, wire)
            elif num == 20 and wire == _VARINT:
                out.type = _signed(v)
            elif num == 2 and wire == _I32:
                out.f = struct.unpack("<f", bytes(v))[0]
            elif num == 3 and wire == _VARINT:
                out.i = _signed(v)
            elif num == 4:
                out.s = _bytes(v, wire)
            elif num == 5:
                out.t = TensorProto.decode(_message(v, wire))
            elif num == 6:
                out.g = GraphProto.decode(_message(v, wire))
            elif num == 7:
                floats.add(wire, v)
            elif num == 8:
                ints.add(wire, v)
            elif num == 9:
                out.strings.append(_bytes(v, wire))
            elif num == 10:
                out.tensors.append(TensorProto.decode(_message(v, wire)))
            elif num == 11:
                out.graphs.append(GraphProto.decode(_message(v, wire)))
            elif num in (14, 15, 22, 23):
                kind = {14: "type_proto", 15: "type_proto", 22: "sparse_tensor", 23: "sparse_tensor"}[num]
                out.opaque.append(OpaqueProto(kind, _bytes(v, wire)))
        f = floats.array(np.float32)
        out.floats = [] if f is None else [float(x) for x in f]
        i = ints.array(np.int64)
        out.ints = [] if i is None else [int(x) for x in i]
        if out.type == A_UNDEFINED:
            # files written before the type field existed (IR version 1) leave it out; the
            # field that is present then says what the attribute holds
            kinds = {2: A_FLOAT, 3: A_INT, 4: A_STRING, 5: A_TENSOR, 6: A_GRAPH, 7: A_FLOATS,
                     8: A_INTS, 9: A_STRINGS, 10: A_TENSORS, 11: A_GRAPHS}
            out.type = next((kinds[n] for n in present if n in kinds), A_UNDEFINED)
        return out

    def encode(self) -> bytes:
        w = _Writer()
        w.str(1, self.name)
        if self.type == A_FLOAT:
            w.float(2, self.f)
        elif self.type == A_INT:
            w.int(3, self.i)
        elif self.type == A_STRING:
            w.bytes(4, self.s)
        elif self.type == A_TENSOR and self.t is not None:
            w.bytes(5, self.t.encode())
        elif self.type == A_GRAPH and self.g is not None:
            w.bytes(6, self.g.encode())
        for x in self.floats:
            w.float(7, x)
        for n in self.ints:
            w.int(8, n)
        for s in self.strings:
            w.bytes(9, s)
        for t in self.tensors:
            w.bytes(10, t.encode())
        for g in self.graphs:
            w.bytes(11, g.encode())
        for o in self.opaque:
            w.bytes(22 if o.kind == "sparse_tensor" else 14, o.payload)
        w.int(20, self.type)
        return w.done()


@dataclass
class NodeProto:
    input: list[str] = field(default_factory=list)
    output: list[str] = field(default_factory=list)
    name: str = ""
    op_type: str = ""
    domain: str = ""
    attribute: list[AttributeProto] = field(default_factory=list)

    @classmethod
    def decode(cls, buf: memoryview) -> NodeProto:
        out = cls()
        for num, wire, v in _fields(buf):
            if num == 1:
                out.input.append(_text(v, wire))
            elif num == 2:
                out.output.append(_text(v, wire))
            elif num == 3:
                out.name = _text(v, wire)
            elif num == 4:
                out.op_type = _text(v, wire)
            elif num == 5:
                out.attribute.append(AttributeProto.decode(_message(v, wire)))
            elif num == 7:
                out.domain = _text(v, wire)
        return out

    def encode(self) -> bytes:
        w = _Writer()
        for s in self.input:
            w.str(1, s)
        for s in self.output:
            w.str(2, s)
        if self.name:
            w.str(3, self.name)
        w.str(4, self.op_type)
        for a in self.attribute:
            w.bytes(5, a.encode())
        if self.domain:
            w.str(7, self.domain)
        return w.done()


@dataclass
class GraphProto:
    node: list[NodeProto] = field(default_factory=list)
    name: str = ""
    initializer: list[TensorProto] = field(default_factory=list)
    input: list[ValueInfoProto] = field(default_factory=list)
    output: list[ValueInfoProto] = field(default_factory=list)
    value_info: list[ValueInfoProto] = field(default_factory=list)

    @classmethod
    def decode(cls, buf: memoryview) -> GraphProto:
        out = cls()
        for num, wire, v in _fields(buf):
            if num == 1:
                out.node.append(NodeProto.decode(_message(v, wire)))
            elif num == 2:
                out.name = _text(v, wire)
            elif num == 5:
                out.initializer.append(TensorProto.decode(_message(v, wire)))
            elif num == 11:
                out.input.append(ValueInfoProto.decode(_message(v, wire)))
            elif num == 12:
                out.output.append(ValueInfoProto.decode(_message(v, wire)))
            elif num == 13:
                out.value_info.append(ValueInfoProto.decode(_message(v, wire)))
        return out

    def encode(self) -> bytes:
        w = _Writer()
        for n in self.node:
            w.bytes(1, n.encode())
        w.str(2, self.name)
        for t in self.initializer:
            w.bytes(5, t.encode())
        for vi in self.input:
            w.bytes(11, vi.encode())
        for vi in self.output:
            w.bytes(12, vi.encode())
        for vi in self.value_info:
            w.bytes(13, vi.encode())
        return w.done()


@dataclass
class ModelProto:
    ir_version: int = 0
    opset_import: list[OperatorSetIdProto] = field(default_factory=list)
    producer_name: str = ""
    producer_version: str = ""
    domain: str = ""
    model_version: int = 0
    doc_string: str = ""
    graph: GraphProto = field(default_factory=GraphProto)
    base_dir: Path | None = None  # directory external tensor data is relative to

    @classmethod
    def decode(cls, data: bytes | bytearray | memoryview) -> ModelProto:
        out = cls()
        seen_graph = False
        for num, wire, v in _fields(memoryview(data)):
            if num == 1 and wire == _VARINT:
                out.ir_version = _signed(v)
            elif num == 2:
                out.producer_name = _text(v, wire)
            elif num == 3:
                out.producer_version = _text(v, wire)
            elif num == 4:
                out.domain = _text(v, wire)
            elif num == 5 and wire == _VARINT:
                out.model_version = _signed(v)
            elif num == 6:
                out.doc_string = _text(v, wire)
            elif num == 7:
                out.graph = GraphProto.decode(_message(v, wire))
                seen_graph = True
            elif num == 8:
                out.opset_import.append(OperatorSetIdProto.decode(_message(v, wire)))
        if not seen_graph and len(data):
            raise DecodeError("not an ONNX model: the file has no graph")
        return out

    def encode(self) -> bytes:
        w = _Writer()
        w.int(1, self.ir_version)
        if self.producer_name:
            w.str(2, self.producer_name)
        if self.producer_version:
            w.str(3, self.producer_version)
        if self.domain:
            w.str(4, self.domain)
        if self.model_version:
            w.int(5, self.model_version)
        if self.doc_string:
            w.str(6, self.doc_string)
        w.bytes(7, self.graph.encode())
        for o in self.opset_import:
            w.bytes(8, o.encode())
        return w.done()

    SerializeToString = encode


# ---------------------------------------------------------------------------------------------
# files and tensors


def load_model(source: str | Path | bytes | bytearray | memoryview) -> ModelProto:
    """A model from a file path or from serialized bytes (``onnx.load`` /
    ``onnx.load_model_from_string``). Tensors stored as external data are read later, by
    :func:`to_array`, relative to the model file's directory."""
    if isinstance(source, (bytes, bytearray, memoryview)):
        return ModelProto.decode(source)
    path = Path(source)
    try:
        data = path.read_bytes()
    except OSError as exc:
        raise ModelImportError(f"cannot read {str(path)!r}: {exc.strerror or exc}") from exc
    try:
        model = ModelProto.decode(data)
    except DecodeError as exc:
        raise ModelImportError(f"{str(path)!r} is not a valid ONNX model: {exc}") from exc
    model.base_dir = path.resolve().parent
    return model


def save_model(model: ModelProto, path: str | Path) -> Path:
    path = Path(path)
    path.write_bytes(model.encode())
    return path


def _external_bytes(tensor: TensorProto, base_dir: Path | None) -> bytes:
    info = tensor.external_data
    location = info.get("location", "")
    if base_dir is None:
        raise ModelImportError(
            f"tensor {tensor.name!r} keeps its data in external file {location!r}; load the model "
            "from its path so the file can be found"
        )
    target = (base_dir / location).resolve()
    if not location or base_dir.resolve() not in (target, *target.parents):
        raise ModelImportError(f"tensor {tensor.name!r}: external data location {location!r} is not "
                               "a file inside the model's directory")
    offset = int(info.get("offset", "0") or 0)
    length = info.get("length")
    try:
        with open(target, "rb") as fh:
            fh.seek(offset)
            data = fh.read(int(length)) if length else fh.read()
    except OSError as exc:
        raise ModelImportError(f"tensor {tensor.name!r}: cannot read external data {location!r}: {exc}") from exc
    if length and len(data) != int(length):
        raise ModelImportError(f"tensor {tensor.name!r}: external data {location!r} is shorter than "
                               f"offset {offset} + length {length}")
    return data


def to_array(tensor: TensorProto, base_dir: Path | None = None) -> np.ndarray:
    """The tensor's value as a C-ordered numpy array (``onnx.numpy_helper.to_array``)."""
    if tensor.data_type not in NP_TYPES:
        raise ModelImportError(
            f"tensor {tensor.name!r} has unsupported data type {tensor.data_type}"
        )
    dtype = NP_TYPES[tensor.data_type]
    shape = tuple(int(d) for d in tensor.dims)
    if any(d < 0 for d in shape):
        raise ModelImportError(f"tensor {tensor.name!r} has a negative dimension {list(shape)}")
    count = int(np.prod(shape, dtype=np.int64))
    raw = tensor.raw_data
    if tensor.data_location == EXTERNAL:
        raw = _external_bytes(tensor, base_dir)
    if raw is not None:
        if len(raw) != count * dtype.itemsize:
            raise ModelImportError(
                f"tensor {tensor.name!r}: raw_data holds {len(raw)} bytes, shape {list(shape)} of "
                f"{dtype.name} needs {count * dtype.itemsize}"
            )
        flat = np.frombuffer(raw, dtype).astype(dtype.newbyteorder("="), copy=True)
    else:
        code = tensor.data_type
        if code == FLOAT:
            src = tensor.float_data
        elif code == DOUBLE:
            src = tensor.double_data
        elif code == INT64:
            src = tensor.int64_data
        elif code in (UINT32, UINT64):
            src = tensor.uint64_data
        else:  # INT32, INT16, INT8, UINT16, UINT8, BOOL, FLOAT16 (bit patterns)
            src = tensor.int32_data
        if src is None:
            src = np.zeros(0, np.int64)
        if src.size != count:
            raise ModelImportError(
                f"tensor {tensor.name!r} holds {src.size} values, shape {list(shape)} needs {count}"
            )
        if code == FLOAT16:
            flat = src.astype(np.uint16).view(np.float16)
        elif code == BOOL:
            flat = src != 0
        else:
            flat = src.astype(dtype.newbyteorder("="))
    return flat.reshape(shape)


def from_array(array: Any, name: str = "") -> TensorProto:
    """A TensorProto holding ``array`` as raw little-endian data (``numpy_helper.from_array``)."""
    a = np.asarray(array)
    key = a.dtype.newbyteorder("=")
    if key not in _DATA_TYPE_OF:
        raise ModelImportError(f"arrays of dtype {a.dtype} have no ONNX tensor type here")
    code = _DATA_TYPE_OF[key]
    data = np.ascontiguousarray(a, NP_TYPES[code]).tobytes()
    return TensorProto(name=name, dims=[int(d) for d in a.shape], data_type=code, raw_data=data)


# ---------------------------------------------------------------------------------------------
# construction helpers (the subset of onnx.helper that model writers and tests use)


def make_attribute(name: str, value: Any) -> AttributeProto:
    """An attribute whose type follows the Python value, as ``onnx.helper.make_attribute``."""
    a = AttributeProto(name=name)
    if isinstance(value, (str, bytes)):
        a.type, a.s = A_STRING, value.encode("utf-8") if isinstance(value, str) else value
    elif isinstance(value, (bool, np.bool_, Integral)):
        a.type, a.i = A_INT, int(value)
    elif isinstance(value, Real):
        a.type, a.f = A_FLOAT, float(value)
    elif isinstance(value, TensorProto):
        a.type, a.t = A_TENSOR, value
    elif isinstance(value, np.ndarray):
        a.type, a.t = A_TENSOR, from_array(value)
    elif isinstance(value, GraphProto):
        a.type, a.g = A_GRAPH, value
    elif isinstance(value, (list, tuple)):
        items = list(value)
        if all(isinstance(v, (bool, np.bool_, Integral)) for v in items):
            a.type, a.ints = A_INTS, [int(v) for v in items]
        elif all(isinstance(v, Real) for v in items):
            a.type, a.floats = A_FLOATS, [float(v) for v in items]
        elif all(isinstance(v, (str, bytes)) for v in items):
            a.type = A_STRINGS
            a.strings = [v.encode("utf-8") if isinstance(v, str) else v for v in items]
        elif all(isinstance(v, (TensorProto, np.ndarray)) for v in items):
            a.type = A_TENSORS
            a.tensors = [v if isinstance(v, TensorProto) else from_array(v) for v in items]
        elif all(isinstance(v, GraphProto) for v in items):
            a.type, a.graphs = A_GRAPHS, items
        else:
            raise ModelImportError(f"attribute {name!r}: a list of mixed kinds cannot be encoded")
    else:
        raise ModelImportError(f"attribute {name!r}: values of type {type(value).__name__} cannot be encoded")
    return a


def attribute_value(attr: AttributeProto) -> Any:
    """The Python value of an attribute (``onnx.helper.get_attribute_value``): bytes for
    strings, TensorProto / GraphProto objects for tensors and graphs."""
    kind = attr.type
    if kind == A_FLOAT:
        return attr.f
    if kind == A_INT:
        return attr.i
    if kind == A_STRING:
        return attr.s
    if kind == A_TENSOR:
        return attr.t
    if kind == A_GRAPH:
        return attr.g
    if kind == A_FLOATS:
        return list(attr.floats)
    if kind == A_INTS:
        return list(attr.ints)
    if kind == A_STRINGS:
        return list(attr.strings)
    if kind == A_TENSORS:
        return list(attr.tensors)
    if kind == A_GRAPHS:
        return list(attr.graphs)
    if kind in (A_SPARSE_TENSOR, A_TYPE_PROTO):
        return attr.opaque[0] if attr.opaque else OpaqueProto("sparse_tensor" if kind == A_SPARSE_TENSOR else "type_proto")
    if kind in (A_SPARSE_TENSORS, A_TYPE_PROTOS):
        return list(attr.opaque)
    raise ModelImportError(f"attribute {attr.name!r} has unsupported type {kind}")


def make_node(op_type: str, inputs: Sequence[str], outputs: Sequence[str], name: str = "",
              domain: str = "", **attrs: Any) -> NodeProto:
    return NodeProto(list(inputs), list(outputs), name, op_type, domain,
                     [make_attribute(k, v) for k, v in sorted(attrs.items())])


def make_value_info(name: str, elem_type: int, shape: Sequence[int | str | None] | None) -> ValueInfoProto:
    """``shape`` entries: an int (dim_value), a str (dim_param) or None (unknown); ``shape``
    None leaves the shape out."""
    dims = None
    if shape is not None:
        dims = [Dimension(dim_value=int(d)) if isinstance(d, Integral)
                else Dimension(dim_param=d) if isinstance(d, str) else Dimension() for d in shape]
    return ValueInfoProto(name, elem_type, dims)


def make_graph(nodes: Sequence[NodeProto], name: str, inputs: Sequence[ValueInfoProto],
               outputs: Sequence[ValueInfoProto], initializer: Sequence[TensorProto] = ()) -> GraphProto:
    return GraphProto(list(nodes), name, list(initializer), list(inputs), list(outputs))


def make_model(graph: GraphProto, opset: int = 17, domain: str = "", ir_version: int = 8,
               producer_name: str = "ml-graph-compiler") -> ModelProto:
    return ModelProto(ir_version=ir_version, opset_import=[OperatorSetIdProto(domain, opset)],
                      producer_name=producer_name, graph=graph)
