"""ONNX model loading for the device path: ModelProto -> ModelGraph, with every
initializer's bytes located in its file.

Restates the reference's OnnxModelLoader (src/ModelSharp/Onnx/OnnxModelLoader.cs) and its
ProtoReader (src/ModelSharp/Onnx/ProtoReader.cs): the same protobuf fields, dtype
decoding and error messages. Two things differ by design:

* the model file and every external-data file are memory-mapped and initializers are
  numpy views of the mapping (no copy into the heap; the reference copies each slice,
  OnnxModelLoader.cs:497-503);
* each raw initializer also records where its bytes lie (file, offset, length), so
  HipMatMulNBitsKernel.preload can stream MatMulNBits weights from the file straight
  into HBM through ms_hip_nbits_weights_create_from_files, without a host copy.
"""
from __future__ import annotations

import dataclasses
import mmap
import os
import struct

import numpy as np

from .graph import GraphNode, ModelGraph, ModelSharpException

# TensorProto.DataType (onnx.proto3)
DT_FLOAT, DT_UINT8, DT_INT8, DT_INT32, DT_INT64, DT_BOOL, DT_FLOAT16, DT_BFLOAT16 = 1, 2, 3, 6, 7, 9, 10, 16
_RAW_DTYPE = {DT_FLOAT: np.float32, DT_UINT8: np.uint8, DT_INT8: np.int8, DT_INT32: np.int32, DT_INT64: np.int64,
              DT_FLOAT16: np.float16}


@dataclasses.dataclass(frozen=True)
class FileSlice:
    """Where an initializer's raw little-endian bytes lie."""
    path: str
    offset: int
    length: int
    data_type: int


class _Reader:
    """Protobuf wire-format reader over buf[pos:end] (ProtoReader.cs)."""

    __slots__ = ("buf", "pos", "end")

    def __init__(self, buf, pos: int = 0, end: int | None = None):
        self.buf, self.pos, self.end = buf, pos, len(buf) if end is None else end

    @property
    def eof(self) -> bool:
        return self.pos >= self.end

    def varint(self) -> int:
        shift = result = 0
        buf = self.buf
        while True:
            if self.pos >= self.end:
                raise ModelSharpException("Truncated varint in ONNX protobuf.")
            b = buf[self.pos]
            self.pos += 1
            result |= (b & 0x7F) << shift
            if b < 0x80:
                return result
            shift += 7
            if shift >= 70:
                raise ModelSharpException("Malformed varint in ONNX protobuf.")

    def int64(self) -> int:
        v = self.varint() & 0xFFFFFFFFFFFFFFFF
        return v - (1 << 64) if v >= (1 << 63) else v

    def int32(self) -> int:
        v = self.varint() & 0xFFFFFFFF
        return v - (1 << 32) if v >= (1 << 31) else v

    def tag(self):
        if self.eof:
            return None
        t = self.varint()
        return t >> 3, t & 7

    def span(self) -> tuple[int, int]:
        n = self.varint()
        start = self.pos
        if n < 0 or start + n > self.end:
            raise ModelSharpException("Length-delimited field runs past the end of its message.")
        self.pos = start + n
        return start, start + n

    def string(self) -> str:
        s, e = self.span()
        return bytes(self.buf[s:e]).decode("utf-8")

    def float32(self) -> float:
        if self.pos + 4 > self.end:
            raise ModelSharpException("Truncated fixed32 in ONNX protobuf.")
        v = struct.unpack_from("<f", self.buf, self.pos)[0]
        self.pos += 4
        return v

    def skip(self, wire: int) -> None:
        if wire == 0:
            self.varint()
        elif wire == 1:
            self.pos += 8
        elif wire == 2:
            self.span()
        elif wire == 5:
            self.pos += 4
        else:
            raise ModelSharpException(f"Unsupported protobuf wire type {wire}.")
        if self.pos > self.end:
            raise ModelSharpException("Field runs past the end of its message.")


class _Files:
    """Memory maps of the model's external-data files, one per file
    (ExternalDataResolver, OnnxModelLoader.cs:468-511)."""

    def __init__(self, base_dir: str | None):
        self.base_dir = base_dir
        self.maps: dict[str, tuple] = {}

    def slice(self, location: str, offset: int, length: int, tensor: str):
        path = location if self.base_dir is None else os.path.join(self.base_dir, location)
        entry = self.maps.get(path)
        if entry is None:
            if not os.path.isfile(path):
                raise ModelSharpException(f"External data file '{path}' for initializer '{tensor}' was not found.")
            size = os.path.getsize(path)
            with open(path, "rb") as f:
                mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else None
            entry = (mm, size)
            self.maps[path] = entry
        mm, size = entry
        if length < 0:
            length = size - offset
        if offset < 0 or length < 0 or offset + length > size:
            raise ModelSharpException(
                f"External data slice [{offset}, {offset + length}) for initializer '{tensor}' is out of bounds "
                f"for file '{path}' (length {size}).")
        return path, mm, offset, length


def _packed(r: _Reader, s: int, e: int, kind: str, out: list):
    rr = _Reader(r.buf, s, e)
    while not rr.eof:
        out.append(rr.float32() if kind == "f" else (rr.int32() if kind == "i32" else rr.int64()))


class _Parser:
    def __init__(self, buf, model_path: str | None, files: _Files | None):
        self.buf = buf
        self.model_path = model_path
        self.files = files

    # ---- TensorProto (OnnxModelLoader.cs:236-431) ----------------------------------------------
    def tensor(self, s: int, e: int):
        r = _Reader(self.buf, s, e)
        dims: list[int] = []
        name = ""
        data_type = 0
        floats = int32s = int64s = None
        raw = None              # (buffer, start, end, path or None, file offset)
        ext_loc = None
        ext_off, ext_len, has_len = 0, -1, False
        location = 0
        while (t := r.tag()) is not None:
            f, w = t
            if f == 1 and w == 0:
                dims.append(r.int64())
            elif f == 1 and w == 2:
                _packed(r, *r.span(), "i64", dims)
            elif f == 2 and w == 0:
                data_type = r.int64()
            elif f == 4 and w == 5:
                (floats := floats or []).append(r.float32())
            elif f == 4 and w == 2:
                _packed(r, *r.span(), "f", floats := floats or [])
            elif f == 5 and w == 0:
                (int32s := int32s or []).append(r.int32())
            elif f == 5 and w == 2:
                _packed(r, *r.span(), "i32", int32s := int32s or [])
            elif f == 7 and w == 0:
                (int64s := int64s or []).append(r.int64())
            elif f == 7 and w == 2:
                _packed(r, *r.span(), "i64", int64s := int64s or [])
            elif f == 8 and w == 2:
                name = r.string()
            elif f == 9 and w == 2:
                rs, re_ = r.span()
                raw = (self.buf, rs, re_, self.model_path, rs)
            elif f == 13 and w == 2:
                key, value = self.entry(*r.span())
                if key == "location":
                    ext_loc = value
                elif key == "offset":
                    ext_off = int(value) if value else 0
                elif key == "length" and value:
                    ext_len, has_len = int(value), True
            elif f == 14 and w == 0:
                location = r.int64()
            else:
                r.skip(w)
        shape = tuple(int(d) for d in dims)
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        if location == 1:   # EXTERNAL (:288-303)
            if ext_loc is None:
                raise ModelSharpException(f"Initializer '{name}' is EXTERNAL but has no 'location' in external_data.")
            if self.files is None:
                raise ModelSharpException(
                    f"Initializer '{name}' references external data file '{ext_loc}', but the model was parsed "
                    "from an in-memory byte buffer with no base directory; load it from a file path "
                    "(OnnxModelLoader.LoadModel) so external data can be resolved.")
            path, mm, off, ln = self.files.slice(ext_loc, ext_off, ext_len if has_len else -1, name)
            raw = (mm if mm is not None else b"", off, off + ln, path, off)
        if data_type == 0:   # :306-312
            data_type = DT_INT64 if int64s is not None else DT_INT32 if int32s is not None else DT_FLOAT
        avail = (raw[2] - raw[1]) if raw is not None else 0
        if raw is None:
            for lst in (int64s, int32s, floats):
                if lst is not None and len(lst) > avail:
                    avail = len(lst)
        if count > avail:   # :314-329
            raise ModelSharpException(
                f"Initializer '{name}' declares {count} elements but only {avail} are available in its data "
                "(malformed, truncated, or adversarial model).")
        arr, src = self.decode(name, data_type, shape, count, raw, floats, int32s, int64s)
        return name, arr, src

    def decode(self, name, dt, shape, count, raw, floats, int32s, int64s):
        src = None
        if dt in _RAW_DTYPE or dt in (DT_BOOL, DT_BFLOAT16):
            if raw is not None and count > 0:
                buf, s, e, path, off = raw
                # Every raw type reads itemsize * count bytes of its own field and no more.
                itemsize = 1 if dt == DT_BOOL else 2 if dt == DT_BFLOAT16 else np.dtype(_RAW_DTYPE[dt]).itemsize
                if itemsize * count > e - s:
                    raise ModelSharpException(
                        f"Initializer '{name}' declares {count} elements but only {(e - s) // itemsize} "
                        "are available in its data (malformed, truncated, or adversarial model).")
                if dt == DT_BOOL:
                    arr = np.frombuffer(buf, np.uint8, count, s) != 0
                elif dt == DT_BFLOAT16:
                    bits = np.frombuffer(buf, np.uint16, count, s).astype(np.uint32) << 16
                    arr = bits.view(np.float32)
                else:
                    npdt = np.dtype(_RAW_DTYPE[dt])
                    arr = np.frombuffer(buf, npdt, count, s)
                    if path is not None:
                        src = FileSlice(path, off, npdt.itemsize * count, dt)
                return arr.reshape(shape), src
            lst = int64s if dt == DT_INT64 else floats if dt == DT_FLOAT else int32s
            npdt = {DT_BOOL: np.bool_, DT_BFLOAT16: np.float32}.get(dt, _RAW_DTYPE.get(dt))
            arr = np.zeros(count, dtype=npdt)
            if lst is not None:
                vals = lst[:count]
                if dt == DT_FLOAT16:
                    arr[:len(vals)] = np.array([v & 0xFFFF for v in vals], np.uint16).view(np.float16)
                elif dt == DT_BFLOAT16:
                    arr[:len(vals)] = (np.array([v & 0xFFFF for v in vals], np.uint32) << 16).view(np.float32)
                elif dt == DT_BOOL:
                    arr[:len(vals)] = np.array(vals) != 0
                else:
                    arr[:len(vals)] = np.array(vals).astype(npdt)
            return arr.reshape(shape), None
        raise ModelSharpException(f"Unsupported tensor data_type {dt} for '{name}'.")

    def entry(self, s: int, e: int) -> tuple[str, str]:
        r = _Reader(self.buf, s, e)
        key = value = ""
        while (t := r.tag()) is not None:
            f, w = t
            if f == 1 and w == 2:
                key = r.string()
            elif f == 2 and w == 2:
                value = r.string()
            else:
                r.skip(w)
        return key, value

    # ---- AttributeProto (:170-234) ---------------------------------------------------------------
    def attribute(self, s: int, e: int):
        r = _Reader(self.buf, s, e)
        name = ""
        atype = 0
        val = {}
        while (t := r.tag()) is not None:
            f, w = t
            if f == 1 and w == 2:
                name = r.string()
            elif f == 20 and w == 0:
                atype = r.int64()
            elif f == 2 and w == 5:
                val["f"] = r.float32()
            elif f == 3 and w == 0:
                val["i"] = r.int64()
            elif f == 4 and w == 2:
                val["s"] = r.string()
            elif f == 5 and w == 2:
                val["t"] = self.tensor(*r.span())[1]
            elif f == 6 and w == 2:
                val["g"] = self.graph(*r.span(), None)
            elif f == 7 and w == 5:
                val.setdefault("floats", []).append(r.float32())
            elif f == 7 and w == 2:
                _packed(r, *r.span(), "f", val.setdefault("floats", []))
            elif f == 8 and w == 0:
                val.setdefault("ints", []).append(r.int64())
            elif f == 8 and w == 2:
                _packed(r, *r.span(), "i64", val.setdefault("ints", []))
            elif f == 9 and w == 2:
                val.setdefault("strings", []).append(r.string())
            elif f == 10 and w == 2:
                val.setdefault("graphs", []).append(self.graph(*r.span(), None))
            else:
                r.skip(w)
        order = {1: "f", 2: "i", 3: "s", 4: "t", 5: "g", 6: "floats", 7: "ints", 8: "strings", 10: "graphs"}
        key = order.get(atype)
        if key is None or key not in val:
            key = next(iter(val), None)
        return name, (val.get(key) if key else None)

    # ---- NodeProto (:142-168) ------------------------------------------------------------------
    def node(self, s: int, e: int) -> GraphNode:
        r = _Reader(self.buf, s, e)
        inputs, outputs, attrs = [], [], {}
        name = op = ""
        while (t := r.tag()) is not None:
            f, w = t
            if f == 1 and w == 2:
                inputs.append(r.string())
            elif f == 2 and w == 2:
                outputs.append(r.string())
            elif f == 3 and w == 2:
                name = r.string()
            elif f == 4 and w == 2:
                op = r.string()
            elif f == 5 and w == 2:
                k, v = self.attribute(*r.span())
                attrs[k] = v
            else:
                r.skip(w)
        return GraphNode(op, name, inputs, outputs, attrs)

    # ---- GraphProto (:77-118) ------------------------------------------------------------------
    def graph(self, s: int, e: int, metadata) -> ModelGraph:
        r = _Reader(self.buf, s, e)
        nodes, inits, sources, ins, outs = [], {}, {}, [], []
        while (t := r.tag()) is not None:
            f, w = t
            if f == 1 and w == 2:
                nodes.append(self.node(*r.span()))
            elif f == 5 and w == 2:
                name, arr, src = self.tensor(*r.span())
                inits[name] = arr
                if src is not None:
                    sources[name] = src
            elif f == 11 and w == 2:
                ins.append(self.value_info_name(*r.span()))
            elif f == 12 and w == 2:
                outs.append(self.value_info_name(*r.span()))
            else:
                r.skip(w)
        g = ModelGraph(nodes, inits, [n for n in ins if n not in inits], outs)
        g.sources = sources
        g.metadata = dict(metadata or {})
        return g

    def value_info_name(self, s: int, e: int) -> str:
        r = _Reader(self.buf, s, e)
        while (t := r.tag()) is not None:
            f, w = t
            if f == 1 and w == 2:
                return r.string()
            r.skip(w)
        return ""

    def model(self) -> ModelGraph:
        r = _Reader(self.buf)
        graph = None
        metadata = {}
        while (t := r.tag()) is not None:
            f, w = t
            if f == 7 and w == 2:
                graph = r.span()
            elif f == 14 and w == 2:
                k, v = self.entry(*r.span())
                if k:
                    metadata[k] = v
            else:
                r.skip(w)
        if graph is None:
            raise ModelSharpException("ONNX model contains no graph (field 7).")
        return self.graph(*graph, metadata)


def load_model(path: str) -> ModelGraph:
    """OnnxModelLoader.LoadModel: the model file and its external-data files are
    memory-mapped; initializers are views of the mappings. graph.sources maps each raw
    initializer to its FileSlice."""
    path = os.path.abspath(path)
    with open(path, "rb") as f:
        size = os.path.getsize(path)
        buf = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ) if size else b""
    return _Parser(buf, path, _Files(os.path.dirname(path))).model()


def parse_model(data: bytes) -> ModelGraph:
    """OnnxModelLoader.ParseModel(bytes): no base directory, so EXTERNAL initializers fail."""
    return _Parser(memoryview(data), None, None).model()


def load_tensor(path: str) -> np.ndarray:
    """OnnxModelLoader.LoadTensorTyped: a standalone TensorProto (.pb)."""
    path = os.path.abspath(path)
    with open(path, "rb") as f:
        data = f.read()
    return _Parser(memoryview(data), None, _Files(os.path.dirname(path))).tensor(0, len(data))[1]
