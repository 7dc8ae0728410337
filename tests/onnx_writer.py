"""A minimal ONNX ModelProto writer for the loader tests: protobuf wire encoding of the
fields the loader reads (onnx.proto field numbers), with initializers inline (raw_data or
typed lists) or in external-data files.
"""
from __future__ import annotations

import os
import struct

import numpy as np

DTYPE = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3, np.dtype(np.int32): 6,
         np.dtype(np.int64): 7, np.dtype(np.bool_): 9, np.dtype(np.float16): 10}


def varint(v: int) -> bytes:
    v &= 0xFFFFFFFFFFFFFFFF
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(field: int, wire: int) -> bytes:
    return varint((field << 3) | wire)


def ld(field: int, payload: bytes) -> bytes:
    return key(field, 2) + varint(len(payload)) + payload


def s(field: int, text: str) -> bytes:
    return ld(field, text.encode())


def vi(field: int, v: int) -> bytes:
    return key(field, 0) + varint(v)


def f32(field: int, v: float) -> bytes:
    return key(field, 5) + struct.pack("<f", v)


def entry(k: str, v: str) -> bytes:
    return s(1, k) + s(2, v)


def tensor(name: str, arr: np.ndarray, mode: str = "raw", ext: tuple | None = None, data_type: int | None = None):
    """TensorProto. mode 'raw' (raw_data), 'typed' (float_data / int32_data / int64_data),
    'external' (ext = (location, offset, length or None))."""
    arr = np.asarray(arr)
    out = b"".join(vi(1, int(d)) for d in arr.shape)
    out += vi(2, data_type if data_type is not None else DTYPE[arr.dtype])
    out += s(8, name)
    if mode == "raw":
        out += ld(9, np.ascontiguousarray(arr).tobytes())
    elif mode == "typed":
        if arr.dtype == np.float32:
            out += ld(4, arr.astype("<f4").tobytes())
        elif arr.dtype == np.int64:
            out += ld(7, b"".join(varint(int(x)) for x in arr.ravel()))
        else:
            out += ld(5, b"".join(varint(int(x)) for x in arr.ravel().astype(np.int64)))
    elif mode == "external":
        loc, off, length = ext
        out += ld(13, entry("location", loc)) + ld(13, entry("offset", str(off)))
        if length is not None:
            out += ld(13, entry("length", str(length)))
        out += vi(14, 1)
    return out


def attribute(name: str, value) -> bytes:
    out = s(1, name)
    if isinstance(value, float):
        return out + f32(2, value) + vi(20, 1)
    if isinstance(value, int):
        return out + vi(3, value) + vi(20, 2)
    if isinstance(value, str):
        return out + s(4, value) + vi(20, 3)
    if isinstance(value, (list, tuple)):
        return out + ld(8, b"".join(varint(int(x)) for x in value)) + vi(20, 7)
    raise TypeError(value)


def node(op: str, name: str, inputs, outputs, attrs=None, domain: str = "") -> bytes:
    out = b"".join(s(1, i) for i in inputs) + b"".join(s(2, o) for o in outputs) + s(3, name) + s(4, op)
    out += b"".join(ld(5, attribute(k, v)) for k, v in (attrs or {}).items())
    if domain:
        out += s(7, domain)
    return out


def value_info(name: str) -> bytes:
    return s(1, name)


def model(nodes, initializers, inputs, outputs, metadata=None) -> bytes:
    g = b"".join(ld(1, n) for n in nodes) + s(2, "g") + b"".join(ld(5, t) for t in initializers)
    g += b"".join(ld(11, value_info(i)) for i in inputs) + b"".join(ld(12, value_info(o)) for o in outputs)
    m = vi(1, 8) + ld(7, g)
    for k, v in (metadata or {}).items():
        m += ld(14, entry(k, v))
    return m


def write_matmul_nbits_model(directory: str, weights: dict, external: bool, name="model.onnx",
                             data_name="model.onnx.data"):
    """One MatMulNBits node per entry of weights {name: (b, scales, zp, N, K, bits, bs)};
    chained A -> Y0 -> Y1 ... requires each K to equal the previous N. Returns the model path."""
    inits, nodes = [], []
    prev = "A"
    blobs = bytearray()
    for i, (nm, (b, sc, zp, N, K, bits, bs)) in enumerate(weights.items()):
        for tname, arr in ((f"{nm}.B", b), (f"{nm}.scales", sc), (f"{nm}.zp", zp)):
            if arr is None:
                continue
            if external:
                while len(blobs) % 64:
                    blobs.append(0)
                off = len(blobs)
                blobs += np.ascontiguousarray(arr).tobytes()
                inits.append(tensor(tname, arr, "external", ("" + data_name, off, arr.nbytes)))
            else:
                inits.append(tensor(tname, arr, "raw"))
        out = f"Y{i}"
        nodes.append(node("MatMulNBits", nm, [prev, f"{nm}.B", f"{nm}.scales"] + ([f"{nm}.zp"] if zp is not None else []),
                          [out], {"N": N, "K": K, "bits": bits, "block_size": bs}, "com.microsoft"))
        prev = out
    path = os.path.join(directory, name)
    with open(path, "wb") as f:
        f.write(model(nodes, inits, ["A"], [prev]))
    if external:
        with open(os.path.join(directory, data_name), "wb") as f:
            f.write(bytes(blobs))
    return path
