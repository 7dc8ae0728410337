"""The ONNX loader (modelsharp_amd/onnx_loader.py) against the reference's own ONNX
fixtures (tests/ModelSharp.Tests/assets, copied as data under tests/golden/onnx) and
against models written by tests/onnx_writer.py: inline raw_data, typed lists, external
data with offsets, and the loader's error messages (OnnxModelLoader.cs)."""
from __future__ import annotations

import os

import numpy as np
import pytest

import onnx_writer as W
from conftest import ROOT
from modelsharp_amd import onnx_loader as L
from modelsharp_amd import workloads
from modelsharp_amd.graph import ModelSharpException

ASSETS = ROOT / "tests" / "golden" / "onnx"


@pytest.mark.parametrize("case", ["test_matmul_2d", "test_matmul_3d", "test_matmul_4d"])
def test_reference_matmul_fixtures(case):
    g = L.load_model(str(ASSETS / case / "model.onnx"))
    assert [(n.op_type, n.inputs, n.outputs) for n in g.nodes] == [("MatMul", ["a", "b"], ["c"])]
    assert g.inputs == ["a", "b"] and g.outputs == ["c"]
    d = ASSETS / case / "test_data_set_0"
    a, b, c = (L.load_tensor(str(d / f)) for f in ("input_0.pb", "input_1.pb", "output_0.pb"))
    assert a.dtype == np.float32 and c.shape == np.matmul(a, b).shape
    assert np.allclose(np.matmul(a, b), c, rtol=1e-6, atol=1e-6)


def test_reference_mnist_fixture():
    g = L.load_model(str(ASSETS / "mnist-12.onnx"))
    assert [n.op_type for n in g.nodes] == ["Conv", "Add", "Relu", "MaxPool", "Conv", "Add", "Relu", "MaxPool",
                                            "Reshape", "Reshape", "MatMul", "Add"]
    assert g.inputs == ["Input3"] and g.outputs == ["Plus214_Output_0"]
    shapes = {k: v.shape for k, v in g.initializers.items()}
    assert shapes["Parameter5"] == (8, 1, 5, 5) and shapes["Parameter87"] == (16, 8, 5, 5)
    assert shapes["Parameter193"] == (16, 4, 4, 10) and shapes["Parameter194"] == (1, 10)
    conv = g.nodes[0]
    assert conv.attributes["kernel_shape"] == [5, 5] and conv.attributes["auto_pad"] == "SAME_UPPER"
    # topologically consistent: every input is a feed, an initializer or an earlier output
    seen = set(g.inputs) | set(g.initializers)
    for n in g.nodes:
        assert all(i in seen for i in n.inputs if i)
        seen |= set(n.outputs)
    assert g.outputs[0] in seen


def _weights(op, seed):
    b, s, z = workloads.make_weights(op, seed)
    return b, s, z, op.N, op.K, op.bits, op.block_size


@pytest.mark.parametrize("external", [False, True])
def test_matmul_nbits_model_round_trip(tmp_path, external):
    ops = {"gate": _weights(workloads.Op("g", 256, 96, 32, True), 1),
           "down": _weights(workloads.Op("d", 96, 64, 32, False), 2)}
    path = W.write_matmul_nbits_model(str(tmp_path), ops, external)
    g = L.load_model(path)
    assert [n.op_type for n in g.nodes] == ["MatMulNBits", "MatMulNBits"]
    assert g.nodes[0].attributes == {"N": 96, "K": 256, "bits": 4, "block_size": 32}
    assert g.inputs == ["A"] and g.outputs == ["Y1"]
    for nm, (b, s, z, *_rest) in ops.items():
        for t, arr in ((f"{nm}.B", b), (f"{nm}.scales", s), (f"{nm}.zp", z)):
            if arr is None:
                assert t not in g.initializers
                continue
            assert np.array_equal(g.initializers[t], arr) and g.initializers[t].dtype == arr.dtype
            sl = g.sources[t]   # the recorded slice holds exactly the tensor's bytes
            with open(sl.path, "rb") as f:
                f.seek(sl.offset)
                assert f.read(sl.length) == arr.tobytes()
            assert os.path.basename(sl.path) == ("model.onnx.data" if external else "model.onnx")


def test_dtypes_and_typed_lists(tmp_path):
    f16 = np.array([1.5, -2.25, 65504.0], np.float16)
    inits = [W.tensor("f16", f16), W.tensor("f32t", np.array([1.0, 2.5], np.float32), "typed"),
             W.tensor("i64t", np.array([-3, 7], np.int64), "typed"),
             W.tensor("u8t", np.array([1, 255], np.uint8), "typed"),
             W.tensor("bf16", np.array([0x3FC0, 0xC000], np.uint16), "raw", data_type=L.DT_BFLOAT16),
             W.tensor("b", np.array([True, False, True]), "raw")]
    p = tmp_path / "m.onnx"
    p.write_bytes(W.model([], inits, [], [], metadata={"k": "v"}))
    g = L.load_model(str(p))
    I = g.initializers
    assert I["f16"].dtype == np.float16 and np.array_equal(I["f16"], f16)
    assert np.array_equal(I["f32t"], [1.0, 2.5]) and I["i64t"].tolist() == [-3, 7]
    assert I["u8t"].dtype == np.uint8 and I["u8t"].tolist() == [1, 255]
    assert I["bf16"].tolist() == [1.5, -2.0] and I["b"].tolist() == [True, False, True]
    assert g.metadata == {"k": "v"}
    assert "f32t" not in g.sources and "f16" in g.sources


def test_error_messages(tmp_path):
    def load(inits, extra=None):
        p = tmp_path / "e.onnx"
        p.write_bytes(W.model([], inits, [], []))
        return L.load_model(str(p))

    arr = np.arange(8, dtype=np.float32)
    with pytest.raises(ModelSharpException, match="was not found"):
        load([W.tensor("t", arr, "external", ("missing.bin", 0, 32))])
    (tmp_path / "w.bin").write_bytes(arr.tobytes())
    with pytest.raises(ModelSharpException, match=r"slice \[16, 48\) for initializer 't' is out of bounds"):
        load([W.tensor("t", arr, "external", ("w.bin", 16, 32))])
    assert np.array_equal(load([W.tensor("t", arr, "external", ("w.bin", 0, None))]).initializers["t"], arr)
    bad = W.vi(1, 100) + W.vi(2, 1) + W.s(8, "t") + W.ld(9, arr.tobytes())
    with pytest.raises(ModelSharpException, match="declares 100 elements but only 32 are available"):
        load([bad])
    noloc = W.vi(1, 2) + W.vi(2, 1) + W.s(8, "t") + W.vi(14, 1)
    with pytest.raises(ModelSharpException, match="is EXTERNAL but has no 'location'"):
        load([noloc])
    with pytest.raises(ModelSharpException, match="in-memory byte buffer"):
        L.parse_model(W.model([], [W.tensor("t", arr, "external", ("w.bin", 0, 32))], [], []))
    with pytest.raises(ModelSharpException, match=r"no graph \(field 7\)"):
        L.parse_model(W.vi(1, 8))
    with pytest.raises(ModelSharpException, match="Unsupported tensor data_type 13"):
        load([W.vi(1, 1) + W.vi(2, 13) + W.s(8, "u") + W.ld(9, b"\0" * 8)])


def test_truncated_bfloat16_raw_data_is_rejected(tmp_path):
    """A bf16 initializer declaring more elements than its raw bytes hold raises the
    loader's element-count error instead of reading the next fields or tensors of the file
    (the count guard alone, count <= bytes, would let 3 elements read 6 bytes of a 4-byte
    field)."""
    p = tmp_path / "b.onnx"
    raw = np.array([0x3FC0, 0xC000], np.uint16).tobytes()
    bad = W.vi(1, 3) + W.vi(2, L.DT_BFLOAT16) + W.s(8, "h") + W.ld(9, raw)
    after = W.tensor("next", np.arange(4, dtype=np.float32))
    p.write_bytes(W.model([], [bad, after], [], []))
    with pytest.raises(ModelSharpException, match="'h' declares 3 elements but only 2 are available"):
        L.load_model(str(p))
    ok = W.vi(1, 2) + W.vi(2, L.DT_BFLOAT16) + W.s(8, "h") + W.ld(9, raw)
    p.write_bytes(W.model([], [ok, after], [], []))
    assert np.array_equal(L.load_model(str(p)).initializers["h"], np.array([1.5, -2.0], np.float32))
