"""The load path from the model file to HBM: ONNX models written with MatMulNBits
initializers inline and in external-data files, loaded by pipeline.load, whose weights
are streamed from the file slices into device handles (ms_hip_nbits_weights_create_from_files)
and must equal handles made from the same arrays in memory, bit for bit."""
from __future__ import annotations

import time

import numpy as np
import pytest

import onnx_writer as W
import oracle
from modelsharp_amd import native, pipeline, workloads

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("external", [False, True])
def test_pipeline_streams_weights_from_the_file(gpu, tmp_path, external):
    import torch
    ops = {}
    specs = [("qkv", workloads.Op("q", 512, 384, 32, True)), ("o", workloads.Op("o", 384, 512, 64, False)),
             ("up", workloads.Op("u", 512, 256, 128, True)), ("down", workloads.Op("d", 256, 96, 32, True, bits=8))]
    for i, (nm, op) in enumerate(specs):
        b, s, z = workloads.make_weights(op, 10 + i)
        if nm == "o":
            s = s.astype(np.float16)   # q4f16 exports keep fp16 scales
        if nm == "up":
            z = np.random.default_rng(i).uniform(0, 15, op.N * op.nb).astype(np.float32)   # float zero points
        ops[nm] = (b, s, z, op.N, op.K, op.bits, op.block_size)
    path = W.write_matmul_nbits_model(str(tmp_path), ops, external)
    eng = pipeline.load(path)
    k = eng.kernels.try_get("MatMulNBits")[1]
    assert k.file_uploads == 4 and k.handle_count == 4
    a = workloads.make_activations(3, 512, seed=1)
    y = eng.run({"A": torch.from_numpy(a).cuda()})["Y3"].cpu().numpy()
    ref = a
    for nm, (b, s, z, N, K, bits, bs) in ops.items():
        zp_packed = z if (z is not None and z.dtype == np.uint8) else None
        zp_float = z if (z is not None and z.dtype == np.float32) else None
        ref = oracle.matmul_nbits(ref, b, s.astype(np.float32), zp_packed, N, K, bits, bs, zp_float=zp_float)
        w = native.NBitsWeights(b, s, z, N, K, bits, bs)
        h = next(e[1] for key, e in k._handles.items() if key[0] == f"{nm}.B")
        assert np.array_equal(h.dequant(), w.dequant()), nm
        w.close()
    err = np.max(np.abs(y - ref)) / np.abs(ref).max()
    log(f"  chain of 4 MatMulNBits from {'external' if external else 'inline'} data: err {err:.2e}")
    assert err <= 1e-5
    k.close()


def test_upload_7b_gate_from_external_data(gpu, tmp_path):
    op = workloads.Op("gate", 4096, 11008, 32, True)
    b, s, z = workloads.make_weights(op, 3)
    path = W.write_matmul_nbits_model(str(tmp_path), {"gate": (b, s, z, op.N, op.K, 4, 32)}, True)
    from modelsharp_amd import onnx_loader
    g = onnx_loader.load_model(path)
    src = [g.sources[n] for n in ("gate.B", "gate.scales", "gate.zp")]
    t0 = time.perf_counter()
    w = native.NBitsWeights.from_files(*src, op.N, op.K, 4, 32)
    dt = time.perf_counter() - t0
    nbytes = sum(x.length for x in src)
    log(f"  streamed {nbytes / 1e6:.1f} MB from the file into HBM in {dt * 1e3:.1f} ms ({nbytes / dt / 1e9:.2f} GB/s)")
    w2 = native.NBitsWeights(b, s, z, op.N, op.K, 4, 32)
    assert np.array_equal(w.dequant(), w2.dequant())
    a = workloads.make_activations(1, op.K, seed=2)
    assert np.array_equal(w.gemm(a), w2.gemm(a))
    w.close()
    w2.close()
