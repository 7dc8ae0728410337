"""Writes the golden fixtures of the MatMulNBits parity tests.

kat_vectors.json
    The eight hand-derived known-answer cases of the reference's
    tests/ModelSharp.Tests/MatMulNBitsTests.cs (:57-267), transcribed as data:
    inputs (A, packed B, scales, zero points, attributes) and the expected Y
    and its shape, with the reference's tolerance 1e-4 (:23).

ref_qgemm_vectors.npz
    Outputs of the reference's own native ms_qgemm_nbits (native/src/qgemm.cpp,
    compiled from source by oracle/Makefile `ref`, without -ffast-math) on
    seeded inputs over a reduced version of its parity grid
    (native/test/qgemm_test.cpp:258-276: M in {1,8}, bits 4 sym/asym, 8 sym/asym,
    block size 32/128), plus one-hot activations A = I_K, for which the
    reference returns its dequantized weights W^T exactly (every output is a
    single product 1*w plus zeros).

ref_w4a8_vectors.npz
    Outputs of the reference's own native ms_qgemm_w4a8 (native/src/qgemm_w4a8.cpp,
    compiled from source by oracle/Makefile `ref` with -ffp-contract=off) on seeded
    inputs over a reduced version of its accuracy grid
    (native/test/qgemm_w4a8_test.cpp:140-166: M in {1, 8}, bits 4 sym/asym and 8
    sym/asym, block size 32/128, and its three odd shapes).

onnx/
    The reference's own ONNX test assets (tests/ModelSharp.Tests/assets:
    test_matmul_{2d,3d,4d}/ with their test_data_set_0 tensors, and mnist-12.onnx),
    copied as data for the loader tests; read only by the repository's own parser.

Run in the container that holds the reference checkout:
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))


def pack4(lo: int, hi: int) -> int:
    return (lo & 0xF) | ((hi & 0xF) << 4)


def kat_cases() -> list[dict]:
    b_default = [pack4(8, 9), pack4(7, 10), pack4(0, 15), pack4(8, 4)]
    return [
        dict(name="Bits4_DefaultZeroPoint_SingleBlock", a_shape=[1, 4], a=[1, 2, 3, 4],
             b_shape=[2, 1, 2], b=b_default, scales=[2.0, 0.5], zp=None, zp_dtype=None,
             attrs=dict(N=2, K=4, bits=4, block_size=4), y_shape=[1, 2], y=[14.0, -5.0]),
        dict(name="Bits4_DefaultZeroPoint_TwoBlocks_PerBlockScale", a_shape=[1, 8], a=[1, 2, 3, 4, 5, 6, 7, 8],
             b_shape=[2, 2, 2],
             b=[pack4(8, 10), pack4(8, 8), pack4(8, 8), pack4(12, 8),
                pack4(9, 8), pack4(8, 7), pack4(8, 8), pack4(8, 15)],
             scales=[1.0, 2.0, 0.5, 1.0], zp=None, zp_dtype=None,
             attrs=dict(N=2, K=8, bits=4, block_size=4), y_shape=[1, 2], y=[60.0, 54.5]),
        dict(name="Bits4_PackedZeroPoints", a_shape=[1, 4], a=[1, 2, 3, 4], b_shape=[2, 1, 2], b=b_default,
             scales=[2.0, 0.5], zp=[pack4(6, 0), pack4(10, 0)], zp_dtype="uint8",
             attrs=dict(N=2, K=4, bits=4, block_size=4), y_shape=[1, 2], y=[54.0, -15.0]),
        dict(name="Bits4_FloatZeroPoints", a_shape=[1, 4], a=[1, 2, 3, 4], b_shape=[2, 1, 2], b=b_default,
             scales=[2.0, 0.5], zp=[6.0, 10.0], zp_dtype="float32",
             attrs=dict(N=2, K=4, bits=4, block_size=4), y_shape=[1, 2], y=[54.0, -15.0]),
        dict(name="Bits4_BatchedA", a_shape=[2, 4], a=[1, 2, 3, 4, 2, 0, 1, 0], b_shape=[2, 1, 2], b=b_default,
             scales=[2.0, 0.5], zp=None, zp_dtype=None,
             attrs=dict(N=2, K=4, bits=4, block_size=4), y_shape=[2, 2], y=[14.0, -5.0, -2.0, -8.0]),
        dict(name="Bits4_ThreeDimA_PreservesLeadingDims", a_shape=[2, 1, 4], a=[1, 2, 3, 4, 2, 0, 1, 0],
             b_shape=[2, 1, 2], b=b_default, scales=[2.0, 0.5], zp=None, zp_dtype=None,
             attrs=dict(N=2, K=4, bits=4, block_size=4), y_shape=[2, 1, 2], y=[14.0, -5.0, -2.0, -8.0]),
        dict(name="Bits4_KNotMultipleOfBlockSize", a_shape=[1, 6], a=[1, 2, 3, 4, 5, 6], b_shape=[1, 2, 2],
             b=[pack4(8, 9), pack4(8, 7), pack4(10, 8), pack4(6, 6)], scales=[1.0, 2.0], zp=None, zp_dtype=None,
             attrs=dict(N=1, K=6, bits=4, block_size=4), y_shape=[1, 1], y=[18.0]),
        dict(name="Bits8_DefaultZeroPoint", a_shape=[1, 4], a=[1, 2, 3, 4], b_shape=[2, 1, 4],
             b=[128, 130, 126, 132, 120, 128, 140, 128], scales=[2.0, 0.5], zp=None, zp_dtype=None,
             attrs=dict(N=2, K=4, bits=8, block_size=4), y_shape=[1, 2], y=[28.0, 14.0]),
    ]


# (M, N, K) x block size x (bits, asym): a reduced grid of qgemm_test.cpp:258-276.
GRID_SHAPES = [(1, 64, 128), (8, 48, 256)]
GRID_BS = [32, 128]
GRID_MODES = [(4, False), (4, True), (8, False), (8, True)]
# one-hot dequant probes: (N, K, bits, block_size, asym)
ONEHOT = [(40, 128, 4, 32, True), (24, 256, 4, 128, False), (16, 96, 8, 32, True), (12, 100, 4, 32, True)]


def ref_vectors() -> dict:
    import oracle
    from modelsharp_amd import workloads

    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libms_ref_qgemm.so is not built (make -C oracle ref)")
    out = {}
    seed = 100
    for (M, N, K) in GRID_SHAPES:
        for bs in GRID_BS:
            for bits, asym in GRID_MODES:
                seed += 1
                op = workloads.Op("grid", K, N, bs, asym, 0.005, 0.05, bits)
                b, s, z = workloads.make_weights(op, seed)
                a = workloads.make_activations(M, K, seed + 1000)
                y = oracle.ref_qgemm_nbits(a, b, s, z, M, N, K, bits, bs)
                key = f"grid_M{M}_N{N}_K{K}_bits{bits}_bs{bs}_{'asym' if asym else 'sym'}"
                out.update({f"{key}/a": a, f"{key}/b": b, f"{key}/scales": s, f"{key}/y": y,
                            f"{key}/dims": np.array([M, N, K, bits, bs], np.int32)})
                if z is not None:
                    out[f"{key}/zp"] = z
    for (N, K, bits, bs, asym) in ONEHOT:
        seed += 1
        op = workloads.Op("onehot", K, N, bs, asym, 0.005, 0.05, bits)
        b, s, z = workloads.make_weights(op, seed)
        eye = np.eye(K, dtype=np.float32)
        y = oracle.ref_qgemm_nbits(eye, b, s, z, K, N, K, bits, bs)   # y[k, n] = W[n, k]
        key = f"onehot_N{N}_K{K}_bits{bits}_bs{bs}_{'asym' if asym else 'sym'}"
        out.update({f"{key}/b": b, f"{key}/scales": s, f"{key}/w": np.ascontiguousarray(y.T),
                    f"{key}/dims": np.array([N, K, bits, bs], np.int32)})
        if z is not None:
            out[f"{key}/zp"] = z
    return out


W4A8_SHAPES = [(1, 64, 128), (8, 40, 512)]
W4A8_ODD = [(1, 16, 4000, 4, 128, False), (8, 9, 320, 4, 128, True), (32, 130, 200, 8, 128, False),
            (5, 65, 128, 4, 32, True), (13, 257, 128, 8, 32, False)]


def ref_w4a8_vectors() -> dict:
    import oracle
    from modelsharp_amd import workloads

    if oracle.ref_w4a8_lib() is None:
        raise SystemExit("oracle/_ref/libms_ref_w4a8.so is not built (make -C oracle ref)")
    cases = [(M, N, K, bits, bs, asym) for (M, N, K) in W4A8_SHAPES for bs in GRID_BS
             for bits, asym in GRID_MODES] + W4A8_ODD
    out = {}
    seed = 500
    for (M, N, K, bits, bs, asym) in cases:
        seed += 1
        op = workloads.Op("w4a8", K, N, bs, asym, 0.005, 0.05, bits)
        b, s, z = workloads.make_weights(op, seed)
        a = workloads.make_activations(M, K, seed + 1000, kind="rmsnorm" if seed % 2 else "normal")
        y = oracle.ref_qgemm_w4a8(a, b, s, z, M, N, K, bits, bs)
        key = f"w4a8_M{M}_N{N}_K{K}_bits{bits}_bs{bs}_{'asym' if asym else 'sym'}"
        out.update({f"{key}/a": a, f"{key}/b": b, f"{key}/scales": s, f"{key}/y": y,
                    f"{key}/dims": np.array([M, N, K, bits, bs], np.int32)})
        if z is not None:
            out[f"{key}/zp"] = z
    return out


def main() -> None:
    (HERE / "kat_vectors.json").write_text(json.dumps(
        {"source": "tests/ModelSharp.Tests/MatMulNBitsTests.cs:57-267", "tolerance": 1e-4,
         "cases": kat_cases()}, indent=1))
    vec = ref_vectors()
    np.savez_compressed(HERE / "ref_qgemm_vectors.npz", **vec)
    w4a8 = ref_w4a8_vectors()
    np.savez_compressed(HERE / "ref_w4a8_vectors.npz", **w4a8)
    print(f"wrote {len(kat_cases())} KATs, {len(vec)} reference arrays and {len(w4a8)} W4A8 arrays")


if __name__ == "__main__":
    main()
