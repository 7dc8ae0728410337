"""Bounded soak of the launches whose workgroups hand partial sums to each other.

The split-K prefill (two workgroups per tile, flag and slot through device-coherent
memory, possibly on different XCDs), the small-M matrix-core kernel's split K, and the
few-tile prefill's slices and reduce launch: each is called many times in a row on one
stream with no host synchronisation between calls, and every result must be bit-identical
to the first (the hand-offs are ordered, so the sums are deterministic). The comparison
runs on the device and stops at the first mismatch; the handle's device error word must
stay clear (a hand-off that gave up waiting would set it).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from modelsharp_amd import native, workloads

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

# (name, K, N, block size, zero points, M, knobs {knob: value}, calls, expected kernel)
CASES = [
    ("pipe_splitk_whole_round", 11008, 4096, 32, True, 2048, {}, 400, "mfma_w4_pipe"),
    ("pipe_split_last_round", 4096, 11008, 32, True, 2048, {}, 400, "mfma_w4_pipe"),
    ("pipe_splitk_m512", 11008, 4096, 32, True, 512, {}, 1500, "mfma_w4_pipe"),
    ("skinny_splitk4", 11008, 4096, 128, False, 16, {5: 4}, 3000, "skinny_w4"),
    ("skinny_splitk8_bs32", 4096, 11008, 32, True, 8, {5: 8}, 3000, "skinny_w4"),
    ("rb_slices", 4096, 11008, 32, True, 128, {}, 2000, "mfma_w4_rb"),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_split_handoffs_repeat_bitwise(case):
    name, K, N, bs, zp, M, knobs, calls, kernel = case
    if not native.available():
        pytest.skip("no gfx950 device")
    op = workloads.Op(name, K, N, bs, zp, 0.001, 0.01)
    b, s, z = workloads.make_weights(op, 11)
    w = native.NBitsWeights(b, s, z, N, K, 4, bs)
    try:
        if name == "pipe_splitk_m512":
            w.set_tuning(6, 1)   # M=512 K=11008 on the pipelined kernel: 32 tiles, each split in K
        for k, v in knobs.items():
            w.set_tuning(k, v)
        info = w.launch_info(M)
        print(f"{name}: M={M} K={K} N={N} bs={bs} launch {info}, {calls} calls", flush=True)
        assert info["kernel"] == kernel, info
        a = torch.from_numpy(workloads.make_activations(M, K, 5, "rmsnorm" if M > 16 else "normal")).cuda()
        y0 = torch.empty((M, N), dtype=torch.float32, device="cuda")
        y = torch.empty_like(y0)
        stream = torch.cuda.current_stream().cuda_stream
        w.gemm_dev(a.data_ptr(), y0.data_ptr(), M, stream)
        torch.cuda.synchronize()
        w.device_error()
        # the first result is the oracle's product (sampled columns), so the soak compares
        # against a correct value
        cols = np.arange(0, N, max(1, N // 64))
        ref = oracle.matmul_nbits(a.cpu().numpy(), b[cols], s.reshape(N, -1)[cols].ravel(),
                                  None if z is None else z[cols], len(cols), K, 4, bs)
        got = y0.cpu().numpy()[:, cols]
        if M <= 16:
            rowmax = np.max(np.abs(ref), axis=1, keepdims=True)
            assert np.all(np.abs(got - ref) <= 1e-5 * rowmax), name
        else:
            rel = np.linalg.norm((got - ref).astype(np.float64)) / np.linalg.norm(ref.astype(np.float64))
            assert rel <= 2e-3, (name, rel)
        bad = torch.zeros((), dtype=torch.int32, device="cuda")
        first_bad = torch.full((), -1, dtype=torch.int32, device="cuda")
        for i in range(calls):
            w.gemm_dev(a.data_ptr(), y.data_ptr(), M, stream)
            ne = torch.ne(y, y0).any().to(torch.int32)
            first_bad = torch.where((ne > 0) & (first_bad < 0), torch.full_like(first_bad, i), first_bad)
            bad += ne
        torch.cuda.synchronize()
        w.device_error()
        print(f"  {name}: {int(bad)} of {calls} calls differ (first {int(first_bad)})", flush=True)
        assert int(bad) == 0, (name, int(first_bad))
    finally:
        w.close()
