"""Device parity for the weight formats outside the 4-bit fast kernels, against the
oracle (the managed kernel's arithmetic, MatMulNBitsKernel.cs:193-262):

* 8-bit codes (MatMulNBitsSimd.cs:117-132), float zero points
  (MatMulNBitsKernel.cs:239-240), block sizes other than 32/64/128/256, K not a
  multiple of 32 — the general GEMV (M <= 16) and the general MFMA GEMM (M > 16);
* the 8-bit decode GEMV (packed or default zero points, power-of-two block sizes
  >= 16, K % 16 == 0, M <= 4): every launch configuration, the K % block-size tail,
  blocks longer than one step, activation panels above 64 KiB of LDS;
* Float16 scales, zero points and activations, widened exactly on the device as
  GraphContext.Get widens them on the host (GraphContext.cs:106): the results equal
  those of the same values handed over as Float32, bit for bit.

Tolerances: the dequantized weights are bit-exact; the GEMV sums the same fp32 products
in another order, so each output lies within 2*gamma_K * sum_k |a_k w_nk| of the
oracle's; the MFMA GEMM multiplies fp16 hi/lo splits of A and W (each split exact to
2^-22 relative, below 2^-24 of the row's largest element absolute) and sums in fp32, so
each output lies within 4*(2*gamma_K) + 2^-20 of sum_k |a_k w_nk| plus 2^-30 of
max_k |a_k| * sum_k |w_nk|.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from modelsharp_amd import native, workloads
from modelsharp_amd.workloads import Op

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


def float_zero_points(op: Op, seed: int) -> np.ndarray:
    """Per-block float zero points in [0, 2^bits - 1], with fractional parts."""
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.uniform(0.0, float((1 << op.bits) - 1), size=op.N * op.nb).astype(np.float32)


def dot_abs(a, W):
    return np.abs(a).astype(np.float64) @ np.abs(W).astype(np.float64).T


def gamma2(K):
    u = np.finfo(np.float32).eps / 2
    return 2 * K * u / (1 - K * u)


def assert_within(y, ref, allowed, what):
    err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
    ratio = float(np.max(err / np.maximum(allowed, 1e-300)))
    log(f"  {what}: max err / bound {ratio:.3e}")
    assert np.all(err <= allowed), f"{what}: err/bound {ratio:.3e}"


def expected_kernel(op: Op, M: int, float_zp: bool = False, fp16_scales: bool = True, skinny: bool = True) -> str:
    """The kernel the dispatch rules give a call with M rows (fp16_scales: every nonzero
    |scale| lies in [2^-14, 256], as make_weights draws them; skinny=False: knob 4 = 1)."""
    pow2 = op.block_size >= 16 and (op.block_size & (op.block_size - 1)) == 0
    gemv8 = (op.bits == 8 and not float_zp and pow2 and op.K % 16 == 0 and M <= 4
             and M * op.K * 4 <= 159 * 1024)
    low = 3 if op.block_size == 128 else 4   # the default takes 8-bit M <= 4 from here
    if (skinny and op.bits == 8 and not float_zp and op.block_size in (32, 64, 128) and op.K % 128 == 0
            and (5 <= M <= 16 or (3 <= M <= 4 and (not gemv8 or M >= low)))):
        return "skinny_w4"
    if gemv8:
        return "gemv_w8"
    if (op.bits == 8 and not float_zp and pow2 and op.block_size >= 32 and op.K % 128 == 0 and M > 16
            and fp16_scales):
        return "mfma_w4_pipe" if op.block_size == 32 and pipe_over_rb(M, op.N, op.K) else "mfma_w4_rb"
    return "gemv_general" if M <= 16 else "mfma_general"


def pipe_items(M, N, K, ksplit=0):
    """Work items of a pipelined prefill launch on 256 CUs (ksplit: knob 3; 0 the default
    rule: every tile K-split when the tiles fill at most half of the CUs, else the tiles of
    a last round that would; 1 none; 2 all; 3 the second half)."""
    tiles = -(-M // 256) * -(-N // 256)
    full = tiles
    if K // 128 >= 2:
        if ksplit == 2 or (ksplit == 0 and 2 * tiles <= 256):
            full = 0
        elif ksplit == 3:
            full = tiles // 2
        elif ksplit == 0 and 0 < tiles % 256 <= 128:
            full = tiles - tiles % 256
    return full, tiles


def pipe_over_rb(M, N, K):
    """The library's choice of the pipelined kernel over mfma_w4_rb: more than one 128-row
    tile of A, and work items that fill at least half of the 256 CUs."""
    full, tiles = pipe_items(M, N, K)
    return M > 128 and 2 * (full + 2 * (tiles - full)) >= 256


def pipe_grid(M, N, K, ksplit):
    """The pipelined launch's grid: 8 XCDs x (whole tiles per XCD + two halves per split
    tile per XCD)."""
    full, tiles = pipe_items(M, N, K, ksplit)
    return 8 * (-(-full // 8) + 2 * -(-(tiles - full) // 8))


def check_against_oracle(w, a, b, s, zp, zpf, op, what):
    M = a.shape[0]
    kernel = w.launch_info(M)["kernel"]
    y = w.gemm(a)
    ref = oracle.matmul_nbits(a, b, s, zp, op.N, op.K, op.bits, op.block_size, zp_float=zpf)
    W = oracle.dequant_weights(b, s, zp, op.N, op.K, op.bits, op.block_size, zp_float=zpf)
    cond = dot_abs(a, W)
    if kernel == "mfma_general":
        allowed = (4 * gamma2(op.K) + 2.0 ** -20) * cond + 2.0 ** -30 * (
            np.max(np.abs(a), axis=1, keepdims=True).astype(np.float64) * np.abs(W).sum(axis=1)[None, :])
    elif kernel in ("mfma_w4_rb", "mfma_w4_pipe"):
        # fp16 prefill numerics: A rounded once to fp16 after its row's power-of-two scaling
        # (2^-11 relative; below the fp16 normal range, 2^-39 of the row's max absolute)
        # and W = fl16((q - zp) fl16(s)) (2^-10 relative: fl16(s) and the product), exact
        # products, fp32 sums; and the relative Frobenius tolerance of the prefill path, 2e-3.
        allowed = (2.0 ** -11 + 2.0 ** -10 + 2.0 ** -20 + gamma2(op.K)) * 1.01 * cond + 2.0 ** -30 * (
            np.max(np.abs(a), axis=1, keepdims=True).astype(np.float64) * np.abs(W).sum(axis=1)[None, :])
        rel = float(np.linalg.norm(y.astype(np.float64) - ref) / max(np.linalg.norm(ref.astype(np.float64)), 1e-300))
        log(f"  {what}: relative Frobenius error {rel:.3e}")
        assert rel <= 2e-3, f"{what}: rel_fro {rel:.3e}"
    elif kernel == "skinny_w4":
        # the small-M matrix-core kernel: A as 2^e (hi + lo) per (row, 128-k block), exact to
        # 2^-22 of the block's max |a| (so within 2^-22 of the row's), exact products and
        # fp32 sums of the MFMA steps, the blocks and the scales
        allowed = 2 * gamma2(op.K) * cond + 2.0 ** -21 * (
            np.max(np.abs(a), axis=1, keepdims=True).astype(np.float64) * np.abs(W).sum(axis=1)[None, :])
    else:
        allowed = gamma2(op.K) * cond
    assert_within(y, ref, allowed, f"{what} [{kernel}]")
    return kernel, W


FORMATS = [
    Op("b8_zp", 512, 72, 32, True, bits=8),
    Op("b8_sym_bs128", 1024, 40, 128, False, bits=8),
    Op("b8_bs24_tail", 264, 20, 24, True, bits=8),      # 11 blocks of 24
    Op("b4_bs16", 256, 50, 16, True),
    Op("b4_bs48", 480, 33, 48, True),
    Op("b4_k1000_bs40", 1000, 64, 40, True),            # K % 32 != 0
    Op("b4_k1000_bs32_tail", 1000, 70, 32, False),      # partial last block of 8
]
MS = [1, 3, 16, 17, 40, 130]


@pytest.mark.parametrize("op", FORMATS, ids=lambda o: o.name)
@pytest.mark.parametrize("M", MS)
def test_general_formats(gpu, op, M):
    b, s, z = workloads.make_weights(op, seed=op.K + op.N + M)
    a = workloads.make_activations(M, op.K, seed=3 * M + op.N)
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    log(f"general {op.name} M={M} {w.launch_info(M)}")
    kernel, W = check_against_oracle(w, a, b, s, z, None, op, f"{op.name} M={M}")
    assert kernel == expected_kernel(op, M)
    assert np.array_equal(w.dequant(), W)
    w.close()


FLOAT_ZP = [
    Op("fzp_b4_bs32", 512, 96, 32, True),
    Op("fzp_b4_bs128", 2048, 64, 128, True),
    Op("fzp_b8_bs64", 640, 48, 64, True, bits=8),
    Op("fzp_b4_bs40", 1000, 30, 40, True),
]


@pytest.mark.parametrize("op", FLOAT_ZP, ids=lambda o: o.name)
@pytest.mark.parametrize("M", [1, 7, 16, 33, 200])
def test_float_zero_points(gpu, op, M):
    b, s, _ = workloads.make_weights(op, seed=op.K * 3 + M)
    zpf = float_zero_points(op, seed=op.N + M)
    a = workloads.make_activations(M, op.K, seed=M + 11)
    w = native.NBitsWeights(b, s, zpf, op.N, op.K, op.bits, op.block_size)
    log(f"float zp {op.name} M={M} {w.launch_info(M)}")
    kernel, W = check_against_oracle(w, a, b, s, None, zpf, op, f"{op.name} M={M}")
    assert kernel == expected_kernel(op, M, float_zp=True)
    assert np.array_equal(w.dequant(), W)
    w.close()


def test_general_mfma_full_size_8bit(gpu):
    """8-bit weights at a 7B projection's shape (K=4096, N=4096) over 128 rows (the fp16
    prefill kernel) and over one row (the 8-bit GEMV)."""
    op = Op("b8_7b", 4096, 4096, 32, True, bits=8)
    b, s, z = workloads.make_weights(op, seed=5)
    a = workloads.make_activations(128, op.K, seed=6, kind="rmsnorm")
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    log(f"8-bit 4096x4096 M=128 {w.launch_info(128)}")
    kernel, _ = check_against_oracle(w, a, b, s, z, None, op, "b8 K=4096 N=4096 M=128")
    assert kernel == "mfma_w4_rb"
    y1 = w.gemm(a)
    assert np.array_equal(y1, w.gemm(a))   # deterministic
    a1 = a[:1]
    kernel, _ = check_against_oracle(w, a1, b, s, z, None, op, "b8 K=4096 N=4096 M=1")
    assert kernel == "gemv_w8"
    w.close()


# ---- 8-bit decode GEMV ---------------------------------------------------------------------
W8_OPS = [
    Op("w8_gate_7b", 4096, 11008, 32, True, bits=8),     # 7B gate/up projection
    Op("w8_down_7b", 11008, 4096, 32, True, bits=8),     # panel staged in a loop (K = 11008)
    Op("w8_sym_bs16", 1024, 300, 16, False, bits=8),     # default zero point 128
    Op("w8_bs64_tail", 1040, 77, 64, True, bits=8),      # 17 blocks, the last of 16 codes
    Op("w8_bs512", 2048, 130, 512, True, bits=8),        # a block spans several steps
    Op("w8_k16", 16, 40, 16, True, bits=8),              # one chunk per row
    Op("w8_k8192", 8192, 96, 128, True, bits=8),         # M = 3, 4: 96 / 128 KiB of LDS
]


@pytest.mark.parametrize("op", W8_OPS, ids=lambda o: o.name)
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_gemv_w8(gpu, op, M):
    b, s, z = workloads.make_weights(op, seed=op.K + 7 * op.N + M)
    a = workloads.make_activations(M, op.K, seed=5 * M + op.K, kind="rmsnorm")
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    log(f"gemv_w8 {op.name} M={M} {w.launch_info(M)}")
    kernel, _ = check_against_oracle(w, a, b, s, z, None, op, f"{op.name} M={M}")
    assert kernel == expected_kernel(op, M)
    y = w.gemm(a)
    assert np.array_equal(y, w.gemm(a))   # deterministic
    if kernel == "skinny_w4":   # the 8-bit GEMV itself, with the small-M matrix-core kernel off
        w.set_tuning(4, 1)
        kernel, _ = check_against_oracle(w, a, b, s, z, None, op, f"{op.name} M={M} knob 4 = 1")
        assert kernel == expected_kernel(op, M, skinny=False)
        w.set_tuning(4, 0)
    w.close()


@pytest.mark.parametrize("M", [1, 4])
def test_gemv_w8_every_config(gpu, M):
    """Every launch configuration of the 8-bit GEMV (forced through tuning knob 11) on a
    shape whose rows do not fill the last workgroup; knob value -1 keeps the call on the
    general GEMV."""
    op = Op("w8_cfg", 2560, 1000, 64, True, bits=8)
    b, s, z = workloads.make_weights(op, seed=31 + M)
    a = workloads.make_activations(M, op.K, seed=32 + M)
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    try:
        for cfg in range(1, 10):
            w.set_tuning(11, cfg)
            info = w.launch_info(M)
            log(f"gemv_w8 config {cfg - 1} M={M} {info}")
            assert info["kernel"] == "gemv_w8"
            check_against_oracle(w, a, b, s, z, None, op, f"config {cfg - 1} M={M}")
        w.set_tuning(11, -1)
        assert w.launch_info(M)["kernel"] == "gemv_general"
        check_against_oracle(w, a, b, s, z, None, op, f"knob -1 M={M}")
    finally:
        w.set_tuning(11, 0)
    w.close()


def test_gemv_w8_extreme_codes(gpu):
    """Codes and zero points at 0 and 255 (q - zp = +-255, the widest difference), on the
    8-bit GEMV and (M = 4, by default) the small-M matrix-core kernel."""
    op = Op("w8_ext", 512, 64, 32, True, bits=8)
    rng = np.random.Generator(np.random.PCG64(77))
    b = rng.choice(np.array([0, 255], dtype=np.uint8), size=(op.N, op.nb, op.blob))
    z = rng.choice(np.array([0, 255], dtype=np.uint8), size=(op.N, op.zrb))
    s = rng.uniform(op.scale_lo, op.scale_hi, size=op.N * op.nb).astype(np.float32)
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    try:
        for M in (1, 4):
            a = workloads.make_activations(M, op.K, seed=M)
            for knob in (0, 1):
                w.set_tuning(4, knob)
                kernel, _ = check_against_oracle(w, a, b, s, z, None, op, f"extreme codes M={M} knob 4 = {knob}")
                assert kernel == expected_kernel(op, M, skinny=knob == 0)
    finally:
        w.set_tuning(4, 0)
    w.close()


def test_dynamic_range_general_mfma(gpu):
    """Rows of A and W scaled over 2^-40 .. 2^40: the per-row power-of-two splits keep
    every row at fp32-level accuracy."""
    op = Op("range", 512, 64, 32, True, bits=8)
    b, s, z = workloads.make_weights(op, seed=21)
    s = (s.reshape(op.N, op.nb) * np.float32(2.0) ** np.arange(-32, 32, dtype=np.float32)[:, None]).reshape(-1)
    s = s.astype(np.float32)
    a = workloads.make_activations(48, op.K, seed=22)
    a = (a * np.float32(2.0) ** np.linspace(-40, 40, 48).round().astype(np.float32)[:, None]).astype(np.float32)
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    kernel, _ = check_against_oracle(w, a, b, s, z, None, op, "range M=48")
    assert kernel == "mfma_general"
    w.close()


# ---- Float16 inputs ------------------------------------------------------------------------
F16_OPS = [Op("f16_fast", 4096, 256, 32, True), Op("f16_fast_bs128", 2048, 192, 128, False),
           Op("f16_b8", 512, 64, 32, True, bits=8)]


@pytest.mark.parametrize("op", F16_OPS, ids=lambda o: o.name)
def test_f16_scales_equal_widened(gpu, op):
    b, s, z = workloads.make_weights(op, seed=op.N)
    s16 = s.astype(np.float16)
    w16 = native.NBitsWeights(b, s16, z, op.N, op.K, op.bits, op.block_size)
    w32 = native.NBitsWeights(b, s16.astype(np.float32), z, op.N, op.K, op.bits, op.block_size)
    assert np.array_equal(w16.dequant(), w32.dequant())
    for M in (1, 8, 64):
        a = workloads.make_activations(M, op.K, seed=M)
        log(f"f16 scales {op.name} M={M} {w16.launch_info(M)}")
        assert np.array_equal(w16.gemm(a), w32.gemm(a)), f"{op.name} M={M}"
    w16.close()
    w32.close()


def test_f16_zero_points_equal_widened(gpu):
    op = Op("f16_zp", 512, 40, 32, True)
    b, s, _ = workloads.make_weights(op, seed=3)
    z16 = float_zero_points(op, seed=4).astype(np.float16)
    w16 = native.NBitsWeights(b, s, z16, op.N, op.K, op.bits, op.block_size)
    w32 = native.NBitsWeights(b, s, z16.astype(np.float32), op.N, op.K, op.bits, op.block_size)
    assert np.array_equal(w16.dequant(), w32.dequant())
    for M in (1, 20):
        a = workloads.make_activations(M, op.K, seed=M + 1)
        assert np.array_equal(w16.gemm(a), w32.gemm(a))
    w16.close()
    w32.close()


@pytest.mark.parametrize("op", F16_OPS, ids=lambda o: o.name)
def test_f16_activations_equal_widened(gpu, op):
    import torch
    b, s, z = workloads.make_weights(op, seed=op.K)
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    dev = torch.device("cuda", 0)
    for M in (1, 5, 16, 64, 300):
        a16 = torch.from_numpy(workloads.make_activations(M, op.K, seed=M + 2)).to(torch.float16).to(dev)
        a32 = a16.float().contiguous()
        y16 = torch.empty((M, op.N), dtype=torch.float32, device=dev)
        y32 = torch.empty_like(y16)
        log(f"f16 A {op.name} M={M} {w.launch_info(M)}")
        w.gemm_dev_f16(a16.data_ptr(), y16.data_ptr(), M)
        w.gemm_dev(a32.data_ptr(), y32.data_ptr(), M)
        torch.cuda.synchronize()
        assert torch.equal(y16, y32), f"{op.name} M={M}"
    w.close()


def test_operator_routes_float16_and_float_zero_points(gpu):
    """The operator mirror runs Float16 scales, float zero points and Float16
    activations on the device and matches the oracle on the widened values."""
    import torch
    from modelsharp_amd.graph import GraphContext, GraphNode
    from modelsharp_amd.hip_kernel import HipMatMulNBitsKernel

    op = Op("op_f16", 640, 56, 64, True)
    b, s, _ = workloads.make_weights(op, seed=8)
    s16 = s.astype(np.float16)
    zpf = float_zero_points(op, seed=9)
    a16 = workloads.make_activations(24, op.K, seed=10).astype(np.float16)
    node = GraphNode("MatMulNBits", "n0", ["A", "B", "scales", "zp"], ["Y"],
                     {"N": op.N, "K": op.K, "bits": 4, "block_size": op.block_size})
    k = HipMatMulNBitsKernel()
    ctx = GraphContext({"A": torch.from_numpy(a16).cuda(), "B": b, "scales": s16, "zp": zpf})
    k.execute(node, ctx)
    y = ctx.get_tensor("Y").cpu().numpy()
    a32 = a16.astype(np.float32)
    ref = oracle.matmul_nbits(a32, b, s16.astype(np.float32), None, op.N, op.K, 4, op.block_size, zp_float=zpf)
    W = oracle.dequant_weights(b, s16.astype(np.float32), None, op.N, op.K, 4, op.block_size, zp_float=zpf)
    allowed = (4 * gamma2(op.K) + 2.0 ** -20) * dot_abs(a32, W) + 2.0 ** -30 * (
        np.max(np.abs(a32), axis=1, keepdims=True).astype(np.float64) * np.abs(W).sum(axis=1)[None, :])
    assert_within(y, ref, allowed, "operator f16 / float zp M=24")
    k.close()


# ---- 8-bit prefill on the fp16 matrix cores -----------------------------------------------
B8_PREFILL = [
    Op("b8p_bs32_zp", 1024, 1000, 32, True, bits=8),     # ragged N (not a multiple of the tiles)
    Op("b8p_bs64_sym", 2048, 600, 64, False, bits=8),    # default zero point 128
    Op("b8p_bs128_zp", 1536, 384, 128, True, bits=8),
    Op("b8p_bs256_zp", 2304, 256, 256, True, bits=8),    # K % 256 != 0: a partial last block
]


@pytest.mark.parametrize("op", B8_PREFILL, ids=lambda o: o.name)
@pytest.mark.parametrize("M", [17, 130, 300])
def test_prefill_8bit(gpu, op, M):
    b, s, z = workloads.make_weights(op, seed=op.N + M)
    a = workloads.make_activations(M, op.K, seed=M + 5, kind="rmsnorm")
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    log(f"8-bit prefill {op.name} M={M} {w.launch_info(M)}")
    kernel, _ = check_against_oracle(w, a, b, s, z, None, op, f"{op.name} M={M}")
    assert kernel == "mfma_w4_rb"
    assert np.array_equal(w.gemm(a), w.gemm(a))   # deterministic
    w.close()


def test_prefill_8bit_every_split(gpu):
    """Every tile width and K split of the 8-bit prefill (knobs 9 and 7); the pipelined
    kernel when it is switched off (knob 6 = 1), and the exact general kernel when both are
    (knob 2 = 1) or when a scale is outside the fp16 range (|s| > 256)."""
    op = Op("b8p_split", 2048, 520, 32, True, bits=8)
    b, s, z = workloads.make_weights(op, seed=41)
    a = workloads.make_activations(96, op.K, seed=42, kind="rmsnorm")
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    try:
        for nf in (1, 2, 4):            # 4 is not instantiated for 8-bit codes: the pick is used
            for ksw in (1, 3, 16):
                w.set_tuning(9, nf)
                w.set_tuning(7, ksw)
                log(f"8-bit prefill nf={nf} ksw={ksw} {w.launch_info(96)}")
                kernel, _ = check_against_oracle(w, a, b, s, z, None, op, f"nf={nf} ksw={ksw}")
                assert kernel == "mfma_w4_rb"
        w.set_tuning(9, 0)
        w.set_tuning(7, 0)
        w.set_tuning(6, 1)
        kernel, _ = check_against_oracle(w, a, b, s, z, None, op, "rb off")
        assert kernel == "mfma_w4_pipe"   # block size 32: the pipelined kernel's 8-bit form
        w.set_tuning(2, 1)
        kernel, _ = check_against_oracle(w, a, b, s, z, None, op, "rb and pipe off")
        assert kernel == "mfma_general"
    finally:
        w.set_tuning(9, 0)
        w.set_tuning(7, 0)
        w.set_tuning(6, 0)
        w.set_tuning(2, 0)
    w.close()
    s_big = s.copy()
    s_big[7] = np.float32(300.0)        # 255 * 300 overflows fp16
    w = native.NBitsWeights(b, s_big, z, op.N, op.K, op.bits, op.block_size)
    kernel, _ = check_against_oracle(w, a, b, s_big, z, None, op, "scale 300")
    assert kernel == "mfma_general"
    w.close()


# ---- 8-bit codes on the pipelined prefill kernel -------------------------------------------
@pytest.mark.parametrize("zp", [True, False], ids=["zp", "default_zp"])
@pytest.mark.parametrize("M", [17, 33, 100, 129, 300])
def test_prefill_8bit_pipelined_partial_tiles(gpu, M, zp):
    """The pipelined kernel's 8-bit form (mfma_w4_rb, which these small launches take by
    default, switched off: knob 6) on tiles cut by M and N (N=333 is not a multiple of 256;
    K=896 is 7 groups of 4 steps, so the two K halves are unequal), with no, every and half
    of its tiles K-split (knob 3), against the oracle at the prefill bar; without zero
    points the codes are centred on 128."""
    op = Op("b8pp", 896, 333, 32, zp, bits=8)
    b, s, z = workloads.make_weights(op, seed=M + 3)
    a = workloads.make_activations(M, op.K, seed=M + 4, kind="rmsnorm")
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    try:
        w.set_tuning(6, 1)
        for ks in (1, 2, 3):
            w.set_tuning(3, ks)
            info = w.launch_info(M)
            log(f"8-bit pipelined M={M} zp={zp} ksplit={ks} {info}")
            assert info["kernel"] == "mfma_w4_pipe" and info["grid"] == pipe_grid(M, op.N, op.K, ks), info
            check_against_oracle(w, a, b, s, z, None, op, f"8-bit pipelined ksplit={ks} M={M}")
    finally:
        w.set_tuning(3, 0)
        w.set_tuning(6, 0)
    w.close()


B8_PIPE_FULL = [(Op("b8_up", 4096, 11008, 32, True, bits=8), 2048),
                (Op("b8_down", 11008, 4096, 32, True, bits=8), 2048),
                (Op("b8_up", 4096, 11008, 32, True, bits=8), 512),
                (Op("b8_up_sym", 4096, 11008, 32, False, bits=8), 300)]


@pytest.mark.parametrize("op,M", B8_PIPE_FULL, ids=lambda v: str(v) if isinstance(v, int) else v.name)
def test_prefill_8bit_pipelined_full_size(gpu, op, M):
    """8-bit codes at the Llama-2-7B MLP shapes on the library's own choice (the pipelined
    kernel; K=11008 with its tiles K-split at M=2048), with activation outliers of 1e5 and
    -3e6 and rows near 1e-6: every output finite, relative Frobenius error <= 2e-3 against
    the oracle on 96 sampled columns (the rows near 1e-6 on their own too), and bit-identical
    on a second call."""
    b, s, z = workloads.make_weights(op, seed=M + op.K)
    rng = np.random.default_rng(M + 1)
    a = workloads.make_activations(M, op.K, seed=M + 2, kind="rmsnorm")
    rows = rng.permutation(M)
    big, tiny = rows[:4], rows[4:8]
    for i, r in enumerate(big):
        a[r, rng.integers(op.K)] = (1e5 if i % 2 == 0 else -3e6)
    a[tiny] *= np.float32(1e-6)
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    info = w.launch_info(M)
    log(f"8-bit pipelined full size {op.name} M={M} K={op.K} N={op.N} {info}")
    assert info["kernel"] == "mfma_w4_pipe" == expected_kernel(op, M), info
    y = w.gemm(a)
    assert np.all(np.isfinite(y))
    cols = np.sort(rng.choice(op.N, 96, replace=False))
    ref = oracle.matmul_nbits(a, b[cols], s.reshape(op.N, -1)[cols], None if z is None else z[cols], len(cols),
                              op.K, op.bits, op.block_size)
    for sel, what in ((slice(None), "all rows"), (tiny, "rows near 1e-6")):
        got, exp = y[sel][:, cols].astype(np.float64), ref[sel].astype(np.float64)
        rel = float(np.linalg.norm(got - exp) / np.linalg.norm(exp))
        log(f"  {what}: relative Frobenius error {rel:.3e}")
        assert rel <= 2e-3, what
    assert np.array_equal(w.gemm(a), y)
    w.close()


# (K, knob 5): K=640 is 5 blocks of 128 k, split 5 ways (the in-kernel hand-off) or 2;
# K=512 in one workgroup per row tile; K=1408 (11 blocks) split wider than the hand-off
# takes: partial-sum slices and the reduce launch.
B8_SKINNY_SPLITS = [(640, 0), (640, 2), (512, 1), (1408, 0)]


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("K,ksw", B8_SKINNY_SPLITS, ids=lambda v: str(v))
@pytest.mark.parametrize("zp", [False, True], ids=["nozp", "zp"])
def test_skinny_8bit(gpu, zp, K, ksw, bs):
    """The small-M matrix-core kernel on 8-bit codes for every M in 1..16 (below M = 5 forced
    by knob 4 = 2), ragged N, codes and zero points spanning 0..255 (|q - zp| up to 255,
    still exact in fp16), activations spanning 1e-4..1e5 across rows with one outlier; two
    calls agree bit for bit. Block size 128 applies the scale per 128-k block, 64 and 32 per
    32-k step after the transpose of the code dword pairs across the wave's rows."""
    op = Op("sk8", K, 333, bs, zp, bits=8)
    b, s, z = workloads.make_weights(op, seed=90 + bs + zp)
    rng = np.random.default_rng(91)
    b = rng.integers(0, 256, size=b.shape, dtype=np.uint8)
    b[:7, :] = 255                                   # extreme codes in a few rows
    b[7:14, :] = 0
    if z is not None:
        z = rng.integers(0, 256, size=z.shape, dtype=np.uint8)
        z[:7] = 0
        z[7:14] = 255
    w = native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)
    try:
        w.set_tuning(4, 2)
        w.set_tuning(5, ksw)
        for M in range(1, 17):
            a = workloads.make_activations(M, op.K, seed=92 + M)
            a *= (10.0 ** rng.uniform(-4, 5, size=(M, 1))).astype(np.float32)
            a[M // 2, 300] = np.float32(3e6)
            kernel, _ = check_against_oracle(w, a, b, s, z, None, op, f"8-bit skinny M={M} K={K} bs={bs} zp={zp}")
            assert kernel == "skinny_w4"
            assert np.array_equal(w.gemm(a), w.gemm(a)), M
        w.set_tuning(4, 0)
        for M in (3, 4, 5, 16):
            assert w.launch_info(M)["kernel"] == expected_kernel(op, M), M
    finally:
        w.set_tuning(4, 0)
        w.set_tuning(5, 0)
    w.close()
