"""GPU parity of libms_hip_nbits.so against the oracle and the golden fixtures.

Bars (from the operator's definition):
  * dequantized weights: bit-exact (value equality) with the oracle and with
    the reference's native kernel's one-hot output;
  * decode GEMV (M <= 16): per row m, max_n |y - y_ref| <= 1e-5 * max_n |y_ref[m, n]|;
  * prefill MFMA (M > 16): ||y - y_ref||_F / ||y_ref||_F <= 2e-3.
All calls go through the C ABI.
"""
from __future__ import annotations

import threading

import numpy as np
import pytest

import oracle
from conftest import kat_arrays
from modelsharp_amd import native, workloads
from modelsharp_amd.graph import Engine, GraphNode, KernelRegistry, ModelGraph
from modelsharp_amd.hip_kernel import HipMatMulNBitsKernel, register_kernels

pytestmark = pytest.mark.gpu

GEMV_RTOL = 1e-5
MFMA_FRO = 2e-3


def log(msg):
    print(msg, flush=True)


def assert_gemv_close(y, ref, what, cond=None):
    """Row bar 1e-5 * ||y_ref[m,:]||_inf. With `cond` = sum_k |a_k w_nk| given
    (rows of a few outputs, where the row norm is one possibly cancelling dot
    product), an error within the order-independent fp32 bound 2*gamma_K*cond of
    either summation also passes."""
    ref = ref.reshape(y.shape)
    rowmax = np.max(np.abs(ref), axis=-1, keepdims=True)
    allowed = GEMV_RTOL * rowmax
    if cond is not None:
        allowed = np.maximum(allowed, cond)
    err = np.max(np.abs(y - ref) / np.maximum(rowmax, 1e-30))
    log(f"  {what}: max row-relative err {err:.3e}")
    assert np.all(np.abs(y - ref) <= allowed), f"{what}: {err:.3e}"


def fp32_dot_bound(a, W):
    """2*gamma_K * sum_k |a_mk * W_nk|: bounds the gap between two fp32 sums in any order."""
    K = a.shape[-1]
    u = np.finfo(np.float32).eps / 2
    gamma = K * u / (1 - K * u)
    return 2 * gamma * (np.abs(a).astype(np.float64) @ np.abs(W).astype(np.float64).T)


def assert_fro_close(y, ref, what):
    rel = float(np.linalg.norm((y - ref).astype(np.float64)) / np.linalg.norm(ref.astype(np.float64)))
    log(f"  {what}: rel Frobenius {rel:.3e}")
    assert rel <= MFMA_FRO, f"{what}: {rel:.3e}"


def weights_for(op, seed):
    b, s, z = workloads.make_weights(op, seed)
    return b, s, z, native.NBitsWeights(b, s, z, op.N, op.K, op.bits, op.block_size)


# ---- the reference's known answers ---------------------------------------------------------
def test_kats_through_the_device(gpu, kat_cases):
    for case in kat_cases:
        a, b, s, zp, y = kat_arrays(case)
        at = case["attrs"]
        log(f"KAT {case['name']}")
        w = native.NBitsWeights(b, s, zp, at["N"], at["K"], at["bits"], at["block_size"])
        got = w.gemm(a.reshape(-1, at["K"])).reshape(y.shape)
        np.testing.assert_allclose(got, y, rtol=0, atol=1e-4, err_msg=case["name"])
        assert np.array_equal(got, y)
        w.close()


def test_golden_reference_vectors_through_the_device(gpu, ref_vectors):
    for key, g in sorted(ref_vectors.items()):
        if key.startswith("grid"):
            M, N, K, bits, bs = (int(x) for x in g["dims"])
            log(f"golden {key}")
            w = native.NBitsWeights(g["b"], g["scales"], g.get("zp"), N, K, bits, bs)
            assert_gemv_close(w.gemm(g["a"]), g["y"], key)
        else:
            N, K, bits, bs = (int(x) for x in g["dims"])
            log(f"golden {key}")
            w = native.NBitsWeights(g["b"], g["scales"], g.get("zp"), N, K, bits, bs)
            assert np.array_equal(w.dequant(), g["w"]), key
        w.close()


# ---- dequantized weights: bit-exact on every workload shape -----------------------------------
ALL_OPS = ([workloads.QWEN05B_UP] + workloads.QWEN05B_DECODE + workloads.DECODE_7B + workloads.LLAMA7B_SMALLM_OPS
           + workloads.LLAMA7B_PREFILL_OPS)


@pytest.mark.parametrize("op", ALL_OPS, ids=lambda o: f"{o.name}_K{o.K}_N{o.N}_bs{o.block_size}_{'zp' if o.has_zp else 'nozp'}")
def test_dequant_bit_exact(gpu, op):
    b, s, z, w = weights_for(op, seed=op.K * 7 + op.N)
    log(f"dequant K={op.K} N={op.N} bs={op.block_size}")
    assert np.array_equal(w.dequant(), oracle.dequant_weights(b, s, z, op.N, op.K, 4, op.block_size))
    w.close()


# ---- decode GEMV parity at the workloads' full sizes --------------------------------------------
DECODE_CASES = ([(workloads.QWEN05B_UP, 1)] + [(o, 1) for o in workloads.QWEN05B_DECODE]
                + [(o, 1) for o in workloads.DECODE_7B]
                + [(o, m) for o in workloads.LLAMA7B_SMALLM_OPS for m in workloads.LLAMA7B_SMALLM_M])


@pytest.mark.parametrize("op,M", DECODE_CASES, ids=lambda v: str(v) if isinstance(v, int) else f"{v.name}_K{v.K}_N{v.N}")
def test_gemv_parity(gpu, op, M):
    b, s, z, w = weights_for(op, seed=op.N + 3 * op.K + M)
    a = workloads.make_activations(M, op.K, seed=M + op.K)
    assert w.launch_info(M)["kernel"] in ("gemv_w4", "gemv_w4_panel", "skinny_w4")
    log(f"gemv M={M} K={op.K} N={op.N} bs={op.block_size} {w.launch_info(M)}")
    y = w.gemm(a)
    assert_gemv_close(y, oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, op.block_size), f"M={M} {op}")
    w.close()


# (K, knob 5): K=640 is 5 blocks, split 5 ways by default (one block per workgroup) or
# 2 ways (2 and 3 blocks), both through the in-kernel hand-off; K=512 in one workgroup
# per row tile (no slots, direct stores); K=1408 is 11 blocks, split 11 ways by default or
# 9 ways, both wider than the hand-off takes: partial-sum slices and the reduce launch.
SKINNY_SPLITS = [(640, 0), (640, 2), (512, 1), (1408, 0), (1408, 9)]


@pytest.mark.parametrize("bs", [128, 64, 32])
@pytest.mark.parametrize("K,ksw", SKINNY_SPLITS, ids=lambda v: str(v))
@pytest.mark.parametrize("zp", [False, True], ids=["nozp", "zp"])
def test_skinny_every_m_dynamic_range(gpu, zp, K, ksw, bs):
    """The small-M matrix-core path for every M in 1..16 (M = 1 forced), on a ragged shape
    (N=333 is no multiple of the 128-row tiles), with activations spanning 1e-4..1e5 across
    rows and blocks and a lone outlier: the per-block power-of-two split of A keeps the GEMV
    bar, whatever the number of workgroups per row tile. Block size 128 applies the scale
    per 128-k block; 64 and 32 per 32-k step, after the transpose of the code dwords across
    the wave's rows that makes each MFMA step one quantization block. Two calls agree bit
    for bit."""
    op = workloads.Op("sk", K, 333, bs, zp)
    b, s, z, w = weights_for(op, seed=70 + zp)
    rng = np.random.default_rng(71)
    try:
        native.set_tuning(4, 2)
        native.set_tuning(5, ksw)
        for M in range(1, 17):
            a = workloads.make_activations(M, op.K, seed=72 + M)
            a *= (10.0 ** rng.uniform(-4, 5, size=(M, 1))).astype(np.float32)        # per-row magnitude
            a[:, 128:256] *= np.float32(1e-3)                                         # one quiet block
            a[M // 2, 300] = np.float32(3e6)                                          # one outlier
            info = w.launch_info(M)
            assert info["kernel"] == "skinny_w4", info
            y = w.gemm(a)
            assert_gemv_close(y, oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, bs), f"skinny M={M} zp={zp} K={K} bs={bs}")
            assert np.array_equal(w.gemm(a), y), M
    finally:
        native.set_tuning(4, 0)
        native.set_tuning(5, 0)
    w.close()


def test_skinny_captured_before_and_after_eager_call(gpu):
    """Captured before any eager call (no workspace yet) the small-M call takes gemv_w4;
    captured afterwards it runs the matrix-core path, whose slot counters reset
    themselves: every replay equals the eager call bit for bit."""
    import torch
    op = workloads.Op("skc", 4096, 1000, 128, False)
    b, s, z, w = weights_for(op, seed=73)
    M = 8
    a = workloads.make_activations(M, op.K, seed=74)
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 128)
    dA = torch.from_numpy(a).cuda()
    dY = torch.zeros((M, op.N), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w.gemm_dev(dA.data_ptr(), dY.data_ptr(), M, torch.cuda.current_stream().cuda_stream)
    for i in range(2):
        dY.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_gemv_close(dY.cpu().numpy(), ref, f"pre-eager replay {i}")
    eager = w.gemm(a)
    assert w.launch_info(M)["kernel"] == "skinny_w4"
    assert_gemv_close(eager, ref, "eager")
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        w.gemm_dev(dA.data_ptr(), dY.data_ptr(), M, torch.cuda.current_stream().cuda_stream)
    for i in range(3):
        dY.fill_(float("nan"))
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dY.cpu().numpy(), eager), f"replay {i}"
    w.close()


def test_gemv_one_hot_is_bit_exact(gpu):
    """A = rows of the identity: each output is one product 1*W[n,k] plus zeros."""
    op = workloads.DECODE_7B[4]
    b, s, z, w = weights_for(op, seed=9)
    ks = np.random.default_rng(1).choice(op.K, 16, replace=False)
    a = np.zeros((16, op.K), np.float32)
    a[np.arange(16), ks] = 1.0
    W = oracle.dequant_weights(b, s, z, op.N, op.K, 4, op.block_size)
    for M in (1, 4, 16):
        y = w.gemm(a[:M])
        assert np.array_equal(y, W[:, ks[:M]].T), M
    w.close()


def gemv_config_count():
    """Number of gemv_w4 launch configurations (knob 1 accepts 1..count)."""
    n = 0
    while True:
        try:
            native.set_tuning(1, n + 1)
        except native.HipError:
            native.set_tuning(1, 0)
            return n
        n += 1


GEMV_SHAPES = [workloads.Op("a", 3584, 1000), workloads.Op("b", 896, 77, 128, False), workloads.Op("c", 4864, 96),
               workloads.Op("d", 1536, 65, 128, True), workloads.Op("e", 11008, 129, 32, True),
               workloads.Op("f", 320, 300, 32, False)]


def test_gemv_every_launch_config(gpu):
    """Every gemv_w4 configuration (where it fits) and the panel kernel at every lane
    split, M = 1..4, block sizes 32 and 128, with and without zero points, K not a
    multiple of the step, N not a multiple of the workgroup's rows. (The small-M
    matrix-core path, which would take block size 128 at M = 4, is switched off.)"""
    count = gemv_config_count()
    assert count >= 8
    try:
        native.set_tuning(4, 1)
        for cfg in list(range(1, count + 1)) + [-1]:
            native.set_tuning(1, cfg)
            for lanes in ([16, 32, 64] if cfg == -1 else [0]):
                native.set_gemv_lanes(lanes)
                for op in GEMV_SHAPES:
                    for M in (1, 2, 3, 4):
                        b, s, z, w = weights_for(op, seed=(cfg + 2) * 31 + M)
                        a = workloads.make_activations(M, op.K, seed=M + cfg + 2)
                        info = w.launch_info(M)
                        if cfg == -1:
                            assert info["kernel"] == "gemv_w4_panel"
                        log(f"cfg={cfg} lanes={lanes} M={M} K={op.K} N={op.N} {info}")
                        assert_gemv_close(w.gemm(a), oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, op.block_size),
                                          f"cfg={cfg} M={M} {op}")
                        w.close()
    finally:
        native.set_tuning(1, 0)
        native.set_tuning(4, 0)
        native.set_gemv_lanes(0)


@pytest.mark.parametrize("lanes", [16, 32, 64])
def test_gemv_panel_every_lane_split(gpu, lanes):
    """The panel kernel for M = 5..16 (its own range) at every lane split (the small-M
    matrix-core path, which would take the block-size-128 shape, switched off)."""
    ops = [workloads.Op("a", 3584, 1000), workloads.Op("b", 896, 77, 128, False), workloads.Op("c", 4864, 96, 64)]
    try:
        native.set_tuning(4, 1)
        native.set_gemv_lanes(lanes)
        for op in ops:
            for M in (5, 11, 16):
                b, s, z, w = weights_for(op, seed=lanes + M)
                a = workloads.make_activations(M, op.K, seed=M)
                assert w.launch_info(M)["kernel"] == "gemv_w4_panel"
                log(f"panel lanes={lanes} M={M} K={op.K} N={op.N}")
                assert_gemv_close(w.gemm(a), oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, op.block_size),
                                  f"lanes={lanes} M={M} {op}")
                w.close()
    finally:
        native.set_tuning(4, 0)
        native.set_gemv_lanes(0)


# ---- shapes the fast kernels do not take, and edges ----------------------------------------------
EDGE = [
    workloads.Op("ktail", 100, 33, 32, True),          # K % 32 != 0 -> generic
    workloads.Op("bs16", 96, 40, 16, True),            # block size 16 -> generic
    workloads.Op("bits8", 256, 24, 32, True, bits=8),  # 8-bit -> generic
    workloads.Op("bits8sym", 192, 20, 64, False, bits=8),
    workloads.Op("bs64", 640, 70, 64, True),           # fast, 2 chunks per block
    workloads.Op("bs256", 1024, 65, 256, False),       # fast, 8 chunks per block
    workloads.Op("n1", 512, 1, 32, True),              # a single output column
    workloads.Op("odd_nb", 96, 37, 32, True),          # 3 blocks: odd packed zero-point row
]


@pytest.mark.parametrize("op", EDGE, ids=lambda o: o.name)
@pytest.mark.parametrize("M", [1, 5, 16, 40])
def test_edge_shapes(gpu, op, M):
    b, s, z, w = weights_for(op, seed=M + op.N)
    a = workloads.make_activations(M, op.K, seed=M * 3)
    log(f"edge {op.name} M={M} {w.launch_info(M)}")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, op.bits, op.block_size)
    y = w.gemm(a)
    W = oracle.dequant_weights(b, s, z, op.N, op.K, op.bits, op.block_size)
    kernel = w.launch_info(M)["kernel"]
    if kernel in ("mfma_w4", "mfma_w4_pipe", "mfma_w4_rb"):
        assert_fro_close(y, ref, f"{op.name} M={M}")
    elif kernel == "mfma_general":
        # fp16 hi/lo splits of A and W: 2^-22 relative per split, fp32 sums
        absdot = np.abs(a).astype(np.float64) @ np.abs(W).astype(np.float64).T
        rowpart = np.max(np.abs(a), axis=1, keepdims=True).astype(np.float64) * np.abs(W).sum(axis=1)[None, :]
        assert_gemv_close(y, ref, f"{op.name} M={M}",
                          cond=4 * fp32_dot_bound(a, W) + 2.0 ** -20 * absdot + 2.0 ** -30 * rowpart)
    else:
        assert_gemv_close(y, ref, f"{op.name} M={M}", cond=fp32_dot_bound(a, W))
    assert np.array_equal(w.dequant(), W)
    w.close()


def test_m_zero_is_a_no_op(gpu):
    op = workloads.Op("m0", 128, 16)
    b, s, z, w = weights_for(op, 1)
    assert w.gemm(np.zeros((0, op.K), np.float32)).shape == (0, op.N)
    w.close()


# ---- prefill MFMA -------------------------------------------------------------------------------
@pytest.mark.parametrize("op", workloads.LLAMA7B_PREFILL_OPS, ids=lambda o: f"K{o.K}_N{o.N}")
@pytest.mark.parametrize("M", workloads.LLAMA7B_PREFILL_M)
def test_mfma_parity_sampled_columns(gpu, op, M):
    """Full-size call with the library's own kernel choice (mfma_w4_rb where the pipelined
    kernel's tiles would fill less than half of the CUs); the oracle checks a seeded
    sample of 96 output columns."""
    b, s, z, w = weights_for(op, seed=M + op.N)
    a = workloads.make_activations(M, op.K, seed=M, kind="rmsnorm")
    assert w.launch_info(M)["kernel"] == ("mfma_w4_pipe" if M >= 512 and (M > 512 or op.N > 4096) else "mfma_w4_rb")
    log(f"mfma M={M} K={op.K} N={op.N}")
    y = w.gemm(a)
    cols = np.sort(np.random.default_rng(M).choice(op.N, 96, replace=False))
    zc = None if z is None else z[cols]
    ref = oracle.matmul_nbits(a, b[cols], s.reshape(op.N, -1)[cols], zc, len(cols), op.K, 4, op.block_size)
    assert_fro_close(y[:, cols], ref, f"M={M} sampled")
    assert np.all(np.isfinite(y))
    w.close()


def pipe_items(M, N, ksplit):
    """Workgroups the pipelined prefill launches for knob 3 = ksplit (1: no tile split,
    2: all tiles split, 3: the second half split): 8 XCDs x (whole tiles per XCD + two
    halves per split tile per XCD)."""
    tiles = -(-M // 256) * -(-N // 256)
    full = tiles if ksplit == 1 else 0 if ksplit == 2 else tiles // 2
    return 8 * (-(-full // 8) + 2 * -(-(tiles - full) // 8))


@pytest.mark.parametrize("M", [17, 33, 64, 100, 129, 300])
def test_mfma_partial_tiles(gpu, M):
    """Both prefill kernels, and the pipelined one with no, every and half of its tiles K-split, on
    tiles cut by M and N (N=333 is not a multiple of 256; K=896 is 7 groups of 4
    steps, so the two K halves are unequal: 3 and 4 groups). mfma_w4_rb, which these
    small launches would take, is switched off."""
    op = workloads.Op("pt", 896, 333, 32, True)
    b, s, z, w = weights_for(op, seed=M)
    a = workloads.make_activations(M, op.K, seed=M, kind="rmsnorm")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 32)
    try:
        native.set_tuning(6, 1)
        for ks in (1, 2, 3):
            native.set_tuning(3, ks)
            info = w.launch_info(M)
            assert info["kernel"] == "mfma_w4_pipe" and info["grid"] == pipe_items(M, op.N, ks)
            log(f"mfma partial M={M} N={op.N} ksplit={ks} {info}")
            assert_fro_close(w.gemm(a), ref, f"pipe ksplit={ks} M={M}")
        native.set_tuning(3, 0)
        native.set_tuning(2, 1)
        assert w.launch_info(M)["kernel"] == "mfma_w4"
        assert_fro_close(w.gemm(a), ref, f"mfma_w4 M={M}")
    finally:
        native.set_tuning(2, 0)
        native.set_tuning(3, 0)
        native.set_tuning(6, 0)
    w.close()


def test_prefill_split_k_deterministic(gpu):
    """The pipelined prefill's K split (two workgroups per tile, combined by arrival
    order) gives bit-identical results on every call, and matches the unsplit launch to
    the bar (mfma_w4_rb, which this launch would take, switched off)."""
    op = workloads.Op("sk", 4096, 1000, 32, True)
    b, s, z, w = weights_for(op, seed=21)
    a = workloads.make_activations(300, op.K, seed=22, kind="rmsnorm")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 32)
    try:
        native.set_tuning(6, 1)
        assert w.launch_info(300)["grid"] == pipe_items(300, op.N, 2)   # 8 tiles: split by default
        y0 = w.gemm(a)
        assert_fro_close(y0, ref, "split")
        for i in range(4):
            assert np.array_equal(w.gemm(a), y0), i
        native.set_tuning(3, 1)
        y1 = w.gemm(a)
    finally:
        native.set_tuning(3, 0)
        native.set_tuning(6, 0)
    assert_fro_close(y1, ref, "unsplit")
    assert_fro_close(y0, y1, "split vs unsplit")
    w.close()


# ---- prefill with the weights dequantized into MFMA operand registers (mfma_w4_rb) -------------
RB_SHAPES = [workloads.Op("rb32", 896, 333, 32, True),      # 7 blocks of 128 k; N not a multiple of 256
             workloads.Op("rb64", 640, 200, 64, True),      # 2 chunks per quantization block
             workloads.Op("rb128", 1024, 300, 128, False)]  # 4 chunks per block, no zero points


@pytest.mark.parametrize("op", RB_SHAPES, ids=lambda o: o.name)
@pytest.mark.parametrize("M", [17, 100, 129, 300])
def test_rb_partial_tiles_and_splits(gpu, op, M):
    """mfma_w4_rb on tiles cut by M and N, tiles 64, 128 and 256 outputs wide, block sizes
    32/64/128, with and without zero points, unsplit and with K split 2, 3 and 7 ways
    (unequal ranges), always through the reduce launch (which applies the row exponents)."""
    b, s, z, w = weights_for(op, seed=M + op.K)
    a = workloads.make_activations(M, op.K, seed=M, kind="rmsnorm")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, op.block_size)
    G = op.K // 128
    try:
        w.set_tuning(6, 2)
        for nf in (1, 2, 4):
            w.set_tuning(9, nf)
            for ks in sorted({1, 2, 3, G}):
                w.set_tuning(7, ks)
                info = w.launch_info(M)
                items = -(-M // 128) * -(-op.N // (64 * nf)) * min(ks, G)
                assert info["kernel"] == "mfma_w4_rb" and info["grid"] == -(-items // 8) * 8, info
                assert info["lanes_per_row"] == 64 * nf
                log(f"rb {op.name} M={M} nf={nf} ksw={ks} {info}")
                y = w.gemm(a)
                assert_fro_close(y, ref, f"rb {op.name} M={M} nf={nf} ksw={ks}")
                assert np.array_equal(w.gemm(a), y), ks
    finally:
        w.close()


@pytest.mark.parametrize("op", workloads.LLAMA7B_PREFILL_OPS, ids=lambda o: f"K{o.K}_N{o.N}")
@pytest.mark.parametrize("M", workloads.LLAMA7B_PREFILL_M)
def test_rb_parity_sampled_columns(gpu, op, M):
    """mfma_w4_rb at the full prefill sizes (its own K split); the oracle checks 96 columns."""
    b, s, z, w = weights_for(op, seed=M + op.N)
    a = workloads.make_activations(M, op.K, seed=M, kind="rmsnorm")
    try:
        native.set_tuning(6, 2)
        info = w.launch_info(M)
        assert info["kernel"] == "mfma_w4_rb", info
        log(f"rb M={M} K={op.K} N={op.N} {info}")
        y = w.gemm(a)
    finally:
        native.set_tuning(6, 0)
    cols = np.sort(np.random.default_rng(M).choice(op.N, 96, replace=False))
    zc = None if z is None else z[cols]
    ref = oracle.matmul_nbits(a, b[cols], s.reshape(op.N, -1)[cols], zc, len(cols), op.K, 4, op.block_size)
    assert_fro_close(y[:, cols], ref, f"rb M={M} sampled")
    assert np.all(np.isfinite(y))
    w.close()


@pytest.mark.parametrize("op,kernel", [
    (workloads.Op("bs128", 1024, 300, 128, False), "mfma_w4_rb"),  # block size 128
    (workloads.Op("k96", 96, 200, 32, True), "mfma_w4"),           # K not a multiple of 128
    (workloads.Op("k640", 640, 260, 32, False), "mfma_w4_rb"),     # no zero points, few tiles
], ids=lambda v: v.name if hasattr(v, "name") else v)
def test_prefill_kernel_choice(gpu, op, kernel):
    b, s, z, w = weights_for(op, seed=op.K)
    a = workloads.make_activations(70, op.K, seed=3, kind="rmsnorm")
    assert w.launch_info(70)["kernel"] == kernel
    log(f"prefill {op.name} {w.launch_info(70)}")
    assert_fro_close(w.gemm(a), oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, op.block_size), op.name)
    w.close()


def test_prefill_scale_range_fallback(gpu):
    """Scales outside the fp16-normal range send the call to mfma_w4 (fp32 scales, exact
    integer weights)."""
    op = workloads.Op("tiny", 512, 96, 32, True)
    b, s, z = workloads.make_weights(op, 4)
    s = s.copy()
    s[::7] = 3e-6          # below 2^-14
    w = native.NBitsWeights(b, s, z, op.N, op.K, 4, 32)
    a = workloads.make_activations(40, op.K, seed=5, kind="rmsnorm")
    assert w.launch_info(40)["kernel"] == "mfma_w4"
    assert_fro_close(w.gemm(a), oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 32), "tiny scales")
    w.close()


def test_prefill_captured_before_eager_call(gpu):
    """A prefill call captured in a graph before any eager call (no activation
    workspace yet) runs the workspace-free kernel; every replay matches."""
    import torch
    op = workloads.Op("cap", 1024, 512, 32, True)
    b, s, z, w = weights_for(op, seed=6)
    a = workloads.make_activations(96, op.K, seed=7, kind="rmsnorm")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 32)
    dA = torch.from_numpy(a).cuda()
    dY = torch.zeros((96, op.N), dtype=torch.float32, device="cuda")
    native.set_tuning(6, 1)   # the pipelined kernel (this small launch would take mfma_w4_rb)
    try:
        _captured_before_and_after_eager(w, a, ref, dA, dY, split_grid=pipe_items(96, op.N, 2))
    finally:
        native.set_tuning(6, 0)
    w.close()


def test_rb_captured_before_and_after_eager_call(gpu):
    """mfma_w4_rb under capture: before any eager call (no workspace) the call takes the
    workspace-free kernel; afterwards the graph holds the conversion, the K-split kernel
    and the reduce launch, and every replay equals the eager call bit for bit."""
    import torch
    op = workloads.Op("capr", 1024, 512, 32, True)
    b, s, z, w = weights_for(op, seed=8)
    a = workloads.make_activations(96, op.K, seed=9, kind="rmsnorm")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 32)
    dA = torch.from_numpy(a).cuda()
    dY = torch.zeros((96, op.N), dtype=torch.float32, device="cuda")
    info = w.launch_info(96)
    assert info["kernel"] == "mfma_w4_rb" and info["grid"] > 8, info    # split K
    _captured_before_and_after_eager(w, a, ref, dA, dY, split_grid=info["grid"])
    w.close()


def _captured_before_and_after_eager(w, a, ref, dA, dY, split_grid):
    import torch
    M = a.shape[0]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w.gemm_dev(dA.data_ptr(), dY.data_ptr(), M, torch.cuda.current_stream().cuda_stream)
    for i in range(3):
        dY.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert_fro_close(dY.cpu().numpy(), ref, f"replay {i}")
    eager = w.gemm(a)           # grows the workspace
    assert_fro_close(eager, ref, "eager")
    # Captured again now that the workspace exists: the K-split kernel runs in the graph
    # (no memset recorded; counters or slices are rewritten every launch), so every
    # replay equals the eager call bit for bit.
    assert w.launch_info(M)["grid"] == split_grid
    g2 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g2):
        w.gemm_dev(dA.data_ptr(), dY.data_ptr(), M, torch.cuda.current_stream().cuda_stream)
    for i in range(3):
        dY.fill_(float("nan"))
        torch.cuda.synchronize()
        g2.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dY.cpu().numpy(), eager), f"split replay {i}"
        assert np.array_equal(w.gemm(a), eager), f"eager after replay {i}"



@pytest.mark.parametrize("op", workloads.LLAMA7B_PREFILL_OPS, ids=lambda o: f"K{o.K}_N{o.N}")
def test_mfma_full_vs_torch_fp32(gpu, op):
    """Every output of an M=2048 call against an fp32 product of the (bit-exact)
    dequantized weights on the device, on both 7B MLP shapes: the up shape's launch splits
    its last round of tiles over two workgroups each, the down shape's splits every tile.
    Two more calls return the same bits (the split hand-off is order-independent)."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    b, s, z, w = weights_for(op, seed=5)
    a = workloads.make_activations(2048, op.K, seed=6, kind="rmsnorm")
    dA = torch.from_numpy(a).cuda()
    dY = torch.empty((2048, op.N), dtype=torch.float32, device="cuda")
    dW = torch.empty((op.N, op.K), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    w.gemm_dev(dA.data_ptr(), dY.data_ptr(), 2048, stream)
    w.dequant_dev(dW.data_ptr(), stream)
    ref = dA.double() @ dW.double().T
    rel = float(torch.linalg.norm(dY.double() - ref) / torch.linalg.norm(ref))
    log(f"  mfma M=2048 K={op.K} N={op.N} {w.launch_info(2048)} full vs fp64 device product: rel Frobenius {rel:.3e}")
    assert rel <= MFMA_FRO
    y0 = dY.clone()
    for i in range(2):
        w.gemm_dev(dA.data_ptr(), dY.data_ptr(), 2048, stream)
        torch.cuda.synchronize()
        assert torch.equal(dY, y0), i
    w.close()


# ---- determinism, concurrency, the operator interface ------------------------------------------
def test_repeatable_and_thread_safe(gpu):
    op = workloads.Op("thr", 2048, 1536, 32, True)
    b, s, z, w = weights_for(op, 4)
    a = workloads.make_activations(3, op.K, 5)
    a_big = workloads.make_activations(70, op.K, 6)
    y0, y0b = w.gemm(a), w.gemm(a_big)
    results = {}

    def worker(i):
        results[i] = (w.gemm(a), w.gemm(a_big))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for i in range(8):
        assert np.array_equal(results[i][0], y0) and np.array_equal(results[i][1], y0b), i
    w.close()


def test_operator_interface_drop_in(gpu):
    import torch
    op = workloads.Op("proj", 896, 4864, 32, True)
    b, s, z = workloads.make_weights(op, 8)
    graph = ModelGraph(
        nodes=[GraphNode("MatMulNBits", "mmnb", ["A", "B", "scales", "zp"], ["Y"],
                         {"N": op.N, "K": op.K, "bits": 4, "block_size": 32})],
        initializers={"B": b, "scales": s, "zp": z}, inputs=["A"], outputs=["Y"])
    registry = register_kernels(KernelRegistry())
    kernel = registry.try_get("MatMulNBits")[1]
    assert isinstance(kernel, HipMatMulNBitsKernel)
    assert kernel.preload(graph) == 1
    a = workloads.make_activations(6, op.K, 9).reshape(2, 3, op.K)
    y = Engine(graph, registry).run({"A": a})["Y"]
    assert y.shape == (2, 3, op.N)
    ref = oracle.matmul_nbits(a.reshape(6, op.K), b, s, z, op.N, op.K, 4, 32)
    assert_gemv_close(y.reshape(6, op.N), ref, "engine host path")
    yd = Engine(graph, registry).run({"A": torch.from_numpy(a).cuda()})["Y"]
    torch.cuda.synchronize()
    assert np.array_equal(yd.cpu().numpy(), y)
    assert len(kernel._handles) == 1
    kernel.close()


def test_one_shot_entry_matches_handle_path(gpu):
    op = workloads.Op("one", 512, 200, 32, True)
    b, s, z, w = weights_for(op, 12)
    a = workloads.make_activations(4, op.K, 13)
    assert np.array_equal(native.qgemm_nbits(a, b, s, z, 4, op.N, op.K, 4, 32), w.gemm(a))
    w.close()


@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_batch_shared_activations_grouped(gpu, M):
    """The decode layer as an engine issues it: q/k/v on one input go through one grouped
    gemv_w4 launch, and so do gate/up on another up to M = 3 (from M = 4 each takes the
    matrix-core small-M kernel on its own); every output against the oracle."""
    import torch
    ops = workloads.DECODE_7B            # q, k, v, o, gate, up, down
    share = workloads.DECODE_7B_SHARE   # activation buffer each call reads
    host = [weights_for(o, 40 + i) for i, o in enumerate(ops)]
    acts = {j: workloads.make_activations(M, ops[j].K, 50 + j) for j in set(share)}
    dA = {j: torch.from_numpy(a).cuda() for j, a in acts.items()}
    Ys = [torch.full((M, o.N), float("nan"), device="cuda") for o in ops]
    ptrs = [dA[share[i]].data_ptr() for i in range(len(ops))]
    info = native.batch_launch_info([h[3] for h in host], ptrs, M)
    assert info["calls"] == 3 and info["kernel"] == "gemv_w4", info          # q, k, v in one launch
    assert native.batch_launch_info([h[3] for h in host[3:]], ptrs[3:], M)["calls"] == 1   # o alone
    gu = native.batch_launch_info([h[3] for h in host[4:]], ptrs[4:], M)
    if M >= 4:
        assert gu["calls"] == 1 and gu["kernel"] == "skinny_w4", gu                  # gate alone
    else:
        assert gu["calls"] == 2 and gu["kernel"] == "gemv_w4", gu                    # gate, up
    native.gemm_dev_batch([h[3] for h in host], ptrs, [y.data_ptr() for y in Ys], M,
                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for i, (o, (b, s, z, w)) in enumerate(zip(ops, host)):
        a = acts[share[i]]
        log(f"grouped {o.name} M={M}")
        assert_gemv_close(Ys[i].cpu().numpy(), oracle.matmul_nbits(a, b, s, z, o.N, o.K, 4, o.block_size),
                          f"grouped {o.name} M={M}")
        w.close()


def test_batch_group_every_launch_config(gpu):
    """Ragged groups under every gemv_w4 configuration: 5 calls on one input (split
    4 + 1), members with and without zero points, N not a multiple of any row count."""
    import torch
    K, M = 896, 2
    ops = [workloads.Op(f"g{i}", K, n, 32, zp) for i, (n, zp) in
           enumerate([(300, True), (77, False), (1000, True), (5, True), (129, False)])]
    host = [weights_for(o, 60 + i) for i, o in enumerate(ops)]
    a = workloads.make_activations(M, K, 61)
    dA = torch.from_numpy(a).cuda()
    refs = [oracle.matmul_nbits(a, b, s, z, o.N, K, 4, 32) for o, (b, s, z, _) in zip(ops, host)]
    stream = torch.cuda.current_stream().cuda_stream
    try:
        for cfg in range(1, gemv_config_count() + 1):
            native.set_tuning(1, cfg)
            Ys = [torch.full((M, o.N), float("nan"), device="cuda") for o in ops]
            native.gemm_dev_batch([h[3] for h in host], [dA.data_ptr()] * len(ops), [y.data_ptr() for y in Ys],
                                  M, stream)
            torch.cuda.synchronize()
            for o, y, ref in zip(ops, Ys, refs):
                assert_gemv_close(y.cpu().numpy(), ref, f"cfg {cfg} {o.name}")
    finally:
        native.set_tuning(1, 0)
    for h in host:
        h[3].close()


@pytest.mark.parametrize("M,rb", [(300, 0), (300, 2), (2048, 0)])
def test_batch_prefill_shares_the_fp16_copy(gpu, M, rb):
    """Prefill calls of one batch on the same input (gate and up) convert A to fp16 once:
    the second reads the first's copy. Outputs equal single calls bit for bit, on the
    pipelined and the few-tile kernel (knob 6 = 2), and when a handle appears twice (its
    own earlier copy is dropped first) or a call on another input sits in between."""
    import torch
    gate, up = workloads.Op("gate", 1024, 700, 32, True), workloads.Op("up", 1024, 520, 32, True)
    other = workloads.Op("other", 640, 300, 32, True)
    hg, hu, ho = weights_for(gate, 81)[3], weights_for(up, 82)[3], weights_for(other, 83)[3]
    a = torch.from_numpy(workloads.make_activations(M, 1024, 84, kind="rmsnorm")).cuda()
    b = torch.from_numpy(workloads.make_activations(M, 640, 85, kind="rmsnorm")).cuda()
    stream = torch.cuda.current_stream().cuda_stream
    try:
        native.set_tuning(6, rb)
        calls = [(hg, a), (hu, a), (hg, a), (hu, a), (ho, b), (hu, a), (hg, a)]
        Ys = [torch.full((M, h.N), float("nan"), device="cuda") for h, _ in calls]
        kernels = {h.launch_info(M)["kernel"] for h, _ in calls}
        log(f"shared fp16 copy M={M} rb={rb}: {kernels}")
        assert kernels <= {"mfma_w4_pipe", "mfma_w4_rb"} and (rb == 0 or kernels == {"mfma_w4_rb"}), kernels
        native.gemm_dev_batch([h for h, _ in calls], [x.data_ptr() for _, x in calls], [y.data_ptr() for y in Ys],
                              M, stream)
        torch.cuda.synchronize()
        for (h, x), y in zip(calls, Ys):
            ref = torch.full_like(y, float("nan"))
            h.gemm_dev(x.data_ptr(), ref.data_ptr(), M, stream)
            torch.cuda.synchronize()
            assert torch.equal(y, ref), h.N
    finally:
        native.set_tuning(6, 0)
        for h in (hg, hu, ho):
            h.close()


def test_batch_entry_matches_single_calls(gpu):
    import torch
    ops = workloads.DECODE_7B[:4]
    ws = [weights_for(o, i)[3] for i, o in enumerate(ops)]
    As = [torch.from_numpy(workloads.make_activations(1, o.K, i)).cuda() for i, o in enumerate(ops)]
    Ys = [torch.empty((1, o.N), device="cuda") for o in ops]
    stream = torch.cuda.current_stream().cuda_stream
    native.gemm_dev_batch(ws, [x.data_ptr() for x in As], [y.data_ptr() for y in Ys], 1, stream)
    torch.cuda.synchronize()
    for w, x, y in zip(ws, As, Ys):
        assert np.array_equal(y.cpu().numpy(), w.gemm(x.cpu().numpy()))
        w.close()


# ---- fp16 range: every M > 16 path with inputs outside fp16's range ------------------------
RANGE_CASES = [(op, M) for op in workloads.LLAMA7B_PREFILL_OPS for M in (17, 128, 2048)]


@pytest.mark.parametrize("op,M", RANGE_CASES, ids=lambda v: str(v) if isinstance(v, int) else f"K{v.K}_N{v.N}")
def test_prefill_dynamic_range(gpu, op, M):
    """Activation outliers of 1e5 and 3e6, rows near 1e-6, and scales near 1e4 and 1e-6
    (outside what fp16 carries) on both 7B MLP shapes: every output finite, relative
    Frobenius error <= 2e-3 against the oracle on sampled columns, and the tiny rows
    <= 2e-3 on their own (each row is staged in fp16 with its own power-of-two scale,
    so they keep fp16's precision instead of falling into its subnormal range).
    fp16-safe scales run the fp16 kernels (mfma_w4_rb / mfma_w4_pipe), the others the
    exact mfma_w4."""
    b, s, z = workloads.make_weights(op, seed=M + 11)
    rng = np.random.default_rng(M + 12)
    a = workloads.make_activations(M, op.K, seed=M + 13, kind="rmsnorm")
    rows = rng.permutation(M)
    big = rows[: max(2, M // 8)]
    tiny = rows[max(2, M // 8): max(2, M // 8) + max(2, M // 16)]
    for i, r in enumerate(big):
        a[r, rng.integers(op.K)] = (1e5 if i % 2 == 0 else -3e6)
    a[tiny] *= np.float32(1e-6)
    cols = np.sort(rng.choice(op.N, 96, replace=False))
    zc = None if z is None else z[cols]
    fast = "mfma_w4_pipe" if M == 2048 else "mfma_w4_rb"
    for scales, what, kernel in ((s, "fp16-safe scales", fast),
                                 (s * np.float32(1e6), "scales 1e3..1e4", "mfma_w4"),
                                 (s * np.float32(1e-4), "scales 1e-7..1e-6", "mfma_w4")):
        w = native.NBitsWeights(b, scales, z, op.N, op.K, 4, 32)
        assert w.launch_info(M)["kernel"] == kernel, (what, w.launch_info(M))
        log(f"range M={M} K={op.K} N={op.N} {what} -> {kernel}")
        y = w.gemm(a)
        w.close()
        assert np.all(np.isfinite(y)), what
        ref = oracle.matmul_nbits(a, b[cols], scales.reshape(op.N, -1)[cols], zc, len(cols), op.K, 4, 32)
        assert np.all(np.isfinite(ref))
        assert_fro_close(y[:, cols], ref, what)
        assert_fro_close(y[tiny][:, cols], ref[tiny], what + ", rows near 1e-6")


# ---- decode GEMV: exact zero-point differences -------------------------------------------
def _cancelling_weights(op, seed):
    """Rows made of blocks whose codes equal the block's zero point except for a few codes
    one step away: sum_k a_k (q_k - zp) is small while sum_k a_k q_k and zp * sum_k a_k are
    large, so folding the zero point out of the block sum would cancel."""
    rng = np.random.default_rng(seed)
    nb = op.nb
    zp = rng.integers(1, 15, size=(op.N, nb))
    codes = np.repeat(zp, op.block_size, axis=1)[:, : nb * op.block_size]
    for n in range(op.N):
        ks = rng.choice(op.K, size=4, replace=False)
        codes[n, ks] += rng.choice([-1, 1], size=4)
    b = workloads.pack_nibbles(codes.reshape(op.N, nb, op.block_size))
    s = rng.uniform(op.scale_lo, op.scale_hi, size=op.N * nb).astype(np.float32)
    return b, s, workloads.pack_nibbles(zp)


@pytest.mark.parametrize("M,bs,kernel", [(1, 32, "gemv_w4"), (2, 32, "gemv_w4"), (8, 32, "gemv_w4_panel"),
                                         (8, 32, "skinny_w4"), (1, 128, "gemv_w4"), (8, 128, "skinny_w4")])
def test_gemv_exact_zero_point_differences(gpu, M, bs, kernel):
    """Weight rows that are mostly q == zp blocks against activations up to 1e4: the decode
    kernels form a_k (q_k - zp) exactly, so they meet the 1e-5 * ||y_row||_inf bar where a
    folded sum_k a_k q_k - zp * sum_k a_k would not. (The panel kernel is reached with the
    small-M matrix-core path switched off, knob 4 = 1.)"""
    op = workloads.Op("cancel", 4096, 2048, bs, True)
    b, s, z = _cancelling_weights(op, seed=bs + M)
    w = native.NBitsWeights(b, s, z, op.N, op.K, 4, bs)
    if kernel == "gemv_w4_panel":
        w.set_tuning(4, 1)
    assert w.launch_info(M)["kernel"] == kernel
    a = np.random.default_rng(M).uniform(5e3, 1e4, size=(M, op.K)).astype(np.float32)
    y = w.gemm(a)
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, bs)
    assert_gemv_close(y, ref, f"{kernel} M={M} bs={bs} cancelling blocks")
    w.close()


# ---- split-K hand-off failures are reported, with every kernel exiting normally ------------
def _split_pipe_handle(seed):
    op = workloads.Op("split", 1024, 512, 32, True)
    b, s, z, w = weights_for(op, seed)
    w.set_tuning(6, 1)   # the pipelined kernel, not mfma_w4_rb
    w.set_tuning(3, 2)   # every tile split over two workgroups
    a = workloads.make_activations(64, op.K, seed=seed + 1, kind="rmsnorm")
    ref = oracle.matmul_nbits(a, b, s, z, op.N, op.K, 4, 32)
    assert w.launch_info(64)["kernel"] == "mfma_w4_pipe"
    assert_fro_close(w.gemm(a), ref, "split, first call")   # grows the counters
    return w, a, ref


def test_split_k_overlap_is_reported(gpu):
    """Counters holding another launch's tag (what two overlapping launches on one handle
    leave) make both halves of every split tile stand down and the call return an error;
    the counters are reset and the next call is correct."""
    w, a, ref = _split_pipe_handle(21)
    w.debug_set_counters(12345)
    with pytest.raises(native.HipError) as e:
        w.gemm(a)
    assert e.value.status == native.MS_HIP_ERR_HIP and "another launch" in e.value.message
    assert_fro_close(w.gemm(a), ref, "split, after the reported overlap")
    w.device_error()   # nothing left to report
    w.close()


def test_split_k_timeout_is_reported(gpu):
    """A second half whose partner's flag never comes (the tags say both halves arrived
    second; the poll bound is one) gives up, and the call returns an error instead of a
    half-summed output; the next call is correct."""
    w, a, ref = _split_pipe_handle(22)
    w.set_tuning(8, 1)
    w.debug_set_counters(0, next_epoch_tag=True)
    with pytest.raises(native.HipError) as e:
        w.gemm(a)
    assert e.value.status == native.MS_HIP_ERR_HIP and "timed out" in e.value.message
    w.set_tuning(8, 0)
    assert_fro_close(w.gemm(a), ref, "split, after the reported time-out")
    w.close()


def test_split_k_error_reported_to_the_next_device_call(gpu):
    """On the device-pointer entry the failure is reported by the next call on the handle
    (or by ms_hip_nbits_device_error) once the stream has been synchronised."""
    import torch
    w, a, ref = _split_pipe_handle(23)
    dA = torch.from_numpy(a).cuda()
    dY = torch.zeros((64, 512), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    w.debug_set_counters(777)
    w.gemm_dev(dA.data_ptr(), dY.data_ptr(), 64, stream)
    torch.cuda.synchronize()
    with pytest.raises(native.HipError):
        w.gemm_dev(dA.data_ptr(), dY.data_ptr(), 64, stream)
    w.gemm_dev(dA.data_ptr(), dY.data_ptr(), 64, stream)
    torch.cuda.synchronize()
    w.device_error()
    assert_fro_close(dY.cpu().numpy(), ref, "device entry after the reported overlap")
    w.close()


def test_tuning_is_per_handle(gpu):
    """A knob set on one handle changes that handle's kernel only."""
    op = workloads.Op("tune", 1024, 512, 32, True)
    _, _, _, w1 = weights_for(op, 31)
    _, _, _, w2 = weights_for(op, 31)
    assert w1.launch_info(64)["kernel"] == w2.launch_info(64)["kernel"] == "mfma_w4_rb"
    w1.set_tuning(6, 1)
    assert w1.launch_info(64)["kernel"] == "mfma_w4_pipe" and w2.launch_info(64)["kernel"] == "mfma_w4_rb"
    w1.set_tuning(6, native.MS_HIP_TUNING_INHERIT)
    assert w1.launch_info(64)["kernel"] == "mfma_w4_rb"
    w1.close()
    w2.close()


def test_destroyed_handle_is_rejected(gpu):
    op = workloads.Op("gone", 256, 64, 32, True)
    _, _, _, w = weights_for(op, 41)
    h = w.handle
    w.close()
    lib = native.load()
    assert lib.ms_hip_nbits_weights_info(h, None, None, None, None, None) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_nbits_weights_destroy(h) == native.MS_HIP_ERR_INVALID


def test_forced_failure_leaves_output_untouched(gpu):
    """A forced failure (the fallback test switch) refuses a live handle's call before any
    launch; switched off, the same handle computes normally."""
    import torch
    op = workloads.Op("ff", 256, 64)
    b, s, z, w = weights_for(op, 2)
    a = torch.from_numpy(workloads.make_activations(3, op.K, seed=1)).cuda()
    y = torch.full((3, op.N), 7.0, device="cuda")
    lib = native.load()
    try:
        lib.ms_hip_debug_force_failure(1)
        st = lib.ms_hip_nbits_gemm_dev(w.handle, native._vp(a.data_ptr()), native._vp(y.data_ptr()), 3, None)
        assert st == native.MS_HIP_ERR_FORCED
    finally:
        lib.ms_hip_debug_force_failure(0)
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
    w.gemm_dev(a.data_ptr(), y.data_ptr(), 3)
    torch.cuda.synchronize()
    ref = oracle.matmul_nbits(a.cpu().numpy(), b, s, z, op.N, op.K, 4, 32)
    assert_gemv_close(y.cpu().numpy(), ref, "after forced failure")
    w.close()
