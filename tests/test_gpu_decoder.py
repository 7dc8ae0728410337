"""Device parity of the decoder-layer neighbours of MatMulNBits against the oracle
(oracle/ms_decoder_oracle.c), and one decoder layer run end to end on the device.

Bars: the residual sums, Add, Mul and the present V rows are bit-exact; rotated K rows
are bit-exact (the same four roundings per pair); norms, SiLU and attention differ only in
summation order and exp's last bits: elementwise rtol 2e-6 for the norms and activations
(4e-6 for those through exp), attention within 1e-5 of max|out| per call.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from modelsharp_amd import native, workloads
from modelsharp_amd.decoder_kernels import (HipGroupQueryAttentionKernel, fuse_gate_up_silu, fuse_silu_mul,
                                            fuse_skipnorm, register_decoder_kernels)
from modelsharp_amd.graph import Engine, GraphContext, GraphNode, KernelRegistry, ModelGraph
from modelsharp_amd.hip_kernel import register_kernels

pytestmark = pytest.mark.gpu


def log(msg):
    print(msg, flush=True)


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


@pytest.mark.parametrize("rows,norm", [(1, 4096), (7, 100), (2048, 4096), (3, 3)])
def test_rmsnorm(gpu, rows, norm):
    import torch
    r = np.random.default_rng(rows + norm)
    x = (r.standard_normal((rows, norm)) * 2).astype(np.float32)
    w = r.uniform(0.5, 1.5, norm).astype(np.float32)
    dx, dw = dev(x), dev(w)
    y, inv = torch.empty_like(dx), torch.empty(rows, device="cuda")
    native.rmsnorm(dx.data_ptr(), dw.data_ptr(), y.data_ptr(), inv.data_ptr(), rows, norm, 1e-5)
    ref, inv_ref = oracle.rmsnorm(x, w, 1e-5)
    assert np.allclose(host(inv), inv_ref, rtol=2e-6, atol=0)
    assert np.allclose(host(y), ref, rtol=2e-6, atol=1e-7 * np.abs(ref).max())
    native.rmsnorm(dx.data_ptr(), dw.data_ptr(), dx.data_ptr(), None, rows, norm, 1e-5)   # in place
    assert np.array_equal(host(dx), host(y))


@pytest.mark.parametrize("with_bias", [False, True])
def test_skip_rmsnorm_in_place_residual(gpu, with_bias):
    import torch
    r = np.random.default_rng(5)
    rows, norm = 5, 4096
    a = r.standard_normal((rows, norm)).astype(np.float32)
    s = r.standard_normal((rows, norm)).astype(np.float32)
    g = r.uniform(0.5, 1.5, norm).astype(np.float32)
    beta = r.standard_normal(norm).astype(np.float32) if with_bias else None
    bias = r.standard_normal(norm).astype(np.float32) if with_bias else None
    out_ref, inv_ref, sum_ref = oracle.skip_rmsnorm(a, s, g, beta, bias, 1e-6)
    da, ds, dg = dev(a), dev(s), dev(g)
    db = None if beta is None else dev(beta)
    dbi = None if bias is None else dev(bias)
    out, inv = torch.empty_like(da), torch.empty(rows, device="cuda")
    ptr = lambda t: None if t is None else t.data_ptr()   # noqa: E731
    # the residual stream updated in place: sum written over the skip input
    native.skip_rmsnorm(da.data_ptr(), ds.data_ptr(), dg.data_ptr(), ptr(db), ptr(dbi), out.data_ptr(),
                        ds.data_ptr(), inv.data_ptr(), rows, norm, 1e-6)
    assert np.array_equal(host(ds), sum_ref)
    assert np.allclose(host(out), out_ref, rtol=2e-6, atol=1e-7 * np.abs(out_ref).max())
    assert np.allclose(host(inv), inv_ref, rtol=2e-6, atol=0)


def test_elementwise(gpu):
    import torch
    r = np.random.default_rng(9)
    n = 11008 * 3 + 5
    g = (r.standard_normal(n) * 5).astype(np.float32)
    u = r.standard_normal(n).astype(np.float32)
    dg, du, y = dev(g), dev(u), torch.empty(n, device="cuda")
    native.silu_mul(dg.data_ptr(), du.data_ptr(), y.data_ptr(), n)
    ref = oracle.silu_mul(g, u)
    assert np.allclose(host(y), ref, rtol=4e-6, atol=1e-30)
    native.add(dg.data_ptr(), du.data_ptr(), y.data_ptr(), n)
    assert np.array_equal(host(y), g + u)
    native.mul(dg.data_ptr(), du.data_ptr(), y.data_ptr(), n)
    assert np.array_equal(host(y), g * u)
    native.sigmoid(dg.data_ptr(), y.data_ptr(), n)
    assert np.allclose(host(y), 1 / (1 + np.exp(-g.astype(np.float64))), rtol=4e-6, atol=1e-30)
    # SiluMul equals Sigmoid -> Mul -> Mul on the device bit for bit
    s, a, y2 = torch.empty_like(dg), torch.empty_like(dg), torch.empty_like(dg)
    native.sigmoid(dg.data_ptr(), s.data_ptr(), n)
    native.mul(dg.data_ptr(), s.data_ptr(), a.data_ptr(), n)
    native.mul(a.data_ptr(), du.data_ptr(), y2.data_ptr(), n)
    native.silu_mul(dg.data_ptr(), du.data_ptr(), y.data_ptr(), n)
    assert torch.equal(y, y2)


# ---- gate + up + SiLU-Mul in one call (ms_hip_nbits_gemm_dev_swiglu) --------------------
SWIGLU_OPS = [workloads.Op("7b_gate", 3584, 18944, 32, True, 0.001, 0.01),      # the 7B layer's MLP
              workloads.Op("qwen_gate", 896, 4864, 32, True, 0.002, 0.02),
              workloads.Op("llama_bs128", 4096, 11008, 128, False),               # block size 128, no zp
              workloads.Op("ragged", 1024, 1000, 32, True)]                       # N not a multiple of the tile


def _swiglu_handles(op, seed):
    wg = native.NBitsWeights(*workloads.make_weights(op, seed), op.N, op.K, op.bits, op.block_size)
    wu = native.NBitsWeights(*workloads.make_weights(op, seed + 1), op.N, op.K, op.bits, op.block_size)
    return wg, wu


@pytest.mark.parametrize("op", SWIGLU_OPS, ids=lambda o: o.name)
def test_swiglu_fused_decode_equals_grouped_then_silu(gpu, op):
    """At M = 1 the fused launch (the same rows of gate and up in one workgroup, H stored
    directly) is bit-identical to the grouped gate+up launch followed by ms_hip_silu_mul,
    and within the GEMV bar of the oracle's gate and up composed with SiLU-Mul in float64."""
    import torch
    wg, wu = _swiglu_handles(op, 41)
    a = workloads.make_activations(1, op.K, seed=42)
    da = dev(a)
    info = native.swiglu_launch_info(wg, wu, da.data_ptr(), 1)
    log(f"swiglu {op.name} K={op.K} N={op.N}: {info}")
    assert info["fused"]
    h = torch.full((1, op.N), float("nan"), device="cuda")
    native.gemm_dev_swiglu(wg, wu, da.data_ptr(), h.data_ptr(), 1)
    g, u, h2 = (torch.empty((1, op.N), device="cuda") for _ in range(3))
    native.gemm_dev_batch([wg, wu], [da.data_ptr()] * 2, [g.data_ptr(), u.data_ptr()], 1)
    native.silu_mul(g.data_ptr(), u.data_ptr(), h2.data_ptr(), op.N)
    torch.cuda.synchronize()
    assert torch.equal(h, h2)
    bg, sg, zg = workloads.make_weights(op, 41)
    bu, su, zu = workloads.make_weights(op, 42)
    gr = oracle.matmul_nbits(a, bg, sg, zg, op.N, op.K, op.bits, op.block_size).astype(np.float64)
    ur = oracle.matmul_nbits(a, bu, su, zu, op.N, op.K, op.bits, op.block_size).astype(np.float64)
    hr = gr / (1 + np.exp(-gr)) * ur
    got = host(h).astype(np.float64)
    rel = np.linalg.norm(got - hr) / np.linalg.norm(hr)
    log(f"  relative Frobenius error against the oracle {rel:.2e}")
    assert rel <= 1e-5
    wg.close()
    wu.close()


@pytest.mark.parametrize("M", [0, 2, 4, 17, 130])
def test_swiglu_other_forms_equal_separate_calls(gpu, M):
    """Other M (and block size 64, which the decode GEMV does not take) run the three steps
    (gate into H, up into the gate handle's workspace, SiLU-Mul in place): bit-identical to
    the separate calls."""
    import torch
    for op in (workloads.Op("g32", 1024, 1000, 32, True), workloads.Op("g64", 1024, 600, 64, True)):
        wg, wu = _swiglu_handles(op, 51 + M)
        a = workloads.make_activations(max(M, 1), op.K, seed=M + 3, kind="rmsnorm")[:M]
        da = dev(a) if M else torch.empty((0, op.K), device="cuda")
        if M:
            assert not native.swiglu_launch_info(wg, wu, da.data_ptr(), M)["fused"]
        h = torch.full((M, op.N), float("nan"), device="cuda")
        native.gemm_dev_swiglu(wg, wu, da.data_ptr(), h.data_ptr(), M)
        if M:
            g, u, h2 = (torch.empty((M, op.N), device="cuda") for _ in range(3))
            wg.gemm_dev(da.data_ptr(), g.data_ptr(), M)
            wu.gemm_dev(da.data_ptr(), u.data_ptr(), M)
            native.silu_mul(g.data_ptr(), u.data_ptr(), h2.data_ptr(), M * op.N)
            torch.cuda.synchronize()
            assert torch.equal(h, h2), (op.name, M)
        wg.close()
        wu.close()


def test_swiglu_rejects_mismatched_projections(gpu):
    import torch
    wg = native.NBitsWeights(*workloads.make_weights(workloads.Op("a", 512, 64, 32, True), 1), 64, 512, 4, 32)
    wu = native.NBitsWeights(*workloads.make_weights(workloads.Op("b", 512, 96, 32, True), 2), 96, 512, 4, 32)
    a = dev(workloads.make_activations(1, 512, seed=3))
    h = torch.zeros((1, 96), device="cuda")
    with pytest.raises(native.HipError) as e:
        native.gemm_dev_swiglu(wg, wu, a.data_ptr(), h.data_ptr(), 1)
    assert e.value.status == native.MS_HIP_ERR_INVALID and "share K, N" in e.value.message
    wg.close()
    wu.close()


# ---- SkipSimplifiedLayerNormalization fused into its projections ----------------------------
# (projection shapes, M): the 7B q/k/v of one normed input and the Qwen q/k/v (one grouped
# launch each at M = 1), a lone projection, block size 128 without zero points, and M > 1
# (the norm and the batch call apart).
SKIPNORM_CASES = [([workloads.DECODE_7B[i] for i in (0, 1, 2)], 1),
                  (workloads.QWEN05B_DECODE[:3], 1),
                  ([workloads.Op("lone", 1024, 700, 32, True)], 1),
                  ([workloads.Op("bs128", 4096, 1100, 128, False)], 1),
                  ([workloads.Op("m3a", 1024, 300, 32, True), workloads.Op("m3b", 1024, 200, 32, True)], 3)]


def _norm_inputs(M, K, seed):
    r = np.random.default_rng(seed)
    x = r.standard_normal((M, K)).astype(np.float32)
    s = (r.standard_normal((M, K)) * 3).astype(np.float32)
    g = r.uniform(0.5, 1.5, K).astype(np.float32)
    return x, s, g


def _check_norm_outputs(norm, sm, x, s, g, eps):
    out_ref, _, sum_ref = oracle.skip_rmsnorm(x, s, g, None, None, eps)
    assert np.array_equal(sm, sum_ref)
    assert np.allclose(norm, out_ref, rtol=2e-6, atol=1e-7 * np.abs(out_ref).max())
    return out_ref


@pytest.mark.parametrize("ops,M", SKIPNORM_CASES, ids=lambda v: str(v) if isinstance(v, int) else v[0].name)
def test_skipnorm_projections(gpu, ops, M):
    """T = X + Skip and the normed rows as ms_hip_skip_rmsnorm writes them (T bit-exact, the
    norm within its rtol), and each projection of the normed rows within the GEMV bar of the
    oracle (norm, then matmul_nbits). At M = 1 it is one launch that computes the norm in
    every workgroup's staging and scales the sums by inv; two calls agree bit for bit."""
    import torch
    K, eps = ops[0].K, 1e-6
    x, s, g = _norm_inputs(M, K, seed=K + M)
    hs, host_w = [], []
    for i, op in enumerate(ops):
        b, sc, z = workloads.make_weights(op, 60 + i)
        host_w.append((b, sc, z))
        hs.append(native.NBitsWeights(b, sc, z, op.N, op.K, op.bits, op.block_size))
    dx, ds, dg = dev(x), dev(s), dev(g)
    norm, sm = torch.empty_like(dx), torch.empty_like(dx)
    info = native.skipnorm_launch_info(hs, False, dx.data_ptr(), ds.data_ptr(), dg.data_ptr(), norm.data_ptr(),
                                       sm.data_ptr(), M)
    log(f"skipnorm {[o.name for o in ops]} K={K} M={M}: {info}")
    assert info["fused"] == (M == 1)
    ys = [torch.full((M, op.N), float("nan"), device="cuda") for op in ops]
    native.gemm_dev_skipnorm(hs, dx.data_ptr(), ds.data_ptr(), dg.data_ptr(), eps, norm.data_ptr(), sm.data_ptr(),
                             [y.data_ptr() for y in ys], M)
    first = [host(y) for y in ys]
    out_ref = _check_norm_outputs(host(norm), host(sm), x, s, g, eps)
    for (b, sc, z), op, y in zip(host_w, ops, first):
        ref = oracle.matmul_nbits(out_ref, b, sc, z, op.N, op.K, op.bits, op.block_size)
        rowmax = np.max(np.abs(ref), axis=-1, keepdims=True)
        err = np.max(np.abs(y - ref) / rowmax)
        log(f"  {op.name}: max row-relative err {err:.2e}")
        assert err <= 1e-5
    native.gemm_dev_skipnorm(hs, dx.data_ptr(), ds.data_ptr(), dg.data_ptr(), eps, norm.data_ptr(), None,
                             [y.data_ptr() for y in ys], M)
    for y, y1 in zip(ys, first):
        assert np.array_equal(host(y), y1)
    for h in hs:
        h.close()


@pytest.mark.parametrize("op", SWIGLU_OPS[:3], ids=lambda o: o.name)
def test_skipnorm_swiglu(gpu, op):
    """The norm, then gate, up and SiLU-Mul: one launch at M = 1, within the GEMV bar of the
    unfused calls (ms_hip_skip_rmsnorm, then ms_hip_nbits_gemm_dev_swiglu) and of the
    oracle in float64."""
    import torch
    eps = 1e-5
    x, s, g = _norm_inputs(1, op.K, seed=op.N)
    wg, wu = _swiglu_handles(op, 71)
    dx, ds, dg = dev(x), dev(s), dev(g)
    norm, sm = torch.empty_like(dx), torch.empty_like(dx)
    info = native.skipnorm_launch_info([wg, wu], True, dx.data_ptr(), ds.data_ptr(), dg.data_ptr(), norm.data_ptr(),
                                       sm.data_ptr(), 1)
    log(f"skipnorm swiglu {op.name}: {info}")
    assert info["fused"]
    h = torch.full((1, op.N), float("nan"), device="cuda")
    native.gemm_dev_skipnorm_swiglu(wg, wu, dx.data_ptr(), ds.data_ptr(), dg.data_ptr(), eps, norm.data_ptr(),
                                    sm.data_ptr(), h.data_ptr(), 1)
    out_ref = _check_norm_outputs(host(norm), host(sm), x, s, g, eps)
    n2, h2 = torch.empty_like(dx), torch.empty_like(h)
    native.skip_rmsnorm(dx.data_ptr(), ds.data_ptr(), dg.data_ptr(), None, None, n2.data_ptr(), None, None, 1, op.K,
                        eps)
    native.gemm_dev_swiglu(wg, wu, n2.data_ptr(), h2.data_ptr(), 1)
    got, sep = host(h).astype(np.float64), host(h2).astype(np.float64)
    bg, sg, zg = workloads.make_weights(op, 71)
    bu, su, zu = workloads.make_weights(op, 72)
    gr = oracle.matmul_nbits(out_ref, bg, sg, zg, op.N, op.K, op.bits, op.block_size).astype(np.float64)
    ur = oracle.matmul_nbits(out_ref, bu, su, zu, op.N, op.K, op.bits, op.block_size).astype(np.float64)
    hr = gr / (1 + np.exp(-gr)) * ur
    for what, v in (("oracle", hr), ("unfused", sep)):
        rel = np.linalg.norm(got - v) / np.linalg.norm(v)
        log(f"  against the {what}: relative Frobenius {rel:.2e}")
        assert rel <= 1e-5
    wg.close()
    wu.close()


def test_skipnorm_rejects_outputs_over_inputs(gpu):
    """The fused launch's workgroups read X and Skip while workgroup 0 writes the sum and the
    normed rows, so those outputs may not overlap the inputs (the residual stream needs a
    second buffer)."""
    import torch
    op = workloads.Op("a", 512, 64, 32, True)
    w = native.NBitsWeights(*workloads.make_weights(op, 1), op.N, op.K, op.bits, op.block_size)
    x, s, g = (dev(v) for v in _norm_inputs(1, op.K, seed=2))
    norm, y = torch.empty_like(x), torch.empty((1, op.N), device="cuda")
    for dnorm, dsum, dy in ((norm, s, y), (x, None, y), (norm, norm, y), (norm, None, x), (norm, None, norm)):
        with pytest.raises(native.HipError) as e:
            native.gemm_dev_skipnorm([w], x.data_ptr(), s.data_ptr(), g.data_ptr(), 1e-6, dnorm.data_ptr(),
                                     None if dsum is None else dsum.data_ptr(), [dy.data_ptr()], 1)
        assert e.value.status == native.MS_HIP_ERR_INVALID and "overlap" in e.value.message
    w.close()


# ---- GroupQueryAttention ---------------------------------------------------------------------
from test_oracle_decoder import GQA_CASES, make_case   # noqa: E402


def run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin, capacity=None, workspace=False):
    import torch
    total = d.past_seq + d.kv_seq
    cap = capacity or total
    nd = native.GqaDesc(**{f: getattr(d, f) for f, _ in d._fields_})
    nd.present_capacity = cap
    ws_bytes = native.gqa_workspace_size(nd) if workspace else 0
    ws = torch.empty(max(1, ws_bytes // 4), device="cuda") if ws_bytes else None
    PK = torch.zeros((d.batch, d.kv_num_heads, cap, d.head_dim), device="cuda")
    PV = torch.zeros_like(PK)
    out = torch.empty((d.batch, d.q_seq, d.num_heads * d.head_dim), device="cuda")
    t = {n: (None if a is None else dev(a)) for n, a in dict(q=q, k=k, v=v, pk=pk, pv=pv, sl=sl, cos=cos,
                                                                sin=sin).items()}
    ptr = lambda x: None if x is None else x.data_ptr()   # noqa: E731
    native.gqa(nd, ptr(t["q"]), ptr(t["k"]), ptr(t["v"]), ptr(t["pk"]), ptr(t["pv"]), ptr(t["sl"]), ptr(t["cos"]),
               ptr(t["sin"]), out.data_ptr(), PK.data_ptr(), PV.data_ptr(), ptr(ws), ws_bytes)
    return host(out), host(PK)[:, :, :total], host(PV)[:, :, :total]


def check_gqa(out, PK, PV, ref, rk, rv, what):
    assert np.array_equal(PK, rk), what
    assert np.array_equal(PV, rv), what
    err = np.max(np.abs(out - ref)) / max(np.abs(ref).max(), 1e-30)
    log(f"  {what}: max err / max|out| {err:.2e}")
    assert err <= 1e-5, what


@pytest.mark.parametrize("case", GQA_CASES, ids=lambda c: f"seed{c['seed']}")
def test_gqa_cases(gpu, case):
    d, q, k, v, pk, pv, sl, cos, sin = make_case(**case)
    ref, rk, rv = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    check_gqa(*run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin, capacity=d.past_seq + d.kv_seq + 7),
              ref, rk, rv, f"seed {case['seed']}")


# The grouped kernel (head_dim 64 / 128, up to 8 query heads per kv head, up to 8 queries):
# every option of the operator at those head dims, with and without key splits.
GROUPED_CASES = [
    dict(seed=101, B=1, Sq=1, H=28, KH=4, D=128, past=2047, cos_rows=2048),          # the 7B decode step
    dict(seed=102, B=2, Sq=5, H=8, KH=1, D=64, past=3),                              # MQA, 8 heads per kv head
    dict(seed=103, B=1, Sq=4, H=6, KH=3, D=128, past=0, packed=True),                # packed QKV, no past
    dict(seed=104, B=1, Sq=3, H=4, KH=2, D=64, past=600, interleaved=True, cos_rows=700),
    dict(seed=105, B=2, Sq=8, H=4, KH=2, D=128, past=45, window=7),                  # sliding window
    dict(seed=106, B=2, Sq=2, H=4, KH=2, D=64, past=70, seqlens=[40, 71], cos_rows=80),   # seqlens_k bound
    dict(seed=107, B=1, Sq=3, H=6, KH=2, D=128, past=33, cos_cols=24),               # partial rotary span
    dict(seed=108, B=1, Sq=2, H=2, KH=2, D=64, past=90, cos_rows=64),                # positions past the cache
    dict(seed=109, B=1, Sq=1, H=14, KH=2, D=128, past=5000, rotary=False, cos_rows=8),
    dict(seed=110, B=1, Sq=2, H=8, KH=2, D=128, past=40, kv_seq=12, cos_rows=64),   # more than 8 new rows
    dict(seed=111, B=2, Sq=4, H=4, KH=2, D=64, past=30, kv_seq=2, cos_rows=64),     # fewer new rows than queries
]


@pytest.mark.parametrize("workspace", [False, True], ids=["one_split", "key_splits"])
@pytest.mark.parametrize("case", GROUPED_CASES, ids=lambda c: f"seed{c['seed']}")
def test_gqa_grouped_cases(gpu, case, workspace):
    d, q, k, v, pk, pv, sl, cos, sin = make_case(**case)
    ref, rk, rv = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    check_gqa(*run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin, capacity=d.past_seq + d.kv_seq + 3,
                              workspace=workspace), ref, rk, rv, f"grouped seed {case['seed']} workspace={workspace}")


# The flash kernel (head_dim 64 / 128, more than 8 queries): every option of the operator.
FLASH_CASES = [
    dict(seed=201, B=1, Sq=200, H=28, KH=4, D=128, past=0, cos_rows=256),            # 7B heads, ragged block
    dict(seed=202, B=2, Sq=70, H=8, KH=1, D=64, past=5, cos_rows=128),               # MQA, past
    dict(seed=203, B=1, Sq=33, H=6, KH=3, D=128, past=100, packed=True, cos_rows=160),
    dict(seed=204, B=1, Sq=64, H=4, KH=2, D=64, past=0, interleaved=True, cos_rows=64),
    dict(seed=205, B=2, Sq=90, H=4, KH=2, D=128, past=30, window=17, cos_rows=128),  # sliding window
    dict(seed=206, B=2, Sq=40, H=4, KH=2, D=64, past=10, seqlens=[20, 49], cos_rows=64),   # seqlens_k bound
    dict(seed=207, B=1, Sq=65, H=6, KH=2, D=128, past=0, cos_cols=24, cos_rows=80),  # partial rotary span
    dict(seed=208, B=1, Sq=20, H=2, KH=2, D=64, past=90, cos_rows=64),               # positions past the cache
    dict(seed=209, B=1, Sq=129, H=14, KH=2, D=128, past=700, rotary=False, cos_rows=8),
    dict(seed=210, B=1, Sq=20, H=4, KH=2, D=64, past=10, kv_seq=28, cos_rows=64),    # more new keys than queries
]


@pytest.mark.parametrize("case", FLASH_CASES, ids=lambda c: f"seed{c['seed']}")
def test_gqa_flash_cases(gpu, case):
    d, q, k, v, pk, pv, sl, cos, sin = make_case(**case)
    ref, rk, rv = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    check_gqa(*run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin, capacity=d.past_seq + d.kv_seq + 5), ref, rk, rv,
              f"flash seed {case['seed']}")


@pytest.mark.parametrize("workspace", [False, True], ids=["one_split", "key_splits"])
@pytest.mark.parametrize("Sq,past,KH", [(1, 2047, 8), (1, 4095, 32), (128, 0, 8), (16, 300, 8)])
def test_gqa_7b_shapes(gpu, Sq, past, KH, workspace):
    d, q, k, v, pk, pv, sl, cos, sin = make_case(20 + Sq, B=1, Sq=Sq, H=32, KH=KH, D=128, past=past, packed=True,
                                                 cos_rows=4096 + 128)
    ref, rk, rv = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    check_gqa(*run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin, workspace=workspace), ref, rk, rv,
              f"7B Sq={Sq} past={past} KH={KH} workspace={workspace}")


@pytest.mark.parametrize("D", [32, 64, 256, 40])
def test_gqa_head_dims_and_long_history(gpu, D):
    """Every lane-group width, the per-unit kernel (head_dim 40), and a history longer than
    one workgroup's LDS holds (key splits required)."""
    past = 60000 if D == 64 else 700
    d, q, k, v, pk, pv, sl, cos, sin = make_case(40 + D, B=1, Sq=1, H=4, KH=2, D=D, past=past, packed=False,
                                                 cos_rows=past + 8)
    ref, rk, rv = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    check_gqa(*run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin, workspace=True), ref, rk, rv, f"D={D} past={past}")
    if D != 64:
        check_gqa(*run_device_gqa(d, q, k, v, pk, pv, sl, cos, sin), ref, rk, rv, f"D={D} unsplit")


def test_gqa_resident_cache_appends_in_place(gpu):
    """Five decode steps through the operator kernel, each passing the previous present
    K/V back as past: the cache buffer stays put and every step matches the oracle run
    on the whole history."""
    r = np.random.default_rng(3)
    H, KH, D, S0 = 4, 2, 64, 6
    cos_rows = 64
    ang = np.outer(np.arange(cos_rows), 1.0 / 10000 ** (np.arange(D // 2) / (D // 2)))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    node = GraphNode("GroupQueryAttention", "attn0", ["qkv", "", "", "past_k", "past_v", "", "", "cos", "sin"],
                     ["out", "present_k", "present_v"],
                     {"num_heads": H, "kv_num_heads": KH, "do_rotary": 1})
    node0 = GraphNode("GroupQueryAttention", "attn0", ["qkv", "", "", "", "", "", "", "cos", "sin"],
                      ["out", "present_k", "present_v"], node.attributes)
    k = HipGroupQueryAttentionKernel()
    hist_k = hist_v = None
    ptr0 = None
    for step in range(6):
        S = S0 if step == 0 else 1
        qkv = r.standard_normal((1, S, (H + 2 * KH) * D)).astype(np.float32)
        ctx = GraphContext({"qkv": dev(qkv), "cos": cos, "sin": sin})
        if step:
            ctx.set("past_k", pres_k)
            ctx.set("past_v", pres_v)
        k.execute(node if step else node0, ctx)
        out, pres_k, pres_v = ctx.get_tensor("out"), ctx.get_tensor("present_k"), ctx.get_tensor("present_v")
        if step == 0:
            ptr0 = pres_k.data_ptr()
        assert pres_k.data_ptr() == ptr0   # appended in place (capacity 64)
        past = 0 if step == 0 else hist_k.shape[2]
        d = oracle.GqaDesc(batch=1, q_seq=S, kv_seq=S, num_heads=H, kv_num_heads=KH, head_dim=D, packed_qkv=1,
                           past_seq=past, present_capacity=past + S, do_rotary=1, cos_rows=cos_rows, cos_cols=D // 2,
                           local_window_size=-1)
        ref, hist_k, hist_v = oracle.gqa(d, qkv, None, None, hist_k, hist_v, None, cos, sin)
        check_gqa(host(out), host(pres_k), host(pres_v), ref, hist_k, hist_v, f"step {step}")
    k._caches.clear()


def test_gqa_two_steps_from_one_past_leave_earlier_presents_alone(gpu):
    """Two candidate tokens decoded from the same past (beam search, a retry): the second
    call must not write into the rows the first call returned as its present K/V. Each
    call's outputs and presents are checked against the oracle after both calls, and a
    third step that follows the second call's present appends in place again."""
    r = np.random.default_rng(8)
    H, KH, D, S0 = 4, 2, 64, 5
    cos_rows = 64
    ang = np.outer(np.arange(cos_rows), 1.0 / 10000 ** (np.arange(D // 2) / (D // 2)))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    attrs = {"num_heads": H, "kv_num_heads": KH, "do_rotary": 1}
    node0 = GraphNode("GroupQueryAttention", "attn0", ["qkv", "", "", "", "", "", "", "cos", "sin"],
                      ["out", "present_k", "present_v"], attrs)
    node = GraphNode("GroupQueryAttention", "attn0", ["qkv", "", "", "past_k", "past_v", "", "", "cos", "sin"],
                     ["out", "present_k", "present_v"], attrs)
    k = HipGroupQueryAttentionKernel()

    def desc(S, past):
        return oracle.GqaDesc(batch=1, q_seq=S, kv_seq=S, num_heads=H, kv_num_heads=KH, head_dim=D, packed_qkv=1,
                              past_seq=past, present_capacity=past + S, do_rotary=1, cos_rows=cos_rows,
                              cos_cols=D // 2, local_window_size=-1)

    qkv0 = r.standard_normal((1, S0, (H + 2 * KH) * D)).astype(np.float32)
    ctx = GraphContext({"qkv": dev(qkv0), "cos": cos, "sin": sin})
    k.execute(node0, ctx)
    pk0, pv0 = ctx.get_tensor("present_k"), ctx.get_tensor("present_v")
    _, hk0, hv0 = oracle.gqa(desc(S0, 0), qkv0, None, None, None, None, None, cos, sin)
    runs = []
    for cand in range(2):
        qkv = r.standard_normal((1, 1, (H + 2 * KH) * D)).astype(np.float32)
        c = GraphContext({"qkv": dev(qkv), "cos": cos, "sin": sin, "past_k": pk0, "past_v": pv0})
        k.execute(node, c)
        runs.append((qkv, c.get_tensor("out"), c.get_tensor("present_k"), c.get_tensor("present_v")))
    log(f"candidate presents at {runs[0][2].data_ptr():#x} and {runs[1][2].data_ptr():#x}")
    for i, (qkv, out, pk, pv) in enumerate(runs):
        ref, rk, rv = oracle.gqa(desc(1, S0), qkv, None, None, hk0, hv0, None, cos, sin)
        check_gqa(host(out), host(pk), host(pv), ref, rk, rv, f"candidate {i} after both calls")
    check_gqa(host(runs[0][1]), host(pk0), host(pv0), oracle.gqa(desc(1, S0), runs[0][0], None, None, hk0, hv0,
                                                                   None, cos, sin)[0], hk0, hv0, "the shared past")
    # the next step from the second candidate's present follows the cache: in place
    qkv2 = r.standard_normal((1, 1, (H + 2 * KH) * D)).astype(np.float32)
    c = GraphContext({"qkv": dev(qkv2), "cos": cos, "sin": sin, "past_k": runs[1][2], "past_v": runs[1][3]})
    k.execute(node, c)
    assert c.get_tensor("present_k").data_ptr() == runs[1][2].data_ptr()
    _, rk1, rv1 = oracle.gqa(desc(1, S0), runs[1][0], None, None, hk0, hv0, None, cos, sin)
    ref, rk, rv = oracle.gqa(desc(1, S0 + 1), qkv2, None, None, rk1, rv1, None, cos, sin)
    check_gqa(host(c.get_tensor("out")), host(c.get_tensor("present_k")), host(c.get_tensor("present_v")), ref, rk,
              rv, "step after candidate 1")
    # the first candidate's present is still its own
    _, rk0, rv0 = oracle.gqa(desc(1, S0), runs[0][0], None, None, hk0, hv0, None, cos, sin)
    assert np.array_equal(host(runs[0][2]), rk0) and np.array_equal(host(runs[0][3]), rv0)
    k._caches.clear()


# ---- one decoder layer end to end ---------------------------------------------------------------
def layer_graph(hid, H, KH, D, inter, bs, seed):
    """A Llama-family decoder layer as the onnxruntime-genai INT4 exports lay it out:
    SkipSimplifiedLayerNormalization, packed q/k/v MatMulNBits, GroupQueryAttention with
    in-op rotary, o projection, SkipSimplifiedLayerNormalization, gate/up MatMulNBits,
    Sigmoid -> Mul -> Mul, down MatMulNBits."""
    r = np.random.default_rng(seed)
    inits = {}

    def mm(name, K, N):
        op = workloads.Op(name, K, N, bs, True)
        b, s, z = workloads.make_weights(op, seed + K + N)
        inits.update({f"{name}.B": b, f"{name}.s": s, f"{name}.z": z})
        return GraphNode("MatMulNBits", name, ["", f"{name}.B", f"{name}.s", f"{name}.z"], [""],
                         {"K": K, "N": N, "bits": 4, "block_size": bs})

    def wire(n, inputs, outputs):
        n.inputs[0] = inputs
        n.outputs = outputs
        return n

    inits["ln1.g"] = r.uniform(0.5, 1.5, hid).astype(np.float32)
    inits["ln2.g"] = r.uniform(0.5, 1.5, hid).astype(np.float32)
    ang = np.outer(np.arange(256), 1.0 / 10000 ** (np.arange(D // 2) / (D // 2)))
    inits["cos"], inits["sin"] = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    nodes = [
        GraphNode("SkipSimplifiedLayerNormalization", "ln1", ["x", "resid", "ln1.g"], ["n1", "", "", "t1"],
                  {"epsilon": 1e-5}),
        wire(mm("qkv", hid, (H + 2 * KH) * D), "n1", ["qkv_out"]),
        GraphNode("GroupQueryAttention", "attn", ["qkv_out", "", "", "past_k", "past_v", "", "", "cos", "sin"],
                  ["attn_out", "present_k", "present_v"], {"num_heads": H, "kv_num_heads": KH, "do_rotary": 1}),
        wire(mm("o", H * D, hid), "attn_out", ["o_out"]),
        GraphNode("SkipSimplifiedLayerNormalization", "ln2", ["o_out", "t1", "ln2.g"], ["n2", "", "", "t2"],
                  {"epsilon": 1e-5}),
        wire(mm("gate", hid, inter), "n2", ["g"]),
        wire(mm("up", hid, inter), "n2", ["u"]),
        GraphNode("Sigmoid", "sig", ["g"], ["sg"]),
        GraphNode("Mul", "m1", ["g", "sg"], ["act0"]),
        GraphNode("Mul", "m2", ["act0", "u"], ["act"]),
        wire(mm("down", inter, hid), "act", ["y"]),
    ]
    return ModelGraph(nodes, inits, ["x", "resid", "past_k", "past_v"], ["y", "t2", "present_k", "present_v"])


def layer_oracle(g, x, resid, past_k, past_v, hid, H, KH, D, inter, bs):
    I = g.initializers

    def mm(name, a, K, N):
        return oracle.matmul_nbits(a.reshape(-1, K), I[f"{name}.B"], I[f"{name}.s"], I[f"{name}.z"], N, K, 4, bs)

    S = x.shape[1]
    n1, _, t1 = oracle.skip_rmsnorm(x.reshape(-1, hid), resid.reshape(-1, hid), I["ln1.g"], None, None, 1e-5)
    qkv = mm("qkv", n1, hid, (H + 2 * KH) * D).reshape(1, S, -1)
    past = 0 if past_k is None else past_k.shape[2]
    d = oracle.GqaDesc(batch=1, q_seq=S, kv_seq=S, num_heads=H, kv_num_heads=KH, head_dim=D, packed_qkv=1,
                       past_seq=past, present_capacity=past + S, do_rotary=1, cos_rows=256, cos_cols=D // 2,
                       local_window_size=-1)
    attn, pk, pv = oracle.gqa(d, qkv, None, None, past_k, past_v, None, I["cos"], I["sin"])
    o = mm("o", attn, H * D, hid)
    n2, _, t2 = oracle.skip_rmsnorm(o, t1, I["ln2.g"], None, None, 1e-5)
    act = oracle.silu_mul(mm("gate", n2, hid, inter), mm("up", n2, hid, inter))
    y = mm("down", act, inter, hid)
    return y.reshape(1, S, hid), t2.reshape(1, S, hid), pk, pv


@pytest.mark.parametrize("fused", [False, True])
def test_decoder_layer_end_to_end(gpu, fused):
    """Prefill of 5 tokens, then 3 decode steps, the whole layer on the device (no host
    round trip between operators), against the oracle composed on the CPU; fused: SiLU-Mul,
    gate/up and both norms folded into the launches of the projections (the norm computed
    in the projection launch's staging at the decode steps, apart at the prefill)."""
    import torch
    hid, H, KH, D, inter, bs = 512, 8, 2, 64, 1024, 32
    g = layer_graph(hid, H, KH, D, inter, bs, seed=1)
    if fused:
        assert fuse_silu_mul(g) == 1 and [n.op_type for n in g.nodes].count("SiluMul") == 1
        assert fuse_gate_up_silu(g) == 1 and [n.op_type for n in g.nodes].count("GateUpSiluMul") == 1
        assert fuse_skipnorm(g) == 2
        ops = [n.op_type for n in g.nodes]
        assert ops.count("SkipNormMatMulNBits") == 1 and ops.count("SkipNormGateUpSiluMul") == 1
    reg = register_decoder_kernels(register_kernels(KernelRegistry()))
    eng = Engine(g, reg)
    r = np.random.default_rng(2)
    pk = pv = None
    hk = hv = None
    for step, S in enumerate([5, 1, 1, 1]):
        x = r.standard_normal((1, S, hid)).astype(np.float32)
        resid = r.standard_normal((1, S, hid)).astype(np.float32)
        feeds = {"x": dev(x), "resid": dev(resid)}
        if pk is not None:
            feeds.update(past_k=pk, past_v=pv)
        else:
            g.nodes[[n.op_type for n in g.nodes].index("GroupQueryAttention")].inputs[3:5] = ["", ""]
        res = eng.run(feeds)
        y, t2, pk, pv = res["y"], res["t2"], res["present_k"], res["present_v"]
        assert isinstance(y, torch.Tensor) and y.is_cuda
        ry, rt2, hk, hv = layer_oracle(g, x, resid, hk, hv, hid, H, KH, D, inter, bs)
        if step == 0:
            g.nodes[[n.op_type for n in g.nodes].index("GroupQueryAttention")].inputs[3:5] = ["past_k", "past_v"]
        err = np.max(np.abs(host(y) - ry)) / np.abs(ry).max()
        log(f"  step {step} (S={S}) fused={fused}: max err / max|y| {err:.2e}")
        assert err <= 1e-4
        assert np.allclose(host(t2), rt2, rtol=1e-5, atol=1e-5 * np.abs(rt2).max())


# ---- the reference's own known answers (tests/golden/decoder_kats.json) -------------------------
import decoder_kats  # noqa: E402

_KAT_TOL, _KAT_CASES = decoder_kats.load()


@pytest.mark.parametrize("case", _KAT_CASES, ids=[c["name"] for c in _KAT_CASES])
def test_reference_known_answers(gpu, case):
    """FusedLlmNormTests.cs:47-131, GqaGenaiTests.cs:106-381, GqaSlidingWindowTests.cs:110-245
    through the device kernels behind the operator interface, at the reference tests' 1e-4
    (host arrays in the context, as those tests build it)."""
    log(f"decoder known answer {case['name']}")
    decoder_kats.check(case, decoder_kats.device_run(case), _KAT_TOL)
