"""Pins the oracle's decoder-layer operators (oracle/ms_decoder_oracle.c) against float64
closed forms and brute force, and against special cases whose answer is exact.

References: SimplifiedLayerNormalizationKernel.cs, SkipSimplifiedLayerNormalizationKernel.cs,
SigmoidKernel.cs, GroupQueryAttentionKernel.cs (src/ModelSharp/Cpu/Kernels/...).
"""
from __future__ import annotations

import json

import numpy as np
import pytest

import decoder_kats
import oracle


def rng(seed):
    return np.random.default_rng(seed)


# ---- norms ------------------------------------------------------------------------------------
def rms_f64(x, w, eps):
    x = x.astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * inv * w.astype(np.float64), inv[..., 0]


@pytest.mark.parametrize("rows,norm", [(1, 4096), (5, 100), (3, 7), (2, 8)])
def test_rmsnorm_vs_f64(rows, norm):
    r = rng(norm)
    x = (r.standard_normal((rows, norm)) * 3).astype(np.float32)
    w = r.uniform(0.5, 1.5, norm).astype(np.float32)
    y, inv = oracle.rmsnorm(x, w, 1e-5)
    ref, inv_ref = rms_f64(x, w, 1e-5)
    assert np.allclose(inv, inv_ref, rtol=2e-6, atol=0)
    assert np.all(np.abs(y - ref) <= 4e-7 * np.abs(ref) + 1e-30 + 4e-7 * np.abs(x * inv[:, None]).max())


def test_rmsnorm_exact_on_constant_rows():
    """x = 2 everywhere, eps = 0: mean(x^2) = 4 exactly, inv = 1/2 exactly, y = scale."""
    x = np.full((3, 64), 2.0, np.float32)
    w = rng(1).standard_normal(64).astype(np.float32)
    y, inv = oracle.rmsnorm(x, w, 0.0)
    assert np.all(inv == 0.5) and np.array_equal(y, np.broadcast_to(w, y.shape))


def test_skip_rmsnorm_sum_and_norm():
    r = rng(2)
    rows, norm = 4, 96
    a = r.standard_normal((rows, norm)).astype(np.float32)
    s = r.standard_normal((rows, norm)).astype(np.float32)
    bias = r.standard_normal(norm).astype(np.float32)
    beta = r.standard_normal(norm).astype(np.float32)
    g = r.uniform(0.5, 1.5, norm).astype(np.float32)
    out, inv, total = oracle.skip_rmsnorm(a, s, g, beta, bias, 1e-6)
    assert np.array_equal(total, (a + s) + bias)   # fp32 adds, in the reference's order
    ref, inv_ref = rms_f64(total, g, 1e-6)
    ref = ref + beta.astype(np.float64)
    assert np.allclose(inv, inv_ref, rtol=2e-6, atol=0)
    assert np.allclose(out, ref, rtol=1e-6, atol=1e-6)
    out2, _, total2 = oracle.skip_rmsnorm(a, s, g, None, None, 1e-6)
    assert np.array_equal(total2, a + s)


def test_silu_mul_closed_form():
    r = rng(3)
    g = (r.standard_normal(1000) * 6).astype(np.float32)
    u = r.standard_normal(1000).astype(np.float32)
    y = oracle.silu_mul(g, u)
    g64 = g.astype(np.float64)
    ref = g64 / (1 + np.exp(-g64)) * u
    assert np.allclose(y, ref, rtol=2e-6, atol=1e-30)
    assert np.array_equal(oracle.silu_mul(np.zeros(4, np.float32), np.ones(4, np.float32)), np.zeros(4, np.float32))
    # odd symmetry of the logistic: g*s(g) - (-g)*s(-g) = g
    x = np.linspace(-8, 8, 33).astype(np.float32)
    d = oracle.silu_mul(x, np.ones_like(x)).astype(np.float64) - oracle.silu_mul(-x, np.ones_like(x))
    assert np.allclose(d, x, rtol=1e-6, atol=1e-6)


# ---- GroupQueryAttention ---------------------------------------------------------------------
def rope_f64(x, pos, cos, sin, half, rot_half, interleaved):
    x = x.astype(np.float64).copy()
    c = cos[pos, :rot_half].astype(np.float64)
    s = sin[pos, :rot_half].astype(np.float64)
    if interleaved:
        i0, i1 = np.arange(rot_half) * 2, np.arange(rot_half) * 2 + 1
    else:
        i0, i1 = np.arange(rot_half), np.arange(rot_half) + rot_half
    a, b = x[i0].copy(), x[i1].copy()
    x[i0] = a * c - b * s
    x[i1] = b * c + a * s
    return x


def gqa_f64(d, q, k, v, pk, pv, seqlens, cos, sin):
    B, Sq, Skv, H, KH, D, past = d.batch, d.q_seq, d.kv_seq, d.num_heads, d.kv_num_heads, d.head_dim, d.past_seq
    qh, kvh = H * D, KH * D
    if d.packed_qkv:
        qq, kk, vv = q[..., :qh], q[..., qh:qh + kvh], q[..., qh + kvh:]
    else:
        qq, kk, vv = q, k, v
    total = past + Skv
    rot_half = min(2 * d.cos_cols, D) // 2 if d.do_rotary else 0
    Kf = np.zeros((B, KH, total, D))
    Vf = np.zeros((B, KH, total, D))
    if past:
        Kf[:, :, :past] = pk
        Vf[:, :, :past] = pv
    for b in range(B):
        for s in range(Skv):
            for g in range(KH):
                row = kk[b, s, g * D:(g + 1) * D]
                if d.do_rotary:
                    row = rope_f64(row, min(past + s, d.cos_rows - 1), cos, sin, d.cos_cols, rot_half,
                                   d.rotary_interleaved)
                Kf[b, g, past + s] = row
                Vf[b, g, past + s] = vv[b, s, g * D:(g + 1) * D]
    scale = d.scale if d.scale != 0 else 1.0 / np.sqrt(D)
    out = np.zeros((B, Sq, qh))
    for b in range(B):
        for h in range(H):
            g = h // (H // KH)
            for qi in range(Sq):
                qa = past + qi
                lim = min(qa, total - 1 if seqlens is None else min(total - 1, seqlens[min(b, len(seqlens) - 1)]))
                st = max(0, qa - d.local_window_size + 1) if d.local_window_size >= 0 else 0
                if lim < st:
                    continue
                qr = qq[b, qi, h * D:(h + 1) * D]
                if d.do_rotary:
                    qr = rope_f64(qr, min(qa, d.cos_rows - 1), cos, sin, d.cos_cols, rot_half, d.rotary_interleaved)
                sc = Kf[b, g, st:lim + 1] @ qr.astype(np.float64) * scale
                p = np.exp(sc - sc.max())
                out[b, qi, h * D:(h + 1) * D] = (p / p.sum()) @ Vf[b, g, st:lim + 1]
    return out, Kf, Vf


def make_case(seed, B, Sq, H, KH, D, past, packed=False, rotary=True, interleaved=False, window=-1, seqlens=None,
              cos_rows=64, cos_cols=None, kv_seq=None):
    # kv_seq: new key/value rows, Sq unless given (the reference takes key.Shape[1],
    # GroupQueryAttentionKernel.cs:131; packed QKV shares the query length, :104)
    Skv = Sq if kv_seq is None else kv_seq
    r = rng(seed)
    d = oracle.GqaDesc(batch=B, q_seq=Sq, kv_seq=Skv, num_heads=H, kv_num_heads=KH, head_dim=D,
                       packed_qkv=int(packed), past_seq=past, past_in_present=0, present_capacity=past + Skv,
                       do_rotary=int(rotary), rotary_interleaved=int(interleaved), cos_rows=cos_rows,
                       cos_cols=cos_cols if cos_cols is not None else D // 2, local_window_size=window, scale=0.0,
                       seqlens_len=0 if seqlens is None else len(seqlens))
    if packed:
        q = r.standard_normal((B, Sq, (H + 2 * KH) * D)).astype(np.float32)
        k = v = None
    else:
        q = r.standard_normal((B, Sq, H * D)).astype(np.float32)
        k = r.standard_normal((B, Skv, KH * D)).astype(np.float32)
        v = r.standard_normal((B, Skv, KH * D)).astype(np.float32)
    pk = r.standard_normal((B, KH, past, D)).astype(np.float32) if past else None
    pv = r.standard_normal((B, KH, past, D)).astype(np.float32) if past else None
    ang = np.outer(np.arange(cos_rows), 1.0 / 10000 ** (np.arange(d.cos_cols) / d.cos_cols))
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    sl = None if seqlens is None else np.array(seqlens, np.int32)
    return d, q, k, v, pk, pv, sl, cos, sin


GQA_CASES = [
    dict(seed=1, B=1, Sq=1, H=4, KH=2, D=16, past=9),                            # decode
    dict(seed=2, B=2, Sq=5, H=4, KH=1, D=8, past=3),                             # prefill, MQA
    dict(seed=3, B=1, Sq=4, H=6, KH=3, D=12, past=0, packed=True),               # packed QKV
    dict(seed=4, B=1, Sq=3, H=2, KH=2, D=16, past=6, interleaved=True),
    dict(seed=5, B=2, Sq=4, H=4, KH=2, D=16, past=5, window=3),                  # sliding window
    dict(seed=6, B=2, Sq=2, H=4, KH=2, D=16, past=7, seqlens=[5, 8]),            # seqlens_k bound
    dict(seed=7, B=1, Sq=3, H=2, KH=1, D=20, past=2, cos_cols=6),                # partial rotary span
    dict(seed=8, B=1, Sq=2, H=2, KH=2, D=8, past=70, cos_rows=64),               # position past the cache
    dict(seed=9, B=1, Sq=3, H=4, KH=2, D=16, past=4, rotary=False),
    dict(seed=10, B=1, Sq=2, H=4, KH=2, D=16, past=5, kv_seq=6),                 # more new keys than queries
    dict(seed=12, B=2, Sq=4, H=4, KH=2, D=16, past=3, kv_seq=2),                 # fewer new keys than queries
]


@pytest.mark.parametrize("case", GQA_CASES, ids=lambda c: f"seed{c['seed']}")
def test_gqa_vs_f64(case):
    d, q, k, v, pk, pv, sl, cos, sin = make_case(**case)
    out, Kp, Vp = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    ref, Kf, Vf = gqa_f64(d, q, k, v, pk, pv, sl, cos, sin)
    assert np.allclose(Kp, Kf, rtol=1e-6, atol=1e-6)
    assert np.array_equal(Vp, Vf.astype(np.float32))
    assert np.allclose(out, ref, rtol=1e-5, atol=1e-5)


def test_gqa_window_one_returns_the_current_value_row():
    d, q, k, v, pk, pv, sl, cos, sin = make_case(11, B=1, Sq=3, H=4, KH=2, D=8, past=4, window=1)
    out, Kp, Vp = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    for qi in range(3):
        for h in range(4):
            assert np.array_equal(out[0, qi, h * 8:(h + 1) * 8], Vp[0, h // 2, 4 + qi])


def test_gqa_equal_scores_average_the_values():
    d, q, k, v, pk, pv, sl, cos, sin = make_case(12, B=1, Sq=2, H=2, KH=1, D=8, past=3, rotary=False)
    q[:] = 0.0
    out, Kp, Vp = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    for qi in range(2):
        mean = Vp[0, 0, :3 + qi + 1].astype(np.float64).mean(axis=0)
        assert np.allclose(out[0, qi, :8], mean, rtol=1e-6, atol=1e-6)


def test_gqa_rotary_identity_and_norms():
    d, q, k, v, pk, pv, sl, cos, sin = make_case(13, B=1, Sq=2, H=2, KH=2, D=16, past=0)
    out, Kp, _ = oracle.gqa(d, q, k, v, pk, pv, sl, np.ones_like(cos), np.zeros_like(sin))
    assert np.array_equal(Kp[0, :, :, :], k.reshape(2, 2, 16).transpose(1, 0, 2))
    _, Kr, _ = oracle.gqa(d, q, k, v, pk, pv, sl, cos, sin)
    kk = k.reshape(2, 2, 16).transpose(1, 0, 2).astype(np.float64)
    pairs = lambda x: x[..., :8] ** 2 + x[..., 8:] ** 2
    assert np.allclose(pairs(Kr.astype(np.float64)), pairs(kk), rtol=1e-5)


# ---- the reference's own known answers (tests/golden/decoder_kats.json) -------------------------
_KAT_TOL, _KAT_CASES = decoder_kats.load()


@pytest.mark.parametrize("case", _KAT_CASES, ids=[c["name"] for c in _KAT_CASES])
def test_reference_known_answers(case):
    """FusedLlmNormTests.cs:47-131, GqaGenaiTests.cs:106-381, GqaSlidingWindowTests.cs:110-245:
    the oracle meets each case's expected outputs at the reference tests' 1e-4, including
    the reading of seqlens_k as the last valid key index (Decode_WithPast_AndSeqlensK,
    SeqlensK_BoundsKeyRange, DecodeWithPast_WindowExcludesOldCachedKeys)."""
    decoder_kats.check(case, decoder_kats.oracle_run(case), _KAT_TOL)


def test_reference_known_answers_catch_a_planted_mistake():
    """The fixture rejects a seqlens_k read as a key count instead of the last valid index:
    SeqlensK_BoundsKeyRange then lets both queries see key 1 as well."""
    case = next(c for c in _KAT_CASES if c["name"] == "SeqlensK_BoundsKeyRange")
    wrong = json.loads(json.dumps(case))
    wrong["inputs"]["seqlens_k"]["data"] = [1]
    with pytest.raises(AssertionError):
        decoder_kats.check(case, decoder_kats.oracle_run(wrong), _KAT_TOL)
