"""The reference's decoder-operator known answers (tests/golden/decoder_kats.json, written by
tests/golden/make_decoder_kats.py from FusedLlmNormTests.cs, GqaGenaiTests.cs and
GqaSlidingWindowTests.cs) run through the oracle or through the device kernels behind the
operator interface, the way the reference's tests drive its managed kernels: one
GraphNode and a GraphContext of host arrays per case."""
from __future__ import annotations

import json
import pathlib

import numpy as np

FIXTURE = pathlib.Path(__file__).resolve().parent / "golden" / "decoder_kats.json"
GQA_INPUTS = ["q", "k", "v", "past_key", "past_value", "seqlens_k", "total_sequence_length", "cos", "sin"]


def load():
    d = json.loads(FIXTURE.read_text())
    return d["tolerance"], d["cases"]


def arrays(case):
    out = {}
    for name, t in case["inputs"].items():
        dt = np.int32 if t["dtype"] == "int32" else np.float32
        out[name] = np.array(t["data"], dt).reshape(t["shape"])
    return out


def oracle_run(case):
    """The case through the oracle (oracle/ms_decoder_oracle.c)."""
    import oracle
    x = arrays(case)
    at = case["attrs"]
    if case["op"] == "SimplifiedLayerNormalization":
        y, inv = oracle.rmsnorm(x["x"], x["scale"], at.get("epsilon", 1e-5))
        return {"y": y, "inv": inv}
    if case["op"] == "SkipSimplifiedLayerNormalization":
        out, inv, total = oracle.skip_rmsnorm(x["input"], x["skip"], x["gamma"], x.get("beta"), x.get("bias"),
                                              at.get("epsilon", 1e-5))
        return {"out": out, "inv": inv, "sum": total}
    q = x["q"]
    H, KH = at["num_heads"], at["kv_num_heads"]
    packed = "k" not in x
    B, S = q.shape[0], q.shape[1]
    D = q.shape[2] // (H + 2 * KH) if packed else q.shape[2] // H
    skv = S if packed else x["k"].shape[1]
    past = x["past_key"].shape[2] if "past_key" in x else 0
    cos = x.get("cos")
    d = oracle.GqaDesc(batch=B, q_seq=S, kv_seq=skv, num_heads=H, kv_num_heads=KH, head_dim=D,
                       packed_qkv=int(packed), past_seq=past, past_in_present=0, present_capacity=past + skv,
                       do_rotary=at.get("do_rotary", 0), rotary_interleaved=at.get("rotary_interleaved", 0),
                       cos_rows=0 if cos is None else cos.shape[0], cos_cols=0 if cos is None else cos.shape[-1],
                       local_window_size=at.get("local_window_size", -1), scale=0.0,
                       seqlens_len=x["seqlens_k"].size if "seqlens_k" in x else 0)
    out, pk, pv = oracle.gqa(d, q, x.get("k"), x.get("v"), x.get("past_key"), x.get("past_value"),
                             x.get("seqlens_k"), cos, x.get("sin"))
    return {"out": out, "present_key": pk, "present_value": pv}


def device_run(case):
    """The case through the device kernels of modelsharp_amd.decoder_kernels (needs a GPU)."""
    import torch
    from modelsharp_amd.decoder_kernels import (HipGroupQueryAttentionKernel, HipSimplifiedLayerNormalizationKernel,
                                                HipSkipSimplifiedLayerNormalizationKernel)
    from modelsharp_amd.graph import GraphContext, GraphNode
    x = arrays(case)
    at = dict(case["attrs"])
    ctx = GraphContext(x)
    if case["op"] == "SimplifiedLayerNormalization":
        node = GraphNode(case["op"], "n", ["x", "scale"], ["y", "inv"], at)
        HipSimplifiedLayerNormalizationKernel().execute(node, ctx)
        names = ["y", "inv"]
    elif case["op"] == "SkipSimplifiedLayerNormalization":
        ins = ["input", "skip", "gamma", "beta" if "beta" in x else "", "bias" if "bias" in x else ""]
        node = GraphNode(case["op"], "n", ins, ["out", "", "inv", "sum"], at)
        HipSkipSimplifiedLayerNormalizationKernel().execute(node, ctx)
        names = ["out", "inv", "sum"]
    else:
        ins = [n if n in x else "" for n in GQA_INPUTS]
        node = GraphNode(case["op"], "n", ins, ["out", "present_key", "present_value"], at)
        HipGroupQueryAttentionKernel().execute(node, ctx)
        names = ["out", "present_key", "present_value"]
    torch.cuda.synchronize()
    return {n: ctx.get_tensor(n).cpu().numpy() for n in names}


def check(case, got, tol):
    """The reference test's assertions: every expected output within tol (absolute), the
    present shape, and the structural bounds some tests add."""
    for name, exp in case["expected"].items():
        g = np.asarray(got[name], np.float64).ravel()
        e = np.asarray(exp, np.float64)
        if name == "present_key" and g.size != e.size:
            raise AssertionError(f"{case['name']}: present_key has {g.size} values, expected {e.size}")
        err = np.abs(g - e)
        assert err.size == e.size and np.all(err <= tol), \
            f"{case['name']} {name}: max |err| {err.max():.3e} > {tol} (got {g.tolist()}, expected {e.tolist()})"
    if "present_shape" in case:
        assert list(got["present_key"].shape) == case["present_shape"], case["name"]
    out = np.asarray(got.get("out", got.get("y")), np.float64).ravel()
    for i, (lo, hi) in enumerate(case.get("bounds", [])):
        # Window2: query 0 equals v0; query 1 lies strictly inside (v0, v1); query 2 (v0
        # excluded by the window) strictly inside (v1, v2).
        if lo == hi:
            assert abs(out[i] - lo) <= tol, case["name"]
        else:
            assert lo < out[i] < hi, f"{case['name']}: out[{i}] = {out[i]} not in ({lo}, {hi})"
    if "below" in case:
        assert np.all(out < case["below"]), f"{case['name']}: old cached values leaked through the window"
