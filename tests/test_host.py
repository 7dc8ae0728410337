"""Host-side tests that need no GPU: the C-ABI library loads and exports what
include/ms_hip_kernels.h declares, the validation rules and messages match
MatMulNBitsKernel.cs:87-161, and the operator-interface mirror behaves like
KernelRegistry / ManagedCpuEngine."""
from __future__ import annotations

import ctypes
import subprocess

import numpy as np
import pytest

from conftest import ROOT, kat_arrays
from modelsharp_amd import native
from modelsharp_amd.graph import (Engine, GraphContext, GraphNode, IKernel, KernelRegistry, ModelGraph,
                                  ModelSharpException,
                                  UnsupportedOperatorException)
from modelsharp_amd.hip_kernel import HipMatMulNBitsKernel, register_kernels

X = "×"


def test_library_exports_every_header_symbol():
    lib = native.load()
    names = native.header_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(native.lib_path())], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported
    assert set(native._PROTOTYPES) == set(names)


def test_library_is_gfx950_code():
    blob = native.lib_path().read_bytes()
    assert b"amdgcn-amd-amdhsa--gfx950" in blob
    for other in (b"--gfx942", b"--gfx90a", b"--gfx1100"):
        assert other not in blob


def test_no_device_is_reported_not_crashed():
    if native.available():
        pytest.skip("a gfx950 device is present")
    lib = native.load()
    assert lib.ms_hip_available() == 0
    h = ctypes.c_void_p()
    b = np.zeros(64, np.uint8)
    s = np.ones(4, np.float32)
    st = lib.ms_hip_nbits_weights_create(b.ctypes.data, b.size, s.ctypes.data, s.size, None, 0, 4, 32, 4, 32,
                                         ctypes.byref(h))
    assert st == native.MS_HIP_ERR_NO_DEVICE
    assert "no gfx950 device" in native.last_error()
    assert not h.value


def check(N, K, bits, bs, b_len, s_len, zp_kind=0, zp_len=0, a_last=-1):
    st = native.load().ms_hip_nbits_check(N, K, bits, bs, b_len, s_len, zp_kind, zp_len, a_last)
    return st, (native.last_error() if st else "")


def test_check_messages_match_reference():
    # MatMulNBitsKernel.cs:87-93
    assert check(0, 4, 4, 4, 0, 0) == (1, "MatMulNBits requires positive N and K attributes (got N=0, K=4).")
    assert check(2, -1, 4, 4, 0, 0) == (1, "MatMulNBits requires positive N and K attributes (got N=2, K=-1).")
    assert check(2, 4, 3, 4, 0, 0) == (1, "MatMulNBits supports bits=4 or bits=8; got 3.")
    assert check(2, 4, 4, 0, 0, 0) == (1, "MatMulNBits requires a positive block_size; got 0.")
    # :100-104
    assert check(2, 8, 4, 4, 7, 4) == (
        1, f"MatMulNBits B has 7 elements; expected 8 (N=2 {X} n_blocks_per_row=2 {X} blob_size=2).")
    # :108-112
    assert check(2, 8, 4, 4, 8, 3) == (
        1, f"MatMulNBits scales has 3 elements; expected 4 (N=2 {X} n_blocks_per_row=2).")
    # :126-129 float zp, :134-138 packed zp
    assert check(2, 8, 4, 4, 8, 4, 2, 3) == (1, "MatMulNBits float zero_points has 3 elements; expected 4.")
    assert check(2, 8, 4, 4, 8, 4, 1, 3) == (1, f"MatMulNBits packed zero_points has 3 bytes; expected 2 (N=2 {X} 1).")
    # valid inputs, K tail and 8-bit
    assert check(2, 8, 4, 4, 8, 4, 1, 2) == (0, "")
    assert check(1, 6, 4, 4, 4, 2) == (0, "")
    assert check(2, 4, 8, 4, 8, 2, 1, 2) == (0, "")
    assert check(3, 100, 4, 32, 3 * 4 * 16, 12, 1, 6) == (0, "")


def _node(inputs, N, K, bits=4, bs=4, name="n"):
    return GraphNode("MatMulNBits", name, inputs, ["Y"], {"N": N, "K": K, "bits": bits, "block_size": bs})


def test_kernel_validation_messages(kat_cases):
    k = HipMatMulNBitsKernel()
    a, b, s, zp, y = kat_arrays(kat_cases[0])
    ctx = GraphContext({"A": a, "B": b, "scales": s})
    with pytest.raises(ModelSharpException, match=r"^MatMulNBits requires positive N and K attributes \(got N=0, K=4\)\.$"):
        k.execute(_node(["A", "B", "scales"], 0, 4), ctx)
    with pytest.raises(ModelSharpException, match=r"^Tensor dtype is Int32; expected UInt8\.$"):
        k.execute(_node(["A", "B2", "scales"], 2, 4), GraphContext({"A": a, "B2": b.astype(np.int32), "scales": s}))
    with pytest.raises(ModelSharpException, match=r"^MatMulNBits zero_points must be Float32 or UInt8; got Int64\.$"):
        k.execute(_node(["A", "B", "scales", "zp"], 2, 4),
                  GraphContext({"A": a, "B": b, "scales": s, "zp": np.array([6, 10], np.int64)}))
    with pytest.raises(ModelSharpException, match=r"^MatMulNBits A inner dimension must equal K=4; got shape \[1,3\]\.$"):
        k.execute(_node(["A", "B", "scales"], 2, 4), GraphContext({"A": a[:, :3].copy(), "B": b, "scales": s}))
    with pytest.raises(ModelSharpException, match="non-trivial block permutation"):
        k.execute(_node(["A", "B", "scales", "", "g"], 2, 4),
                  GraphContext({"A": a, "B": b, "scales": s, "g": np.array([0, 0, 1, 0], np.int32)}))


def test_registry_last_registration_wins():
    class Other:
        op_type = "MatMulNBits"

        def execute(self, node, ctx):
            pass

    r = KernelRegistry().register(Other())
    register_kernels(r)
    ok, k = r.try_get("MatMulNBits")
    assert ok and isinstance(k, HipMatMulNBitsKernel) and r.count == 1
    assert r.try_get("Relu") == (False, None)


def test_engine_unknown_op_message():
    g = ModelGraph(nodes=[GraphNode("Relu", "r0", ["X"], ["Y"])], initializers={}, inputs=["X"], outputs=["Y"])
    with pytest.raises(UnsupportedOperatorException, match=r"^Operator 'Relu' is not supported yet by the managed engine \(node 'r0'\)\.$"):
        Engine(g, KernelRegistry()).run({"X": np.zeros(1, np.float32)})


def test_context_semantics():
    ctx = GraphContext({"h": np.ones(3, np.float16)})
    assert ctx.get("h").dtype == np.float32
    assert not ctx.has("")
    with pytest.raises(ModelSharpException, match="Tensor 'x' is not available in the execution context."):
        ctx.get_tensor("x")


def test_workload_costs_match_published_table():
    from modelsharp_amd import workloads as W
    # the workload table's rows (algorithmic bytes, flops)
    assert W.algorithmic_bytes(W.QWEN05B_UP, 1) == 2_814_976
    assert W.flops(W.QWEN05B_UP, 1) == 8_716_288
    gate = next(o for o in W.DECODE_7B if o.name == "gate")
    assert W.algorithmic_bytes(gate, 1) == 43_585_536
    assert sum(W.algorithmic_bytes(o, 1) for o in W.DECODE_7B) == 149_655_552
    assert sum(W.algorithmic_bytes(o, 1) for o in W.QWEN05B_DECODE) == 97_465_600
    up, down = W.LLAMA7B_PREFILL_OPS
    # (4096,11008) and (11008,4096) cost the same each
    for op in (up, down):
        assert W.algorithmic_bytes(op, 2048) == 152_616_960
        assert W.flops(op, 2048) == 184_683_593_728
        assert W.algorithmic_bytes(op, 128) == 36_618_240
    for op in W.LLAMA7B_SMALLM_OPS:
        assert W.algorithmic_bytes(op, 1) == 24_013_824
        assert W.algorithmic_bytes(op, 16) == 24_920_064


def test_pack_nibbles_layout():
    from modelsharp_amd.workloads import pack_nibbles
    assert pack_nibbles(np.array([[8, 9, 7, 10]])).tolist() == [[0x98, 0xA7]]
    assert pack_nibbles(np.array([[1, 2, 3]])).tolist() == [[0x21, 0x03]]


def test_header_is_plain_c():
    src = (ROOT / "include" / "ms_hip_kernels.h").read_text()
    assert "torch" not in src and "hip_runtime" not in src
    out = subprocess.run(["gcc", "-fsyntax-only", "-x", "c", "-std=c99", "-Wall", "-Werror", "-"], input=src,
                         capture_output=True, text=True)
    assert out.returncode == 0, out.stderr


class _FakeWeights:
    """Stands in for native.NBitsWeights on a host without a GPU: records each upload."""

    made: list = []

    def __init__(self, b, scales, zp, N, K, bits, block_size):
        assert scales.dtype in (np.float32, np.float16)   # Float16 is widened on the device
        self.N, self.closed = N, False
        _FakeWeights.made.append(self)

    def gemm(self, a):
        return np.zeros((a.shape[0], self.N), np.float32)

    def close(self):
        self.closed = True


def _fp16_scale_graph():
    from modelsharp_amd import workloads
    op = workloads.Op("t", 64, 8, 32, True)
    b, s, z = workloads.make_weights(op, 0)
    node = GraphNode("MatMulNBits", "mm", ["A", "B", "S", "Z"], ["Y"],
                     {"N": op.N, "K": op.K, "bits": 4, "block_size": 32})
    inits = {"B": b, "S": s.astype(np.float16), "Z": z}
    return ModelGraph([node], inits, ["A"], ["Y"]), op


def test_handle_cache_one_upload_per_initializer(monkeypatch):
    """Repeated execute() on fp16 scales (a q4f16 export) reuses one device handle, the one
    preload() made: the handle is keyed by the node's input names and the raw initializer
    tensors, never by the fp32 copy that widening makes on each call."""
    monkeypatch.setattr(native, "NBitsWeights", _FakeWeights)
    _FakeWeights.made = []
    graph, op = _fp16_scale_graph()
    kernel = HipMatMulNBitsKernel()
    assert kernel.preload(graph) == 1
    engine = Engine(graph, KernelRegistry().register(kernel))
    a = np.ones((1, op.K), np.float32)
    for _ in range(20):
        engine.run({"A": a})
    assert len(_FakeWeights.made) == 1 and kernel.handle_count == 1
    # The same names bound to other tensors: a new handle, and the old one is closed.
    graph.initializers["S"] = graph.initializers["S"].copy()
    engine.run({"A": a})
    assert len(_FakeWeights.made) == 2 and _FakeWeights.made[0].closed and kernel.handle_count == 1
    kernel.close()
    assert _FakeWeights.made[1].closed


def test_tuning_knobs_validated_without_a_device():
    lib = native.load()
    assert lib.ms_hip_set_tuning(99, 0) == native.MS_HIP_ERR_INVALID
    assert "invalid tuning knob" in native.last_error()
    assert lib.ms_hip_set_tuning(1, 10_000) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_set_tuning(3, 0) == native.MS_HIP_OK
    assert lib.ms_hip_set_tuning(11, 10) == native.MS_HIP_ERR_INVALID   # 9 gemv_w8 configurations
    assert lib.ms_hip_set_tuning(11, -2) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_set_tuning(12, 0) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_set_tuning(11, 0) == native.MS_HIP_OK
    bogus = ctypes.c_void_p(0x1234560)
    assert lib.ms_hip_nbits_set_tuning(bogus, 0, 0) == native.MS_HIP_ERR_INVALID
    assert "invalid weights handle" in native.last_error()


def test_host_entries_from_many_threads():
    """The host entries a caller may reach from several threads at once without a device:
    validation (its message in each thread's own last error), the global tuning knobs
    (atomics), the live-handle registry's rejection of unknown handles (a mutex) and the
    attention checks. ctypes drops the GIL around each foreign call, so the threads run in
    the library together; this is also the workload the host library's ThreadSanitizer
    build is run on (the csrc Makefile's tsan target)."""
    import threading
    lib = native.load()
    junk = (ctypes.c_uint32 * 64)(*([0x4D534E42] * 64))
    bogus = ctypes.c_void_p(ctypes.addressof(junk))
    n_out = ctypes.c_int()
    failures = []

    def work(t):
        try:
            for i in range(300):
                K = -(t * 1000 + i) - 1
                st = lib.ms_hip_nbits_check(2, K, 4, 4, 0, 0, 0, 0, -1)
                msg = native.last_error()
                assert st == 1 and f"(got N=2, K={K})" in msg, msg
                assert lib.ms_hip_set_tuning(3, (t + i) % 3) == native.MS_HIP_OK
                assert lib.ms_hip_set_tuning(99, 0) == native.MS_HIP_ERR_INVALID
                assert lib.ms_hip_nbits_weights_info(bogus, ctypes.byref(n_out), None, None, None, None) == \
                    native.MS_HIP_ERR_INVALID
                assert lib.ms_hip_nbits_set_tuning(bogus, 0, 0) == native.MS_HIP_ERR_INVALID
                assert lib.ms_hip_gqa_check(None) != native.MS_HIP_OK
                lib.ms_hip_available()
                # the last error is still this thread's own after the other threads' calls
                st = lib.ms_hip_nbits_check(2, 8, 3, 4, 0, 0, 0, 0, -1)
                assert st == 1 and native.last_error() == "MatMulNBits supports bits=4 or bits=8; got 3."
        except AssertionError as e:   # noqa: PERF203
            failures.append((t, str(e)))

    threads = [threading.Thread(target=work, args=(t,)) for t in range(8)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    lib.ms_hip_set_tuning(3, 0)
    assert not failures, failures[:3]


def test_unknown_handles_are_rejected_not_read():
    """A pointer that is not a live handle (never created, or destroyed) is rejected by
    every entry without being dereferenced."""
    lib = native.load()
    junk = (ctypes.c_uint32 * 64)(*([0x4D534E42] * 64))   # memory that looks like a handle's bytes
    p = ctypes.c_void_p(ctypes.addressof(junk))
    n = ctypes.c_int()
    assert lib.ms_hip_nbits_weights_info(p, ctypes.byref(n), None, None, None, None) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_nbits_weights_destroy(p) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_nbits_gemm_dev(p, None, None, 1, None) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_nbits_device_error(p) == native.MS_HIP_ERR_INVALID
    assert lib.ms_hip_nbits_weights_destroy(None) == native.MS_HIP_ERR_INVALID


# ---- switches: MODELSHARP_HIP kill switch and forced failure (NativeGemm.cs:42-57) --------
_SWITCH_PROBE = r"""
import ctypes, json, sys
sys.path.insert(0, sys.argv[1])
from modelsharp_amd import native
lib = native.load()
h = ctypes.c_void_p()
b = (ctypes.c_uint8 * 16)()
s = (ctypes.c_float * 1)()
st_create = lib.ms_hip_nbits_weights_create(b, 16, s, 1, None, 0, 1, 32, 4, 32, ctypes.byref(h))
err = native.last_error()
st_check = lib.ms_hip_nbits_check(1, 32, 4, 32, 16, 1, 0, 0, -1)
print(json.dumps({"available": lib.ms_hip_available(), "create": st_create, "err": err, "check": st_check,
                  "gemm": lib.ms_hip_nbits_gemm_dev(None, None, None, 1, None)}))
"""


def _probe_switches(env_extra):
    import json
    import os
    import sys
    env = {k: v for k, v in os.environ.items() if k not in ("MODELSHARP_HIP", "MS_HIP_FORCE_FAIL")}
    env.update(env_extra)
    out = subprocess.run([sys.executable, "-c", _SWITCH_PROBE, str(ROOT)], env=env, capture_output=True, text=True,
                         timeout=120)
    assert out.returncode == 0, out.stderr
    return json.loads(out.stdout.strip().splitlines()[-1])


@pytest.mark.parametrize("value", ["0", "off", "FALSE"])
def test_kill_switch_turns_the_library_off(value):
    r = _probe_switches({"MODELSHARP_HIP": value})
    assert r["available"] == 0
    assert r["create"] == native.MS_HIP_ERR_DISABLED and "MODELSHARP_HIP" in r["err"]
    assert r["gemm"] == native.MS_HIP_ERR_DISABLED
    assert r["check"] == 0   # validation keeps working


@pytest.mark.parametrize("value", ["1", "on", "True"])
def test_forced_failure_env(value):
    r = _probe_switches({"MS_HIP_FORCE_FAIL": value})
    assert r["create"] == native.MS_HIP_ERR_FORCED and "forced failure" in r["err"]
    assert r["gemm"] == native.MS_HIP_ERR_FORCED
    assert r["check"] == 0


def test_switches_off_by_default():
    r = _probe_switches({"MODELSHARP_HIP": "1", "MS_HIP_FORCE_FAIL": "0"})
    assert r["create"] not in (native.MS_HIP_ERR_DISABLED, native.MS_HIP_ERR_FORCED)


def test_forced_failure_settable_at_run_time():
    lib = native.load()
    h = ctypes.c_void_p()
    b = (ctypes.c_uint8 * 16)()
    s = (ctypes.c_float * 1)()
    try:
        assert lib.ms_hip_debug_force_failure(1) == 0
        assert lib.ms_hip_nbits_weights_create(b, 16, s, 1, None, 0, 1, 32, 4, 32, ctypes.byref(h)) == \
            native.MS_HIP_ERR_FORCED
        assert not h.value
    finally:
        lib.ms_hip_debug_force_failure(0)
    st = lib.ms_hip_nbits_weights_create(b, 16, s, 1, None, 0, 1, 32, 4, 32, ctypes.byref(h))
    assert st != native.MS_HIP_ERR_FORCED
    if st == 0:
        lib.ms_hip_nbits_weights_destroy(h)


def test_kill_switch_leaves_registry_alone(monkeypatch):
    class Managed:
        op_type = "MatMulNBits"

        def execute(self, node, ctx):
            pass

    m = Managed()
    monkeypatch.setenv("MODELSHARP_HIP", "off")
    r = register_kernels(KernelRegistry().register(m))
    assert r.try_get("MatMulNBits") == (True, m)
    monkeypatch.setenv("MODELSHARP_HIP", "1")
    assert isinstance(register_kernels(r).try_get("MatMulNBits")[1], HipMatMulNBitsKernel)


# ---- decoder-layer kernels: graph fusion and validation (no device needed) -----------------
def test_fuse_silu_mul_patterns():
    from modelsharp_amd.decoder_kernels import fuse_silu_mul
    mk = lambda: ModelGraph(nodes=[   # noqa: E731
        GraphNode("MatMulNBits", "gate", ["n", "B"], ["g"]),
        GraphNode("Sigmoid", "sig", ["g"], ["s"]),
        GraphNode("Mul", "m1", ["s", "g"], ["a"]),
        GraphNode("Mul", "m2", ["u", "a"], ["y"]),
    ], initializers={}, inputs=["n", "u"], outputs=["y"])
    g = mk()
    assert fuse_silu_mul(g) == 1
    assert [(n.op_type, n.inputs, n.outputs) for n in g.nodes] == [
        ("MatMulNBits", ["n", "B"], ["g"]), ("SiluMul", ["g", "u"], ["y"])]
    g = mk()
    g.outputs.append("s")   # the sigmoid is used elsewhere: no fusion
    assert fuse_silu_mul(g) == 0 and len(g.nodes) == 4
    g = mk()
    g.nodes[2].inputs = ["s", "other"]   # Mul of the sigmoid with another tensor
    assert fuse_silu_mul(g) == 0


def test_fuse_gate_up_silu_patterns():
    from modelsharp_amd.decoder_kernels import fuse_gate_up_silu, fuse_silu_mul
    at = {"N": 8, "K": 4, "bits": 4, "block_size": 32}
    mk = lambda: ModelGraph(nodes=[   # noqa: E731
        GraphNode("MatMulNBits", "gate", ["n", "Bg", "Sg", "Zg"], ["g"], dict(at)),
        GraphNode("MatMulNBits", "up", ["n", "Bu", "Su"], ["u"], dict(at)),
        GraphNode("Sigmoid", "sig", ["g"], ["s"]),
        GraphNode("Mul", "m1", ["g", "s"], ["a"]),
        GraphNode("Mul", "m2", ["a", "u"], ["h"]),
        GraphNode("MatMulNBits", "down", ["h", "Bd", "Sd"], ["y"], dict(at)),
    ], initializers={}, inputs=["n"], outputs=["y"])
    g = mk()
    assert fuse_silu_mul(g) == 1 and fuse_gate_up_silu(g) == 1
    assert [(n.op_type, n.inputs, n.outputs) for n in g.nodes] == [
        ("GateUpSiluMul", ["n", "Bg", "Sg", "Zg", "Bu", "Su", ""], ["h"]),
        ("MatMulNBits", ["h", "Bd", "Sd"], ["y"])]
    assert g.nodes[0].attributes == at
    g = mk()
    g.outputs.append("u")   # the up projection is used elsewhere: no fusion
    assert fuse_silu_mul(g) == 1 and fuse_gate_up_silu(g) == 0
    g = mk()
    g.nodes[1].inputs[0] = "other"   # gate and up of different inputs
    assert fuse_silu_mul(g) == 1 and fuse_gate_up_silu(g) == 0
    g = mk()
    g.nodes[1].attributes["N"] = 16   # different shapes
    assert fuse_silu_mul(g) == 1 and fuse_gate_up_silu(g) == 0
    g = mk()
    g.nodes[0].inputs += ["g_idx"]   # a g_idx input is not folded
    assert fuse_silu_mul(g) == 1 and fuse_gate_up_silu(g) == 0


def test_fuse_skipnorm_patterns():
    from modelsharp_amd.decoder_kernels import fuse_gate_up_silu, fuse_silu_mul, fuse_skipnorm
    at = {"K": 4, "bits": 4, "block_size": 32}
    inits = {k: None for k in ("g1", "g2", "Bq", "Sq", "Zq", "Bk", "Sk", "Bg", "Sg", "Zg", "Bu", "Su", "Bd", "Sd")}
    mk = lambda: ModelGraph(nodes=[   # noqa: E731
        GraphNode("SkipSimplifiedLayerNormalization", "ln1", ["x", "r", "g1"], ["n1", "", "", "t1"], {"epsilon": 1e-6}),
        GraphNode("MatMulNBits", "q", ["n1", "Bq", "Sq", "Zq"], ["q"], dict(at, N=8)),
        GraphNode("MatMulNBits", "k", ["n1", "Bk", "Sk"], ["k"], dict(at, N=2)),
        GraphNode("Add", "mix", ["q", "t1"], ["o"]),
        GraphNode("SkipSimplifiedLayerNormalization", "ln2", ["o", "t1", "g2"], ["n2", "", "", "t2"]),
        GraphNode("MatMulNBits", "gate", ["n2", "Bg", "Sg", "Zg"], ["g"], dict(at, N=8)),
        GraphNode("MatMulNBits", "up", ["n2", "Bu", "Su"], ["u"], dict(at, N=8)),
        GraphNode("Sigmoid", "sig", ["g"], ["s"]),
        GraphNode("Mul", "m1", ["g", "s"], ["a"]),
        GraphNode("Mul", "m2", ["a", "u"], ["h"]),
        GraphNode("MatMulNBits", "down", ["h", "Bd", "Sd"], ["y"], dict(at, N=4)),
    ], initializers=dict(inits), inputs=["x", "r"], outputs=["y", "k", "t2"])
    g = mk()
    assert fuse_silu_mul(g) == 1 and fuse_gate_up_silu(g) == 1 and fuse_skipnorm(g) == 2
    assert [(n.op_type, n.inputs, n.outputs) for n in g.nodes] == [
        ("SkipNormMatMulNBits", ["x", "r", "g1", "Bq", "Sq", "Zq", "Bk", "Sk", ""], ["q", "k", "t1"]),
        ("Add", ["q", "t1"], ["o"]),
        ("SkipNormGateUpSiluMul", ["o", "t1", "g2", "Bg", "Sg", "Zg", "Bu", "Su", ""], ["h", "t2"]),
        ("MatMulNBits", ["h", "Bd", "Sd"], ["y"])]
    assert g.nodes[0].attributes == dict(at, Ns=[8, 2], epsilon=1e-6)
    assert g.nodes[2].attributes == dict(at, N=8, epsilon=1e-5)
    g = mk()
    g.outputs.append("n1")   # the normed output is used elsewhere: that norm stays
    assert fuse_skipnorm(g) == 1 and g.nodes[0].op_type == "SkipSimplifiedLayerNormalization"
    g = mk()
    g.nodes[0].outputs[2] = "inv"
    g.outputs.append("inv")   # inv_std is used: no fusion of that norm
    assert fuse_skipnorm(g) == 1 and g.nodes[0].op_type == "SkipSimplifiedLayerNormalization"
    g = mk()
    g.nodes[0].inputs.append("beta")   # beta is not folded
    assert fuse_skipnorm(g) == 1 and g.nodes[0].op_type == "SkipSimplifiedLayerNormalization"
    g = mk()
    g.nodes[2].attributes["K"] = 8   # projections of different shapes
    assert fuse_skipnorm(g) == 1 and g.nodes[0].op_type == "SkipSimplifiedLayerNormalization"
    g = mk()
    del g.initializers["Bk"]   # a weight computed after the norm: not available at its place
    g.nodes.insert(0, GraphNode("Add", "late", ["x", "x"], ["Bk"]))
    g.nodes[0], g.nodes[1] = g.nodes[1], g.nodes[0]
    assert fuse_skipnorm(g) == 1 and g.nodes[0].op_type == "SkipSimplifiedLayerNormalization"
    g = mk()   # without the SiLU fusions, gate and up are two plain projections of n2
    assert fuse_skipnorm(g) == 2 and g.nodes[2].op_type == "SkipNormMatMulNBits"
    assert g.nodes[2].outputs == ["g", "u", "t2"]


def test_gqa_kernel_validation_messages():
    from modelsharp_amd.decoder_kernels import HipGroupQueryAttentionKernel
    k = HipGroupQueryAttentionKernel()
    node = GraphNode("GroupQueryAttention", "a", ["q"], ["o"], {"num_heads": 0, "kv_num_heads": 1})
    with pytest.raises(ModelSharpException, match=r"^GroupQueryAttention requires positive 'num_heads' and 'kv_num_heads'\.$"):
        k.execute(node, GraphContext({}))
    node.attributes = {"num_heads": 6, "kv_num_heads": 4}
    with pytest.raises(ModelSharpException, match=r"^GroupQueryAttention num_heads=6 must be a multiple of kv_num_heads=4\.$"):
        k.execute(node, GraphContext({}))


def test_gqa_descriptor_checks():
    lib = native.load()
    d = native.GqaDesc(batch=1, q_seq=2, kv_seq=2, num_heads=4, kv_num_heads=2, head_dim=64, packed_qkv=1,
                       present_capacity=1)
    assert lib.ms_hip_gqa_check(ctypes.byref(d)) == native.MS_HIP_ERR_INVALID
    assert "present capacity" in native.last_error()
    d.present_capacity = 2
    d.do_rotary = 1
    assert lib.ms_hip_gqa_check(ctypes.byref(d)) == native.MS_HIP_ERR_INVALID
    assert "cos_cache" in native.last_error()
    d.do_rotary = 0
    assert lib.ms_hip_gqa_check(ctypes.byref(d)) == 0
    d.past_seq, d.present_capacity = 50000, 50002
    # head_dim 64: the keys split over workgroups, given the workspace it asks for
    assert lib.ms_hip_gqa_check(ctypes.byref(d)) == 0
    assert native.gqa_workspace_size(d) == 2 * 4 * 64 * (64 + 2) * 4   # units x splits x (D + 2) floats
    d.head_dim = 40   # the per-unit kernel keeps every score of a unit in LDS
    assert lib.ms_hip_gqa_check(ctypes.byref(d)) == native.MS_HIP_ERR_UNSUPPORTED


def test_device_inputs_keep_initializers_only():
    """Feeds arrive as new host arrays every run: uploading them must not grow the
    kernels' upload cache, while an initializer is uploaded once and reused."""
    import torch
    from modelsharp_amd.decoder_kernels import _DeviceInputs
    dev = _DeviceInputs(device="cpu")
    w = np.arange(8, dtype=np.float32)
    first = None
    for i in range(6):
        ctx = GraphContext({"w": w, "x": np.full(8, i, np.float32)}, constants={"w"})
        dw, dx = dev.input(ctx, "w"), dev.input(ctx, "x")
        first = dw if first is None else first
        assert dw is first and torch.equal(dx, torch.full((8,), float(i)))
        assert dev.cached == 1


def test_engine_marks_initializers_constant():
    """Engine.run binds the graph's initializers as constants; a feed that shadows one
    is not."""
    seen = {}

    class Probe(IKernel):
        op_type = "Probe"

        def execute(self, node, ctx):
            seen.update({n: ctx.is_constant(n) for n in node.inputs})
            ctx.set(node.outputs[0], ctx.get_tensor(node.inputs[0]))

    g = ModelGraph([GraphNode("Probe", "p", ["x", "w", "v"], ["y"])],
                   {"w": np.ones(2, np.float32), "v": np.zeros(2, np.float32)}, ["x"], ["y"])
    Engine(g, KernelRegistry().register(Probe())).run({"x": np.ones(2, np.float32), "v": np.ones(2, np.float32)})
    assert seen == {"x": False, "w": True, "v": False}
