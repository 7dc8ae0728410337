"""The decoder-layer operators next to MatMulNBits, on the device, behind the reference's
operator interface (IKernel, KernelRegistry).

Each kernel mirrors the reference's managed kernel of the same OpType — same inputs,
attributes, outputs and error messages — and computes on the device through the C ABI
of libms_hip_nbits.so, so a decoder layer's activations stay in HBM from one
MatMulNBits to the next:

  SimplifiedLayerNormalization      Cpu/Kernels/Llm/SimplifiedLayerNormalizationKernel.cs
  SkipSimplifiedLayerNormalization  Cpu/Kernels/Llm/SkipSimplifiedLayerNormalizationKernel.cs
  GroupQueryAttention               Cpu/Kernels/Llm/GroupQueryAttentionKernel.cs
  Sigmoid, Mul, Add                 Activations/SigmoidKernel.cs, the elementwise Mul/Add
                                    (equal shapes: the residual stream and the MLP gate)
  SiluMul                           Sigmoid -> Mul -> Mul fused by fuse_silu_mul()
  GateUpSiluMul                     MatMulNBits(x, gate), MatMulNBits(x, up) -> SiluMul, fused by
                                    fuse_gate_up_silu()
  SkipNormMatMulNBits,              SkipSimplifiedLayerNormalization and the MatMulNBits (or the
  SkipNormGateUpSiluMul             GateUpSiluMul) that read its output, fused by fuse_skipnorm()

Activations are torch tensors on the device (host arrays are uploaded once per call);
initializers (norm weights, rotary caches) are uploaded once and kept. Nothing here
computes on the CPU: an input the device kernels do not take raises
ModelSharpException.
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import native
from .graph import GraphContext, GraphNode, IKernel, KernelRegistry, ModelGraph, ModelSharpException


def _torch():
    import torch
    return torch


class _DeviceInputs:
    """Device copies of host arrays. Initializers (names the context marks constant: norm
    weights, rotary caches) are uploaded once and kept, keyed by the array object; any
    other host array (a feed of this run) is uploaded for the call and not kept."""

    def __init__(self, device="cuda"):
        self._cache: dict[int, tuple] = {}
        self._device = device

    @property
    def cached(self) -> int:
        return len(self._cache)

    def input(self, ctx: GraphContext, name: str):
        return self.f32(ctx.get_tensor(name), keep=ctx.is_constant(name))

    def f32(self, t, keep=False):
        torch = _torch()
        if isinstance(t, np.ndarray):
            if keep:
                hit = self._cache.get(id(t))
                if hit is not None and hit[0] is t:
                    return hit[1]
            d = torch.from_numpy(np.ascontiguousarray(t, dtype=np.float32)).to(self._device)
            if keep:
                self._cache[id(t)] = (t, d)
            return d
        if t.dtype != torch.float32:
            t = t.float()
        return t.contiguous()

    def i32(self, t):
        torch = _torch()
        if isinstance(t, np.ndarray):
            return torch.from_numpy(np.ascontiguousarray(t, dtype=np.int32)).to(self._device)
        return t.to(torch.int32).contiguous()


def _stream(t):
    return _torch().cuda.current_stream(t.device).cuda_stream


def _attr_float(node: GraphNode, key: str, default: float) -> float:
    """Attr.Float (Cpu/Kernels/Internal/Attr.cs)."""
    return float(node.attributes.get(key, default))


def _present(node: GraphNode, i: int) -> bool:
    return len(node.outputs) > i and len(node.outputs[i]) > 0


class HipSimplifiedLayerNormalizationKernel(IKernel):
    op_type = "SimplifiedLayerNormalization"

    def __init__(self):
        self._dev = _DeviceInputs()

    def execute(self, node: GraphNode, ctx: GraphContext) -> None:
        torch = _torch()
        x = self._dev.input(ctx, node.inputs[0])
        scale = self._dev.input(ctx, node.inputs[1])
        rank = x.dim()
        axis = node.attr_int("axis", -1)
        if axis < 0:
            axis += rank
        eps = _attr_float(node, "epsilon", 1e-5)
        outer = int(np.prod(x.shape[:axis])) if axis > 0 else 1
        norm = int(np.prod(x.shape[axis:]))
        if scale.numel() != norm:
            raise ModelSharpException(f"SimplifiedLayerNormalization scale has {scale.numel()} elements; "
                                      f"expected {norm}.")
        y = torch.empty_like(x)
        inv = torch.empty(outer, dtype=torch.float32, device=x.device) if _present(node, 1) else None
        native.rmsnorm(x.data_ptr(), scale.data_ptr(), y.data_ptr(), None if inv is None else inv.data_ptr(),
                       outer, norm, eps, _stream(x))
        ctx.set(node.outputs[0], y)
        if inv is not None:
            ctx.set(node.outputs[1], inv)


class HipSkipSimplifiedLayerNormalizationKernel(IKernel):
    op_type = "SkipSimplifiedLayerNormalization"

    def __init__(self):
        self._dev = _DeviceInputs()

    def execute(self, node: GraphNode, ctx: GraphContext) -> None:
        torch = _torch()
        inp = self._dev.input(ctx, node.inputs[0])
        skip = self._dev.input(ctx, node.inputs[1])
        gamma = self._dev.input(ctx, node.inputs[2])
        beta = self._dev.input(ctx, node.inputs[3]) if len(node.inputs) > 3 and node.inputs[3] else None
        bias = self._dev.input(ctx, node.inputs[4]) if len(node.inputs) > 4 and node.inputs[4] else None
        eps = _attr_float(node, "epsilon", 1e-5)
        norm = gamma.numel()
        total = inp.numel()
        outer = 0 if norm == 0 else total // norm
        if skip.numel() != total:
            raise ModelSharpException("SkipSimplifiedLayerNormalization skip must have the input's shape.")
        out = torch.empty_like(inp)
        want_sum = _present(node, 3)
        total_t = torch.empty_like(inp) if want_sum else None
        inv = torch.empty(outer, dtype=torch.float32, device=inp.device) if _present(node, 2) else None
        ptr = lambda t: None if t is None else t.data_ptr()   # noqa: E731
        native.skip_rmsnorm(inp.data_ptr(), skip.data_ptr(), gamma.data_ptr(), ptr(beta), ptr(bias), out.data_ptr(),
                            ptr(total_t), ptr(inv), outer, norm, eps, _stream(inp))
        ctx.set(node.outputs[0], out)
        if _present(node, 1):   # mean: undefined for RMSNorm, zeros (:80-81)
            ctx.set(node.outputs[1], torch.zeros(outer, dtype=torch.float32, device=inp.device))
        if inv is not None:
            ctx.set(node.outputs[2], inv)
        if want_sum:
            ctx.set(node.outputs[3], total_t)


class _Elementwise(IKernel):
    def __init__(self):
        self._dev = _DeviceInputs()

    def _same_shape(self, node, ctx):
        a = self._dev.input(ctx, node.inputs[0])
        b = self._dev.input(ctx, node.inputs[1])
        if tuple(a.shape) != tuple(b.shape):
            raise ModelSharpException(
                f"{self.op_type} on the device takes equal shapes; got {list(a.shape)} and {list(b.shape)}.")
        return a, b


class HipAddKernel(_Elementwise):
    op_type = "Add"

    def execute(self, node, ctx):
        a, b = self._same_shape(node, ctx)
        y = _torch().empty_like(a)
        native.add(a.data_ptr(), b.data_ptr(), y.data_ptr(), a.numel(), _stream(a))
        ctx.set(node.outputs[0], y)


class HipMulKernel(_Elementwise):
    op_type = "Mul"

    def execute(self, node, ctx):
        a, b = self._same_shape(node, ctx)
        y = _torch().empty_like(a)
        native.mul(a.data_ptr(), b.data_ptr(), y.data_ptr(), a.numel(), _stream(a))
        ctx.set(node.outputs[0], y)


class HipSigmoidKernel(_Elementwise):
    op_type = "Sigmoid"

    def execute(self, node, ctx):
        x = self._dev.input(ctx, node.inputs[0])
        y = _torch().empty_like(x)
        native.sigmoid(x.data_ptr(), y.data_ptr(), x.numel(), _stream(x))
        ctx.set(node.outputs[0], y)


class HipSiluMulKernel(_Elementwise):
    """SiluMul(gate, up) = (gate * Sigmoid(gate)) * up: the three nodes fuse_silu_mul
    replaces, with the same roundings."""
    op_type = "SiluMul"

    def execute(self, node, ctx):
        g, u = self._same_shape(node, ctx)
        y = _torch().empty_like(g)
        native.silu_mul(g.data_ptr(), u.data_ptr(), y.data_ptr(), g.numel(), _stream(g))
        ctx.set(node.outputs[0], y)


def fuse_silu_mul(graph: ModelGraph) -> int:
    """Rewrites Sigmoid(x) -> s, Mul(x, s) -> a, Mul(a, u) -> y (either operand order) into
    one SiluMul(x, u) -> y node when s and a feed nothing else. Returns the number of
    patterns fused."""
    uses: dict[str, int] = {}
    for n in graph.nodes:
        for i in n.inputs:
            uses[i] = uses.get(i, 0) + 1
    for o in graph.outputs:
        uses[o] = uses.get(o, 0) + 1
    producer = {o: n for n in graph.nodes for o in n.outputs}
    fused = 0
    drop: set[int] = set()
    replace: dict[int, GraphNode] = {}
    for mul2 in graph.nodes:
        if mul2.op_type != "Mul" or len(mul2.inputs) != 2:
            continue
        for ai in (0, 1):
            a_name, u_name = mul2.inputs[ai], mul2.inputs[1 - ai]
            mul1 = producer.get(a_name)
            if mul1 is None or mul1.op_type != "Mul" or uses.get(a_name, 0) != 1 or id(mul1) in drop:
                continue
            sig = None
            for si in (0, 1):
                s_name, x_name = mul1.inputs[si], mul1.inputs[1 - si]
                cand = producer.get(s_name)
                if (cand is not None and cand.op_type == "Sigmoid" and cand.inputs[0] == x_name
                        and uses.get(s_name, 0) == 1 and id(cand) not in drop):
                    sig = cand
                    break
            if sig is None:
                continue
            drop.update({id(sig), id(mul1)})
            replace[id(mul2)] = GraphNode("SiluMul", mul2.name + "/silu_mul", [sig.inputs[0], u_name],
                                          list(mul2.outputs))
            fused += 1
            break
    graph.nodes = [replace.get(id(n), n) for n in graph.nodes if id(n) not in drop]
    return fused


def fuse_gate_up_silu(graph: ModelGraph) -> int:
    """Rewrites MatMulNBits(x, W_gate) -> g, MatMulNBits(x, W_up) -> u, SiluMul(g, u) -> h
    into one GateUpSiluMul(x, B_g, scales_g, zp_g, B_u, scales_u, zp_u) -> h node when g and
    u feed nothing else and the two projections share their attributes and carry no
    g_idx or bias inputs (run fuse_silu_mul first). Returns the number of patterns fused."""
    uses: dict[str, int] = {}
    for n in graph.nodes:
        for i in n.inputs:
            uses[i] = uses.get(i, 0) + 1
    for o in graph.outputs:
        uses[o] = uses.get(o, 0) + 1
    producer = {o: n for n in graph.nodes for o in n.outputs}
    fused = 0
    drop: set[int] = set()
    replace: dict[int, GraphNode] = {}

    def plain(n):
        return (n is not None and n.op_type == "MatMulNBits" and id(n) not in drop and len(n.outputs) == 1
                and not any(n.inputs[4:]))

    for sm in graph.nodes:
        if sm.op_type != "SiluMul" or len(sm.inputs) != 2:
            continue
        gn, un = producer.get(sm.inputs[0]), producer.get(sm.inputs[1])
        if not (plain(gn) and plain(un)) or gn is un or gn.inputs[0] != un.inputs[0]:
            continue
        if uses.get(sm.inputs[0], 0) != 1 or uses.get(sm.inputs[1], 0) != 1:
            continue
        keys = ("N", "K", "bits", "block_size")
        if any(gn.attributes.get(k) != un.attributes.get(k) for k in keys):
            continue
        tri = lambda n: (list(n.inputs[1:4]) + ["", "", ""])[:3]
        drop.update({id(gn), id(un)})
        replace[id(sm)] = GraphNode("GateUpSiluMul", sm.name + "/gate_up_silu",
                                    [gn.inputs[0]] + tri(gn) + tri(un), list(sm.outputs), dict(gn.attributes))
        fused += 1
    graph.nodes = [replace.get(id(n), n) for n in graph.nodes if id(n) not in drop]
    return fused


class HipGateUpSiluMulKernel(IKernel):
    """GateUpSiluMul(x, gate triple, up triple) = SiluMul(MatMulNBits(x, gate), MatMulNBits(x,
    up)) (the nodes fuse_gate_up_silu replaces): both projections validated as
    MatMulNBits nodes (MatMulNBitsKernel.cs:79-161), then one ms_hip_nbits_gemm_dev_swiglu
    call on device activations (one launch at M = 1, bit-identical to the three kernels);
    other inputs (host arrays, fp16 activations, the W4A8 opt-in) run the three kernels."""
    op_type = "GateUpSiluMul"

    def __init__(self, matmul=None):
        from .hip_kernel import HipMatMulNBitsKernel
        self._mm = matmul if matmul is not None else HipMatMulNBitsKernel()
        self._silu = HipSiluMulKernel()

    def close(self):
        self._mm.close()

    def preload(self, graph: ModelGraph) -> int:
        """Load-time upload of the fused nodes' two weight triples, as
        HipMatMulNBitsKernel.preload does for MatMulNBits nodes (file-backed initializers
        streamed from their slices). Returns the number of handles created."""
        pseudo = []
        for n in graph.nodes:
            if n.op_type == self.op_type:
                pseudo += [GraphNode("MatMulNBits", n.name + "/gate", [n.inputs[0]] + list(n.inputs[1:4]),
                                     [n.name + "/g"], n.attributes),
                           GraphNode("MatMulNBits", n.name + "/up", [n.inputs[0]] + list(n.inputs[4:7]),
                                     [n.name + "/u"], n.attributes)]
        g = ModelGraph(pseudo, graph.initializers)
        g.sources = getattr(graph, "sources", {})
        return self._mm.preload(g)

    def execute(self, node, ctx):
        x = node.inputs[0]
        gnode = GraphNode("MatMulNBits", node.name + "/gate", [x] + list(node.inputs[1:4]), [node.name + "/g"],
                          node.attributes)
        unode = GraphNode("MatMulNBits", node.name + "/up", [x] + list(node.inputs[4:7]), [node.name + "/u"],
                          node.attributes)
        a, bg, sg, zg, N, K, bits, bs = self._mm._validate(gnode, ctx)
        _, bu, su, zu, _, _, _, _ = self._mm._validate(unode, ctx)
        torch = _torch()
        if not isinstance(a, np.ndarray) and a.dtype == torch.float32 and not self._mm.w4a8:
            wg = self._mm._weights(gnode, bg, sg, zg, N, K, bits, bs)
            wu = self._mm._weights(unode, bu, su, zu, N, K, bits, bs)
            lead = tuple(a.shape[:-1])
            M = int(np.prod(lead)) if lead else 1
            a2 = a.reshape(M, K).contiguous()
            h = torch.empty(lead + (N,), dtype=torch.float32, device=a.device)
            native.gemm_dev_swiglu(wg, wu, a2.data_ptr(), h.data_ptr(), M, _stream(a2))
            ctx.set(node.outputs[0], h)
            return
        self._mm.execute(gnode, ctx)
        self._mm.execute(unode, ctx)
        self._silu.execute(GraphNode("SiluMul", node.name + "/silu_mul", [gnode.outputs[0], unode.outputs[0]],
                                     list(node.outputs)), ctx)


def fuse_skipnorm(graph: ModelGraph) -> int:
    """Rewrites a SkipSimplifiedLayerNormalization(x, skip, gamma) -> (n, mean, inv_std, t)
    without beta or bias, whose normed output n feeds nothing but 1-4 MatMulNBits nodes on n
    (sharing K, bits and block_size, no g_idx or bias inputs) or one GateUpSiluMul on n, and
    whose mean and inv_std outputs are unused, into one node at the norm's place:
    SkipNormMatMulNBits(x, skip, gamma, B_1, scales_1, zp_1, ...) -> (y_1, ..., t) with
    attributes K, bits, block_size, Ns (each projection's N) and epsilon, or
    SkipNormGateUpSiluMul(x, skip, gamma, gate triple, up triple) -> (h, t). The projections'
    weights must be graph inputs, initializers or outputs of nodes before the norm. Run
    fuse_gate_up_silu first. Returns the number of norms fused."""
    consumers: dict[str, list[GraphNode]] = {}
    for n in graph.nodes:
        for i in n.inputs:
            if i:
                consumers.setdefault(i, []).append(n)
    outs = set(graph.outputs)
    available = set(graph.inputs) | set(graph.initializers) | {""}
    fused = 0
    drop: set[int] = set()
    replace: dict[int, GraphNode] = {}
    keys = ("K", "bits", "block_size")

    def plain_mm(c, n):
        return (c.op_type == "MatMulNBits" and len(c.outputs) == 1 and c.inputs[0] == n and n not in c.inputs[1:]
                and not any(c.inputs[4:]))

    def tri(c, lo):
        return (list(c.inputs[lo:lo + 3]) + ["", "", ""])[:3]

    for node in graph.nodes:
        s = node
        ok = (s.op_type == "SkipSimplifiedLayerNormalization" and len(s.inputs) >= 3 and not any(s.inputs[3:])
              and s.outputs and s.outputs[0] and s.outputs[0] not in outs
              and not any(o and (o in outs or consumers.get(o)) for o in s.outputs[1:3]))
        cons = consumers.get(s.outputs[0], []) if ok else []
        if ok and cons and not any(id(c) in drop for c in cons):
            n = s.outputs[0]
            t = s.outputs[3] if len(s.outputs) > 3 else ""
            eps = s.attributes.get("epsilon", 1e-5)
            fnode = None
            if len(cons) == 1 and cons[0].op_type == "GateUpSiluMul" and cons[0].inputs[0] == n \
                    and n not in cons[0].inputs[1:]:
                c = cons[0]
                w = tri(c, 1) + tri(c, 4)
                if all(x in available for x in w):
                    fnode = GraphNode("SkipNormGateUpSiluMul", s.name + "/skipnorm", list(s.inputs[:3]) + w,
                                      [c.outputs[0], t], {**c.attributes, "epsilon": eps})
            elif 1 <= len(cons) <= 4 and all(plain_mm(c, n) for c in cons) \
                    and all(c.attributes.get(k) == cons[0].attributes.get(k) for c in cons for k in keys):
                w = [x for c in cons for x in tri(c, 1)]
                if all(x in available for x in w):
                    at = {k: cons[0].attributes.get(k) for k in keys}
                    at.update(Ns=[c.attributes.get("N") for c in cons], epsilon=eps)
                    fnode = GraphNode("SkipNormMatMulNBits", s.name + "/skipnorm", list(s.inputs[:3]) + w,
                                      [c.outputs[0] for c in cons] + [t], at)
            if fnode is not None:
                drop.update(id(c) for c in cons)
                replace[id(s)] = fnode
                fused += 1
        available.update(o for o in node.outputs if o)
    graph.nodes = [replace.get(id(n), n) for n in graph.nodes if id(n) not in drop]
    return fused


class _HipSkipNormFused(IKernel):
    """The nodes fuse_skipnorm makes: SkipSimplifiedLayerNormalization
    (SkipSimplifiedLayerNormalizationKernel.cs:29-86) and the projections of its output
    (MatMulNBitsKernel.cs:79-161 validation), as one ms_hip_nbits_gemm_dev_skipnorm(_swiglu)
    call on the device (one launch at M = 1); the W4A8 opt-in runs the nodes apart."""

    def __init__(self, matmul=None):
        from .hip_kernel import HipMatMulNBitsKernel
        self._mm = matmul if matmul is not None else HipMatMulNBitsKernel()
        self._norm = HipSkipSimplifiedLayerNormalizationKernel()
        self._dev = _DeviceInputs()

    def close(self):
        self._mm.close()

    def _projections(self, node: GraphNode, a: str) -> list[GraphNode]:
        raise NotImplementedError

    def preload(self, graph: ModelGraph) -> int:
        """Load-time upload of the fused nodes' weight triples (HipMatMulNBitsKernel.preload)."""
        pseudo = [p for n in graph.nodes if n.op_type == self.op_type for p in self._projections(n, n.inputs[0])]
        g = ModelGraph(pseudo, graph.initializers)
        g.sources = getattr(graph, "sources", {})
        return self._mm.preload(g)

    def _apart(self, node: GraphNode, ctx: GraphContext, normed: str) -> None:
        raise NotImplementedError

    def execute(self, node: GraphNode, ctx: GraphContext) -> None:
        torch = _torch()
        normed = node.name + "/normed"
        t_name = node.outputs[-1]
        if self._mm.w4a8:
            self._norm.execute(GraphNode("SkipSimplifiedLayerNormalization", node.name + "/norm", list(node.inputs[:3]),
                                         [normed, "", "", t_name], {"epsilon": _attr_float(node, "epsilon", 1e-5)}),
                               ctx)
            self._apart(node, ctx, normed)
            return
        x = self._dev.input(ctx, node.inputs[0])
        skip = self._dev.input(ctx, node.inputs[1])
        gamma = self._dev.input(ctx, node.inputs[2])
        K = gamma.numel()
        if skip.numel() != x.numel():
            raise ModelSharpException("SkipSimplifiedLayerNormalization skip must have the input's shape.")
        M = 0 if K == 0 else x.numel() // K
        dnorm = torch.empty_like(x)
        ctx.set(normed, dnorm)   # for the projections' validation (shapes), written by the call
        dsum = torch.empty_like(x) if t_name else None
        self._run(node, ctx, normed, x, skip, gamma, dnorm, dsum, M)
        if t_name:
            ctx.set(t_name, dsum)


class HipSkipNormMatMulNBitsKernel(_HipSkipNormFused):
    op_type = "SkipNormMatMulNBits"

    def _projections(self, node, a):
        at = node.attributes
        return [GraphNode("MatMulNBits", f"{node.name}/mm{i}", [a] + list(node.inputs[3 + 3 * i:6 + 3 * i]),
                          [node.outputs[i]], {"K": at["K"], "N": N, "bits": at["bits"],
                                              "block_size": at["block_size"]})
                for i, N in enumerate(at["Ns"])]

    def _apart(self, node, ctx, normed):
        for p in self._projections(node, normed):
            self._mm.execute(p, ctx)

    def _run(self, node, ctx, normed, x, skip, gamma, dnorm, dsum, M):
        torch = _torch()
        hs, ys = [], []
        for p in self._projections(node, normed):
            a, b, sc, zp, N, K, bits, bs = self._mm._validate(p, ctx)
            hs.append(self._mm._weights(p, b, sc, zp, N, K, bits, bs))
            ys.append(torch.empty(tuple(x.shape[:-1]) + (N,), dtype=torch.float32, device=x.device))
        native.gemm_dev_skipnorm(hs, x.data_ptr(), skip.data_ptr(), gamma.data_ptr(),
                                 _attr_float(node, "epsilon", 1e-5), dnorm.data_ptr(),
                                 None if dsum is None else dsum.data_ptr(), [y.data_ptr() for y in ys], M, _stream(x))
        for o, y in zip(node.outputs[:-1], ys):
            ctx.set(o, y)


class HipSkipNormGateUpSiluMulKernel(_HipSkipNormFused):
    op_type = "SkipNormGateUpSiluMul"

    def __init__(self, matmul=None):
        super().__init__(matmul)
        self._gus = HipGateUpSiluMulKernel(self._mm)

    def _projections(self, node, a):
        at = node.attributes
        mk = lambda nm, lo: GraphNode("MatMulNBits", f"{node.name}/{nm}", [a] + list(node.inputs[lo:lo + 3]),   # noqa: E731
                                      [f"{node.name}/{nm}_out"], {k: at[k] for k in ("K", "N", "bits", "block_size")})
        return [mk("gate", 3), mk("up", 6)]

    def _apart(self, node, ctx, normed):
        self._gus.execute(GraphNode("GateUpSiluMul", node.name + "/gate_up_silu", [normed] + list(node.inputs[3:9]),
                                    [node.outputs[0]], {k: v for k, v in node.attributes.items() if k != "epsilon"}),
                          ctx)

    def _run(self, node, ctx, normed, x, skip, gamma, dnorm, dsum, M):
        torch = _torch()
        gnode, unode = self._projections(node, normed)
        _, bg, sg, zg, N, K, bits, bs = self._mm._validate(gnode, ctx)
        _, bu, su, zu, _, _, _, _ = self._mm._validate(unode, ctx)
        wg = self._mm._weights(gnode, bg, sg, zg, N, K, bits, bs)
        wu = self._mm._weights(unode, bu, su, zu, N, K, bits, bs)
        h = torch.empty(tuple(x.shape[:-1]) + (N,), dtype=torch.float32, device=x.device)
        native.gemm_dev_skipnorm_swiglu(wg, wu, x.data_ptr(), skip.data_ptr(), gamma.data_ptr(),
                                        _attr_float(node, "epsilon", 1e-5), dnorm.data_ptr(),
                                        None if dsum is None else dsum.data_ptr(), h.data_ptr(), M, _stream(x))
        ctx.set(node.outputs[0], h)


@dataclasses.dataclass
class _Cache:
    k: object
    v: object
    capacity: int
    returned: int = -1   # rows of the present K/V views the last call handed out


class HipGroupQueryAttentionKernel(IKernel):
    """GroupQueryAttention (GroupQueryAttentionKernel.cs:64-323). Present K/V are views
    into per-node capacity buffers: when the next step passes back exactly the views the
    last call returned (same K and V buffers, past equal to the rows handed out), the
    new rows are appended in place (ms_hip_gqa past_in_present) instead of copying the
    past, and the buffer doubles when it fills. Any other past (an older step's present,
    two candidates from one past, a rollback) is copied into a fresh buffer, so present
    tensors handed out earlier never change, as with the reference's fresh tensors."""
    op_type = "GroupQueryAttention"

    def __init__(self):
        self._dev = _DeviceInputs()
        self._caches: dict[str, _Cache] = {}
        self._workspace: dict[str, object] = {}   # key-split workspace per node (ms_hip_gqa_workspace_size)

    def _cache_for(self, node, B, KH, D, past_k, past_v, past, total, device):
        torch = _torch()
        c = self._caches.get(node.name)
        follows = (c is not None and past_k is not None and past > 0 and past == c.returned
                   and isinstance(past_k, torch.Tensor) and isinstance(past_v, torch.Tensor)
                   and past_k.data_ptr() == c.k.data_ptr() and past_v.data_ptr() == c.v.data_ptr()
                   and tuple(c.k.shape[:2]) == (B, KH) and c.k.shape[3] == D)
        if follows and c.capacity >= total:
            return c, True
        # A fresh buffer (the old one may back present tensors the caller still holds):
        # twice the old capacity when a followed cache fills, else room to append as much
        # again as this call holds.
        cap = max(total, 2 * c.capacity, 64) if follows else max(2 * total, 64)
        k = torch.empty((B, KH, cap, D), dtype=torch.float32, device=device)
        v = torch.empty_like(k)
        c = _Cache(k, v, cap)
        self._caches[node.name] = c
        return c, False

    def execute(self, node: GraphNode, ctx: GraphContext) -> None:
        torch = _torch()
        H = node.attr_int("num_heads", 0)
        KH = node.attr_int("kv_num_heads", 0)
        if H <= 0 or KH <= 0:
            raise ModelSharpException("GroupQueryAttention requires positive 'num_heads' and 'kv_num_heads'.")
        if H % KH != 0:
            raise ModelSharpException(
                f"GroupQueryAttention num_heads={H} must be a multiple of kv_num_heads={KH}.")
        q = self._dev.input(ctx, node.inputs[0])
        if q.dim() != 3:
            raise ModelSharpException(
                f"GroupQueryAttention supports only 3-D query [B, S, hidden]; got rank {q.dim()}.")
        key_name = node.inputs[1] if len(node.inputs) > 1 else ""
        value_name = node.inputs[2] if len(node.inputs) > 2 else ""
        packed = len(key_name) == 0 or len(value_name) == 0
        B, Sq = int(q.shape[0]), int(q.shape[1])
        k = v = None
        if packed:
            hidden = int(q.shape[2])
            unit = H + 2 * KH
            if hidden % unit != 0:
                raise ModelSharpException(
                    f"GroupQueryAttention packed-QKV hidden {hidden} not divisible by "
                    f"(num_heads + 2·kv_num_heads) = {unit}.")
            D = hidden // unit
            Skv = Sq
        else:
            k = self._dev.input(ctx, key_name)
            v = self._dev.input(ctx, value_name)
            if k.dim() != 3 or v.dim() != 3:
                raise ModelSharpException("GroupQueryAttention supports only unpacked 3-D key/value.")
            q_hidden = int(q.shape[2])
            Skv, kv_hidden = int(k.shape[1]), int(k.shape[2])
            if int(k.shape[0]) != B or int(v.shape[0]) != B:
                raise ModelSharpException("GroupQueryAttention query/key/value batch sizes disagree.")
            if int(v.shape[1]) != Skv or int(v.shape[2]) != kv_hidden:
                raise ModelSharpException("GroupQueryAttention key/value shapes disagree.")
            if q_hidden % H != 0:
                raise ModelSharpException(
                    f"GroupQueryAttention query hidden {q_hidden} not divisible by num_heads={H}.")
            D = q_hidden // H
            if kv_hidden != KH * D:
                raise ModelSharpException(
                    f"GroupQueryAttention key/value hidden {kv_hidden} must equal kv_num_heads·head_dim = {KH * D}.")
        past_k = ctx.get_tensor(node.inputs[3]) if len(node.inputs) > 3 and node.inputs[3] else None
        past_v = ctx.get_tensor(node.inputs[4]) if len(node.inputs) > 4 and node.inputs[4] else None
        past = 0
        if past_k is not None:
            if past_v is None:
                raise ModelSharpException("GroupQueryAttention past_key provided without past_value.")
            shp = tuple(int(x) for x in past_k.shape)
            if len(shp) != 4 or shp[0] != B or shp[1] != KH or shp[3] != D:
                raise ModelSharpException(
                    "GroupQueryAttention past_key must be [B, kv_num_heads, pastSeq, head_dim].")
            past = shp[2]
        total = past + Skv
        seqlens = None
        if len(node.inputs) > 5 and node.inputs[5]:
            seqlens = self._dev.i32(ctx.get_tensor(node.inputs[5])).reshape(-1)
        do_rotary = node.attr_int("do_rotary", 0) != 0
        cos = sin = None
        if do_rotary:
            if len(node.inputs) <= 8 or not node.inputs[7] or not node.inputs[8]:
                raise ModelSharpException(
                    "GroupQueryAttention do_rotary=1 requires cos_cache (input 7) and sin_cache (input 8).")
            cos = self._dev.input(ctx, node.inputs[7])
            sin = self._dev.input(ctx, node.inputs[8])
        cache, in_place = self._cache_for(node, B, KH, D, past_k, past_v, past, total, q.device)
        if past and not in_place:
            pk_src, pv_src = self._dev.f32(past_k), self._dev.f32(past_v)
        else:
            pk_src = pv_src = None
        d = native.GqaDesc(batch=B, q_seq=Sq, kv_seq=Skv, num_heads=H, kv_num_heads=KH, head_dim=D,
                           packed_qkv=int(packed), past_seq=past, past_in_present=int(in_place and past > 0),
                           present_capacity=cache.capacity, do_rotary=int(do_rotary),
                           rotary_interleaved=int(node.attr_int("rotary_interleaved", 0) != 0),
                           cos_rows=0 if cos is None else int(cos.shape[0]),
                           cos_cols=0 if cos is None else int(cos.shape[-1]),
                           local_window_size=node.attr_int("local_window_size", -1),
                           scale=_attr_float(node, "scale", 0.0),
                           seqlens_len=0 if seqlens is None else int(seqlens.numel()))
        out = torch.empty((B, Sq, H * D), dtype=torch.float32, device=q.device)
        ws_bytes = native.gqa_workspace_size(d)
        ws = None
        if ws_bytes:
            ws = self._workspace.get(node.name)
            if ws is None or ws.numel() * 4 < ws_bytes:
                ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=q.device)
                self._workspace[node.name] = ws
        ptr = lambda t: None if t is None else t.data_ptr()   # noqa: E731
        native.gqa(d, q.data_ptr(), ptr(k), ptr(v), ptr(pk_src), ptr(pv_src), ptr(seqlens), ptr(cos), ptr(sin),
                   out.data_ptr(), cache.k.data_ptr(), cache.v.data_ptr(), ptr(ws), ws_bytes, _stream(q))
        ctx.set(node.outputs[0], out)
        cache.returned = total
        if _present(node, 1):
            ctx.set(node.outputs[1], cache.k[:, :, :total, :])
        if _present(node, 2):
            ctx.set(node.outputs[2], cache.v[:, :, :total, :])


def register_decoder_kernels(registry: KernelRegistry) -> KernelRegistry:
    """Registers the device kernels of the decoder-layer operators (last registration
    wins, KernelRegistry.cs:20-24)."""
    for k in (HipSimplifiedLayerNormalizationKernel(), HipSkipSimplifiedLayerNormalizationKernel(),
              HipGroupQueryAttentionKernel(), HipAddKernel(), HipMulKernel(), HipSigmoidKernel(),
              HipSiluMulKernel(), HipGateUpSiluMulKernel(), HipSkipNormMatMulNBitsKernel(),
              HipSkipNormGateUpSiluMulKernel()):
        registry.register(k)
    return registry
