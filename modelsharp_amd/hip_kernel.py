"""HipMatMulNBitsKernel — the MatMulNBits operator routed to the MI355X library.

A drop-in for the reference's managed kernel behind the same interface
(IKernel, OpType "MatMulNBits"): it validates its inputs exactly as
src/ModelSharp/Cpu/Kernels/Quantize/MatMulNBitsKernel.cs:79-169 does (same
checks, same order, same messages), keeps one device-resident weight handle per
initializer (created at load time by preload(), or on first use), and calls the
C ABI of libms_hip_nbits.so. It never falls back to a CPU kernel: every input
the managed kernel accepts runs on the device — packed or float zero points,
Float32 or Float16 scales (widened exactly on the device, as GraphContext.Get
widens them, GraphContext.cs:106), Float32 or Float16 activations, bits 4 or 8,
any block size.
"""
from __future__ import annotations

import os
import threading

import numpy as np

from . import native
from .graph import GraphContext, GraphNode, IKernel, KernelRegistry, ModelGraph, ModelSharpException, element_type


def _to_numpy(t):
    if isinstance(t, np.ndarray):
        return t
    return t.detach().cpu().numpy()


def _raw_float(t) -> np.ndarray:
    """Host copy of a float tensor in its stored type when the C ABI takes that type
    (Float32, Float16), else widened to Float32 as GraphContext.Get does."""
    x = _to_numpy(t)
    return x if x.dtype in (np.float32, np.float16) else x.astype(np.float32)


def w4a8_flag() -> bool:
    """MODELSHARP_W4A8, read as MatMulNBitsKernel.ReadW4A8Flag reads it
    (MatMulNBitsKernel.cs:67-75)."""
    return os.environ.get("MODELSHARP_W4A8", "") in ("1", "true", "TRUE", "True", "on", "ON", "yes", "YES")


class HipMatMulNBitsKernel(IKernel):
    op_type = "MatMulNBits"

    def __init__(self, w4a8: bool | None = None):
        """w4a8: the opt-in approximate product (ms_hip_nbits_gemm_dev_w4a8), default
        from MODELSHARP_W4A8 at construction, as the reference reads it once per process.
        It covers packed and default zero points, as the native W4A8 kernel the
        reference routes them to does (MatMulNBitsKernel.cs:172-186, NativeQuant.cs:78-115);
        nodes with float zero points keep the exact product."""
        self._lock = threading.Lock()
        self._handles: dict[tuple, tuple] = {}
        self.w4a8 = w4a8_flag() if w4a8 is None else bool(w4a8)
        self.file_uploads = 0   # handles streamed from file slices by preload()

    # ---- validation: MatMulNBitsKernel.cs:79-161 ----------------------------------------
    @staticmethod
    def _validate(node: GraphNode, ctx: GraphContext):
        a = ctx.get_tensor(node.inputs[0])   # Float16 stays Float16: widened on the device
        b = ctx.get_tensor(node.inputs[1])
        if element_type(b) != "UInt8":                          # QuantizeKernels.cs:54-56
            raise ModelSharpException(f"Tensor dtype is {element_type(b)}; expected UInt8.")
        N = node.attr_int("N", 0)
        K = node.attr_int("K", 0)
        bits = node.attr_int("bits", 4)
        block_size = node.attr_int("block_size", 0)
        # The raw tensor: widened to fp32 (GraphContext.cs:106) only when a handle is made.
        scales = ctx.get_tensor(node.inputs[2])
        lib = native.load()
        st = lib.ms_hip_nbits_check(N, K, bits, block_size, int(np.prod(b.shape)), int(np.prod(scales.shape)),
                                    0, 0, -1)
        if st:
            raise ModelSharpException(native.last_error())
        zp = None
        if len(node.inputs) > 3 and ctx.has(node.inputs[3]):   # :119-145
            zp = ctx.get_tensor(node.inputs[3])
            kind = {"UInt8": 1, "Float32": 2}.get(element_type(zp))
            if kind is None:
                raise ModelSharpException(
                    f"MatMulNBits zero_points must be Float32 or UInt8; got {element_type(zp)}.")
            st = lib.ms_hip_nbits_check(N, K, bits, block_size, int(np.prod(b.shape)),
                                        int(np.prod(scales.shape)), kind, int(np.prod(zp.shape)), -1)
            if st:
                raise ModelSharpException(native.last_error())
        if len(node.inputs) > 4 and ctx.has(node.inputs[4]):   # :148-155
            g_idx = _to_numpy(ctx.get_tensor(node.inputs[4])).reshape(-1).astype(np.int64)
            if np.any(g_idx != np.arange(g_idx.size, dtype=np.int64) // block_size):
                raise ModelSharpException(
                    "MatMulNBits g_idx with a non-trivial block permutation is not supported.")
        shape = tuple(a.shape)
        if len(shape) == 0 or shape[-1] != K:                  # :158-161
            raise ModelSharpException(
                f"MatMulNBits A inner dimension must equal K={K}; got shape [{','.join(str(d) for d in shape)}].")
        return a, b, scales, zp, N, K, bits, block_size

    # ---- device-resident weights -----------------------------------------------------------
    # One handle per (B, scales, zero points) initializer triple, keyed by the input names
    # as the per-initializer residency of IlgpuEngine.ResidentOrTempInt keys by name
    # (src/ModelSharp.Gpu/IlgpuEngine.cs:3396). The entry keeps the raw tensors it was made
    # from: a context that binds those names to other tensors gets a new handle (the old
    # one is closed), the same tensors always find the same handle.
    def _weights(self, node, b, scales, zp, N, K, bits, block_size) -> native.NBitsWeights:
        key = tuple(node.inputs[1:4])
        with self._lock:
            entry = self._handles.get(key)
            if entry is not None and entry[0][0] is b and entry[0][1] is scales and entry[0][2] is zp:
                return entry[1]
            w = native.NBitsWeights(_to_numpy(b), _raw_float(scales),
                                    None if zp is None else _to_numpy(zp), N, K, bits, block_size)
            if entry is not None:
                entry[1].close()
            self._handles[key] = ((b, scales, zp), w)
            return w

    def preload(self, graph: ModelGraph) -> int:
        """Load-time upload: one handle per MatMulNBits node whose B, scales and
        zero points are initializers. Returns the number of handles created.

        Initializers that a file-backed load located in their files (graph.sources,
        onnx_loader.load_model) are streamed from disk straight into HBM
        (ms_hip_nbits_weights_create_from_files); the others are uploaded from memory."""
        made = 0
        sources = getattr(graph, "sources", {}) or {}
        ctx = GraphContext(graph.initializers)
        for node in graph.nodes:
            if node.op_type != self.op_type:
                continue
            names = node.inputs[1:4]
            if not all(ctx.has(n) for n in names if n) or not ctx.has(node.inputs[1]):
                continue
            b = ctx.get_tensor(node.inputs[1])
            scales = ctx.get_tensor(node.inputs[2])
            zp = ctx.get_tensor(node.inputs[3]) if len(node.inputs) > 3 and ctx.has(node.inputs[3]) else None
            before = len(self._handles)
            names = [n for n in node.inputs[1:4] if n]
            if all(n in sources for n in names):
                self._weights_from_files(node, b, scales, zp, [sources[n] for n in node.inputs[1:3]]
                                         + [sources[node.inputs[3]] if zp is not None else None])
            else:
                self._weights(node, b, scales, zp, node.attr_int("N", 0), node.attr_int("K", 0),
                              node.attr_int("bits", 4), node.attr_int("block_size", 0))
            made += len(self._handles) - before
        return made

    def _weights_from_files(self, node, b, scales, zp, slices) -> None:
        key = tuple(node.inputs[1:4])
        with self._lock:
            entry = self._handles.get(key)
            if entry is not None and entry[0][0] is b and entry[0][1] is scales and entry[0][2] is zp:
                return
            w = native.NBitsWeights.from_files(slices[0], slices[1], slices[2], node.attr_int("N", 0),
                                               node.attr_int("K", 0), node.attr_int("bits", 4),
                                               node.attr_int("block_size", 0))
            if entry is not None:
                entry[1].close()
            self._handles[key] = ((b, scales, zp), w)
            self.file_uploads += 1

    def close(self) -> None:
        with self._lock:
            for _, w in self._handles.values():
                w.close()
            self._handles.clear()

    @property
    def handle_count(self) -> int:
        return len(self._handles)

    # ---- IKernel.Execute -------------------------------------------------------------------
    def execute(self, node: GraphNode, ctx: GraphContext) -> None:
        a, b, scales, zp, N, K, bits, block_size = self._validate(node, ctx)
        w = self._weights(node, b, scales, zp, N, K, bits, block_size)
        lead = tuple(a.shape[:-1])
        M = int(np.prod(lead)) if lead else 1
        w4a8 = self.w4a8 and (zp is None or element_type(zp) != "Float32")
        if isinstance(a, np.ndarray):
            a2 = a.reshape(M, K).astype(np.float32, copy=False)
            y = (w.gemm_w4a8(a2) if w4a8 else w.gemm(a2)).reshape(lead + (N,))
        else:
            import torch
            a2 = a.reshape(M, K)
            if a2.dtype not in (torch.float32, torch.float16) or (w4a8 and a2.dtype != torch.float32):
                a2 = a2.float()
            a2 = a2.contiguous()
            y = torch.empty(lead + (N,), dtype=torch.float32, device=a.device)
            stream = torch.cuda.current_stream(a.device).cuda_stream
            if w4a8:
                w.gemm_dev_w4a8(a2.data_ptr(), y.data_ptr(), M, stream)
            elif a2.dtype == torch.float16:
                w.gemm_dev_f16(a2.data_ptr(), y.data_ptr(), M, stream)
            else:
                w.gemm_dev(a2.data_ptr(), y.data_ptr(), M, stream)
        ctx.set(node.outputs[0], y)


def hip_enabled() -> bool:
    """False under MODELSHARP_HIP in {0, off, false}: the kill switch (the convention of
    MODELSHARP_NATIVE, NativeGemm.cs:53-57)."""
    return os.environ.get("MODELSHARP_HIP", "").lower() not in ("0", "off", "false")


def register_kernels(registry: KernelRegistry) -> KernelRegistry:
    """Routes MatMulNBits to the HIP kernel; last registration wins, as for
    ImageSharpRegistration.RegisterKernels (src/ModelSharp.ImageSharp/ImageSharpRegistration.cs:52-60).
    Under the kill switch the registry is left as it is (the kernel registered before
    keeps the op)."""
    if not hip_enabled():
        return registry
    return registry.register(HipMatMulNBitsKernel())
