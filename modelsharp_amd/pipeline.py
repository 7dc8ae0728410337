"""Loading a model for the device: the hook of Pipeline.Load / ModelSharpPipeline.Build
(src/ModelSharp/Pipeline/ModelSharpPipeline.cs:24-30, :125-160) where the managed engine
is built over KernelRegistry.CreateDefault() — here the registry gets the HIP kernels and
the MatMulNBits weights go to HBM at load time, streamed from the model's files.
"""
from __future__ import annotations

from . import onnx_loader
from .decoder_kernels import (HipGateUpSiluMulKernel, HipSkipNormGateUpSiluMulKernel, HipSkipNormMatMulNBitsKernel,
                              fuse_gate_up_silu, fuse_silu_mul, fuse_skipnorm, register_decoder_kernels)
from .graph import Engine, KernelRegistry, ModelGraph
from .hip_kernel import HipMatMulNBitsKernel, register_kernels


def build(graph: ModelGraph, registry: KernelRegistry | None = None) -> Engine:
    """Registers the device kernels on `registry` (last registration wins, so they
    replace the managed ones) and uploads every MatMulNBits weight triple."""
    registry = registry if registry is not None else KernelRegistry()
    register_decoder_kernels(registry)
    register_kernels(registry)
    for op, cls in (("MatMulNBits", HipMatMulNBitsKernel), ("GateUpSiluMul", HipGateUpSiluMulKernel),
                    ("SkipNormMatMulNBits", HipSkipNormMatMulNBitsKernel),
                    ("SkipNormGateUpSiluMul", HipSkipNormGateUpSiluMulKernel)):
        ok, k = registry.try_get(op)
        if ok and isinstance(k, cls):
            k.preload(graph)
    return Engine(graph, registry)


def load(path: str, registry: KernelRegistry | None = None, fuse: bool = True) -> Engine:
    """OnnxModelLoader.LoadModel + Build, with the SiLU-Mul fusion of the MLP gate, the
    gate/up projections folded into it, and each SkipSimplifiedLayerNormalization folded
    into the projections that read its output."""
    graph = onnx_loader.load_model(path)
    if fuse:
        fuse_silu_mul(graph)
        fuse_gate_up_silu(graph)
        fuse_skipnorm(graph)
    return build(graph, registry)
