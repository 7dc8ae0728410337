"""The reference's operator interface, restated for the HIP MatMulNBits kernel.

Mirrors (paths relative to the ModelSharp checkout):
  ModelSharpException         src/ModelSharp/Exceptions/ModelSharpException.cs:6-11
  UnsupportedOperatorException src/ModelSharp/Exceptions/UnsupportedOperatorException.cs:8-21
  GraphNode                   src/ModelSharp/Graph/GraphNode.cs (op type, name, inputs,
                              outputs, attributes; "" = omitted optional input)
  ModelGraph                  src/ModelSharp/Graph/ModelGraph.cs (nodes, initializers)
  GraphContext                src/ModelSharp/Cpu/Kernels/GraphContext.cs:106-122
  IKernel                     src/ModelSharp/Cpu/Kernels/IKernel.cs:10-17
  KernelRegistry              src/ModelSharp/Cpu/Kernels/KernelRegistry.cs:15-30
  Engine.run                  src/ModelSharp/Cpu/ManagedCpuEngine.cs:36-84 (node loop)
Tensors are numpy arrays on the host, or torch tensors already on the device.
"""
from __future__ import annotations

import dataclasses
from typing import Any

import numpy as np


class ModelSharpException(Exception):
    """Base type for operator errors (ModelSharpException.cs:6)."""


class UnsupportedOperatorException(ModelSharpException):
    """UnsupportedOperatorException.cs:17-21 — message names the op and node."""

    def __init__(self, op: str, detail: str | None = None):
        super().__init__(f"Operator '{op}' is not supported yet by the managed engine"
                         + ("." if detail is None else f" ({detail})."))
        self.operator = op


# .NET ElementType names for error messages (MatMulNBitsKernel.cs:143, QuantizeKernels.cs:54-56).
_ELEMENT_TYPE = {
    np.dtype(np.float32): "Float32", np.dtype(np.float16): "Float16", np.dtype(np.float64): "Float64",
    np.dtype(np.uint8): "UInt8", np.dtype(np.int8): "Int8", np.dtype(np.int16): "Int16",
    np.dtype(np.uint16): "UInt16", np.dtype(np.int32): "Int32", np.dtype(np.int64): "Int64",
    np.dtype(np.bool_): "Bool",
}


def element_type(t: Any) -> str:
    dt = np.dtype(str(t.dtype).replace("torch.", "")) if not isinstance(t, np.ndarray) else t.dtype
    return _ELEMENT_TYPE.get(dt, str(dt))


@dataclasses.dataclass
class GraphNode:
    op_type: str
    name: str
    inputs: list[str]
    outputs: list[str]
    attributes: dict[str, Any] = dataclasses.field(default_factory=dict)

    def attr_int(self, key: str, default: int) -> int:
        """Attr.Int (Cpu/Kernels/Internal/Attr.cs:9-10): attributes are boxed longs."""
        return int(self.attributes.get(key, default))


@dataclasses.dataclass
class ModelGraph:
    nodes: list[GraphNode]
    initializers: dict[str, Any]
    inputs: list[str] = dataclasses.field(default_factory=list)
    outputs: list[str] = dataclasses.field(default_factory=list)


class GraphContext:
    """Name -> tensor environment of one run (GraphContext.cs)."""

    def __init__(self, values: dict[str, Any] | None = None, constants=()):
        self.values: dict[str, Any] = dict(values or {})
        # Names bound to the graph's initializers: device kernels may keep their uploads.
        self.constants: frozenset[str] = frozenset(constants)

    def is_constant(self, name: str) -> bool:
        return name in self.constants

    def get_tensor(self, name: str):
        if name not in self.values:
            raise ModelSharpException(f"Tensor '{name}' is not available in the execution context.")
        return self.values[name]

    def get(self, name: str):
        """Float32 view; fp16 is widened (GraphContext.cs:106, Tensor.ToFloat32)."""
        t = self.get_tensor(name)
        if isinstance(t, np.ndarray):
            return t if t.dtype == np.float32 else t.astype(np.float32)
        if str(t.dtype) != "torch.float32":
            return t.float()
        return t

    def has(self, name: str) -> bool:
        return len(name) != 0 and name in self.values

    def set(self, name: str, value) -> None:
        self.values[name] = value


class IKernel:
    """Executes one operator against a GraphContext (IKernel.cs:10-17)."""

    op_type: str = ""

    def execute(self, node: GraphNode, ctx: GraphContext) -> None:   # pragma: no cover - interface
        raise NotImplementedError


class KernelRegistry:
    """Op type -> kernel; the last registration of an op type wins (KernelRegistry.cs:20-24)."""

    def __init__(self):
        self._kernels: dict[str, IKernel] = {}

    def register(self, kernel: IKernel) -> "KernelRegistry":
        self._kernels[kernel.op_type] = kernel
        return self

    def try_get(self, op_type: str):
        k = self._kernels.get(op_type)
        return (k is not None), k

    @property
    def count(self) -> int:
        return len(self._kernels)


class Engine:
    """The node loop of ManagedCpuEngine.Run / ExecuteNodes (ManagedCpuEngine.cs:36-84)."""

    def __init__(self, graph: ModelGraph, kernels: KernelRegistry):
        self.graph = graph
        self.kernels = kernels

    def run(self, feeds: dict[str, Any]) -> dict[str, Any]:
        env = dict(self.graph.initializers)
        env.update(feeds)
        ctx = GraphContext(env, constants=set(self.graph.initializers) - set(feeds))
        for node in self.graph.nodes:
            ok, kernel = self.kernels.try_get(node.op_type)
            if not ok:
                raise UnsupportedOperatorException(node.op_type, f"node '{node.name}'")
            kernel.execute(node, ctx)
        return {name: ctx.get_tensor(name) for name in self.graph.outputs}
