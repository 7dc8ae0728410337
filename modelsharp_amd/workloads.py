"""Seeded synthetic MatMulNBits workloads and their algorithmic cost.

The five workloads the measurements and parity tests use:
  qwen05b_up      one op, M=1, K=896, N=4864 (Qwen2.5-0.5B MLP up), bs=32, zp
  qwen05b_decode  the Qwen2.5-0.5B layer projections + lm_head, M=1, bs=32, zp
  7b_decode       a 7B-class layer (hidden 3584, intermediate 18944, 28 query /
                  4 KV heads of dim 128), M=1, bs=32, zp
  llama7b_smallm  M in {1,2,4,8,16}, Llama-2-7B MLP shapes, bs=128, no zp
  llama7b_prefill M in {128,512,2048}, same shapes, bs=32, zp, activations
                  shaped like post-RMSNorm rows
All inputs of one workload come from one seed (numpy PCG64). Codes and zero
points are uniform 0..15, packed low nibble first; unused nibbles (a partial
last block, an odd block count) are filled with random codes, which the
operator must ignore.
"""
from __future__ import annotations

import dataclasses
import math

import numpy as np


@dataclasses.dataclass(frozen=True)
class Op:
    name: str
    K: int
    N: int
    block_size: int = 32
    has_zp: bool = True
    scale_lo: float = 0.001
    scale_hi: float = 0.01
    bits: int = 4

    @property
    def nb(self) -> int:
        return (self.K + self.block_size - 1) // self.block_size

    @property
    def blob(self) -> int:
        return (self.block_size * self.bits + 7) // 8

    @property
    def zrb(self) -> int:
        return (self.nb * self.bits + 7) // 8


def _qwen(name, K, N):
    return Op(name, K, N, 32, True, 0.002, 0.02)


def _7b(name, K, N):
    return Op(name, K, N, 32, True, 0.001, 0.01)


QWEN05B_UP = _qwen("up", 896, 4864)
QWEN05B_DECODE = [_qwen("q", 896, 896), _qwen("k", 896, 128), _qwen("v", 896, 128), _qwen("o", 896, 896),
                  _qwen("gate", 896, 4864), _qwen("up", 896, 4864), _qwen("down", 4864, 896),
                  _qwen("lm_head", 896, 151936)]
# Activation buffer each QWEN05B_DECODE projection reads in the model: q/k/v share the
# attention input, gate/up the MLP input; o, down and lm_head read their own.
QWEN05B_DECODE_SHARE = [0, 0, 0, 3, 4, 4, 6, 7]
DECODE_7B = [_7b("q", 3584, 3584), _7b("k", 3584, 512), _7b("v", 3584, 512), _7b("o", 3584, 3584),
             _7b("gate", 3584, 18944), _7b("up", 3584, 18944), _7b("down", 18944, 3584)]
# Activation buffer each DECODE_7B projection reads in a decoder layer: q/k/v share the
# attention input, gate/up the MLP input.
DECODE_7B_SHARE = [0, 0, 0, 3, 4, 4, 6]
LLAMA7B_SMALLM_OPS = [Op("up", 4096, 11008, 128, False), Op("down", 11008, 4096, 128, False)]
LLAMA7B_SMALLM_M = [1, 2, 4, 8, 16]
LLAMA7B_PREFILL_OPS = [_7b("up", 4096, 11008), _7b("down", 11008, 4096)]
LLAMA7B_PREFILL_M = [128, 512, 2048]


def weight_bytes(op: Op) -> int:
    """Packed B + fp32 scales + packed zero points."""
    return op.N * op.nb * op.blob + op.N * op.nb * 4 + (op.N * op.zrb if op.has_zp else 0)


def algorithmic_bytes(op: Op, M: int) -> int:
    """Bytes one call must move: weights once, A (fp32) once, Y (fp32) once."""
    return weight_bytes(op) + M * op.K * 4 + M * op.N * 4


def algorithmic_bytes_group(ops: list, M: int) -> int:
    """Bytes one grouped launch over ops that share their activations must move: each
    op's weights and Y once, the shared A once."""
    return sum(algorithmic_bytes(op, M) for op in ops) - (len(ops) - 1) * M * ops[0].K * 4


def flops(op: Op, M: int) -> int:
    return 2 * M * op.N * op.K


def pack_nibbles(codes: np.ndarray) -> np.ndarray:
    """[..., 2j] low nibble, [..., 2j+1] high nibble (MatMulNBitsKernel.cs:28-30)."""
    c = codes.astype(np.uint8)
    if c.shape[-1] % 2:
        c = np.concatenate([c, np.zeros(c.shape[:-1] + (1,), np.uint8)], axis=-1)
    return (c[..., 0::2] & 0x0F) | ((c[..., 1::2] & 0x0F) << 4)


def make_weights(op: Op, seed: int):
    """(B uint8 [N, nb, blob], scales fp32 [N*nb], zp uint8 [N, zrb] or None)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    # Uniform random bytes are two independent uniform 4-bit codes (bits=4) or
    # one uniform 8-bit code (bits=8), for B and for the packed zero points.
    b = rng.integers(0, 256, size=(op.N, op.nb, op.blob), dtype=np.uint8)
    scales = rng.uniform(op.scale_lo, op.scale_hi, size=op.N * op.nb).astype(np.float32)
    zp = rng.integers(0, 256, size=(op.N, op.zrb), dtype=np.uint8) if op.has_zp else None
    return b, scales, zp


def make_activations(M: int, K: int, seed: int, kind: str = "normal") -> np.ndarray:
    """A [M, K] fp32.

    normal:  A ~ N(0, 1).
    rmsnorm: A ~ N(0, 0.5^2); a fixed seeded 1% of the K channels (the same
             channels in every row) scaled x20 as outliers; then every row
             scaled to unit RMS — one reading of "rows shaped like
             post-RMSNorm activations".
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    if kind == "normal":
        return rng.standard_normal((M, K), dtype=np.float32)
    if kind == "rmsnorm":
        a = rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.5)
        ch = rng.choice(K, size=max(1, K // 100), replace=False)
        a[:, ch] *= np.float32(20.0)
        rms = np.sqrt(np.mean(a.astype(np.float64) ** 2, axis=1, keepdims=True))
        return (a / rms).astype(np.float32)
    raise ValueError(kind)


def ideal_us(nbytes: int, peak_gbs: float = 8000.0) -> float:
    return nbytes / (peak_gbs * 1e3)


def rotation_copies(footprint_bytes: int, total_bytes: int = 1 << 30) -> int:
    """Distinct copies needed so a rotation touches total_bytes (> 256 MiB MALL)."""
    return max(2, math.ceil(total_bytes / footprint_bytes))
