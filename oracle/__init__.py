"""CPU oracle of the MatMulNBits operator — TEST INFRASTRUCTURE.

Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, to check the device's results or as the timed CPU baseline; the product never imports
it. liboracle_nbits.so is the C restatement of the reference's managed kernel
and of its native W4A8 kernel (ms_nbits_oracle.c, citations there);
_ref/libms_ref_qgemm.so and _ref/libms_ref_w4a8.so, when present, are the
reference's own native ms_qgemm_nbits and ms_qgemm_w4a8 compiled from its
sources (without FP contraction), and _ref/libms_ref_w4a8_shipped.so its
ms_qgemm_w4a8 with the reference Makefile's own flags (-ffast-math).
"""
from __future__ import annotations

import ctypes
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
_vp = ctypes.c_void_p
_lib = None
_ref = None


class GqaDesc(ctypes.Structure):
    """msor_gqa_desc / ms_hip_gqa_desc (the same field order)."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "batch", "q_seq", "kv_seq", "num_heads", "kv_num_heads", "head_dim", "packed_qkv", "past_seq",
        "past_in_present", "present_capacity", "do_rotary", "rotary_interleaved", "cos_rows", "cos_cols",
        "local_window_size")] + [("scale", ctypes.c_float), ("seqlens_len", ctypes.c_int)]


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_vp)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        path = HERE / "liboracle_nbits.so"
        if not path.is_file():
            raise RuntimeError(f"oracle not built: {path} (run __graft_entry__.build())")
        L = ctypes.CDLL(str(path))
        L.msor_unpack_nbit.restype = ctypes.c_int
        L.msor_unpack_nbit.argtypes = [_vp, ctypes.c_int64, ctypes.c_int, ctypes.c_int]
        L.msor_dequant_block4.argtypes = [_vp, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_float, _vp]
        L.msor_dequant_block8.argtypes = [_vp, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_float, _vp]
        L.msor_fma_accumulate.restype = ctypes.c_float
        L.msor_fma_accumulate.argtypes = [ctypes.c_float, _vp, _vp, ctypes.c_int]
        L.msor_should_parallelize.restype = ctypes.c_int
        L.msor_should_parallelize.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
        L.msor_matmul_nbits.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp] + [ctypes.c_int] * 6
        L.msor_dequant_weights.argtypes = [_vp, _vp, _vp, _vp, _vp] + [ctypes.c_int] * 5
        L.msor_matmul_f64.argtypes = [_vp, _vp, _vp] + [ctypes.c_int] * 4
        L.msor_w4a8_quantize.argtypes = [_vp, _vp, _vp] + [ctypes.c_int] * 3
        L.msor_rmsnorm.argtypes = [_vp, _vp, _vp, _vp, ctypes.c_int64, ctypes.c_int, ctypes.c_float]
        L.msor_skip_rmsnorm.argtypes = [_vp] * 8 + [ctypes.c_int64, ctypes.c_int, ctypes.c_float]
        L.msor_silu_mul.argtypes = [_vp, _vp, _vp, ctypes.c_int64]
        L.msor_gqa.argtypes = [ctypes.POINTER(GqaDesc)] + [_vp] * 11
        L.msor_qgemm_w4a8.argtypes = [_vp, _vp, _vp, _vp, _vp] + [ctypes.c_int] * 6
        L.msor_w4a8_managed.argtypes = [_vp] * 6 + [ctypes.c_int] * 5
        _lib = L
    return _lib


def ref_lib():
    """The reference's own ms_qgemm_nbits (built from its sources), or None."""
    global _ref
    if _ref is None:
        path = HERE / "_ref" / "libms_ref_qgemm.so"
        if not path.is_file():
            return None
        L = ctypes.CDLL(str(path))
        L.ms_qgemm_nbits.restype = None
        L.ms_qgemm_nbits.argtypes = [_vp, _vp, _vp, _vp, _vp] + [ctypes.c_int] * 5
        _ref = L
    return _ref


_W4A8_LIBS = {"plain": "libms_ref_w4a8.so", "shipped": "libms_ref_w4a8_shipped.so"}
_ref_w4a8_libs: dict = {}


def ref_w4a8_lib(build="plain"):
    """The reference's own ms_qgemm_w4a8 built from its sources, or None: "plain" without FP
    contraction (the bit-exact witness), "shipped" with its native/Makefile's CXXFLAGS
    (-ffast-math)."""
    if build not in _ref_w4a8_libs:
        path = HERE / "_ref" / _W4A8_LIBS[build]
        if not path.is_file():
            return None
        L = ctypes.CDLL(str(path))
        L.ms_qgemm_w4a8.restype = None
        L.ms_qgemm_w4a8.argtypes = [_vp, _vp, _vp, _vp, _vp] + [ctypes.c_int] * 5
        _ref_w4a8_libs[build] = L
    return _ref_w4a8_libs[build]


def threads() -> int:
    try:
        return max(1, len(os.sched_getaffinity(0)))
    except AttributeError:
        return os.cpu_count() or 1


def matmul_nbits(a, b, scales, zp_packed, N, K, bits, block_size, zp_float=None, nthreads=None):
    """y[M,N] of the managed kernel's default path (MatMulNBitsKernel.cs:193-262)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    M = a.size // K
    y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp_packed = None if zp_packed is None else np.ascontiguousarray(zp_packed, dtype=np.uint8)
    zp_float = None if zp_float is None else np.ascontiguousarray(zp_float, dtype=np.float32)
    lib().msor_matmul_nbits(_ptr(a), _ptr(b), _ptr(scales), _ptr(zp_packed), _ptr(zp_float), _ptr(y),
                            M, N, K, bits, block_size, nthreads or threads())
    return y


def dequant_weights(b, scales, zp_packed, N, K, bits, block_size, zp_float=None, nthreads=None):
    w = np.empty((N, K), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp_packed = None if zp_packed is None else np.ascontiguousarray(zp_packed, dtype=np.uint8)
    zp_float = None if zp_float is None else np.ascontiguousarray(zp_float, dtype=np.float32)
    lib().msor_dequant_weights(_ptr(b), _ptr(scales), _ptr(zp_packed), _ptr(zp_float), _ptr(w),
                               N, K, bits, block_size, nthreads or threads())
    return w


def matmul_f64(a, w, nthreads=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    M = a.size // K
    y = np.empty((M, N), dtype=np.float64)
    lib().msor_matmul_f64(_ptr(a), _ptr(w), _ptr(y), M, N, K, nthreads or threads())
    return y


def fma_accumulate(acc, a, w):
    a = np.ascontiguousarray(a, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    return lib().msor_fma_accumulate(ctypes.c_float(acc), _ptr(a), _ptr(w), int(a.size))


def unpack_nbit(data, base_byte, index, bits):
    data = np.ascontiguousarray(data, dtype=np.uint8)
    return lib().msor_unpack_nbit(_ptr(data), base_byte, index, bits)


def ref_qgemm_nbits(a, b, scales, zp_packed, M, N, K, bits, block_size):
    """The reference's native ms_qgemm_nbits (qgemm.cpp:77-118), or None if not built."""
    L = ref_lib()
    if L is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.float32)
    y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp_packed = None if zp_packed is None else np.ascontiguousarray(zp_packed, dtype=np.uint8)
    L.ms_qgemm_nbits(_ptr(a), _ptr(b), _ptr(scales), _ptr(zp_packed), _ptr(y), M, N, K, bits, block_size)
    return y


def w4a8_quantize(a, K, block_size):
    """(aq int8 [M, nb*bs], sa fp32 [M, nb]) of qgemm_w4a8.cpp:257-285."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    M = a.size // K
    nb = (K + block_size - 1) // block_size
    aq = np.empty((M, nb * block_size), dtype=np.int8)
    sa = np.empty((M, nb), dtype=np.float32)
    lib().msor_w4a8_quantize(_ptr(a), _ptr(aq), _ptr(sa), M, K, block_size)
    return aq, sa


def qgemm_w4a8(a, b, scales, zp_packed, N, K, bits, block_size, nthreads=None):
    """y[M,N] of the native W4A8 kernel (qgemm_w4a8.cpp)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    M = a.size // K
    y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp_packed = None if zp_packed is None else np.ascontiguousarray(zp_packed, dtype=np.uint8)
    lib().msor_qgemm_w4a8(_ptr(a), _ptr(b), _ptr(scales), _ptr(zp_packed), _ptr(y), M, N, K, bits, block_size,
                          nthreads or threads())
    return y


def w4a8_managed(a, b, scales, zp_packed, N, K, block_size, zp_float=None, nthreads=None):
    """The reference's managed W4A8 product (4-bit codes), msor_w4a8_managed."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    M = a.size // K
    y = np.empty((M, N), np.float32)
    zp_packed = None if zp_packed is None else np.ascontiguousarray(zp_packed, dtype=np.uint8)
    zp_float = None if zp_float is None else np.ascontiguousarray(zp_float, dtype=np.float32)
    lib().msor_w4a8_managed(_ptr(a), _ptr(np.ascontiguousarray(b, dtype=np.uint8)),
                            _ptr(np.ascontiguousarray(scales, dtype=np.float32)), _ptr(zp_packed), _ptr(zp_float),
                            _ptr(y), M, N, K, block_size, threads() if nthreads is None else nthreads)
    return y


def ref_qgemm_w4a8(a, b, scales, zp_packed, M, N, K, bits, block_size, build="plain"):
    """The reference's native ms_qgemm_w4a8 (see ref_w4a8_lib), or None if not built."""
    L = ref_w4a8_lib(build)
    if L is None:
        return None
    a = np.ascontiguousarray(a, dtype=np.float32)
    y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp_packed = None if zp_packed is None else np.ascontiguousarray(zp_packed, dtype=np.uint8)
    L.ms_qgemm_w4a8(_ptr(a), _ptr(b), _ptr(scales), _ptr(zp_packed), _ptr(y), M, N, K, bits, block_size)
    return y


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def rmsnorm(x, scale, eps):
    """SimplifiedLayerNormalization over the last axis: (y, inv_std)."""
    x = _f32(x)
    norm = x.shape[-1]
    rows = x.size // norm
    y = np.empty_like(x)
    inv = np.empty(rows, np.float32)
    lib().msor_rmsnorm(_ptr(x), _ptr(_f32(scale)), _ptr(y), _ptr(inv), rows, norm, ctypes.c_float(eps))
    return y, inv


def skip_rmsnorm(inp, skip, gamma, beta, bias, eps):
    """SkipSimplifiedLayerNormalization: (out, inv_std, input_skip_bias_sum)."""
    inp, skip = _f32(inp), _f32(skip)
    norm = _f32(gamma).size
    rows = inp.size // norm
    out, total = np.empty_like(inp), np.empty_like(inp)
    inv = np.empty(rows, np.float32)
    lib().msor_skip_rmsnorm(_ptr(inp), _ptr(skip), _ptr(_f32(gamma)), _ptr(_f32(beta)), _ptr(_f32(bias)), _ptr(out),
                            _ptr(total), _ptr(inv), rows, norm, ctypes.c_float(eps))
    return out, inv, total


def silu_mul(g, u):
    g, u = _f32(g), _f32(u)
    y = np.empty_like(g)
    lib().msor_silu_mul(_ptr(g), _ptr(u), _ptr(y), g.size)
    return y


def gqa(desc: GqaDesc, q, k=None, v=None, past_k=None, past_v=None, seqlens=None, cos=None, sin=None):
    """GroupQueryAttention: (out [B, Sq, H*D], present_k, present_v [B, kvH, past+Skv, D])."""
    d = desc
    total = d.past_seq + d.kv_seq
    out = np.empty((d.batch, d.q_seq, d.num_heads * d.head_dim), np.float32)
    pk = np.empty((d.batch, d.kv_num_heads, total, d.head_dim), np.float32)
    pv = np.empty_like(pk)
    sl = None if seqlens is None else np.ascontiguousarray(seqlens, dtype=np.int32)
    lib().msor_gqa(ctypes.byref(d), _ptr(_f32(q)), _ptr(_f32(k)), _ptr(_f32(v)), _ptr(_f32(past_k)),
                   _ptr(_f32(past_v)), _ptr(sl), _ptr(_f32(cos)), _ptr(_f32(sin)), _ptr(out), _ptr(pk), _ptr(pv))
    return out, pk, pv
