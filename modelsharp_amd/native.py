"""ctypes binding of libms_hip_nbits.so, the C ABI in include/ms_hip_kernels.h.

The library is built in-tree (``__graft_entry__.build()`` or
``make -C modelsharp_amd/csrc``) into ``modelsharp_amd/lib/``;
``MODELSHARP_HIP_LIB`` overrides the path, as ``MODELSHARP_NATIVE_LIB`` does for
the reference's CPU library (src/ModelSharp/Native/NativeGemm.cs:98-116).
There is no CPU fallback: a missing library raises.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import re
import threading

import numpy as np

_PKG = pathlib.Path(__file__).resolve().parent
LIB_NAME = "libms_hip_nbits.so"
# Kernel ids of ms_hip_nbits_launch_info.
KERNEL_NAMES = ("generic", "gemv_w4", "mfma_w4", "gemv_w4_panel", "mfma_w4_pipe", "skinny_w4", "mfma_w4_rb",
                "gemv_general", "mfma_general", "gemv_w4a8", "mfma_w4a8", "w4a8_generic", "gemv_w8")
HEADER = _PKG.parent / "include" / "ms_hip_kernels.h"

MS_HIP_OK = 0
MS_HIP_ERR_INVALID = 1
MS_HIP_ERR_NO_DEVICE = 2
MS_HIP_ERR_HIP = 3
MS_HIP_ERR_UNSUPPORTED = 4
MS_HIP_ERR_DISABLED = 5
MS_HIP_ERR_FORCED = 6
MS_HIP_TUNING_INHERIT = -(2 ** 31)
MS_HIP_DTYPE_NONE, MS_HIP_DTYPE_F32, MS_HIP_DTYPE_F16, MS_HIP_DTYPE_U8 = 0, 1, 2, 3
_DTYPE_CODE = {np.dtype(np.float32): MS_HIP_DTYPE_F32, np.dtype(np.float16): MS_HIP_DTYPE_F16,
               np.dtype(np.uint8): MS_HIP_DTYPE_U8}

_c_int = ctypes.c_int
_c_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_fp = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_ip = ctypes.POINTER(ctypes.c_int)

# name -> (restype, argtypes); must cover every function in the header.
_PROTOTYPES = {
    "ms_hip_available": (_c_int, []),
    "ms_hip_device_name": (ctypes.c_char_p, []),
    "ms_hip_build_info": (ctypes.c_char_p, []),
    "ms_hip_last_error": (ctypes.c_char_p, []),
    "ms_hip_nbits_check": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_int, _c_i64, _c_i64]),
    "ms_hip_nbits_weights_create": (
        _c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)]),
    "ms_hip_nbits_weights_create_ex": (
        _c_int, [_vp, _c_i64, _vp, _c_i64, _c_int, _vp, _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int,
                 ctypes.POINTER(_vp)]),
    "ms_hip_nbits_weights_create_dev": (
        _c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, ctypes.POINTER(_vp)]),
    "ms_hip_nbits_weights_destroy": (_c_int, [_vp]),
    "ms_hip_nbits_weights_info": (_c_int, [_vp, _ip, _ip, _ip, _ip, _ip]),
    "ms_hip_nbits_gemm": (_c_int, [_vp, _vp, _vp, _c_int]),
    "ms_hip_nbits_gemm_dev": (_c_int, [_vp, _vp, _vp, _c_int, _vp]),
    "ms_hip_nbits_gemm_dev_noalloc": (_c_int, [_vp, _vp, _vp, _c_int, _vp]),
    "ms_hip_nbits_gemm_dev_w4a8": (_c_int, [_vp, _vp, _vp, _c_int, _vp]),
    "ms_hip_nbits_gemm_w4a8": (_c_int, [_vp, _vp, _vp, _c_int]),
    "ms_hip_qgemm_w4a8": (_c_int, [_vp, _vp, _vp, _vp, _vp] + [_c_int] * 5),
    "ms_hip_nbits_launch_info_w4a8": (_c_int, [_vp, _c_int, ctypes.POINTER(_c_int), ctypes.POINTER(_c_int)]),
    "ms_hip_rmsnorm": (_c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_int, ctypes.c_float, _vp]),
    "ms_hip_skip_rmsnorm": (_c_int, [_vp] * 8 + [_c_i64, _c_int, ctypes.c_float, _vp]),
    "ms_hip_silu_mul": (_c_int, [_vp, _vp, _vp, _c_i64, _vp]),
    "ms_hip_add": (_c_int, [_vp, _vp, _vp, _c_i64, _vp]),
    "ms_hip_sigmoid": (_c_int, [_vp, _vp, _c_i64, _vp]),
    "ms_hip_mul": (_c_int, [_vp, _vp, _vp, _c_i64, _vp]),
    "ms_hip_gqa_check": (_c_int, [_vp]),
    "ms_hip_gqa": (_c_int, [_vp] * 13 + [_c_i64, _vp]),
    "ms_hip_gqa_workspace_size": (_c_i64, [_vp]),
    "ms_hip_nbits_weights_create_from_files": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int,
                                                        ctypes.POINTER(_vp)]),
    "ms_hip_debug_force_failure": (_c_int, [_c_int]),
    "ms_hip_nbits_gemm_dev_f16": (_c_int, [_vp, _vp, _vp, _c_int, _vp]),
    "ms_hip_nbits_device_error": (_c_int, [_vp]),
    "ms_hip_nbits_gemm_dev_batch": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _vp]),
    "ms_hip_qgemm_nbits": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ms_hip_nbits_dequant": (_c_int, [_vp, _vp]),
    "ms_hip_nbits_dequant_dev": (_c_int, [_vp, _vp, _vp]),
    "ms_hip_alloc": (_c_int, [ctypes.POINTER(_vp), _c_i64]),
    "ms_hip_free": (_c_int, [_vp]),
    "ms_hip_upload": (_c_int, [_vp, _vp, _c_i64]),
    "ms_hip_download": (_c_int, [_vp, _vp, _c_i64]),
    "ms_hip_sync": (_c_int, []),
    "ms_hip_set_gemv_lanes": (_c_int, [_c_int]),
    "ms_hip_set_tuning": (_c_int, [_c_int, _c_int]),
    "ms_hip_nbits_set_tuning": (_c_int, [_vp, _c_int, _c_int]),
    "ms_hip_nbits_debug_set_counters": (_c_int, [_vp, _c_int, _c_int]),
    "ms_hip_nbits_launch_info": (_c_int, [_vp, _c_int, _ip, _ip, _ip, _ip]),
    "ms_hip_nbits_batch_launch_info": (_c_int, [_vp, _vp, _c_int, _c_int, _ip, _ip, _ip, _ip, _ip]),
    "ms_hip_nbits_gemm_dev_swiglu": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _vp]),
    "ms_hip_nbits_swiglu_launch_info": (_c_int, [_vp, _vp, _vp, _c_int, _ip, _ip, _ip]),
    "ms_hip_nbits_gemm_dev_skipnorm": (_c_int, [_vp, _c_int, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _c_int,
                                                _vp]),
    "ms_hip_nbits_gemm_dev_skipnorm_swiglu": (_c_int, [_vp, _vp, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _vp,
                                                       _c_int, _vp]),
    "ms_hip_nbits_skipnorm_launch_info": (_c_int, [_vp, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _ip, _ip,
                                                   _ip]),
}

_lock = threading.Lock()
_lib = None


class HipError(RuntimeError):
    """A nonzero status from the library, with ms_hip_last_error()'s message."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status
        self.message = message


def lib_path() -> pathlib.Path:
    env = os.environ.get("MODELSHARP_HIP_LIB")
    return pathlib.Path(env) if env else _PKG / "lib" / LIB_NAME


def load() -> ctypes.CDLL:
    """Loads the library once; raises RuntimeError when it has not been built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        # torch ships its own libamdhip64 (same soname, different file name);
        # importing it first makes this library bind to that one copy, so the
        # process never holds two HIP runtimes.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        path = lib_path()
        if not path.is_file():
            raise RuntimeError(
                f"{LIB_NAME} is not built (expected at {path}); run __graft_entry__.build() "
                "or make -C modelsharp_amd/csrc")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def header_functions() -> list[str]:
    """Names of every function the C header declares."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"\b(ms_hip_\w+)\s*\(", text)


def last_error() -> str:
    return load().ms_hip_last_error().decode("utf-8", "replace")


def check(status: int) -> None:
    if status != MS_HIP_OK:
        raise HipError(status, last_error())


def available() -> bool:
    return bool(load().ms_hip_available())


def device_name() -> str:
    return load().ms_hip_device_name().decode()


def _ptr(arr):
    return None if arr is None else arr.ctypes.data_as(_vp)


class FileSlice(ctypes.Structure):
    """ms_hip_file_slice."""
    _fields_ = [("path", ctypes.c_char_p), ("offset", ctypes.c_int64), ("length", ctypes.c_int64),
                ("dtype", ctypes.c_int)]


class NBitsWeights:
    """A device-resident MatMulNBits weight (B, scales, packed zero points).

    Created once per initializer (load-time upload) and reused by every call,
    like the per-initializer residency of IlgpuEngine.ResidentOrTempInt
    (src/ModelSharp.Gpu/IlgpuEngine.cs:3392-3429), minus its int32 widening.
    """

    def __init__(self, b: np.ndarray, scales: np.ndarray, zero_points: np.ndarray | None,
                 N: int, K: int, bits: int = 4, block_size: int = 32):
        """scales float32 or float16; zero_points packed uint8, float32 or float16, or None
        (the operator's element types, ms_hip_nbits_weights_create_ex)."""
        lib = load()
        b = np.ascontiguousarray(b, dtype=np.uint8).reshape(-1)
        scales = np.ascontiguousarray(scales)
        if scales.dtype not in (np.float32, np.float16):
            scales = scales.astype(np.float32)
        scales = scales.reshape(-1)
        zp = None
        if zero_points is not None:
            zp = np.ascontiguousarray(zero_points)
            if zp.dtype not in (np.uint8, np.float32, np.float16):
                raise ValueError(f"zero points of dtype {zp.dtype}")
            zp = zp.reshape(-1)
        handle = _vp()
        check(lib.ms_hip_nbits_weights_create_ex(
            _ptr(b), b.size, _ptr(scales), scales.size, _DTYPE_CODE[scales.dtype], _ptr(zp),
            0 if zp is None else zp.size, MS_HIP_DTYPE_NONE if zp is None else _DTYPE_CODE[zp.dtype],
            int(N), int(K), int(bits), int(block_size), ctypes.byref(handle)))
        self._init(handle, N, K, bits, block_size, zp is not None)

    @classmethod
    def from_device(cls, d_b: int, d_scales: int, d_zp: int | None, N: int, K: int, bits: int = 4,
                    block_size: int = 32) -> "NBitsWeights":
        lib = load()
        handle = _vp()
        check(lib.ms_hip_nbits_weights_create_dev(_vp(d_b), _vp(d_scales), _vp(d_zp) if d_zp else None,
                                                  N, K, bits, block_size, ctypes.byref(handle)))
        self = cls.__new__(cls)
        self._init(handle, N, K, bits, block_size, bool(d_zp))
        return self

    @classmethod
    def from_files(cls, b, scales, zero_points, N: int, K: int, bits: int = 4, block_size: int = 32):
        """Weights streamed from file slices (FileSlice-like: path, offset, length in bytes,
        data_type as the ONNX TensorProto code) straight into device memory
        (ms_hip_nbits_weights_create_from_files)."""
        onnx_to_ms = {2: MS_HIP_DTYPE_U8, 1: MS_HIP_DTYPE_F32, 10: MS_HIP_DTYPE_F16}

        def sl(x):
            if x is None:
                return None
            return FileSlice(x.path.encode(), int(x.offset), int(x.length), onnx_to_ms.get(int(x.data_type), -1))

        self = cls.__new__(cls)
        slices = [sl(b), sl(scales), sl(zero_points)]
        handle = _vp()
        check(load().ms_hip_nbits_weights_create_from_files(
            ctypes.byref(slices[0]), ctypes.byref(slices[1]), None if slices[2] is None else ctypes.byref(slices[2]),
            int(N), int(K), int(bits), int(block_size), ctypes.byref(handle)))
        self._init(handle, N, K, bits, block_size, zero_points is not None)
        return self

    def _init(self, handle, N, K, bits, block_size, has_zp):
        self.handle = handle
        self.N, self.K, self.bits, self.block_size, self.has_zp = int(N), int(K), int(bits), int(block_size), has_zp

    def gemm(self, a: np.ndarray) -> np.ndarray:
        """Host-pointer call: a[M,K] fp32 -> y[M,N] fp32 (synchronous)."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        M = a.size // self.K
        y = np.empty((M, self.N), dtype=np.float32)
        check(load().ms_hip_nbits_gemm(self.handle, _ptr(a), _ptr(y), M))
        return y

    def gemm_dev(self, dA: int, dY: int, M: int, stream: int | None = None) -> None:
        check(load().ms_hip_nbits_gemm_dev(self.handle, _vp(dA), _vp(dY), int(M), _vp(stream or 0)))

    def gemm_w4a8(self, a: np.ndarray) -> np.ndarray:
        """Host-pointer W4A8 call (the approximate opt-in product of ms_qgemm_w4a8)."""
        a = np.ascontiguousarray(a, dtype=np.float32)
        M = a.size // self.K
        y = np.empty((M, self.N), dtype=np.float32)
        check(load().ms_hip_nbits_gemm_w4a8(self.handle, _ptr(a), _ptr(y), M))
        return y

    def gemm_dev_w4a8(self, dA: int, dY: int, M: int, stream: int | None = None) -> None:
        check(load().ms_hip_nbits_gemm_dev_w4a8(self.handle, _vp(dA), _vp(dY), int(M), _vp(stream or 0)))

    def launch_info_w4a8(self, M: int) -> dict:
        k, gr = ctypes.c_int(), ctypes.c_int()
        check(load().ms_hip_nbits_launch_info_w4a8(self.handle, int(M), ctypes.byref(k), ctypes.byref(gr)))
        return {"kernel": KERNEL_NAMES[k.value], "grid": gr.value}

    def dequant(self) -> np.ndarray:
        w = np.empty((self.N, self.K), dtype=np.float32)
        check(load().ms_hip_nbits_dequant(self.handle, _ptr(w)))
        return w

    def dequant_dev(self, dW: int, stream: int | None = None) -> None:
        check(load().ms_hip_nbits_dequant_dev(self.handle, _vp(dW), _vp(stream or 0)))

    def gemm_dev_f16(self, dA16: int, dY: int, M: int, stream: int | None = None) -> None:
        """gemm_dev with fp16 activations (widened exactly on the device)."""
        check(load().ms_hip_nbits_gemm_dev_f16(self.handle, _vp(dA16), _vp(dY), int(M), _vp(stream or 0)))

    def gemm_dev_noalloc(self, dA: int, dY: int, M: int, stream: int | None = None) -> None:
        """gemm_dev with the library's fixed per-GPU scratch instead of the handle's
        workspace: allocates nothing; overlapping calls on one GPU race."""
        check(load().ms_hip_nbits_gemm_dev_noalloc(self.handle, _vp(dA), _vp(dY), int(M), _vp(stream or 0)))

    def set_tuning(self, knob: int, value: int) -> None:
        """This handle's own value of a launch-shape knob (MS_HIP_TUNING_INHERIT: follow
        the process default set by set_tuning())."""
        check(load().ms_hip_nbits_set_tuning(self.handle, int(knob), int(value)))

    def device_error(self) -> None:
        """Raises HipError when a device-side failure was recorded since the last check."""
        check(load().ms_hip_nbits_device_error(self.handle))

    def debug_set_counters(self, value: int, next_epoch_tag: bool = False) -> None:
        check(load().ms_hip_nbits_debug_set_counters(self.handle, int(value), int(bool(next_epoch_tag))))

    def launch_info(self, M: int) -> dict:
        k, g, gr, bl = (ctypes.c_int() for _ in range(4))
        check(load().ms_hip_nbits_launch_info(self.handle, int(M), ctypes.byref(k), ctypes.byref(g),
                                              ctypes.byref(gr), ctypes.byref(bl)))
        return {"kernel": KERNEL_NAMES[k.value], "lanes_per_row": g.value, "grid": gr.value, "block": bl.value}

    def close(self) -> None:
        if getattr(self, "handle", None):
            check(load().ms_hip_nbits_weights_destroy(self.handle))
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def gemm_dev_batch(weights: list, dA: list[int], dY: list[int], M: int, stream: int | None = None) -> None:
    """Enqueues len(weights) calls back to back with one library call."""
    n = len(weights)
    hs = (_vp * n)(*[w.handle for w in weights])
    pa = (_vp * n)(*dA)
    py = (_vp * n)(*dY)
    check(load().ms_hip_nbits_gemm_dev_batch(hs, pa, py, n, int(M), _vp(stream or 0)))


def batch_launch_info(weights: list, dA: list[int], M: int) -> dict:
    """The first launch a gemm_dev_batch call with these weights and activations makes:
    how many leading calls it serves, and the launch shape as NBitsWeights.launch_info."""
    n = len(weights)
    hs = (_vp * n)(*[w.handle for w in weights])
    pa = (_vp * n)(*dA)
    c, k, g, gr, bl = (ctypes.c_int() for _ in range(5))
    check(load().ms_hip_nbits_batch_launch_info(hs, pa, n, int(M), ctypes.byref(c), ctypes.byref(k), ctypes.byref(g),
                                                 ctypes.byref(gr), ctypes.byref(bl)))
    return {"calls": c.value, "kernel": KERNEL_NAMES[k.value], "lanes_per_row": g.value, "grid": gr.value,
            "block": bl.value}


def gemm_dev_swiglu(gate, up, dA: int, dH: int, M: int, stream: int | None = None) -> None:
    """H = SiLU(A W_gate^T) * (A W_up^T) on device pointers (one launch at M = 1)."""
    check(load().ms_hip_nbits_gemm_dev_swiglu(gate.handle, up.handle, _vp(dA), _vp(dH), int(M), _vp(stream or 0)))


def swiglu_launch_info(gate, up, dA: int, M: int) -> dict:
    """Whether gemm_dev_swiglu with these arguments is the single fused launch, and its shape."""
    f, g, b = (ctypes.c_int() for _ in range(3))
    check(load().ms_hip_nbits_swiglu_launch_info(gate.handle, up.handle, _vp(dA), int(M), ctypes.byref(f),
                                                  ctypes.byref(g), ctypes.byref(b)))
    return {"fused": bool(f.value), "grid": g.value, "block": b.value}


def gemm_dev_skipnorm(weights: list, dX: int, dSkip: int, dGamma: int, eps: float, dNorm: int, dSum: int | None,
                      dY: list[int], M: int, stream: int | None = None) -> None:
    """SkipSimplifiedLayerNormalization (no beta or bias) of X + Skip, then each projection of
    the normed rows: dNorm, dSum (optional) and dY[i] on device pointers (one launch at M = 1)."""
    n = len(weights)
    hs = (_vp * n)(*[w.handle for w in weights])
    py = (_vp * n)(*dY)
    check(load().ms_hip_nbits_gemm_dev_skipnorm(hs, n, _vp(dX), _vp(dSkip), _vp(dGamma), ctypes.c_float(eps),
                                                 _vp(dNorm), _vp(dSum or 0), py, int(M), _vp(stream or 0)))


def gemm_dev_skipnorm_swiglu(gate, up, dX: int, dSkip: int, dGamma: int, eps: float, dNorm: int, dSum: int | None,
                             dH: int, M: int, stream: int | None = None) -> None:
    """The same norm, then gemm_dev_swiglu on its output (one launch at M = 1)."""
    check(load().ms_hip_nbits_gemm_dev_skipnorm_swiglu(gate.handle, up.handle, _vp(dX), _vp(dSkip), _vp(dGamma),
                                                        ctypes.c_float(eps), _vp(dNorm), _vp(dSum or 0), _vp(dH),
                                                        int(M), _vp(stream or 0)))


def skipnorm_launch_info(weights: list, swiglu: bool, dX: int, dSkip: int, dGamma: int, dNorm: int,
                         dSum: int | None, M: int) -> dict:
    """Whether the fused norm call with these arguments is one launch, and its shape."""
    n = len(weights)
    hs = (_vp * n)(*[w.handle for w in weights])
    f, g, b = (ctypes.c_int() for _ in range(3))
    check(load().ms_hip_nbits_skipnorm_launch_info(hs, n, int(bool(swiglu)), _vp(dX), _vp(dSkip), _vp(dGamma),
                                                    _vp(dNorm), _vp(dSum or 0), int(M), ctypes.byref(f),
                                                    ctypes.byref(g), ctypes.byref(b)))
    return {"fused": bool(f.value), "grid": g.value, "block": b.value}


def set_gemv_lanes(lanes: int) -> None:
    check(load().ms_hip_set_gemv_lanes(int(lanes)))


def set_tuning(knob: int, value: int) -> None:
    """Launch-shape knobs for sweeps (include/ms_hip_kernels.h); 0 restores the heuristic."""
    check(load().ms_hip_set_tuning(int(knob), int(value)))


def qgemm_nbits(a, b, scales, zero_points, M, N, K, bits, block_size) -> np.ndarray:
    """One-shot call with ms_qgemm_nbits's argument meaning (uploads per call)."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp = None if zero_points is None else np.ascontiguousarray(zero_points, dtype=np.uint8)
    check(load().ms_hip_qgemm_nbits(_ptr(a), _ptr(b), _ptr(scales), _ptr(zp), _ptr(y), M, N, K, bits, block_size))
    return y


def qgemm_w4a8(a, b, scales, zero_points, M, N, K, bits, block_size) -> np.ndarray:
    """One-shot W4A8 call with ms_qgemm_w4a8's argument meaning."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    y = np.empty((M, N), dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint8)
    scales = np.ascontiguousarray(scales, dtype=np.float32)
    zp = None if zero_points is None else np.ascontiguousarray(zero_points, dtype=np.uint8)
    check(load().ms_hip_qgemm_w4a8(_ptr(a), _ptr(b), _ptr(scales), _ptr(zp), _ptr(y), M, N, K, bits, block_size))
    return y


# ---- decoder-layer neighbours (device pointers; 0 / None for an absent optional buffer) ----
class GqaDesc(ctypes.Structure):
    """ms_hip_gqa_desc."""
    _fields_ = [(n, ctypes.c_int) for n in (
        "batch", "q_seq", "kv_seq", "num_heads", "kv_num_heads", "head_dim", "packed_qkv", "past_seq",
        "past_in_present", "present_capacity", "do_rotary", "rotary_interleaved", "cos_rows", "cos_cols",
        "local_window_size")] + [("scale", ctypes.c_float), ("seqlens_len", ctypes.c_int)]


def _d(p):
    return _vp(p or 0)


def rmsnorm(dX, dScale, dY, dInvStd, rows, norm, eps, stream=None):
    check(load().ms_hip_rmsnorm(_d(dX), _d(dScale), _d(dY), _d(dInvStd), int(rows), int(norm), ctypes.c_float(eps),
                                _d(stream)))


def skip_rmsnorm(dInput, dSkip, dGamma, dBeta, dBias, dOut, dSum, dInvStd, rows, norm, eps, stream=None):
    check(load().ms_hip_skip_rmsnorm(_d(dInput), _d(dSkip), _d(dGamma), _d(dBeta), _d(dBias), _d(dOut), _d(dSum),
                                     _d(dInvStd), int(rows), int(norm), ctypes.c_float(eps), _d(stream)))


def silu_mul(dGate, dUp, dY, n, stream=None):
    check(load().ms_hip_silu_mul(_d(dGate), _d(dUp), _d(dY), int(n), _d(stream)))


def add(dA, dB, dY, n, stream=None):
    check(load().ms_hip_add(_d(dA), _d(dB), _d(dY), int(n), _d(stream)))


def sigmoid(dX, dY, n, stream=None):
    check(load().ms_hip_sigmoid(_d(dX), _d(dY), int(n), _d(stream)))


def mul(dA, dB, dY, n, stream=None):
    check(load().ms_hip_mul(_d(dA), _d(dB), _d(dY), int(n), _d(stream)))


def gqa_workspace_size(desc: GqaDesc) -> int:
    return int(load().ms_hip_gqa_workspace_size(ctypes.byref(desc)))


def gqa(desc: GqaDesc, dQ, dK, dV, dPastK, dPastV, dSeqlens, dCos, dSin, dOut, dPresentK, dPresentV,
        dWorkspace=None, workspace_bytes=0, stream=None):
    check(load().ms_hip_gqa(ctypes.byref(desc), _d(dQ), _d(dK), _d(dV), _d(dPastK), _d(dPastV), _d(dSeqlens),
                            _d(dCos), _d(dSin), _d(dOut), _d(dPresentK), _d(dPresentV), _d(dWorkspace),
                            int(workspace_bytes), _d(stream)))
