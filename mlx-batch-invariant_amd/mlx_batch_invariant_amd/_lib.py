"""ctypes binding of the gfx950 kernel library (``libbi_kernels.so``).

The library is the only compute path: there is no CPU or PyTorch fallback
inside the ``batch_invariant_*`` functions. If the library is missing on a
machine with a GPU, every call raises. Unsupported *inputs* (CPU tensors,
unsupported dtypes, masks, ...) are a separate matter handled by ``ops.py``,
which counts them as fallbacks to the stock torch op, or raises in strict mode,
as the reference does (mlx_batch_invariant/ops.py:36-39).
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch

LIB_NAME = "libbi_kernels.so"
LIB_PATH = Path(os.environ.get("BI_KERNELS_LIB", Path(__file__).resolve().parent / LIB_NAME))

BI_F32, BI_F16, BI_BF16 = 0, 1, 2
DTYPE_CODE = {torch.float32: BI_F32, torch.float16: BI_F16, torch.bfloat16: BI_BF16}
FLOAT_DTYPES = tuple(DTYPE_CODE)

ABI_VERSION = 2    # BI_ABI_VERSION of include/bi_kernels.h this binding matches
GROUP_K = 256      # fixed K group of the matmul fold (contract constant)
SPLIT_KEYS = 256   # fixed attention split size (contract constant)
DECODE_SCRATCH_BYTES = 64 << 20   # BI_DECODE_SCRATCH_BYTES: static scratch of bi_attn_decode_noalloc

_c_i64 = ctypes.c_int64
_vp = ctypes.c_void_p

# name -> (restype, argtypes); must match include/bi_kernels.h
_SIGNATURES = {
    "bi_abi_version": (ctypes.c_int, []),
    "bi_last_error": (ctypes.c_char_p, []),
    "bi_split_m_max": (ctypes.c_int, []),
    "bi_rms_norm": (ctypes.c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, ctypes.c_float, ctypes.c_int, _vp]),
    "bi_layer_norm": (ctypes.c_int, [_vp, _c_i64, _vp, _vp, _vp, _c_i64, _c_i64, ctypes.c_float, ctypes.c_int,
                                     _vp]),
    "bi_matmul_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64]),
    "bi_matmul_launch": (ctypes.c_char_p, [_c_i64, _c_i64, _c_i64]),
    "bi_matmul": (ctypes.c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int,
                                 _vp, ctypes.c_size_t, _vp]),
    "bi_matmul_batched": (ctypes.c_int, [_vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _vp, _c_i64, _c_i64, _c_i64,
                                         _c_i64, _c_i64, ctypes.c_int, _vp, ctypes.c_size_t, _vp]),
    "bi_quantized_matmul_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64]),
    "bi_quantized_matmul": (ctypes.c_int, [_vp, _c_i64, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                           ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t, _vp]),
    "bi_attn_decode_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64, _c_i64]),
    "bi_attn_decode": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                      ctypes.POINTER(_c_i64), ctypes.c_float, ctypes.c_int, _vp,
                                      ctypes.c_size_t, _vp]),
    "bi_attn_prefill": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                       _c_i64, ctypes.POINTER(_c_i64), ctypes.c_int, ctypes.c_float,
                                       ctypes.c_int, _vp]),
    "bi_attn_decode_per_key_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64, _c_i64, _c_i64]),
    "bi_attn_decode_per_key": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                              ctypes.POINTER(_c_i64), ctypes.c_float, _c_i64, ctypes.c_int, _vp,
                                              ctypes.c_size_t, _vp]),
    "bi_attn_prefill_per_key": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                               _c_i64, ctypes.POINTER(_c_i64), ctypes.c_int, ctypes.c_float,
                                               _c_i64, ctypes.c_int, _vp]),
    "bi_attn_decode_noalloc": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64,
                                              ctypes.POINTER(_c_i64), ctypes.c_float, ctypes.c_int, _vp]),
    "bi_attn_decode_paged": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i64,
                                            _c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.c_float,
                                            ctypes.c_int, _vp, ctypes.c_size_t, _vp]),
    "bi_attn_prefill_paged": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64, _vp, _vp, _c_i64, _c_i64,
                                             _c_i64, _c_i64, _c_i64, _c_i64, ctypes.POINTER(_c_i64), ctypes.c_int,
                                             ctypes.c_float, ctypes.c_int, _vp]),
    "bi_exp2_f32": (ctypes.c_int, [_vp, _vp, _c_i64, _vp]),
    "bi_stream_read": (ctypes.c_int, [_vp, _c_i64, _vp, ctypes.c_uint32, _vp]),
    "bi_quantized_dequantize": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_i64, _c_i64, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_int, _vp]),
    "bi_quantized_matmul_dequantized_workspace_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, _c_i64]),
    "bi_quantized_matmul_dequantized": (ctypes.c_int, [_vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int,
                                                       _vp, ctypes.c_size_t, _vp]),
    "bi_matmul_pack_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, ctypes.c_int]),
    "bi_matmul_pack": (ctypes.c_int, [_vp, _c_i64, _vp, ctypes.c_size_t, _c_i64, _c_i64, ctypes.c_int, _vp]),
    "bi_matmul_packed": (ctypes.c_int, [_vp, _c_i64, _vp, _c_i64, _vp, _vp, _c_i64, _c_i64, _c_i64, ctypes.c_int,
                                        _vp, ctypes.c_size_t, _vp]),
    "bi_quantized_pack_bytes": (ctypes.c_size_t, [_c_i64, _c_i64, ctypes.c_int, ctypes.c_int]),
    "bi_quantized_pack": (ctypes.c_int, [_vp, _vp, _vp, _vp, ctypes.c_size_t, _c_i64, _c_i64, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, _vp]),
    "bi_quantized_matmul_packed": (ctypes.c_int, [_vp, _c_i64, _vp, _vp, _vp, _vp, _vp, _c_i64, _c_i64, _c_i64,
                                                  ctypes.c_int, ctypes.c_int, ctypes.c_int, _vp, ctypes.c_size_t,
                                                  _vp]),
    "bi_mfma_step_probe": (ctypes.c_int, [_vp, _vp, _vp, _vp, _c_i64, ctypes.c_int, _vp]),
}

_lib = None
_lock = threading.Lock()


class KernelLibraryError(RuntimeError):
    """The kernel library is missing, stale, or a call into it failed."""


def load() -> ctypes.CDLL:
    """Load the library once (after torch, so the HIP runtime is shared)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise KernelLibraryError(
                f"{LIB_PATH} not found: build it with `python mlx-batch-invariant_amd/csrc/build.py` "
                "(or __graft_entry__.build())")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.bi_abi_version() != ABI_VERSION:
            raise KernelLibraryError(f"{LIB_PATH}: ABI version {lib.bi_abi_version()} != {ABI_VERSION}")
        _bind_fast(lib)
        _lib = lib
        return lib


# The three most frequently called entry points go through the CPython binding
# _bi_pycall when it is built (csrc/bi_pycall.c: the same C functions, about
# 3 us less host time per call than ctypes' argument conversion), else
# through ctypes. Same arguments either way; each returns the ABI status code.
qmm_call = None
matmul_call = None
rms_norm_call = None


def _bind_fast(lib) -> None:
    global qmm_call, matmul_call, rms_norm_call
    qmm_call, matmul_call, rms_norm_call = lib.bi_quantized_matmul, lib.bi_matmul, lib.bi_rms_norm
    try:
        from . import _bi_pycall
    except ImportError:
        return
    addr = [ctypes.cast(getattr(lib, n), ctypes.c_void_p).value
            for n in ("bi_quantized_matmul", "bi_matmul", "bi_rms_norm")]
    _bi_pycall.bind(*addr)
    qmm_call, matmul_call, rms_norm_call = _bi_pycall.quantized_matmul, _bi_pycall.matmul, _bi_pycall.rms_norm


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def gpu_available() -> bool:
    return torch.cuda.is_available()


def is_gpu_tensor(t) -> bool:
    return isinstance(t, torch.Tensor) and t.is_cuda


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().bi_last_error().decode(errors="replace")
        kind = {-1: ValueError, -2: NotImplementedError, -3: ValueError}.get(rc, KernelLibraryError)
        raise kind(f"{what} failed (code {rc}): {msg}")


# The current stream of a device as a raw hipStream_t, without building a
# torch.cuda.Stream object per call (a few microseconds of host time on every
# eager launch); the public API is the fallback.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    if _raw_stream is not None:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


_ws_cache: dict = {}


def ws_bytes(query: str, *shape) -> int:
    """A `bi_*_workspace_bytes` answer, remembered per (query, shape): the
    sizes are pure functions of the shape, and a dict lookup is cheaper than
    the foreign call on every eager launch."""
    key = (query,) + shape
    n = _ws_cache.get(key)
    if n is None:
        if len(_ws_cache) > 4096:
            _ws_cache.clear()
        n = _ws_cache[key] = int(getattr(load(), query)(*shape))
    return n


def workspace(nbytes: int, device) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def require_gpu(what: str, *tensors) -> None:
    for t in tensors:
        if t is not None and not is_gpu_tensor(t):
            raise ValueError(f"{what}: the batch-invariant kernels run on the GPU; got a tensor on {t.device}")
    load()
