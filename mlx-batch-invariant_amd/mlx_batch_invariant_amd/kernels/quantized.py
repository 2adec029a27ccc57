"""Batch-invariant affine quantized matmul: y[M, N] = x[M, K] @ W[N, K].T

``W`` is MLX's packed affine format (reference:
mlx_batch_invariant/kernels/quantized.py:1-22): ``bits``-wide unsigned codes
packed low-to-high inside uint32 words (``32 // bits`` codes per word), one
``scale`` and ``bias`` per ``group_size`` consecutive codes of a row:

    w[n, k] = code(n, k) * scales[n, k // group_size] + biases[n, k // group_size]

The kernel runs the dense matmul's tile body (same 256-wide K groups, same
k-slot map, same MFMA, same fold, same launch shapes) and dequantizes the B
operand as it is fetched: ``T(fmaf(float(code), float(scale), float(bias)))``,
one round-to-nearest-even into the input dtype, exact zero past K. Each lane
unpacks whole 16-byte runs of words of its own 64-k block, which is also one
scale/bias group for group size 64.

The packed weight is a ``torch.uint32`` (or bit-identical ``torch.int32``)
tensor ``[N, K * bits / 32]``; scales and biases are ``[N, K / group_size]``
and are cast to the input dtype, as in the reference (quantized.py:116-119).
"""

from __future__ import annotations

import weakref

import torch

from .. import _lib
from .matmul import _prep_rows

SUPPORTED_BITS = (4, 8)
SUPPORTED_GROUPS = (32, 64, 128)
_WORD_DTYPES = (torch.uint32, torch.int32)


def supports(x, w, scales, biases, transpose, group_size, bits, mode) -> bool:
    """Reference predicate kernels/quantized.py:91-103, on torch tensors on the GPU."""
    try:
        return bool(
            mode == "affine"
            and transpose
            and biases is not None
            and bits in SUPPORTED_BITS
            and group_size in SUPPORTED_GROUPS
            and isinstance(x, torch.Tensor) and x.dtype in _lib.FLOAT_DTYPES
            and isinstance(w, torch.Tensor) and w.dtype in _WORD_DTYPES and w.ndim == 2
            and scales.ndim == 2 and biases.ndim == 2
            and x.shape[-1] % group_size == 0
            and w.shape[1] * (32 // bits) == x.shape[-1]
            and tuple(scales.shape) == (w.shape[0], x.shape[-1] // group_size)
            and tuple(biases.shape) == tuple(scales.shape)
            and all(_lib.is_gpu_tensor(t) for t in (x, w, scales, biases))
        )
    except (AttributeError, TypeError):
        return False


def batch_invariant_quantized_matmul(x: torch.Tensor, w: torch.Tensor, scales: torch.Tensor,
                                     biases: torch.Tensor, *, group_size: int, bits: int) -> torch.Tensor:
    if bits not in SUPPORTED_BITS or group_size not in SUPPORTED_GROUPS:
        raise ValueError(f"batch_invariant_quantized_matmul: bits={bits} group_size={group_size}")
    if x.dtype not in _lib.FLOAT_DTYPES:
        raise ValueError(f"batch_invariant_quantized_matmul: unsupported dtype {x.dtype}")
    if w.dtype not in _WORD_DTYPES or w.ndim != 2:
        raise ValueError("batch_invariant_quantized_matmul: w must be a 2-D uint32 tensor")
    _lib.require_gpu("batch_invariant_quantized_matmul", x, w, scales, biases)
    lead = x.shape[:-1]
    K = x.shape[-1]
    N = w.shape[0]
    if K % group_size or w.shape[1] * (32 // bits) != K:
        raise ValueError(f"shape mismatch: x {tuple(x.shape)}, w {tuple(w.shape)} at {bits} bits")
    dt = x.dtype
    if scales.dtype != dt or not scales.is_contiguous():
        scales = scales.to(dt).contiguous()
    if biases.dtype != dt or not biases.is_contiguous():
        biases = biases.to(dt).contiguous()
    if tuple(scales.shape) != (N, K // group_size) or scales.shape != biases.shape:
        raise ValueError("batch_invariant_quantized_matmul: scales/biases must be [N, K / group_size]")
    if not w.is_contiguous():
        w = w.contiguous()
    flat = x.ndim == 2                         # no reshape round trip for the common 2-D call
    x2 = _prep_rows(x if flat else x.reshape(-1, K), K)
    M = x2.shape[0]
    out = torch.empty((M, N), dtype=dt, device=x.device)
    bq = _dequantized_for(w, scales, biases, group_size, bits, dt) if M >= DEQUANTIZED_MIN_M else None
    bp = _cached_for(_PACKED, w, scales, biases, group_size, bits, dt) if 0 < M <= PACKED_MAX_M else None
    if bp is not None:
        lib = _lib.load()
        ws_bytes = _lib.ws_bytes("bi_quantized_matmul_workspace_bytes", M, N, K)
        ws = _lib.workspace(ws_bytes, x.device)
        rc = lib.bi_quantized_matmul_packed(x2.data_ptr(), x2.stride(0), w.data_ptr(), scales.data_ptr(),
                                            biases.data_ptr(), bp.data_ptr(), out.data_ptr(), M, N, K, bits,
                                            group_size, _lib.DTYPE_CODE[dt], _lib.ptr(ws), ws_bytes,
                                            _lib.stream_of(x))
        _lib.check(rc, "bi_quantized_matmul_packed")
    elif bq is not None:
        _lib.load()
        ws_bytes = _lib.ws_bytes("bi_quantized_matmul_dequantized_workspace_bytes", M, N, K)
        ws = _lib.workspace(ws_bytes, x.device)
        rc = _lib.load().bi_quantized_matmul_dequantized(x2.data_ptr(), x2.stride(0), bq.data_ptr(), out.data_ptr(),
                                                         M, N, K, _lib.DTYPE_CODE[dt], _lib.ptr(ws), ws_bytes,
                                                         _lib.stream_of(x))
        _lib.check(rc, "bi_quantized_matmul_dequantized")
    elif M > 0:
        _lib.load()
        ws_bytes = _lib.ws_bytes("bi_quantized_matmul_workspace_bytes", M, N, K)
        ws = _lib.workspace(ws_bytes, x.device)
        rc = _lib.qmm_call(x2.data_ptr(), x2.stride(0), w.data_ptr(), scales.data_ptr(),
                                     biases.data_ptr(), out.data_ptr(), M, N, K, bits, group_size,
                                     _lib.DTYPE_CODE[dt], _lib.ptr(ws), ws_bytes, _lib.stream_of(x))
        _lib.check(rc, "bi_quantized_matmul")
    return out if flat else out.reshape(*lead, N)


# ---- weights dequantized once (large-M calls) ----------------------------------

# Rows of x from which a cached dequantized weight is used: the large-M launch
# of bi_quantized_matmul dequantizes its weight on every call from here on.
DEQUANTIZED_MIN_M = 256
# id(w) -> (weakref to w, w's / scales' / biases' data pointers, group size, bits,
# dtype, the copy); an entry goes when w is collected (tensors compare
# elementwise, so they cannot key a WeakKeyDictionary).
_DEQUANTIZED: dict = {}


def cache_dequantized(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, group_size: int,
                      bits: int) -> torch.Tensor:
    """Keep a dequantized copy of the packed weight ``w`` (``bi_quantized_dequantize``:
    ``[N, K]`` in scales' dtype, bf16 or fp16, its chunks in the dense kernels'
    k order) for as long as ``w`` lives. Calls of
    ``batch_invariant_quantized_matmul`` with at least ``DEQUANTIZED_MIN_M`` rows,
    this ``w`` (the same tensor object) and these scales / biases then run
    ``bi_quantized_matmul_dequantized`` on it: the same bits, without the
    per-call dequantization. The copy holds N * K * 2 bytes (the size of the
    weight dequantized once, as a stock serving path keeps it). Call again after
    changing the weight's values in place; ``drop_dequantized`` releases it."""
    if bits not in SUPPORTED_BITS or group_size not in SUPPORTED_GROUPS:
        raise ValueError(f"cache_dequantized: bits={bits} group_size={group_size}")
    dt = scales.dtype
    if dt not in (torch.bfloat16, torch.float16):
        raise ValueError(f"cache_dequantized: scales dtype {dt} (bf16 or fp16)")
    if w.dtype not in _WORD_DTYPES or w.ndim != 2 or not w.is_contiguous():
        raise ValueError("cache_dequantized: w must be a contiguous 2-D uint32 tensor")
    _lib.require_gpu("cache_dequantized", w, scales, biases)
    N, K = w.shape[0], w.shape[1] * (32 // bits)
    if K % 256:
        raise ValueError(f"cache_dequantized: K={K} must be a multiple of 256")
    if tuple(scales.shape) != (N, K // group_size) or scales.shape != biases.shape or biases.dtype != dt \
            or not scales.is_contiguous() or not biases.is_contiguous():
        raise ValueError("cache_dequantized: scales/biases must be contiguous [N, K / group_size] of one dtype")
    bq = torch.empty((N, K), dtype=dt, device=w.device)
    rc = _lib.load().bi_quantized_dequantize(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), bq.data_ptr(), N, K,
                                             bits, group_size, _lib.DTYPE_CODE[dt], _lib.stream_of(w))
    _lib.check(rc, "bi_quantized_dequantize")
    _remember(_DEQUANTIZED, w, scales, biases, group_size, bits, dt, bq)
    return bq


def drop_dequantized(w: torch.Tensor) -> None:
    """Release the dequantized copy ``cache_dequantized`` keeps for ``w``."""
    e = _DEQUANTIZED.get(id(w))
    if e is not None and e[0]() is w:
        del _DEQUANTIZED[id(w)]


def _cached_for(cache, w, scales, biases, group_size, bits, dt):
    """The copy ``cache`` keeps for exactly this call (same tensor and storage,
    same scales / biases, format and dtype), else None."""
    e = cache.get(id(w)) if cache else None
    if e is None or e[0]() is not w:
        return None
    if (e[1], e[2], e[3], e[4], e[5], e[6]) != (w.data_ptr(), scales.data_ptr(), biases.data_ptr(), group_size,
                                                bits, dt):
        return None
    return e[7]


def _dequantized_for(w, scales, biases, group_size, bits, dt):
    return _cached_for(_DEQUANTIZED, w, scales, biases, group_size, bits, dt)


def _remember(cache, w, scales, biases, group_size, bits, dt, copy) -> None:
    key = id(w)
    ref = weakref.ref(w, lambda _r, k=key: cache.pop(k, None) if cache.get(k, (None,))[0] is _r else None)
    cache[key] = (ref, w.data_ptr(), scales.data_ptr(), biases.data_ptr(), group_size, bits, dt, copy)


# ---- weights repacked once (decode calls) -------------------------------------

# Rows of x up to which a repacked copy is used (the streaming GEMV's and the
# mid-M launches' range, below the large-M launch, which dequantizes B once per
# call; bi_quantized_matmul_packed reads the MLX layout for the shapes those
# do not take).
PACKED_MAX_M = DEQUANTIZED_MIN_M - 1
# id(w) -> the same record as _DEQUANTIZED's, holding the repacked copy.
_PACKED: dict = {}


def cache_packed(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, *, group_size: int,
                 bits: int) -> torch.Tensor:
    """Keep a repacked copy of the packed weight ``w`` (``bi_quantized_pack``:
    the same codes, scales and biases in the layout the decode GEMV reads, as
    uint8 ``bi_quantized_pack_bytes`` bytes) for as long as ``w`` lives. Calls
    of ``batch_invariant_quantized_matmul`` with at most ``PACKED_MAX_M`` rows,
    this ``w`` (the same tensor object) and these scales / biases then run
    ``bi_quantized_matmul_packed``: the same bits, with each wave instruction of
    the decode GEMV reading a whole 1 KB run of codes; the mid-M launches read
    it too. 4 or 8 bits, group size 32 / 64 / 128, bf16 / fp16 scales, K a
    multiple of 256. The copy holds the codes, scales and biases again (each
    byte once, in another order). Call again after changing the weight's
    values in place; ``drop_packed`` releases it."""
    if bits not in SUPPORTED_BITS or group_size not in SUPPORTED_GROUPS:
        raise ValueError(f"cache_packed: bits={bits} group_size={group_size}")
    dt = scales.dtype
    if dt not in (torch.bfloat16, torch.float16):
        raise ValueError(f"cache_packed: scales dtype {dt} (bf16 or fp16)")
    if w.dtype not in _WORD_DTYPES or w.ndim != 2 or not w.is_contiguous():
        raise ValueError("cache_packed: w must be a contiguous 2-D uint32 tensor")
    _lib.require_gpu("cache_packed", w, scales, biases)
    N, K = w.shape[0], w.shape[1] * (32 // bits)
    if K % 256:
        raise ValueError(f"cache_packed: K={K} must be a multiple of 256")
    if tuple(scales.shape) != (N, K // group_size) or scales.shape != biases.shape or biases.dtype != dt \
            or not scales.is_contiguous() or not biases.is_contiguous():
        raise ValueError("cache_packed: scales/biases must be contiguous [N, K / group_size] of one dtype")
    lib = _lib.load()
    nbytes = lib.bi_quantized_pack_bytes(N, K, bits, group_size)
    bp = torch.empty((nbytes,), dtype=torch.uint8, device=w.device)
    rc = lib.bi_quantized_pack(w.data_ptr(), scales.data_ptr(), biases.data_ptr(), bp.data_ptr(), nbytes, N, K, bits,
                               group_size, _lib.DTYPE_CODE[dt], _lib.stream_of(w))
    _lib.check(rc, "bi_quantized_pack")
    _remember(_PACKED, w, scales, biases, group_size, bits, dt, bp)
    return bp


def drop_packed(w: torch.Tensor) -> None:
    """Release the repacked copy ``cache_packed`` keeps for ``w``."""
    e = _PACKED.get(id(w))
    if e is not None and e[0]() is w:
        del _PACKED[id(w)]


# ---- format helpers (host-side torch; not on the kernel path) -----------------

def quantize(W: torch.Tensor, group_size: int = 64, bits: int = 4, dtype: torch.dtype | None = None):
    """Min/max affine quantizer into the MLX packed layout.

    Per group: ``scale = (max - min) / (2^bits - 1)`` (1 if the group is
    constant), ``bias = min``, ``code = clamp(round((w - bias) / scale))``.
    Returns ``(w_packed uint32 [N, K*bits/32], scales, biases)`` with scales and
    biases in ``dtype`` (default: W's dtype). This is this library's own
    quantizer; the kernel contract depends only on the packed format.
    """
    if bits not in SUPPORTED_BITS or group_size not in SUPPORTED_GROUPS:
        raise ValueError(f"quantize: bits={bits} group_size={group_size}")
    N, K = W.shape
    if K % group_size:
        raise ValueError(f"quantize: K={K} not a multiple of group_size={group_size}")
    dtype = dtype or (W.dtype if W.dtype in _lib.FLOAT_DTYPES else torch.float32)
    Wg = W.detach().to(torch.float32).reshape(N, K // group_size, group_size)
    wmin = Wg.amin(-1)
    wmax = Wg.amax(-1)
    nlev = (1 << bits) - 1
    scale = (wmax - wmin) / nlev
    scale = torch.where(scale > 0, scale, torch.ones_like(scale))
    s_q = scale.to(dtype)
    b_q = wmin.to(dtype)
    codes = torch.round((Wg - b_q.float()[..., None]) / s_q.float()[..., None]).clamp_(0, nlev)
    w_packed = pack(codes.to(torch.int64).reshape(N, K), bits)
    return w_packed, s_q, b_q


def pack(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """[N, K] integer codes -> uint32 [N, K*bits/32], low-to-high within a word."""
    per = 32 // bits
    N, K = codes.shape
    c = codes.to(torch.int64).reshape(N, K // per, per)
    shifts = torch.arange(per, device=codes.device, dtype=torch.int64) * bits
    words = (c << shifts).sum(-1)                       # < 2^32, exact in int64
    words = torch.where(words >= 2**31, words - 2**32, words).to(torch.int32)
    return words.view(torch.uint32)


def unpack(w: torch.Tensor, bits: int) -> torch.Tensor:
    """uint32 [N, W] -> int64 codes [N, W * 32/bits]."""
    per = 32 // bits
    words = w.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(per, device=w.device, dtype=torch.int64) * bits
    codes = (words[..., None] >> shifts) & ((1 << bits) - 1)
    return codes.reshape(w.shape[0], -1)


def dequantize(w: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor, group_size: int,
               bits: int, dtype: torch.dtype | None = None) -> torch.Tensor:
    """W[n, k] = T(code * scale + bias) with one rounding to fp32 then to T.

    Used by the stock fallback (dequantize + torch matmul); it is not
    batch-invariant itself and not part of the kernel path.
    """
    dtype = dtype or scales.dtype
    codes = unpack(w, bits).to(torch.float64)
    N, K = codes.shape
    s = scales.to(torch.float64).repeat_interleave(group_size, dim=1)
    b = biases.to(torch.float64).repeat_interleave(group_size, dim=1)
    return (codes * s + b).to(torch.float32).to(dtype)
