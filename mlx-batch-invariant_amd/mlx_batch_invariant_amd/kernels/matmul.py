"""Batch-invariant matmul: C[M, N] = A[M, K] @ B[K, N] on gfx950.

Canonical reduction order (reference: mlx_batch_invariant/kernels/matmul.py:1-38):

* K is cut into fixed groups of ``GROUP_K`` = 256; group ``g`` covers
  ``k in [256 g, 256 g + 256)`` whatever M, N or the launch shape.
* Inside a group, eight ``v_mfma_f32_16x16x32`` steps (operands in the input
  dtype, fp32 accumulator starting from exact zero) walk the group with the
  fixed k-slot map ``k = 256 g + 64 q + 8 s + e`` (lane quarter q, step s,
  element e). fp32 inputs use a chain of ``v_mfma_f32_16x16x4_f32``.
* The output is the left fold ``((0 + p_0) + p_1) + ...`` of group partials
  as plain fp32 adds, rounded once to the output dtype.

Launch shapes that only change who computes an element: M <= ``SPLIT_M_MAX``
with more than one group writes fp32 group partials and folds them in a
second kernel; larger M folds in registers. The choice never changes bits.

B is consumed transposed (``bt[n, k]``, k contiguous), which is how
``nn.Linear`` stores its weight, so ``x @ W.T`` needs no copy. Other layouts
and odd K are copied / zero-padded first; neither changes the arithmetic.
"""

from __future__ import annotations

import weakref

import torch

from .. import _lib

GROUP_K = _lib.GROUP_K
SPLIT_M_MAX = 32


def _kcontig(t: torch.Tensor) -> bool:
    """Rows k-contiguous with 16-byte aligned row starts (what the kernel reads)."""
    es = t.element_size()
    return (t.stride(-1) == 1 and (t.stride(0) * es) % 16 == 0 and t.data_ptr() % 16 == 0
            and t.stride(0) >= t.shape[-1])


def _prep_rows(t: torch.Tensor, K8: int) -> torch.Tensor:
    """[R, K] -> [R, K8] k-contiguous, 16-byte aligned rows, zero-padded to K8."""
    K = t.shape[1]
    if K8 == K and _kcontig(t):
        return t
    out = torch.zeros((t.shape[0], K8), dtype=t.dtype, device=t.device)
    out[:, :K] = t
    return out


def matmul_bt(a2: torch.Tensor, bt: torch.Tensor) -> torch.Tensor:
    """out[M, N] = a2[M, K] @ bt[N, K].T, both already the output dtype, on the GPU."""
    M, K = a2.shape
    N = bt.shape[0]
    out = torch.empty((M, N), dtype=a2.dtype, device=a2.device)
    if M == 0:
        return out
    if N == 0 or K == 0:
        return out.zero_()
    K8 = (K + 7) // 8 * 8
    a2 = _prep_rows(a2, K8)
    bt = _prep_rows(bt, K8)
    _lib.load()
    ws_bytes = _lib.ws_bytes("bi_matmul_workspace_bytes", M, N, K8)
    ws = _lib.workspace(ws_bytes, a2.device)
    bp = _packed_for(bt) if M <= PACKED_MAX_M and _PACKED else None
    if bp is not None:
        rc = _lib.load().bi_matmul_packed(a2.data_ptr(), a2.stride(0), bt.data_ptr(), bt.stride(0), bp.data_ptr(),
                                          out.data_ptr(), M, N, K8, _lib.DTYPE_CODE[a2.dtype], _lib.ptr(ws),
                                          ws_bytes, _lib.stream_of(a2))
        _lib.check(rc, "bi_matmul_packed")
        return out
    rc = _lib.matmul_call(a2.data_ptr(), a2.stride(0), bt.data_ptr(), bt.stride(0), out.data_ptr(),
                          M, N, K8, _lib.DTYPE_CODE[a2.dtype], _lib.ptr(ws), ws_bytes,
                          _lib.stream_of(a2))
    _lib.check(rc, "bi_matmul")
    return out


# ---- weights repacked once (decode calls) -------------------------------------

# Rows up to which a repacked copy is used (the streaming GEMV's range;
# bi_matmul_packed reads the row-major weight for the shapes it does not take).
PACKED_MAX_M = 16
# weight data pointer -> (weakref to the weight, N, K, row stride, dtype,
# version counter at packing, the copy). The weight's views (W.T, as F.linear
# and x @ W.T pass it) share its storage and version counter, so any of them
# finds the copy, and an in-place change of the weight makes it stale.
_PACKED: dict = {}


def _packed_for(bt: torch.Tensor):
    e = _PACKED.get(bt.data_ptr())
    if e is None:
        return None
    w = e[0]()
    if w is None or w.data_ptr() != bt.data_ptr():
        _PACKED.pop(bt.data_ptr(), None)
        return None
    if (e[1], e[2], e[3], e[4], e[5]) != (bt.shape[0], bt.shape[1], bt.stride(0), bt.dtype, bt._version):
        return None
    return e[6]


def cache_packed_weight(weight: torch.Tensor) -> torch.Tensor:
    """Keep a copy of a dense weight ``[N, K]`` (the ``nn.Linear`` layout; bf16 or
    fp16, K a multiple of 8, k-contiguous 16-byte aligned rows) repacked once
    for the decode GEMV (``bi_matmul_pack``) for as long as the weight lives.
    Calls of ``batch_invariant_matmul(x, weight.T)`` (and ``F.linear`` under the
    mode) with at most ``PACKED_MAX_M`` rows then run ``bi_matmul_packed``: the
    same bits, with each wave instruction reading a whole 1 KB run. The copy
    holds N * K * 2 bytes, K rounded up to a multiple of 256 (zero-filled). An in-place change of the weight (its version
    counter) makes the copy unused until ``cache_packed_weight`` is called
    again; ``drop_packed_weight`` releases it."""
    if weight.ndim != 2 or weight.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("cache_packed_weight: a 2-D bf16 / fp16 weight [N, K]")
    _lib.require_gpu("cache_packed_weight", weight)
    N, K = weight.shape
    if K % 8 or not _kcontig(weight):
        raise ValueError("cache_packed_weight: K must be a multiple of 8 and rows k-contiguous, 16-byte aligned")
    lib = _lib.load()
    code = _lib.DTYPE_CODE[weight.dtype]
    nbytes = lib.bi_matmul_pack_bytes(N, K, code)
    bp = torch.empty((nbytes,), dtype=torch.uint8, device=weight.device)
    rc = lib.bi_matmul_pack(weight.data_ptr(), weight.stride(0), bp.data_ptr(), nbytes, N, K, code,
                            _lib.stream_of(weight))
    _lib.check(rc, "bi_matmul_pack")
    _PACKED[weight.data_ptr()] = (weakref.ref(weight), N, K, weight.stride(0), weight.dtype, weight._version, bp)
    return bp


def drop_packed_weight(weight: torch.Tensor) -> None:
    """Release the repacked copy ``cache_packed_weight`` keeps for ``weight``."""
    e = _PACKED.get(weight.data_ptr())
    if e is not None and e[0]() is weight:
        del _PACKED[weight.data_ptr()]


def batch_invariant_matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b`` for 2-D ``b`` with a batch-invariant reduction order.

    ``a`` may have leading dims; they are flattened into M. ``b`` must be 2-D
    (a transposed view such as ``W.T`` is consumed in place). Accumulation is
    fp32; the output dtype is the promoted input dtype
    (reference: kernels/matmul.py:317-340).
    """
    if b.ndim != 2:
        raise ValueError("batch_invariant_matmul: b must be 2-D")
    if a.ndim < 1:
        raise ValueError("batch_invariant_matmul: a must have at least one dim")
    K = a.shape[-1]
    if K != b.shape[0]:
        raise ValueError(f"shape mismatch {tuple(a.shape)} @ {tuple(b.shape)}")
    out_dtype = a.dtype if a.dtype == b.dtype else torch.result_type(a, b)
    if out_dtype not in _lib.FLOAT_DTYPES:
        raise ValueError(f"batch_invariant_matmul: unsupported dtype {out_dtype}")
    _lib.require_gpu("batch_invariant_matmul", a, b)
    lead = a.shape[:-1]
    N = b.shape[1]
    flat = a.ndim == 2                         # no reshape round trip for the common 2-D call
    a2 = a if flat else a.reshape(-1, K)
    if a2.dtype != out_dtype:
        a2 = a2.to(out_dtype)
    if b.dtype != out_dtype:
        b = b.to(out_dtype)
    out = matmul_bt(a2, b.t())
    return out if flat else out.reshape(*lead, N)


def _prep_batched(t: torch.Tensor, K8: int) -> torch.Tensor:
    """[Bt, R, K] -> rows k-contiguous, 16-byte aligned, padded to K8, with one
    batch stride (0 kept for a broadcast operand)."""
    Bt, R, K = t.shape
    es = t.element_size()
    ok = (K8 == K and t.stride(2) == 1 and t.stride(1) >= K and (t.stride(1) * es) % 16 == 0
          and (t.stride(0) * es) % 16 == 0 and t.data_ptr() % 16 == 0)
    if ok:
        return t
    out = torch.zeros((Bt, R, K8), dtype=t.dtype, device=t.device)
    out[:, :, :K] = t
    return out


def batch_invariant_bmm(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b`` for ``a [..., M, K]`` and ``b [..., K, N]`` with broadcast batch
    dims (``torch.matmul`` semantics for operands of 2 or more dims).

    Every batch slice is computed exactly as the 2-D ``batch_invariant_matmul``
    of that slice, so its bits depend neither on M nor on the batch. The
    reference falls back for a non-2-D right-hand side (ops.py:46-51); its
    roadmap lists the batched matmul (README.md:257-268).
    """
    if a.ndim < 2 or b.ndim < 2:
        raise ValueError("batch_invariant_bmm: operands need 2 or more dims")
    M, K = a.shape[-2:]
    N = b.shape[-1]
    if K != b.shape[-2]:
        raise ValueError(f"shape mismatch {tuple(a.shape)} @ {tuple(b.shape)}")
    out_dtype = a.dtype if a.dtype == b.dtype else torch.result_type(a, b)
    if out_dtype not in _lib.FLOAT_DTYPES:
        raise ValueError(f"batch_invariant_bmm: unsupported dtype {out_dtype}")
    _lib.require_gpu("batch_invariant_bmm", a, b)
    batch = torch.broadcast_shapes(a.shape[:-2], b.shape[:-2])
    Bt = 1
    for d in batch:
        Bt *= d
    out = torch.empty((*batch, M, N), dtype=out_dtype, device=a.device)
    if Bt == 0 or M == 0:
        return out
    if N == 0 or K == 0:
        return out.zero_()
    a3 = a.to(out_dtype).expand(*batch, M, K).reshape(Bt, M, K)
    bt3 = b.to(out_dtype).expand(*batch, K, N).reshape(Bt, K, N).transpose(1, 2)
    K8 = (K + 7) // 8 * 8
    a3 = _prep_batched(a3, K8)
    bt3 = _prep_batched(bt3, K8)
    lib = _lib.load()
    ws_bytes = _lib.ws_bytes("bi_matmul_workspace_bytes", M, N, K8)
    ws = _lib.workspace(ws_bytes, a.device)
    o3 = out.view(Bt, M, N)
    rc = lib.bi_matmul_batched(a3.data_ptr(), a3.stride(0), a3.stride(1), bt3.data_ptr(), bt3.stride(0),
                               bt3.stride(1), o3.data_ptr(), M * N, Bt, M, N, K8, _lib.DTYPE_CODE[out_dtype],
                               _lib.ptr(ws), ws_bytes, _lib.stream_of(a3))
    _lib.check(rc, "bi_matmul_batched")
    return out
