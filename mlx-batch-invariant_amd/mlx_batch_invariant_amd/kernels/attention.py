"""Batch-invariant split-KV attention on gfx950.

Canonical order per (sequence, head, query) (reference:
mlx_batch_invariant/kernels/attention.py:1-32):

* keys are processed in fixed splits of ``SPLIT_SIZE`` = 256 in index order;
  key ``j`` always lands in split ``j // 256`` at the same position;
* the score is ``fp32(dot(k_j, q) * scale * log2(e))`` with the dot taken by a
  fixed chain of ``v_mfma_f32_16x16x32`` steps over the head dimension;
* inside a split: the maximum ``m`` of the active scores, the weights
  ``p = exp2(s - m)`` (exactly 0 for masked keys), and ``acc = P.V``,
  ``l = P.1`` as fixed MFMA chains over the split's 32-key steps (for 16-bit
  types ``P`` enters as a high and a low part, 16 / 22 significant bits);
* splits are merged left to right with ``c_old = exp2(M - M'); c_new = exp2(m - M');
  L = fma(L, c_old, l * c_new); A = fma(A, c_old, acc * c_new)``, and the
  output is ``T(A / L)``.

The reference runs the softmax key by key inside a split; this is the same
quantity in an order whose products all run on the matrix cores (the
reference's own matrix-unit variant, kernels/attention_mma.py, also
reorders). Values agree with the reference order to fp32 rounding.

Decode (T_q == 1) writes per-split partials and folds them in a combine
kernel; prefill folds in registers. Both kernels run the same per-split
sequence and merge source, so a token's output from prefill equals the output
of a later decode step for that position, and chunked prefill equals one-shot
prefill. Causal masking is bottom-right aligned (query t of a T_q-token chunk
sees ``len - T_q + t + 1`` keys), as in MLX.

``order="per_key"`` runs the reference's own order instead (q pre-scaled, 32
lane partials of D/32 dims folded by an xor butterfly, the softmax recurrence
key by key inside each split, splits merged in base e, exp rounded once from
float64): the same invariance properties, values equal to the reference
order's bit for bit, on the vector ALUs and so slower. Contiguous K/V only.
Those kernels take the reference's ``split_size`` keyword too (any split of
1 .. 2^20 keys; a split size fixes the reduction order, so it is part of the
result): ``split_size != 256`` runs them.

``kv_lens`` (int32 [B], optional) is an extension the reference does not have:
sequence b uses only its first ``kv_lens[b]`` keys, and its output is bit-for-bit
what it would be alone with K/V cut to that length.
"""

from __future__ import annotations

import math

import torch

from .. import _lib

SPLIT_SIZE = _lib.SPLIT_KEYS
ORDERS = ("mfma", "per_key")
# Head dims: the matrix-core kernels take these six; the per-key kernels every
# multiple of 32 up to 512 (the reference: any D % 32 == 0,
# kernels/attention.py:299-310). order=None runs the per-key kernels for a
# head dim only they take.
MFMA_HEAD_DIMS = (32, 64, 96, 128, 192, 256)
SUPPORTED_HEAD_DIMS = tuple(range(32, 513, 32))


def supports(q, k, v, mask, sinks=None) -> bool:
    """Reference predicate kernels/attention.py:299-310 (mask None or "causal")."""
    try:
        return bool(
            q.ndim == 4 and k.ndim == 4 and v.ndim == 4
            and (mask is None or (isinstance(mask, str) and mask == "causal"))
            and sinks is None
            and q.shape[1] % k.shape[1] == 0
            and k.shape == v.shape
            and q.shape[-1] == k.shape[-1]
            and q.shape[-1] in SUPPORTED_HEAD_DIMS
            and q.shape[0] == k.shape[0]
            and (mask is None or q.shape[2] <= k.shape[2])
            and q.dtype in _lib.FLOAT_DTYPES
            and all(_lib.is_gpu_tensor(t) for t in (q, k, v))
        )
    except (AttributeError, TypeError):
        return False


def _prep(q, k, v):
    dt = q.dtype
    if dt not in _lib.FLOAT_DTYPES:
        raise ValueError(f"attention: unsupported dtype {dt}")
    if k.dtype != dt:
        k = k.to(dt)
    if v.dtype != dt:
        v = v.to(dt)
    return dt, k, v


def _aligned(t: torch.Tensor) -> bool:
    """Layouts the kernels take in place: unit last stride, 16-byte aligned
    rows and base, and a row stride below 2^23 bytes (the decode and prefill
    kernels address a split's or chunk's rows with 32-bit offsets). Others are
    copied."""
    es = t.element_size()
    st = t.stride()
    return (st[-1] == 1 and t.data_ptr() % 16 == 0
            and all((s * es) % 16 == 0 and s >= 0 for s in st[:-1])
            and (t.dim() < 2 or st[-2] * es < 1 << 23))


def _fix(t: torch.Tensor) -> torch.Tensor:
    return t if _aligned(t) else t.contiguous()


def _lens(kv_lens, B: int, L: int, device) -> torch.Tensor | None:
    if kv_lens is None:
        return None
    kl = torch.as_tensor(kv_lens, dtype=torch.int32, device=device).reshape(-1).contiguous()
    if kl.numel() != B:
        raise ValueError(f"kv_lens has {kl.numel()} entries for batch {B}")
    return kl


MAX_SPLIT = 1 << 20


def _per_key(order, split_size, head_dim: int = 128) -> bool:
    """Which kernels run: the reference's per-key order (True) or the
    matrix-core order (False). ``order=None`` picks the matrix-core kernels for
    the contract split of 256 keys at their head dims, and the per-key kernels
    for any other ``split_size`` (the reference's keyword,
    kernels/attention.py:326-327, :368-370) or head dim, which only they take."""
    if isinstance(split_size, bool) or not isinstance(split_size, int) or not 1 <= split_size <= MAX_SPLIT:
        raise ValueError(f"split_size must be an int in [1, {MAX_SPLIT}]; got {split_size!r}")
    if order is None:
        return split_size != SPLIT_SIZE or head_dim not in MFMA_HEAD_DIMS
    if order not in ORDERS:
        raise ValueError(f"attention order must be one of {ORDERS}; got {order!r}")
    if order == "mfma" and split_size != SPLIT_SIZE:
        raise ValueError(f"the matrix-core kernels use {SPLIT_SIZE}-key splits; split_size={split_size} "
                         "runs with order='per_key'")
    if order == "mfma" and head_dim not in MFMA_HEAD_DIMS:
        raise ValueError(f"the matrix-core kernels take head dims {MFMA_HEAD_DIMS}; D={head_dim} runs with "
                         "order='per_key'")
    return order == "per_key"


def batch_invariant_decode_attention(q, k, v, *, scale: float, split_size: int = SPLIT_SIZE,
                                     kv_lens=None, order: str | None = None) -> torch.Tensor:
    """T_q == 1. Per-split partials (the GU query heads of a kv head share each
    K/V row), then an ordered combine (reference: kernels/attention.py:326-365)."""
    B, Hq, Tq, D = q.shape
    _, Hkv, L, _ = k.shape
    per_key = _per_key(order, split_size, D)
    if Tq != 1:
        raise ValueError(f"decode attention needs T_q == 1, got {Tq}")
    if D not in SUPPORTED_HEAD_DIMS or Hq % Hkv:
        raise ValueError(f"decode attention: unsupported shape q {tuple(q.shape)} k {tuple(k.shape)}")
    dt, k, v = _prep(q, k, v)
    _lib.require_gpu("batch_invariant_decode_attention", q, k, v)
    q3 = _fix(q[:, :, 0, :])
    k = _fix(k)
    v = _fix(v)
    kl = _lens(kv_lens, B, L, q.device)
    out = torch.empty((B, Hq, 1, D), dtype=dt, device=q.device)
    if B == 0:
        return out
    lib = _lib.load()
    strides = (_lib._c_i64 * 8)(q3.stride(0), q3.stride(1), k.stride(0), k.stride(1), k.stride(2),
                                v.stride(0), v.stride(1), v.stride(2))
    if per_key:
        ws_bytes = _lib.ws_bytes("bi_attn_decode_per_key_workspace_bytes", B, Hq, L, D, split_size)
        ws = _lib.workspace(ws_bytes, q.device)
        rc = lib.bi_attn_decode_per_key(q3.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(kl), out.data_ptr(),
                                        B, Hq, Hkv, L, D, strides, float(scale), split_size, _lib.DTYPE_CODE[dt],
                                        _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
        _lib.check(rc, "bi_attn_decode_per_key")
        return out
    ws_bytes = _lib.ws_bytes("bi_attn_decode_workspace_bytes", B, Hq, L, D)
    ws = _lib.workspace(ws_bytes, q.device)
    rc = lib.bi_attn_decode(q3.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(kl), out.data_ptr(),
                            B, Hq, Hkv, L, D, strides, float(scale), _lib.DTYPE_CODE[dt],
                            _lib.ptr(ws), ws_bytes, _lib.stream_of(q))
    _lib.check(rc, "bi_attn_decode")
    return out


def batch_invariant_prefill_attention(q, k, v, *, scale: float, causal: bool,
                                      split_size: int = SPLIT_SIZE, kv_lens=None,
                                      order: str | None = None) -> torch.Tensor:
    """Any T_q. Blocks of 16 (token, head) rows share each K/V row; same split
    loop and merge as decode (reference: kernels/attention.py:368-390)."""
    B, Hq, Tq, D = q.shape
    _, Hkv, L, _ = k.shape
    per_key = _per_key(order, split_size, D)
    if D not in SUPPORTED_HEAD_DIMS or Hq % Hkv:
        raise ValueError(f"prefill attention: unsupported shape q {tuple(q.shape)} k {tuple(k.shape)}")
    if causal and Tq > L:
        raise ValueError(f"causal prefill needs T_q <= L (T_q={Tq}, L={L})")
    dt, k, v = _prep(q, k, v)
    _lib.require_gpu("batch_invariant_prefill_attention", q, k, v)
    q = _fix(q)
    k = _fix(k)
    v = _fix(v)
    kl = _lens(kv_lens, B, L, q.device)
    out = torch.empty((B, Hq, Tq, D), dtype=dt, device=q.device)
    if B == 0 or Tq == 0:
        return out
    lib = _lib.load()
    strides = (_lib._c_i64 * 9)(q.stride(0), q.stride(1), q.stride(2), k.stride(0), k.stride(1),
                                k.stride(2), v.stride(0), v.stride(1), v.stride(2))
    if per_key:
        rc = lib.bi_attn_prefill_per_key(q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(kl), out.data_ptr(),
                                         B, Hq, Hkv, Tq, L, D, strides, 1 if causal else 0, float(scale),
                                         split_size, _lib.DTYPE_CODE[dt], _lib.stream_of(q))
        _lib.check(rc, "bi_attn_prefill_per_key")
        return out
    rc = lib.bi_attn_prefill(q.data_ptr(), k.data_ptr(), v.data_ptr(), _lib.ptr(kl), out.data_ptr(),
                             B, Hq, Hkv, Tq, L, D, strides, 1 if causal else 0, float(scale),
                             _lib.DTYPE_CODE[dt], _lib.stream_of(q))
    _lib.check(rc, "bi_attn_prefill")
    return out


def batch_invariant_attention(q, k, v, *, scale: float | None = None, mask=None, kv_lens=None,
                              order: str | None = None, split_size: int = SPLIT_SIZE) -> torch.Tensor:
    """Dispatch: decode path for T_q == 1, prefill otherwise (reference:
    kernels/attention.py:393-397). ``mask`` is None or "causal"; ``order`` is
    "mfma" (matrix cores), "per_key" (the reference's own order) or None (the
    matrix cores for split_size 256, else per-key)."""
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if mask is not None and mask != "causal":
        raise ValueError("batch_invariant_attention: mask must be None or 'causal'")
    if q.shape[2] == 1:
        return batch_invariant_decode_attention(q, k, v, scale=scale, kv_lens=kv_lens, order=order,
                                                split_size=split_size)
    return batch_invariant_prefill_attention(q, k, v, scale=scale, causal=(mask == "causal"),
                                             kv_lens=kv_lens, order=order, split_size=split_size)


def batch_invariant_paged_attention(q, k_pages, v_pages, block_table, kv_lens=None, *, scale: float | None = None,
                                    mask=None) -> torch.Tensor:
    """Attention over a paged K/V cache: decode for T_q == 1, prefill otherwise.

    ``k_pages`` / ``v_pages``: ``[num_pages, Hkv, page_size, D]`` (any strides
    with ``d`` contiguous, e.g. a permuted ``[num_pages, page_size, Hkv, D]``
    pool); ``block_table``: int32 ``[B, max_pages]``, key ``p`` of sequence ``b``
    lives at row ``p % page_size`` of page ``block_table[b, p // page_size]``;
    ``kv_lens``: int32 ``[B]`` (None: every sequence spans the whole table).
    ``page_size`` must be a power of two. A table entry outside
    ``[0, num_pages)`` is clamped into the pool by the kernels (wrong values,
    never a read outside the pool); a sequence of length 0, and a causal query
    row that sees no key, gets an all-zero output. The output is bit for bit the
    contiguous call on the same keys: paging changes addresses only. The
    reference reads one contiguous cache (kernels/attention.py:87-254); paged
    KV is an item of its roadmap of adjacent ops.
    """
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    if mask is not None and mask != "causal":
        raise ValueError("batch_invariant_paged_attention: mask must be None or 'causal'")
    B, Hq, Tq, D = q.shape
    num_pages, Hkv, page_size, Dk = k_pages.shape
    if v_pages.shape != k_pages.shape or Dk != D or D not in MFMA_HEAD_DIMS or Hq % Hkv:
        raise ValueError(f"paged attention: unsupported shapes q {tuple(q.shape)} k {tuple(k_pages.shape)} "
                         f"v {tuple(v_pages.shape)}")
    if page_size & (page_size - 1):
        raise ValueError(f"paged attention: page size {page_size} is not a power of two")
    if block_table.ndim != 2 or block_table.shape[0] != B:
        raise ValueError(f"paged attention: block table {tuple(block_table.shape)} for batch {B}")
    dt, k_pages, v_pages = _prep(q, k_pages, v_pages)
    _lib.require_gpu("batch_invariant_paged_attention", q, k_pages, v_pages, block_table)
    k_pages, v_pages = _fix(k_pages), _fix(v_pages)
    table = block_table.to(torch.int32).contiguous()
    L = table.shape[1] * page_size
    kl = _lens(kv_lens, B, L, q.device)
    causal = mask == "causal"
    if causal and Tq > L:
        raise ValueError(f"causal prefill needs T_q <= L (T_q={Tq}, L={L})")
    out = torch.empty((B, Hq, Tq, D), dtype=dt, device=q.device)
    if B == 0 or Tq == 0:
        return out
    lib = _lib.load()
    ks = (k_pages.stride(0), k_pages.stride(1), k_pages.stride(2))
    vs = (v_pages.stride(0), v_pages.stride(1), v_pages.stride(2))
    if Tq == 1:
        q3 = _fix(q[:, :, 0, :])
        ws_bytes = _lib.ws_bytes("bi_attn_decode_workspace_bytes", B, Hq, L, D)
        ws = _lib.workspace(ws_bytes, q.device)
        strides = (_lib._c_i64 * 8)(q3.stride(0), q3.stride(1), *ks, *vs)
        rc = lib.bi_attn_decode_paged(q3.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), table.data_ptr(),
                                      table.stride(0), page_size, num_pages, _lib.ptr(kl), out.data_ptr(), B, Hq, Hkv, L, D,
                                      strides, float(scale), _lib.DTYPE_CODE[dt], _lib.ptr(ws), ws_bytes,
                                      _lib.stream_of(q))
        _lib.check(rc, "bi_attn_decode_paged")
        return out
    q = _fix(q)
    strides = (_lib._c_i64 * 9)(q.stride(0), q.stride(1), q.stride(2), *ks, *vs)
    rc = lib.bi_attn_prefill_paged(q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr(), table.data_ptr(),
                                   table.stride(0), page_size, num_pages, _lib.ptr(kl), out.data_ptr(), B, Hq, Hkv, Tq, L, D,
                                   strides, 1 if causal else 0, float(scale), _lib.DTYPE_CODE[dt],
                                   _lib.stream_of(q))
    _lib.check(rc, "bi_attn_prefill_paged")
    return out
