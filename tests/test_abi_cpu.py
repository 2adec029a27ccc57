"""The C-ABI library on a host without a GPU: it loads, exports every symbol
include/bi_kernels.h declares, and rejects bad arguments before launching."""

import ctypes
import re
from pathlib import Path

import pytest

from mlx_batch_invariant_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "bi_kernels.h"


def _declared():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(bi_\w+)\s*\(", text, re.M)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared()
    assert len(names) >= 11
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(_lib.exported_symbols()) == names
    assert lib.bi_abi_version() == _lib.ABI_VERSION == 2
    assert lib.bi_split_m_max() == 32


def test_workspace_sizes():
    lib = _lib.load()
    # M <= 32 folds its group partials in LDS up to 64 groups (32 for M > 16)
    assert lib.bi_matmul_workspace_bytes(1, 14336, 4096) == 0
    # dense 16 < M <= 128 with too few column tiles: the mid-M launch splits K
    assert lib.bi_matmul_workspace_bytes(32, 100, 896) == 4 * 32 * 100 * 4
    assert lib.bi_matmul_workspace_bytes(1, 100, 65 * 256) == 65 * 1 * 100 * 4   # split + fold
    assert lib.bi_matmul_workspace_bytes(20, 100, 33 * 256) == 33 * 20 * 100 * 4
    assert lib.bi_matmul_workspace_bytes(33, 100, 896) == 0          # M > 32 splits only with >= 8 groups
    assert lib.bi_matmul_workspace_bytes(64, 14336, 4096) == 0       # mid-M, enough column tiles
    assert lib.bi_matmul_workspace_bytes(64, 4096, 14336) == 0       # 32 x 32 tiles fill half the chip
    assert lib.bi_matmul_workspace_bytes(64, 1024, 4096) == 16 * 64 * 1024 * 4   # 4 chunks of 4 groups
    assert lib.bi_matmul_workspace_bytes(129, 100, 896) == 0         # tall tile, 4 groups: no split
    assert lib.bi_matmul_workspace_bytes(256, 4864, 896) == 0        # tall tile
    assert lib.bi_matmul_workspace_bytes(256, 4096, 4096) == 0       # tall tile fills the chip
    assert lib.bi_matmul_workspace_bytes(200, 768, 2048) == 8 * 200 * 768 * 4    # tall tile, 4 chunks
    assert lib.bi_matmul_workspace_bytes(129, 12800, 896) == 0       # large tile, >= 96 tiles: fused
    assert lib.bi_matmul_workspace_bytes(257, 100, 896) == 0         # fused (LDS tiles)
    assert lib.bi_matmul_workspace_bytes(200, 4864, 900) == 0        # K % 64 != 0: LDS tiles
    assert lib.bi_quantized_matmul_workspace_bytes(32, 100, 896) == 0   # quantized mid-M needs whole groups
    # quantized mid-M with too few (64-column, row block) tiles splits K: ~512 workgroups
    assert lib.bi_quantized_matmul_workspace_bytes(64, 4096, 14336) == 56 * 64 * 4096 * 4   # 8 chunks of 7
    assert lib.bi_quantized_matmul_workspace_bytes(17, 1024, 4096) == 16 * 17 * 1024 * 4    # 16 chunks of 1
    assert lib.bi_quantized_matmul_workspace_bytes(64, 14336, 4096) == 0    # 224 column blocks: no split
    assert lib.bi_quantized_matmul_workspace_bytes(8, 1024, 4096) == 0      # GEMV launch, LDS fold
    assert lib.bi_matmul_workspace_bytes(8, 100, 256) == 0           # one group
    assert lib.bi_quantized_matmul_workspace_bytes(4, 14336, 4096) == 0
    # large M: dequantized weight + reordered activations, 2 bytes each
    assert lib.bi_quantized_matmul_workspace_bytes(800, 14336, 1024) == (14336 + 800) * 1024 * 2
    assert lib.bi_quantized_matmul_workspace_bytes(2048, 4096, 4096) == (4096 + 2048) * 4096 * 2
    assert lib.bi_quantized_matmul_workspace_bytes(300, 14336, 4096) == (14336 + 300) * 4096 * 2
    assert lib.bi_quantized_matmul_workspace_bytes(300, 4096, 4096) == (4096 + 300) * 4096 * 2   # 128 x 64 form
    assert lib.bi_quantized_matmul_workspace_bytes(512, 1024, 4096) == (1024 + 512) * 4096 * 2   # unsplit tall
    # below M = 256 (the mid-M launches) or K not whole groups: none
    assert lib.bi_quantized_matmul_workspace_bytes(200, 14336, 4096) == 0
    assert lib.bi_quantized_matmul_workspace_bytes(2048, 4096, 4000) == 0
    ns = (8192 + 255) // 256
    bh = 256 * 32 * ns
    # pm | pl | pacc | 16-byte item counter
    assert lib.bi_attn_decode_workspace_bytes(256, 32, 8192, 128) == (2 * ((bh + 3) // 4 * 4) + bh * 128 + 4) * 4


def test_dense_launch_policy():
    """The dense mid/large-M launch per shape (a diagnostic of the policy; the
    bits never depend on it): the smallest large-tile form whose tiles fit one
    per CU (128 x 64 from 72 tiles, then 128 x 128, then 256 x 128), the tall
    tile below that (up to M = 1024) with ring-capped configurations chosen by
    how full they leave the chip's workgroup slots, K split only for long K
    with too few tiles."""
    lib = _lib.load()
    name = lambda M, N, K: lib.bi_matmul_launch(M, N, K).decode()
    assert name(256, 4864, 896) == "big 128x64"                 # Qwen2-0.5B linear, M = 256: 152 tiles of 128 x 64
    assert name(192, 4864, 896) == "big 128x64"
    assert name(64, 4864, 896) == "tall 32x32 k128 r4 c1"       # M <= 64: never the large tile
    assert name(32, 14336, 4096) == "tall 32x64 k128 r4 c1"     # M <= 32: widest tile with >= 200
    assert name(32, 4096, 4096) == "tall 32x32 k128 r4 c2"
    assert name(128, 14336, 4096) == "big 128x64"               # 224 tiles of 128 x 64
    assert name(128, 4096, 4096) == "tall 32x32 k128 r4 c1"     # 64 tiles of 128 x 64: too few
    assert name(256, 4096, 4096) == "big 128x64"                # 128 tiles of 128 x 64
    assert name(512, 4096, 4096) == "big 128x64"                # config-5 prefill at B = 1: 256 tiles
    assert name(512, 4096, 14336) == "big 128x64"
    assert name(768, 4096, 4096) == "big 128x128"               # 384 tiles of 128 x 64 > 256; 192 of 128 x 128
    assert name(2048, 4096, 4096) == "big"                      # 512 tiles of 128 x 128: more than one round
    assert name(192, 896, 4864) == "tall 64x32 k128 r3 c4"
    assert name(192, 14336, 4096) == "big 128x128"              # 448 tiles of 128 x 64; 224 of 128 x 128
    assert name(384, 14336, 4096) == "big"                      # 336 tiles of 128 x 128: more than one round
    assert name(300, 12416, 960) == "big"
    assert name(256, 3328, 576) == "tall 32x64 k64 r5 c1"       # K % 128 != 0: 64-k stages; K < 768: no large tile
    assert name(512, 1024, 4096) == "tall 32x32 k128 r4 c1"     # 64 tiles of 128 x 64: the tall tile up to M = 1024
    assert name(768, 1024, 4096) == "big 128x64"                # 96 tiles of 128 x 64
    assert name(16, 4864, 896) == "other"                       # small-M launches
    assert name(2048, 128, 512) == "other"                      # M > 1024 with few tiles: LDS tiles
    assert name(200, 4864, 900) == "other"                      # K % 64 != 0
    assert name(0, 10, 10) == "other"


def _err(lib):
    return lib.bi_last_error().decode()


def test_invalid_arguments_are_rejected_before_launch():
    lib = _lib.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    # K not a multiple of 8
    assert lib.bi_matmul(p, 12, p, 12, p, 2, 4, 12, 2, None, 0, None) == -1
    assert "multiples of 8" in _err(lib)
    # missing workspace for a split launch
    assert lib.bi_matmul(p, 65 * 256, p, 65 * 256, p, 2, 4, 65 * 256, 2, None, 0, None) == -3
    # paged attention: the page table is checked before anything runs
    st = (ctypes.c_int64 * 8)(*([128] * 8))
    assert lib.bi_attn_decode_paged(p, p, p, p, 4, 3, 9, None, p, 1, 8, 2, 12, 128, st, 1.0, 2, p, 1 << 20, None) == -1
    assert lib.bi_attn_decode_paged(p, p, p, None, 4, 4, 9, None, p, 1, 8, 2, 12, 128, st, 1.0, 2, p, 1 << 20,
                                    None) == -1
    assert lib.bi_attn_decode_paged(p, p, p, p, 2, 4, 9, None, p, 1, 8, 2, 12, 128, st, 1.0, 2, p, 1 << 20, None) == -1
    # the pool size bounds the clamp of every table entry: it must be >= 1
    for num_pages in (0, -3, 1 << 31):
        assert lib.bi_attn_decode_paged(p, p, p, p, 4, 4, num_pages, None, p, 1, 8, 2, 12, 128, st, 1.0, 2, p,
                                        1 << 20, None) == -1
        assert "num_pages" in _err(lib)
        st9 = (ctypes.c_int64 * 9)(*([128] * 9))
        assert lib.bi_attn_prefill_paged(p, p, p, p, 4, 4, num_pages, None, p, 1, 8, 2, 4, 12, 128, st9, 1, 1.0, 2,
                                         None) == -1
    # unsupported quantization
    assert lib.bi_quantized_matmul(p, 64, p, p, p, p, 2, 4, 64, 3, 64, 2, None, 0, None) == -2
    assert lib.bi_quantized_matmul(p, 96, p, p, p, p, 2, 4, 96, 4, 64, 2, None, 0, None) == -1
    # unknown dtype, bad shapes
    assert lib.bi_rms_norm(p, 8, None, p, 2, 8, 1e-6, 7, None) == -2
    assert lib.bi_rms_norm(p, 4, None, p, 2, 8, 1e-6, 2, None) == -1
    assert lib.bi_rms_norm(p, 8, None, p, 0, 8, 1e-6, 2, None) == 0     # nothing to do
    strides = (ctypes.c_int64 * 9)(*([128] * 9))
    assert lib.bi_attn_decode(p, p, p, None, p, 1, 4, 4, 10, 80, strides, 1.0, 2, p, 1 << 20, None) == -2   # D % 32 != 0
    assert lib.bi_attn_decode(p, p, p, None, p, 1, 6, 4, 10, 128, strides, 1.0, 2, p, 1 << 20, None) == -1
    assert lib.bi_attn_decode(p, p, p, None, p, 1, 4, 4, 10, 128, strides, 1.0, 2, None, 0, None) == -3
    assert lib.bi_attn_prefill(p, p, p, None, p, 1, 4, 4, 20, 10, 128, strides, 1, 1.0, 2, None) == -1
    # the no-workspace decode rejects shapes whose partials exceed its static scratch, before any HIP call
    assert lib.bi_attn_decode_workspace_bytes(256, 32, 8192, 128) > _lib.DECODE_SCRATCH_BYTES
    assert lib.bi_attn_decode_noalloc(p, p, p, None, p, 256, 32, 8, 8192, 128, strides, 1.0, 2, None) == -3
    assert "static scratch" in _err(lib)
    bad = (ctypes.c_int64 * 9)(*([3] * 9))
    assert lib.bi_attn_prefill(p, p, p, None, p, 1, 4, 4, 5, 10, 128, bad, 0, 1.0, 2, None) == -1
    # K position stride of 2^24 bytes: the contiguous prefill kernel's 32-bit chunk offsets cannot hold it
    huge = (ctypes.c_int64 * 9)(*([128] * 5 + [1 << 23] + [128] * 3))
    assert lib.bi_attn_prefill(p, p, p, None, p, 1, 4, 4, 5, 10, 128, huge, 0, 1.0, 2, None) == -2
    assert "2^24 bytes" in _err(lib)
    # more (sequence, kv head, 64-row workgroup) items than the prefill kernel's padded 1-D grid can hold
    assert lib.bi_attn_prefill(p, p, p, None, p, 1000, 1024, 1024, 200000, 200000, 128, strides, 1, 1.0, 2,
                               None) == -2
    assert "grid too large" in _err(lib)
    # V position stride of 2^23 bytes: the contiguous decode kernel's 32-bit split offsets cannot hold it
    huge8 = (ctypes.c_int64 * 9)(*([128] * 7 + [1 << 22] + [128]))
    assert lib.bi_attn_decode(p, p, p, None, p, 1, 4, 4, 10, 128, huge8, 1.0, 2, p, 1 << 20, None) == -2
    assert "2^23 bytes" in _err(lib)
    # the per-key order entry points share the validation, plus the split size
    assert lib.bi_attn_decode_per_key(p, p, p, None, p, 1, 4, 4, 10, 80, strides, 1.0, 256, 2, p, 1 << 20,
                                      None) == -2
    assert lib.bi_attn_decode_per_key(p, p, p, None, p, 1, 4, 4, 10, 128, strides, 1.0, 256, 2, None, 0, None) == -3
    assert "bi_attn_decode_per_key" in _err(lib)
    assert lib.bi_attn_prefill_per_key(p, p, p, None, p, 1, 4, 4, 20, 10, 128, strides, 1, 1.0, 256, 2, None) == -1
    assert lib.bi_attn_prefill_per_key(p, p, p, None, p, 1, 4, 4, 5, 10, 128, bad, 0, 1.0, 256, 2, None) == -1
    assert lib.bi_attn_decode_per_key(p, p, p, None, p, 0, 4, 4, 10, 128, strides, 1.0, 256, 2, None, 0, None) == 0
    for split in (0, -1, (1 << 20) + 1):
        assert lib.bi_attn_decode_per_key(p, p, p, None, p, 1, 4, 4, 10, 128, strides, 1.0, split, 2, p, 1 << 20,
                                          None) == -1
        assert "split_size" in _err(lib)
        assert lib.bi_attn_prefill_per_key(p, p, p, None, p, 1, 4, 4, 5, 10, 128, strides, 0, 1.0, split, 2,
                                           None) == -1
        assert lib.bi_attn_decode_per_key_workspace_bytes(1, 4, 10, 128, split) == 0
    # a workspace sized for 256-key splits is too small for 100-key splits
    need = lib.bi_attn_decode_per_key_workspace_bytes(2, 8, 1000, 128, 100)
    assert need > lib.bi_attn_decode_workspace_bytes(2, 8, 1000, 128)
    assert lib.bi_attn_decode_per_key_workspace_bytes(2, 8, 1000, 128, 256) == lib.bi_attn_decode_workspace_bytes(
        2, 8, 1000, 128)
    assert lib.bi_attn_decode_per_key(p, p, p, None, p, 2, 8, 2, 1000, 128, strides, 1.0, 100, 2, p, need - 16,
                                      None) == -3
    # head dims: the per-key entry points take multiples of 32 up to 512, the matrix-core ones six of them
    assert lib.bi_attn_decode_per_key(p, p, p, None, p, 1, 4, 4, 10, 544, strides, 1.0, 256, 2, p, 1 << 20,
                                      None) == -2
    assert lib.bi_attn_prefill_per_key(p, p, p, None, p, 1, 4, 4, 5, 10, 176, strides, 0, 1.0, 256, 2, None) == -2
    assert lib.bi_attn_decode(p, p, p, None, p, 1, 4, 4, 10, 160, strides, 1.0, 2, p, 1 << 20, None) == -2
    assert "per-key" in _err(lib)
    # the exp2 diagnostic: count and pointers checked before launch, nothing to do for n = 0
    assert lib.bi_exp2_f32(p, p, -1, None) == -1
    assert lib.bi_exp2_f32(None, p, 4, None) == -1
    assert lib.bi_exp2_f32(p, None, 4, None) == -1
    assert lib.bi_exp2_f32(None, None, 0, None) == 0
    assert lib.bi_stream_read(p, 24, p, 0, None) == -1          # not whole 16-byte pieces
    assert lib.bi_stream_read(None, 32, p, 0, None) == -1
    assert lib.bi_stream_read(None, 0, None, 0, None) == 0
    # the single-step MFMA probe: count, dtype and pointers checked before launch
    assert lib.bi_mfma_step_probe(p, p, p, p, -1, 2, None) == -1
    assert lib.bi_mfma_step_probe(p, p, p, p, (1 << 24) + 1, 2, None) == -1
    assert lib.bi_mfma_step_probe(p, p, p, p, 1, 9, None) == -2
    assert lib.bi_mfma_step_probe(None, p, p, p, 1, 2, None) == -1
    assert lib.bi_mfma_step_probe(ctypes.c_void_p(24), p, p, p, 1, 2, None) == -1   # a not 16-byte aligned
    assert lib.bi_mfma_step_probe(None, None, None, None, 0, 2, None) == 0
    # the dequantize-once pair: formats, dtypes, shapes, pointers and workspace checked before launch
    assert lib.bi_quantized_dequantize(p, p, p, p, 16, 256, 3, 64, 2, None) == -2        # bits
    assert lib.bi_quantized_dequantize(p, p, p, p, 16, 256, 4, 64, 3, None) == -2        # fp32
    assert lib.bi_quantized_dequantize(p, p, p, p, 16, 320, 4, 64, 2, None) == -1        # K % 256
    assert lib.bi_quantized_dequantize(None, p, p, p, 16, 256, 4, 64, 2, None) == -1
    assert lib.bi_quantized_dequantize(None, None, None, None, 0, 256, 4, 64, 2, None) == 0
    need = lib.bi_quantized_matmul_dequantized_workspace_bytes(512, 4096, 4096)
    assert need >= 512 * 4096 * 2
    assert lib.bi_quantized_matmul_dequantized(p, 4096, p, p, 512, 4096, 4096, 2, p, need - 16, None) == -3
    assert lib.bi_quantized_matmul_dequantized(p, 4096, p, p, 512, 4096, 4096, 3, p, need, None) == -2
    assert lib.bi_quantized_matmul_dequantized(p, 4096, p, p, 512, 4096, 4000, 2, p, need, None) == -1
    assert lib.bi_quantized_matmul_dequantized(p, 4095, p, p, 512, 4096, 4096, 2, p, need, None) == -1
    assert lib.bi_quantized_matmul_dequantized(None, 0, None, None, 0, 4096, 4096, 2, None, 0, None) == 0


def test_quantized_pack_sizes_and_rejections():
    """bi_quantized_pack_bytes: ceil(N / 16) tiles x K / 256 groups x (bits x
    512 + 16 x 256 / group_size x 4) bytes (each lane's codes as 16-byte pieces
    of 1 KB runs, then the block's (scale, bias) pairs, each once), 0 for a
    format without a packed form;
    bi_quantized_pack / bi_quantized_matmul_packed reject what they cannot take
    before launching anything (M = 0 is a no-op)."""
    lib = _lib.load()
    assert lib.bi_quantized_pack_bytes(14336, 4096, 4, 64) == 896 * 16 * 2304
    assert lib.bi_quantized_pack_bytes(4096, 14336, 4, 64) == 256 * 56 * 2304
    assert lib.bi_quantized_pack_bytes(17, 256, 8, 64) == 2 * 1 * 4352
    assert lib.bi_quantized_pack_bytes(17, 256, 8, 128) == 2 * 1 * 4224
    assert lib.bi_quantized_pack_bytes(4096, 4096, 4, 32) == 256 * 16 * 2560
    for args in ((4096, 4096, 4, 16), (4096, 4096, 3, 64), (4096, 4160, 4, 64), (0, 4096, 4, 64),
                 (4096, 0, 4, 64)):
        assert lib.bi_quantized_pack_bytes(*args) == 0, args
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    need = lib.bi_quantized_pack_bytes(32, 512, 4, 64)
    assert lib.bi_quantized_pack(p, p, p, p, need, 32, 512, 4, 16, 2, None) == -2           # group size 16
    assert lib.bi_quantized_pack(p, p, p, p, need, 32, 512, 4, 64, 0, None) == -2           # fp32
    assert lib.bi_quantized_pack(p, p, p, p, need, 32, 320, 4, 64, 2, None) == -1           # K % 256
    assert lib.bi_quantized_pack(p, p, p, p, need - 1, 32, 512, 4, 64, 2, None) == -1       # too small
    assert "required" in _err(lib)
    assert lib.bi_quantized_pack(p, p, None, p, need, 32, 512, 4, 64, 2, None) == -1        # null biases
    assert lib.bi_quantized_pack(p, p, p, ctypes.c_void_p(24), need, 32, 512, 4, 64, 2, None) == -1  # misaligned
    assert lib.bi_quantized_pack(p, p, p, p, need, 0, 512, 4, 64, 2, None) == 0             # nothing to pack
    # the matmul with a packed copy: the copy's format first, then the op's own checks
    assert lib.bi_quantized_matmul_packed(p, 512, p, p, p, p, p, 2, 32, 512, 4, 16, 2, None, 0, None) == -2
    assert lib.bi_quantized_matmul_packed(p, 512, p, p, p, p, p, 2, 32, 512, 4, 64, 0, None, 0, None) == -2
    assert lib.bi_quantized_matmul_packed(p, 320, p, p, p, p, p, 2, 32, 320, 4, 64, 2, None, 0, None) == -2
    assert lib.bi_quantized_matmul_packed(p, 512, p, p, p, p, p, 2, 32, 512, 3, 64, 2, None, 0, None) == -2
    assert lib.bi_quantized_matmul_packed(p, 520, p, p, p, ctypes.c_void_p(24), p, 2, 32, 512, 4, 64, 2, None, 0,
                                          None) == -1
    assert lib.bi_quantized_matmul_packed(p, 12, p, p, p, p, p, 2, 32, 512, 4, 64, 2, None, 0, None) == -1   # ldx < K
    assert lib.bi_quantized_matmul_packed(p, 512, p, p, p, p, p, 0, 32, 512, 4, 64, 2, None, 0, None) == 0
    # without a copy it is bi_quantized_matmul, checks included
    assert lib.bi_quantized_matmul_packed(p, 64, p, p, p, None, p, 2, 4, 64, 3, 64, 2, None, 0, None) == -2


def test_dense_pack_sizes_and_rejections():
    """bi_matmul_pack_bytes: ceil(N / 16) tiles x ceil(K / 256) groups x 8 KB
    (each lane's eight 16-byte fragments as pieces of 1 KB runs, zero past K),
    0 for fp32 or K not a multiple of 8; bi_matmul_pack / bi_matmul_packed
    reject what they cannot take before launching anything."""
    lib = _lib.load()
    assert lib.bi_matmul_pack_bytes(14336, 4096, 2) == 896 * 16 * 8192
    assert lib.bi_matmul_pack_bytes(1000, 256, 1) == 63 * 1 * 8192
    assert lib.bi_matmul_pack_bytes(4864, 896, 2) == 304 * 4 * 8192
    for args in ((4096, 4096, 0), (4096, 4100, 2), (0, 4096, 2), (4096, 0, 2)):
        assert lib.bi_matmul_pack_bytes(*args) == 0, args
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    need = lib.bi_matmul_pack_bytes(32, 512, 2)
    assert lib.bi_matmul_pack(p, 512, p, need, 32, 512, 0, None) == -2          # fp32
    assert lib.bi_matmul_pack(p, 328, p, need, 32, 324, 2, None) == -1          # K % 8
    assert lib.bi_matmul_pack(p, 512, p, need - 1, 32, 512, 2, None) == -1      # too small
    assert "required" in _err(lib)
    assert lib.bi_matmul_pack(p, 500, p, need, 32, 512, 2, None) == -1          # ldb < K
    assert lib.bi_matmul_pack(p, 512, ctypes.c_void_p(24), need, 32, 512, 2, None) == -1   # misaligned copy
    assert lib.bi_matmul_pack(p, 512, p, need, 0, 512, 2, None) == 0            # nothing to pack
    assert lib.bi_matmul_packed(p, 512, p, 512, p, p, 2, 32, 512, 0, None, 0, None) == -2      # fp32 copy
    assert lib.bi_matmul_packed(p, 328, p, 328, p, p, 2, 32, 324, 2, None, 0, None) == -2      # K % 8
    assert lib.bi_matmul_packed(p, 512, p, 512, ctypes.c_void_p(24), p, 2, 32, 512, 2, None, 0, None) == -1
    assert lib.bi_matmul_packed(p, 512, p, 512, p, p, 0, 32, 512, 2, None, 0, None) == 0       # M = 0
    # without a copy it is bi_matmul, checks included
    assert lib.bi_matmul_packed(p, 12, p, 12, None, p, 2, 4, 12, 2, None, 0, None) == -1


def test_split_size_routing():
    """split_size other than 256 runs the per-key kernels (the only ones that
    take it); asking the matrix-core kernels for it is an error."""
    from mlx_batch_invariant_amd.kernels.attention import _per_key
    assert _per_key(None, 256) is False
    assert _per_key(None, 128) is True
    assert _per_key("per_key", 256) is True
    assert _per_key("mfma", 256) is False
    assert _per_key(None, 256, 160) is True          # a head dim only the per-key kernels take
    assert _per_key(None, 256, 192) is False
    for bad in [("mfma", 128), (None, 0), (None, 1.5), ("fast", 256), (None, True), ("mfma", 256, 160)]:
        with pytest.raises(ValueError):
            _per_key(*bad)


def test_fast_binding_matches_ctypes():
    """The CPython binding (_bi_pycall, built with the library) calls the same
    C functions as ctypes: the same status for the same (rejected) arguments,
    None as NULL, and a TypeError for a wrong argument count."""
    lib = _lib.load()
    from mlx_batch_invariant_amd import _bi_pycall
    assert _lib.qmm_call is _bi_pycall.quantized_matmul
    assert _lib.matmul_call is _bi_pycall.matmul
    assert _lib.rms_norm_call is _bi_pycall.rms_norm
    # null operands: rejected before any launch, by either binding
    q = (0, 4096, 0, 0, 0, 0, 1, 14336, 4096, 4, 64, _lib.BI_BF16, None, 0, 0)
    assert _lib.qmm_call(*q) == lib.bi_quantized_matmul(*q) == -1
    m = (0, 8, 0, 8, 0, 1, 8, 8, _lib.BI_BF16, None, 0, 0)
    assert _lib.matmul_call(*m) == lib.bi_matmul(*m) == -1
    r = (0, 8, None, 0, 1, 8, 1e-6, _lib.BI_BF16, 0)
    assert _lib.rms_norm_call(*r) == lib.bi_rms_norm(*r) == -1
    # an unknown dtype code is rejected the same way
    q_bad = q[:11] + (7,) + q[12:]
    assert _lib.qmm_call(*q_bad) == lib.bi_quantized_matmul(*q_bad)
    with pytest.raises(TypeError):
        _lib.qmm_call(*q[:-1])
    with pytest.raises(TypeError):
        _lib.rms_norm_call(*r[:6], "eps", *r[7:])
