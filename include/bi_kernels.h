/*
 * bi_kernels.h — C ABI of the MI355X (gfx950) batch-invariant kernel library.
 *
 * Every entry point is asynchronous on the caller's HIP stream (`stream` is a
 * hipStream_t passed as a plain pointer; NULL means the default stream), never
 * allocates, frees or synchronises, and validates its arguments before it
 * launches anything.
 *
 * Return codes: 0 = ok; BI_E_INVALID_ARG / BI_E_UNSUPPORTED / BI_E_WORKSPACE
 * (negative) = rejected before launch, nothing was enqueued; >0 = the
 * hipError_t of a failed launch. bi_last_error() returns a thread-local
 * message describing the last non-zero return on the calling thread.
 *
 * Buffers are device pointers owned by the caller. Element type is chosen by
 * `dtype` (BI_F32 / BI_F16 / BI_BF16) and is the same for every floating-point
 * operand of a call; accumulation is always fp32.
 *
 * The reference ("mlx-batch-invariant") has no native ABI: its kernels are Metal
 * source strings launched through mx.fast.metal_kernel from Python. Each entry
 * point below replaces one of those Python launchers; the citation names it.
 */
#ifndef BI_KERNELS_H
#define BI_KERNELS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define BI_ABI_VERSION 2

enum bi_dtype { BI_F32 = 0, BI_F16 = 1, BI_BF16 = 2 };

enum bi_status {
  BI_OK = 0,
  BI_E_INVALID_ARG = -1, /* shapes, strides, alignment or pointers are wrong */
  BI_E_UNSUPPORTED = -2, /* valid request this library has no kernel for    */
  BI_E_WORKSPACE = -3    /* workspace missing or smaller than required      */
};

/* Contract constants. They fix the reduction order, so changing either one
 * changes result bits. Reference: kernels/matmul.py:46 (GROUP_K = 256),
 * kernels/attention.py:38 (SPLIT_SIZE = 256). */
#define BI_GROUP_K 256
#define BI_SPLIT_KEYS 256

int bi_abi_version(void);
const char* bi_last_error(void);
/* Threshold of the launch-shape policy: GEMMs with M <= this many rows run one
 * workgroup per (tile, K group) plus an ordered fold kernel. Launch shape only;
 * it never changes bits. Reference: kernels/matmul.py:47 (SPLIT_M_MAX). */
int bi_split_m_max(void);

/* ---- RMSNorm --------------------------------------------------------------
 * out[r, :] = T( (float(x[r, :]) * inv_r) * float(w) ),
 * inv_r = 1 / sqrt( ss_r / D + eps ), ss_r reduced in a fixed order that
 * depends on D only. w may be NULL (all ones). x rows are `x_row_stride`
 * elements apart; out is contiguous [rows, D].
 * Replaces: kernels/rmsnorm.py:64-79 (batch_invariant_rms_norm) and its
 * kernel kernels/rmsnorm.py:19-47. */
int bi_rms_norm(const void* x, int64_t x_row_stride, const void* w, void* out,
                int64_t rows, int64_t D, float eps, int dtype, void* stream);

/* ---- LayerNorm over the last dimension -------------------------------------
 * out = T(((x - mean) * inv) * w + b) per row, mean and the biased variance
 * in a fixed two-pass order that depends on D only; w and b may be NULL (the
 * multiply / add is then skipped). x rows are x_row_stride elements apart; out
 * is contiguous [rows, D].
 * Replaces: nothing in the reference's kernels (it falls back to the stock
 * mx.fast.layer_norm, README.md:250-251); its roadmap item "a batch-invariant
 * mx.fast.layer_norm" (README.md:257-260). */
int bi_layer_norm(const void* x, int64_t x_row_stride, const void* w, const void* b, void* out,
                  int64_t rows, int64_t D, float eps, int dtype, void* stream);

/* ---- Dense matmul ---------------------------------------------------------
 * out[M, N] = a[M, K] @ b[K, N], with b given transposed: element b[k, n] is at
 * bt[n * ldb + k] (the k-contiguous nn.Linear weight layout). a rows are lda
 * elements apart; out is contiguous [M, N]. Requires K % 8 == 0, lda % 8 == 0,
 * ldb % 8 == 0 and 16-byte aligned a/bt (the Python layer pads or copies
 * otherwise, which does not change bits).
 * The workspace holds fp32 group partials for small-M launches; query its
 * size with bi_matmul_workspace_bytes (0 means none needed).
 * Replaces: kernels/matmul.py:279-314 (launch_tiled) + :317-340
 * (batch_invariant_matmul), kernels :81-234. */
size_t bi_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K);
int bi_matmul(const void* a, int64_t lda, const void* bt, int64_t ldb, void* out,
              int64_t M, int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes,
              void* stream);

/* Diagnostic, no counterpart in the reference: the mid- and large-M launch
 * the policy picks for a 2-byte dense call of this shape (aligned operands):
 * "big" (256 x 128 tiles), "big 128x128", "tall <BM>x<BN> k<SK> r<ring>
 * c<K chunks>", or "other" (the small-M and LDS-tile launches). Host only;
 * launch shape never changes bits. The string is valid until the calling
 * thread's next call. */
const char* bi_matmul_launch(int64_t M, int64_t N, int64_t K);

/* A repacked copy of a dense weight for the decode GEMV. bi_matmul_pack writes
 * bt's N x K elements (bf16 / fp16, K % 8 == 0, ldb % 8 == 0) into
 * bi_matmul_pack_bytes bytes laid out for the streaming GEMV: per 16 rows and
 * 256-k group (ceil(K / 256) groups, zero past K), each MFMA lane's 16-byte
 * fragment of step s as the lane's piece of the s-th 1 KB run (pack_bytes
 * returns 0 for an unsupported format).
 * bi_matmul_packed is bi_matmul with that copy beside bt (packed may be NULL:
 * then it is bi_matmul): the streaming GEMV reads the copy wherever it takes
 * the shape (M <= 16), every other launch reads bt, and the result equals
 * bi_matmul's bit for bit at every M. Same checks and workspace as bi_matmul;
 * the copy must have been packed from this bt.
 * No counterpart in the reference (MLX reads the weight as stored): for callers
 * that keep a repacked copy of an nn.Linear weight, so that decode reads whole
 * 1 KB runs per wave instruction. */
size_t bi_matmul_pack_bytes(int64_t N, int64_t K, int dtype);
int bi_matmul_pack(const void* bt, int64_t ldb, void* packed, size_t packed_bytes, int64_t N, int64_t K, int dtype,
                   void* stream);
int bi_matmul_packed(const void* a, int64_t lda, const void* bt, int64_t ldb, const void* packed, void* out,
                     int64_t M, int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes, void* stream);

/* Strided batch of dense matmuls (a [batch][M, K], bt [batch][N, K],
 * out [batch][M, N]; batch strides in elements, 0 broadcasts a or bt): slice i
 * is exactly bi_matmul on the slice's pointers, so its bits equal a 2-D call
 * and do not depend on batch. Same requirements and workspace as bi_matmul
 * (shared by the slices, which run in order on the stream).
 * Replaces: the reference's fallback for a non-2-D right-hand side
 * (ops.py:46-51, "matmul:non-2d-rhs-or-non-float"); its roadmap's batched
 * matmul (README.md:257-268). */
int bi_matmul_batched(const void* a, int64_t a_batch_stride, int64_t lda, const void* bt,
                      int64_t b_batch_stride, int64_t ldb, void* out, int64_t out_batch_stride,
                      int64_t batch, int64_t M, int64_t N, int64_t K, int dtype, void* ws,
                      size_t ws_bytes, void* stream);

/* ---- Affine quantized matmul (MLX packed format) ---------------------------
 * out[M, N] = x[M, K] @ W^T with W[n, k] = T(fmaf(code(n,k), scale, bias)),
 * code(n, k) = (w[n, k*bits/32] >> (bits * (k % (32/bits)))) & (2^bits - 1),
 * scale/bias = scales/biases[n, k / group_size] (element type = dtype).
 * w is contiguous uint32 [N, K*bits/32]; scales, biases contiguous
 * [N, K/group_size]. bits in {4, 8}, group_size in {32, 64, 128},
 * K % group_size == 0. x rows are ldx elements apart (ldx % 8 == 0).
 * Workspace (bi_quantized_matmul_workspace_bytes): fp32 group partials
 * [K/256, M, N] for small M and for mid M (M < 256, K % 256 == 0) when there
 * are too few 64-column blocks to fill the GPU; for large M with
 * K % 256 == 0 (bf16/fp16) the dequantized weight and a reordered copy of x,
 * (N + M) * K elements of 2 bytes. The query has no dtype: it reports the
 * need of the 2-byte launches, which an fp32 call also accepts.
 * Replaces: kernels/quantized.py:106-125 (batch_invariant_quantized_matmul),
 * kernels :33-67 (dequant-on-stage). */
size_t bi_quantized_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K);
int bi_quantized_matmul(const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                        const void* biases, void* out, int64_t M, int64_t N, int64_t K,
                        int bits, int group_size, int dtype, void* ws, size_t ws_bytes,
                        void* stream);

/* The quantized op on a weight dequantized once. bi_quantized_dequantize
 * writes bq [N, K] (dtype elements): W dequantized as above, its 8-element
 * chunks permuted within each 256-k group into the order the dense kernels
 * read (the large-M launch's own copy of the weight). bi_quantized_matmul_-
 * dequantized computes out[M, N] from x and bq, bit for bit equal to
 * bi_quantized_matmul on the same x and weight at every M (the dense kernels
 * on the permuted operands put the quantized order's products in every
 * matrix-core slot); workspace from bi_quantized_matmul_dequantized_-
 * workspace_bytes (x reordered, plus the dense launch's partials).
 * bf16 / fp16, K % 256 == 0, ldx % 8 == 0, x and bq 16-byte aligned.
 * No counterpart in the reference (MLX dequantizes inside its kernels): for
 * callers that keep a dequantized copy next to the codes, so that prefill
 * (large M) skips the per-call dequantization. */
int bi_quantized_dequantize(const uint32_t* w, const void* scales, const void* biases, void* bq, int64_t N,
                            int64_t K, int bits, int group_size, int dtype, void* stream);
size_t bi_quantized_matmul_dequantized_workspace_bytes(int64_t M, int64_t N, int64_t K);
int bi_quantized_matmul_dequantized(const void* x, int64_t ldx, const void* bq, void* out, int64_t M, int64_t N,
                                    int64_t K, int dtype, void* ws, size_t ws_bytes, void* stream);

/* A repacked copy of a weight for the decode GEMV. bi_quantized_pack writes
 * the same codes, scales and biases as w / scales / biases (bits 4 or 8,
 * group_size 32 / 64 / 128, bf16 / fp16, K % 256 == 0) into
 * bi_quantized_pack_bytes bytes laid out for the streaming GEMV: per 16 rows
 * and 256-k group, the codes of each MFMA lane as the lane's 16-byte pieces of
 * consecutive 1 KB runs, then the block's (scale, bias) pairs, each once
 * (pack_bytes returns 0 for an unsupported format). bi_quantized_matmul_packed is bi_quantized_matmul with
 * that copy beside the MLX-layout operands (packed may be NULL: then it is
 * bi_quantized_matmul): the streaming GEMV (M <= 16) and the mid-M launches
 * (M < 256) read the copy wherever they take the shape, every other launch
 * reads w / scales / biases, and the
 * result equals bi_quantized_matmul's bit for bit at every M. Same checks and
 * workspace as bi_quantized_matmul; the copy must have been packed from these
 * w / scales / biases.
 * No counterpart in the reference (MLX reads its own layout): for callers that
 * keep a repacked copy next to the codes, so that decode reads whole 1 KB runs
 * per wave instruction. */
size_t bi_quantized_pack_bytes(int64_t N, int64_t K, int bits, int group_size);
int bi_quantized_pack(const uint32_t* w, const void* scales, const void* biases, void* packed, size_t packed_bytes,
                      int64_t N, int64_t K, int bits, int group_size, int dtype, void* stream);
int bi_quantized_matmul_packed(const void* x, int64_t ldx, const uint32_t* w, const void* scales,
                               const void* biases, const void* packed, void* out, int64_t M, int64_t N, int64_t K,
                               int bits, int group_size, int dtype, void* ws, size_t ws_bytes, void* stream);

/* ---- Split-KV decode attention (one query token per sequence) -------------
 * q [B, Hq, D], k/v [B, Hkv, L, D] addressed through element strides
 *   strides[0..1] = q  (batch, head)
 *   strides[2..4] = k  (batch, head, position)
 *   strides[5..7] = v  (batch, head, position)
 * with d contiguous. out contiguous [B, Hq, D]. kv_lens (device int32[B], may
 * be NULL = all L) gives each sequence's own key count, clamped to [0, L]; a
 * sequence's output depends only on its own first len keys, and a sequence of
 * length 0 gets an all-zero output (no key: no softmax). Hq % Hkv == 0,
 * D in {32, 64, 96, 128, 192, 256}. Keys go in fixed splits of BI_SPLIT_KEYS; the workspace
 * holds per-split (m, l, acc) partials and a work-item counter
 * (bi_attn_decode_workspace_bytes); calls that overlap must not share it.
 * The V position stride must stay below 2^23 bytes (BI_E_UNSUPPORTED
 * otherwise; copy such a layout first).
 * Replaces: kernels/attention.py:326-365 (batch_invariant_decode_attention),
 * kernels :47-171; kv_lens is an extension the reference lacks. */
size_t bi_attn_decode_workspace_bytes(int64_t B, int64_t Hq, int64_t L, int64_t D);
int bi_attn_decode(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                   void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                   const int64_t* strides, float scale, int dtype, void* ws,
                   size_t ws_bytes, void* stream);

/* bi_attn_decode without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * Same arguments, arithmetic and bits as bi_attn_decode; the per-split
 * partials and the work-item counter live in a static device array of
 * BI_DECODE_SCRATCH_BYTES per GPU (held from library load until the process
 * ends), so calls with bi_attn_decode_workspace_bytes(B, Hq, L, D) above it
 * are rejected with BI_E_WORKSPACE (64 MiB: e.g. B = 64, Hq = 32, L = 8192,
 * D = 128 needs 34 MB). The call allocates nothing. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (concurrent streams,
 * threads) race and must be serialised by the caller. The scratch is the
 * current device's: a non-null stream of another device is rejected with
 * BI_E_INVALID_ARG. The first call on a device resolves the array's address
 * and must be made outside graph capture (BI_E_UNSUPPORTED otherwise); later
 * calls of the same shape may be captured and replayed. */
#define BI_DECODE_SCRATCH_BYTES (64u << 20)
int bi_attn_decode_noalloc(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                           void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                           const int64_t* strides, float scale, int dtype, void* stream);

/* Paged K/V variant of bi_attn_decode: k_pages / v_pages are pools of
 * num_pages pages of page_size keys (a power of two, 1 .. 2^24);
 * strides[2..4] / [5..7] are the (page, head, position-in-page) element
 * strides. Key p of sequence b is row p mod page_size of page
 * block_table[b * table_stride + p / page_size] (device int32; table_stride
 * >= ceil(L / page_size)). A table entry outside [0, num_pages) is clamped
 * into the pool, so a stale table gives wrong values but never reads outside
 * it. L is the longest sequence the table can hold (it sizes the workspace,
 * as in bi_attn_decode). Same arithmetic as bi_attn_decode: the output equals
 * the contiguous call on the same keys, bit for bit.
 * Replaces: nothing in the reference (its decode reads one contiguous cache,
 * kernels/attention.py:87-147); the paged-KV item of its roadmap of adjacent
 * ops. */
int bi_attn_decode_paged(const void* q, const void* k_pages, const void* v_pages,
                         const int32_t* block_table, int64_t table_stride, int64_t page_size,
                         int64_t num_pages, const int32_t* kv_lens, void* out, int64_t B, int64_t Hq, int64_t Hkv,
                         int64_t L, int64_t D, const int64_t* strides, float scale, int dtype,
                         void* ws, size_t ws_bytes, void* stream);

/* ---- Prefill attention (any number of query tokens) ------------------------
 * q [B, Hq, Tq, D], k/v [B, Hkv, L, D] through element strides
 *   strides[0..2] = q (batch, head, token)
 *   strides[3..5] = k (batch, head, position)
 *   strides[6..8] = v (batch, head, position)
 * out contiguous [B, Hq, Tq, D]. With causal != 0, query t of sequence b sees
 * keys [0, len_b - Tq + t + 1) (bottom-right aligned, so a later chunk of a
 * prompt run against the whole cache is a valid prefill); otherwise all len_b.
 * len_b = kv_lens[b] (device int32[B], may be NULL = L; clamped to [0, L]);
 * with causal != 0, Tq <= L is required, and a query row with no visible key
 * (len_b - Tq + t + 1 <= 0) gets an all-zero output. Same split order and per-split arithmetic as bi_attn_decode, so a token's
 * output equals a later decode step's and chunked equals one-shot prefill.
 * The K and V position strides must stay below 2^24 bytes
 * (BI_E_UNSUPPORTED otherwise; copy such a layout first).
 * Replaces: kernels/attention.py:368-390 (batch_invariant_prefill_attention),
 * kernels :173-254. */
int bi_attn_prefill(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                    void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t L,
                    int64_t D, const int64_t* strides, int causal, float scale, int dtype,
                    void* stream);

/* Paged K/V variant of bi_attn_prefill (pool of num_pages pages,
 * strides[3..5] / [6..8] = (page, head, position-in-page), block table and
 * clamping as in bi_attn_decode_paged): a
 * prompt chunk run against a paged cache. Bit-identical to bi_attn_prefill on
 * the same keys.
 * Replaces: nothing in the reference (kernels/attention.py:173-254 reads a
 * contiguous cache); the paged-KV prefill item of its roadmap of adjacent ops. */
int bi_attn_prefill_paged(const void* q, const void* k_pages, const void* v_pages,
                          const int32_t* block_table, int64_t table_stride, int64_t page_size,
                          int64_t num_pages, const int32_t* kv_lens, void* out, int64_t B, int64_t Hq, int64_t Hkv,
                          int64_t Tq, int64_t L, int64_t D, const int64_t* strides, int causal,
                          float scale, int dtype, void* stream);

/* ---- Attention in the reference's per-key order ----------------------------
 * The arguments, validation and invariance properties of bi_attn_decode /
 * bi_attn_prefill plus split_size, in the reference kernels' own order of
 * operations instead of the matrix-core order: q pre-scaled in fp32, score =
 * 32 lane partials of D/32 dims (fma chains) folded by an xor butterfly
 * 16..1, the online softmax key by key inside each split of split_size keys
 * (m' = max(m, s); corr = exp(m - m'); p = exp(s - m'); l = fma(l, corr, p);
 * acc = fma(acc, corr, p v)), splits merged left to right in base e, out =
 * T(A / L). exp is fp32 rounded once from double precision. split_size is any
 * key count in [1, 2^20] (the reference's split_size; 256 is BI_SPLIT_KEYS);
 * decode's workspace comes from bi_attn_decode_per_key_workspace_bytes.
 * Slower (vector ALUs, one key at a time); for callers that need the
 * reference order's values.
 * Replaces: kernels/attention.py:326-365 (decode, split_size), :87-147 +
 * :149-171 (kernels), :368-390 and :173-254 (prefill); order of operations
 * :1-32, :47-85. */
size_t bi_attn_decode_per_key_workspace_bytes(int64_t B, int64_t Hq, int64_t L, int64_t D, int64_t split_size);
int bi_attn_decode_per_key(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                           void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                           const int64_t* strides, float scale, int64_t split_size, int dtype, void* ws,
                           size_t ws_bytes, void* stream);
int bi_attn_prefill_per_key(const void* q, const void* k, const void* v, const int32_t* kv_lens,
                            void* out, int64_t B, int64_t Hq, int64_t Hkv, int64_t Tq, int64_t L,
                            int64_t D, const int64_t* strides, int causal, float scale, int64_t split_size,
                            int dtype, void* stream);

/* Diagnostic, no counterpart in the reference: y[i] = the hardware base-2
 * exponential (v_exp_f32) of x[i], n >= 0 floats, device pointers, on the
 * stream. It is the instruction the matrix-core attention kernels compute
 * every split weight and merge factor with, exposed so that a CPU emulation
 * of that order can use the hardware's values. */
int bi_exp2_f32(const float* x, float* y, int64_t n, void* stream);

/* Diagnostic, no counterpart in the reference: one pass over `bytes` (a
 * multiple of 16, 16-byte aligned) of device memory at src in one launch,
 * every wave reading whole 1 KB chunks; writes sink[0] only in the unlikely
 * case that a thread's xor of its data equals magic. The achievable-bandwidth
 * reference for the HBM-bound kernels (same bytes, one launch). */
int bi_stream_read(const void* src, int64_t bytes, uint32_t* sink, uint32_t magic, void* stream);

/* Diagnostic, no counterpart in the reference: one matrix-core step of the
 * matmul kernels per block, on caller-chosen operands and accumulator. Block
 * i: a, b [16][32] elements of dtype (row r, k-slot j; slot 8 q + e is what
 * lane quarter q holds as its element e), c, d [16][16] fp32 (row, column):
 *   d = c + A B^T by one v_mfma_f32_16x16x32_{bf16,f16}, or for fp32 by the
 *   kernels' eight v_mfma_f32_16x16x4_f32 (element e of every quarter in
 *   sub-step e).
 * nblocks in [0, 2^24]; a and b 16-byte aligned; device pointers, on the
 * stream. It isolates the instruction whose accumulation the oracle models,
 * independent of any matmul kernel's data movement. */
int bi_mfma_step_probe(const void* a, const void* b, const float* c, float* d, int64_t nblocks, int dtype,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* BI_KERNELS_H */
