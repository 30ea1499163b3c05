/*
 * void_amd.h — C ABI of the MI355X (gfx950) quantized block-sparse SpMM library.
 *
 * The library replaces the Triton launches of the reference's quantized SpMM
 * path.  Every entry point takes plain device pointers and sizes, launches
 * asynchronously on the caller's HIP stream, never allocates or frees device
 * memory, and returns 0 on success or a negative void_status code (the text
 * of the last error is available from void_last_error()).
 *
 * Sparse operand A ("BSR view" of a VOID tensor): 32x32 tiles stored
 * block-row-major — tiles of block-row r occupy [row_ptr[r], row_ptr[r+1])
 * with ascending block column — so that a workgroup streams one block-row's
 * tiles from contiguous HBM.  This is the order the reference visits tiles
 * in (Int8VOIDTensor.get_row_block_info, void/int_quant.py:158-175), with the
 * block_indices indirection resolved once at conversion time.
 *
 * Dense operand B is int8 (INT8 path) or fp8 E4M3FN (FP8 path), K x N,
 * either row-major (element (k,n) at b[k*ldb+n], the reference's layout) or
 * column-major (element (k,n) at b[n*ldb+k]).
 */
#ifndef VOID_AMD_H
#define VOID_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VOID_AMD_ABI_VERSION 5
#define VOID_TILE 32

typedef enum void_status {
  VOID_OK = 0,
  VOID_ERR_ARG = -1,         /* null pointer, negative size, shape mismatch */
  VOID_ERR_UNSUPPORTED = -2, /* combination not implemented (e.g. row_mean on fp8) */
  VOID_ERR_HIP = -3,         /* a HIP runtime call failed */
  VOID_ERR_WORKSPACE = -4,   /* workspace missing or too small for the plan */
  VOID_ERR_CAPACITY = -5     /* planner output array too small */
} void_status;

/* Epilogue applied to the int32 / fp32 accumulators of one 32 x N tile. */
typedef enum void_epilogue {
  /* int32 accumulators of the whole block-row, stored raw (out_dtype must be I32). */
  VOID_EPI_RAW_I32 = 0,
  /* Reference semantics of void_spmm_int8_kernel (void/int_quant.py:519-526):
   *   S = sequential fp32 sum over the row's tiles (ascending column) of fl(s_a[t] * s_b)
   *   C = f32(acc_i32) * (S / n_tiles_in_row), 0 for an empty row. */
  VOID_EPI_ROW_MEAN = 1,
  /* True per-tile dequantisation: C = s_b * sum_t s_a[t] * f32(A_t @ B_t). */
  VOID_EPI_PER_BLOCK = 2
} void_epilogue;

typedef enum void_dtype {
  VOID_DT_F32 = 0,
  VOID_DT_BF16 = 1,
  VOID_DT_F16 = 2,
  VOID_DT_I32 = 3
} void_dtype;

/* Activation codes follow get_activation_code (void/fusion.py:77-91). */
typedef enum void_activation {
  VOID_ACT_NONE = 0,
  VOID_ACT_RELU = 1,
  VOID_ACT_GELU = 2, /* tanh form, void/fusion.py:38-43 */
  VOID_ACT_SILU = 3
} void_activation;

/* Device view of a quantized VOID tensor (Int8VOIDTensor / FP8VOIDTensor). */
typedef struct void_bsr_desc {
  const void* tiles;      /* [n_blocks][32][32] int8 or e4m3fn bytes, block-row-major */
  const float* scales;    /* [n_blocks] per-tile scale (same order), or [1] if per_tensor_a */
  const int32_t* row_ptr; /* [n_block_rows + 1] */
  const int32_t* col_idx; /* [n_blocks] block column of each tile */
  int32_t M, K;           /* dense shape of A */
  int32_t n_blocks;
  int32_t n_block_rows;   /* ceil(M / 32) */
  int32_t per_tensor_a;   /* 1: scales[0] applies to every tile */
  int32_t reserved;
} void_bsr_desc;

#define VOID_ITEM_INLINE_COLS 24

/* One unit of work: tiles [begin, end) of block-row `row`.  A row with more
 * tiles than the plan's chunk size is split into `nchunks` items that each
 * write a partial tile into workspace slot (slot + chunk); the last of them
 * to finish (counted on split tile `tile`) reduces the partials in chunk
 * order and applies the epilogue.  tile == -1 marks an unsplit row.
 * cols[] repeats the block columns of the item's first 24 tiles so that a
 * workgroup reads its first B addresses together with the item (128 bytes,
 * one scalar load burst) instead of after it.
 * Replaces StreamKWorkload (void/stream_k.py:13-33). */
typedef struct void_work_item {
  int32_t row, begin, end, tile;
  int32_t nchunks, chunk, slot, reserved;
  int32_t cols[VOID_ITEM_INLINE_COLS];
} void_work_item;

/* A plan from void_streamk_plan with its items copied to device memory. */
typedef struct void_plan {
  const void_work_item* items; /* device array of n_items entries */
  int32_t n_items;
  int32_t n_split_tiles;
  int32_t n_slots;
  int32_t chunk_tiles;
} void_plan;

/* The dense operand and the output of one SpMM call. */
typedef struct void_dense_args {
  const void* b;          /* K x N: int8 (void_spmm_int8), e4m3fn (void_spmm_fp8), fp32 (void_spmm_f32) */
  int64_t ldb;            /* elements between consecutive rows (row-major) or columns (column-major) */
  int32_t b_col_major;    /* 0: (k,n) at b[k*ldb+n]; 1: (k,n) at b[n*ldb+k] */
  int32_t N;
  float b_scale;          /* per-tensor scale of B, used when b_scale_vec is NULL */
  const float* b_scale_vec; /* [N] per-column scale of B, or NULL */
  const float* bias;      /* [N] added before the activation, or NULL */
  void* c;                /* M x N row-major output */
  int64_t ldc;
  int32_t out_dtype;      /* void_dtype */
  int32_t activation;     /* void_activation */
  int32_t bias_per_row;   /* 0: bias[N] per column; 1: bias[M] per output row (the reference's
                             row-bias kernel, void/fusion.py:202-304; float SpMM only) */
  int32_t reserved;       /* 0 */
} void_dense_args;

/* ---------------------------------------------------------------------- */

/* ABI version (VOID_AMD_ABI_VERSION) of the loaded library. */
int void_abi_version(void);

/* Text of the last error reported on the calling thread ("" if none). */
const char* void_last_error(void);

/* Width in columns of the N panel one workgroup computes (128). */
int void_panel_width(void);

/* Properties of the current device that the roofline peaks are derived from:
 * compute units, peak engine clock (kHz), peak memory clock (kHz) and memory
 * bus width (bits).  No counterpart in the reference; used by bench.py to
 * state the peaks it divides by.  Returns VOID_OK or VOID_ERR_HIP. */
int void_device_info(int32_t* compute_units, int32_t* sclk_khz, int32_t* mclk_khz, int32_t* bus_bits);

/* The id of the HIP graph capture that `stream` is in, or 0 when it is not
 * capturing (hipStreamGetCaptureInfo).  No counterpart in the reference; the
 * Python layer uses it to give the launches of one capture on one stream a
 * single split-row workspace.  Returns VOID_OK or VOID_ERR_HIP. */
int void_stream_capture_id(hipStream_t stream, unsigned long long* id);

/* Host-side Stream-K planner.  Replaces compute_stream_k_workload
 * (void/stream_k.py:36-110): every block-row becomes one item, except rows
 * with more than chunk_tiles tiles, which are split into ceil(n/chunk_tiles)
 * near-equal chunks.  Items are ordered longest-first (when rows were
 * split, the SpMM kernels deal the list round-robin among the XCDs that
 * share a panel group, so that each XCD runs a balanced mix), and empty
 * rows are kept (they produce the zero / activation(bias) rows of C).
 * row_ptr (n_block_rows + 1 entries) and col_idx (row_ptr[n_block_rows]
 * entries, or NULL to leave cols[] at -1) are HOST arrays.
 * On VOID_ERR_CAPACITY, *n_items holds the required capacity. */
int void_streamk_plan(const int32_t* row_ptr, const int32_t* col_idx, int32_t n_block_rows,
                      int32_t chunk_tiles, void_work_item* items, int32_t capacity,
                      int32_t* n_items, int32_t* n_split_tiles, int32_t* n_slots);

/* Bytes of device workspace a plan needs for N output columns (0 if the plan
 * splits no row).  The first n_split_tiles * n_panels int32 counters of the
 * workspace must be zero before the first launch; every launch leaves them
 * zero again.  Calls that share one workspace must not overlap in time. */
size_t void_workspace_bytes(int32_t n_split_tiles, int32_t n_slots, int32_t N);

/* INT8 block-sparse SpMM, replacing void_spmm_int8_kernel + void_spmm_int8
 * (void/int_quant.py:435-612) and, with activation != NONE, the INT8 form of
 * void_spmm_activation_kernel (void/fusion.py:98-198).
 * epilogue: void_epilogue; RAW_I32 requires out_dtype == I32.
 * workspace: void_workspace_bytes(plan) bytes, NULL when the plan splits no row. */
int void_spmm_int8(const void_bsr_desc* a, const void_dense_args* d, int32_t epilogue,
                   const void_plan* plan, void* workspace, size_t workspace_bytes,
                   hipStream_t stream);

/* void_spmm_int8 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  It
 * calls no hipMalloc, hipFree or allocating library routine: the split-row
 * counters and partial blocks live in a static device array of the library
 * (32 MiB per GPU, held from module load to process end).  A plan may need
 * at most VOID_NOALLOC_COUNTER_BYTES of counters (counters_bytes: n_split_tiles
 * x ceil(N / 128) x 4, rounded up to 256) and VOID_NOALLOC_PARTIAL_BYTES of
 * partials (void_workspace_bytes minus the counters); larger plans fail with
 * VOID_ERR_WORKSPACE.  The first call on a device that splits rows looks the
 * array up and clears its counters with a kernel on `stream`.  All calls on
 * one GPU share the array: calls that overlap in time on one GPU race (run
 * them on one stream, or use void_spmm_int8 with a workspace per stream).
 * Results are identical to void_spmm_int8's. */
#define VOID_NOALLOC_COUNTER_BYTES ((size_t)1 << 20)
#define VOID_NOALLOC_PARTIAL_BYTES (((size_t)31) << 20)
int void_spmm_int8_noalloc(const void_bsr_desc* a, const void_dense_args* d, int32_t epilogue,
                           const void_plan* plan, hipStream_t stream);

/* FP8 (E4M3FN x E4M3FN, fp32 accumulate) block-sparse SpMM, replacing
 * void_spmm_fp8_kernel + void_spmm_fp8 (void/fp8.py:577-742).  The epilogue
 * is always PER_BLOCK: C = s_b * sum_t s_a[t] * (A_t @ B_t). */
int void_spmm_fp8(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);

/* FP8 SpMM with a float B, as the reference computes it when B is not FP8:
 * C = sum_t s_a[t] * dec(A_t) @ B with B in fp32 (void_spmm_fp8_kernel and
 * void_spmm_fp8, void/fp8.py:577-742, whose kernel upcasts both operands to
 * fp32).  a->tiles holds E4M3FN tiles with per-tile (or per-tensor) scales;
 * d->b is fp32, row-major, with 16-byte aligned rows and N % 4 == 0; the
 * plan's items have at most 64 tiles.  The E4M3 codes are decoded exactly
 * to bf16 and each B value is split into bf16 hi + lo on the bf16 MFMA, so
 * every product is within 2^-16 relative of the exact one (fp32
 * accumulation).  d->b_scale / b_scale_vec multiply the result (1.0 gives
 * the reference's semantics); out_dtype f32, bf16 or f16; workspace as for
 * void_spmm_int8. */
int void_spmm_fp8_f32b(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                       void* workspace, size_t workspace_bytes, hipStream_t stream);

/* The same for a 16-bit B: d->b holds bf16 (b_dtype VOID_DT_BF16) or fp16
 * (VOID_DT_F16) values, which the reference's upcast (void/fp8.py:624-671)
 * takes as they are.  The E4M3 tiles are decoded exactly to B's type and
 * multiplied on the 16-bit MFMA (exact products, fp32 accumulation), each
 * tile's product scaled into the sum.  B and C row-major with 16-byte
 * aligned rows and N % 8 == 0 (else VOID_ERR_UNSUPPORTED); plan items of at
 * most 64 tiles. */
int void_spmm_fp8_b16(const void_bsr_desc* a, const void_dense_args* d, int32_t b_dtype, const void_plan* plan,
                      void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Float SpMM: fp32 tiles times fp32 B on the fp32 MFMA (exact products,
 * fp32 accumulation), then bias, activation and conversion to d->out_dtype
 * (f32, bf16 or f16).  Replaces void_spmm_kernel + void_spmm
 * (void/ops.py:148-213) and, with d->activation / d->bias set,
 * void_spmm_activation_kernel (void/fusion.py:98-198) for float VOID
 * tensors.  a->tiles holds fp32 tiles; a->scales, d->b_scale and
 * d->b_scale_vec are not used.  B row-major; plan items of at most 64
 * tiles (plan->chunk_tiles <= 64); workspace as for void_spmm_int8. */
int void_spmm_f32(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Float SpMM on 16-bit tensors: bf16 tiles times bf16 B (void_spmm_bf16) or
 * fp16 tiles times fp16 B (void_spmm_f16) on the 16-bit MFMA (exact
 * products, fp32 accumulation), then bias, activation and conversion to
 * d->out_dtype (f32, bf16 or f16).  Replaces void_spmm_kernel + void_spmm
 * (void/ops.py:148-213, whose tl.dot takes 16-bit operands as they are) and
 * void_spmm_activation_kernel (void/fusion.py:98-198) for VOID tensors
 * whose values and B share a 16-bit dtype.  a->tiles holds 16-bit tiles
 * (2048 bytes each); scales unused.  B and C row-major with 16-byte aligned
 * rows, N % 8 == 0 (else VOID_ERR_UNSUPPORTED); plan items of at most 64
 * tiles; workspace as for void_spmm_int8. */
int void_spmm_bf16(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                   void* workspace, size_t workspace_bytes, hipStream_t stream);
int void_spmm_f16(const void_bsr_desc* a, const void_dense_args* d, const void_plan* plan,
                  void* workspace, size_t workspace_bytes, hipStream_t stream);

/* Per-tensor symmetric INT8 quantisation of n contiguous floats b (a float
 * B operand), as quantize_tensor (void/int_quant.py:254-325) with qmin =
 * -128, qmax = 127: *scale = max(max|b| / 128, 1e-8), q = clamp(rint(b /
 * scale), -128, 127).  The scale stays in device memory (the reference reads
 * it back to the host).  partials: device workspace of 1024 uint32.  b
 * 16-byte aligned, q 4-byte aligned. */
int void_quantize_b_i8(const float* b, int64_t n, int8_t* q, float* scale, uint32_t* partials,
                       hipStream_t stream);

/* dst[c * ld_dst + r] = src[r * ld_src + c] for a rows x cols byte matrix:
 * a column-major int8 or E4M3 B (src: its N columns of K bytes, ld_src
 * between columns; rows = N, cols = K) made row-major (dst: K x N,
 * ld_dst >= N) for the LDS-DMA ring, which reads B slabs in whole lines.
 * rows, cols, ld_src and ld_dst multiples of 16, 16-byte aligned arrays.  No
 * counterpart in the reference (its kernels take B's strides as given). */
int void_transpose_b8(const void* src, int64_t ld_src, int32_t rows, int32_t cols, void* dst, int64_t ld_dst,
                      hipStream_t stream);

/* ---- Quantisers on the path's input side (one wave per tile) ---------- */

/* Per-tile symmetric INT8 of n_tiles fp32 32x32 tiles (tile t at
 * tiles[1024 t], row-major): s_t = max(max|x| / 128, 1e-8),
 * q = clamp(round_half_even(x / s_t), -128, 127), bit-identical to the
 * reference's per-block loop (void/int_quant.py:178-214, 254-305, 363-369
 * under quantize_void_tensor, :328-388).  tiles and q 16-byte aligned;
 * q[1024 n_tiles], scales[n_tiles]. */
int void_quantize_tiles_i8(const float* tiles, int32_t n_tiles, int8_t* q, float* scales, hipStream_t stream);

/* Per-tile E4M3FN with the reference's first-call scaling: s_t =
 * max(max|x| / 448, 1e-12), code = e4m3_rne(clamp(x * (1 / s_t), +-448)),
 * bit-identical to void/fp8.py:81-105 and 185-229 as used by
 * void_tensor_to_fp8 (:749-766, per_block).  Same layout as above; amax
 * (nullable, n_tiles floats) receives max|x| of every tile, the value the
 * reference records in its amax history. */
int void_quantize_tiles_fp8(const float* tiles, int32_t n_tiles, uint8_t* q, float* scales, float* amax,
                            hipStream_t stream);

/* ---- CSR -> VOID tiles on the device (csr_to_void, void/format.py:248-349) --
 * Canonical CSR (int32 indptr[M+1] and column indices, no duplicate
 * entries; float32 values; indices and values 16-byte aligned) becomes Morton-ordered 32x32 fp32 tiles, block
 * rows, block columns and Morton codes, the reference's VOIDTensor fields.
 * Explicit zeros activate their tile, as in the reference.  Two calls:
 * void_csr_count_blocks flags the active blocks, ranks them in Morton order
 * and writes their number to *n_blocks (a device int64); the caller sizes the
 * outputs from it (the tile array 16-byte aligned), then void_csr_to_tiles
 * fills them.  Both use the same workspace of void_csr_workspace_bytes(M, N)
 * bytes, which carries the flags and ranks from the first call to the second
 * (0 when the block grid is too large for the device conversion: more than
 * 2^28 blocks). */
size_t void_csr_workspace_bytes(int32_t M, int32_t N);
int void_csr_count_blocks(const int32_t* indptr, const int32_t* indices, int32_t M, int32_t N, void* workspace,
                          size_t workspace_bytes, int64_t* n_blocks, hipStream_t stream);
int void_csr_to_tiles(const int32_t* indptr, const int32_t* indices, const float* data, int32_t M, int32_t N,
                      void* workspace, size_t workspace_bytes, int64_t n_blocks, float* values,
                      int32_t* block_rows, int32_t* block_cols, int64_t* morton, hipStream_t stream);

/* ---- Backward: gradient on the nonzero tiles (SDDMM) ------------------ */

/* grad_tiles[t] = grad_c[32 br .. +32, :] @ b[32 bc .. +32, :]^T for every
 * tile t = (block_rows[t], block_cols[t]) (any order), fp32 products and
 * accumulation, written as out_dtype (f32, bf16, f16) into [n_blocks, 32, 32].
 * grad_c is M x N row-major (leading dimension ldg), b is K x N row-major
 * (ldb); rows past M / K and columns past N count as zero.  Replaces
 * void_spmm_backward_a_kernel (void/autograd.py:14-97). */
int void_sddmm_f32(const float* grad_c, int64_t ldg, const float* b, int64_t ldb, const int32_t* block_rows,
                   const int32_t* block_cols, int32_t n_blocks, int32_t M, int32_t N, int32_t K, void* grad_tiles,
                   int32_t out_dtype, hipStream_t stream);

/* The same gradient with the tiles grouped by block-row, as the SpMM's BSR
 * order gives them: groups[3 g .. 3 g + 2] = (block row, first BSR position,
 * tile count <= 8) for n_groups groups, col_idx[k] the block column of BSR
 * position k, and the gradient of position k written to tile
 * tile_index[k] of grad_tiles (or tile k when tile_index is null).  Tiles of
 * one group share one read of their grad_c rows.  Same operand rules as
 * void_sddmm_f32; also replaces void_spmm_backward_a_kernel
 * (void/autograd.py:14-97). */
int void_sddmm_rows_f32(const float* grad_c, int64_t ldg, const float* b, int64_t ldb, const int32_t* groups,
                        int32_t n_groups, const int32_t* col_idx, const int64_t* tile_index, int32_t M, int32_t N,
                        int32_t K, void* grad_tiles, int32_t out_dtype, hipStream_t stream);

/* void_sddmm_rows_f32 for 16-bit grad_c and b of one dtype (bf16 or fp16),
 * the backward of a VOID tensor in that dtype: products of the 16-bit values
 * on the 16-bit MFMA (exact in fp32), fp32 accumulation, written as
 * out_dtype.  Needs 16-byte aligned operands with ldg, ldb and N multiples
 * of 8 (else VOID_ERR_UNSUPPORTED).  Replaces void_spmm_backward_a_kernel
 * (void/autograd.py:14-97), whose tl.dot takes 16-bit operands as they are. */
int void_sddmm_rows_bf16(const void* grad_c, int64_t ldg, const void* b, int64_t ldb, const int32_t* groups,
                         int32_t n_groups, const int32_t* col_idx, const int64_t* tile_index, int32_t M, int32_t N,
                         int32_t K, void* grad_tiles, int32_t out_dtype, hipStream_t stream);
int void_sddmm_rows_f16(const void* grad_c, int64_t ldg, const void* b, int64_t ldb, const int32_t* groups,
                        int32_t n_groups, const int32_t* col_idx, const int64_t* tile_index, int32_t M, int32_t N,
                        int32_t K, void* grad_tiles, int32_t out_dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* VOID_AMD_H */
