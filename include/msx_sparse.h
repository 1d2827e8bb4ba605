/*
 * msx_sparse.h - C ABI of the MI355X (gfx950) CSR sparse x dense library.
 *
 * This is the drop-in boundary for mlx-sparse's sparse x dense hot path:
 * CSR SpMV (y = A x) and CSR SpMM with a dense row-major right-hand side
 * (Y = A X).  Every entry point takes plain pointers and sizes; no C++ or
 * framework type crosses it.
 *
 * Conventions
 *   - The caller owns every buffer.  Outputs (y / Y) are allocated by the
 *     caller; the library only writes them.  Plans are the one object the
 *     library allocates (device memory for row blocks), released by
 *     msx_csr_plan_destroy.
 *   - GPU entry points are asynchronous and ordered on the HIP stream passed
 *     as `stream` (a hipStream_t; NULL means the default stream).  They
 *     return after the launch, not after completion.  Calls on different
 *     streams may run concurrently, except calls that share one plan (see
 *     msx_csr_plan_create).
 *   - Errors are status codes; msx_last_error() returns a thread-local text
 *     for the last failing call on the calling thread.  The texts for shape
 *     and dtype problems follow the reference validators
 *     (reference: src/common/common.cpp:104-177).
 *   - `indices` and `indptr` share one index type; `data`, `x`/`X` and
 *     `y`/`Y` share one value type (reference: src/common/common.cpp:146-168).
 *   - Sizes are int64_t, but n_rows, n_cols and k must be below 2^31, as in
 *     the reference, whose shapes are `int` (reference:
 *     src/sparse/csr_matvec/csr_matvec.h:25-27).
 *   - Arithmetic: float16/bfloat16 operands are widened to float32,
 *     multiplied and summed in float32, and rounded once to the storage type
 *     (round to nearest even).  float32 sums in float32; complex64 sums in
 *     complex64 with the textbook product.  Products and sums are rounded
 *     separately (no fused multiply-add), as in the reference CPU kernels
 *     (reference: src/common/common.h:52-79).
 */
#ifndef MSX_SPARSE_H
#define MSX_SPARSE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSX_ABI_VERSION 7

typedef enum msx_vtype {
  MSX_F32 = 0,  /* float32 */
  MSX_F16 = 1,  /* IEEE binary16, passed as raw 16-bit storage */
  MSX_BF16 = 2, /* bfloat16, passed as raw 16-bit storage */
  MSX_C64 = 3   /* complex64: interleaved (real, imag) float32 pairs */
} msx_vtype;

typedef enum msx_itype {
  MSX_I32 = 0, /* int32 indices / indptr */
  MSX_I64 = 1  /* int64 indices / indptr */
} msx_itype;

typedef enum msx_status {
  MSX_OK = 0,
  MSX_EINVAL = 1, /* bad shape, size, pointer or plan (ValueError) */
  MSX_ETYPE = 2,  /* unsupported or mismatched dtype (TypeError) */
  MSX_EHIP = 3,   /* a HIP runtime call failed (RuntimeError) */
  MSX_ENOMEM = 4  /* device or host allocation failed (MemoryError) */
} msx_status;

/* Opaque row-block plan built from `indptr` on the device. */
typedef struct msx_csr_plan msx_csr_plan;

/* Column slicing of a bound plan (msx_csr_plan_create_bound). */
typedef enum msx_slice_mode {
  MSX_SLICE_AUTO = 0,  /* when x exceeds 8 MB and most blocks' columns span
                          over a quarter of the columns: panels if the matrix
                          qualifies and its short rows hold at least 65536
                          values per compute unit, else XCD slices if x is
                          16 MB or more, else row blocks */
  MSX_SLICE_OFF = 1,   /* row blocks only */
  MSX_SLICE_ON = 2,    /* XCD column slices */
  MSX_SLICE_PANELS = 3 /* LDS column panels (two-pass SpMV) */
} msx_slice_mode;

typedef struct msx_plan_options {
  int64_t block_nnz;  /* W: 0 = default (512 when rows average 20 or more
                         values and the values are not complex64, else 256),
                         else a power of two in [64, 1024] */
  int32_t slice_mode; /* msx_slice_mode */
  int32_t reserved;   /* must be 0 */
} msx_plan_options;

/* Summary of a plan, for callers that report or test it. */
typedef struct msx_plan_info {
  int64_t n_rows;
  int64_t nnz;
  int64_t block_nnz;   /* W: a short block holds rows whose starts fall in one
                          W-wide window of the nnz range; rows with more than
                          W stored values are "long" */
  int64_t block_rows;  /* R: a short block never crosses a multiple of R rows */
  int64_t chunk_nnz;   /* C: long rows are split into chunks of C values */
  int64_t n_blocks;    /* short blocks */
  int64_t n_bounds;    /* entries of the bounds list: short blocks + long rows */
  int64_t n_long_rows; /* rows with more than W stored values */
  int64_t n_chunks;    /* total chunks over all long rows */
  int64_t device;      /* HIP device ordinal the plan lives on */
  int64_t plan_bytes;  /* device bytes held by the plan */
  int64_t n_slices;    /* 0, or 8 when the plan holds a column-sliced copy */
  int64_t slice_width; /* columns per slice */
  int64_t slice_bytes; /* device bytes of the sliced copy and its partial sums */
  int64_t n_panels;    /* 0, or the number of LDS column panels */
  int64_t panel_width; /* columns per panel */
  int64_t n_tiles;     /* row tiles of a panel plan */
  int64_t panel_values;/* entries of the panel copy: values of short rows with valid
                          columns, each (panel, tile) segment padded to a
                          multiple of 4 */
  int64_t panel_bytes; /* device bytes of the panel copy and its product buffer */
  int64_t window_rows; /* bound plans: the widest column window (in rows of X)
                          of the plan's 64-row tiles, 0 when none; SpMM
                          stages each tile's window of X in LDS when it fits */
} msx_plan_info;

/* ABI version of the loaded library (MSX_ABI_VERSION at build time). */
int msx_abi_version(void);

/* Thread-local text of the last error on this thread ("" if none). */
const char *msx_last_error(void);

/* Number of HIP devices visible to the library (0 when none). */
msx_status msx_device_count(int *count);

/*
 * Build a row-block plan from a device-resident `indptr` (n_rows + 1
 * entries of type `it`) on `stream`.  The plan splits the rows into short
 * blocks (consecutive rows processed by one wavefront) and long rows (split
 * into chunks processed by whole workgroups, then summed in chunk order).
 * Synchronises `stream` once to read the block counts.  `block_nnz` selects
 * W (0 = library default: 512 when nnz >= 20 * n_rows, else 256; otherwise
 * a power of two in [64, 1024]).
 * The plan holds scratch for long-row chunk sums: calls sharing one plan
 * must be ordered (one stream) - concurrent calls on a shared plan race.
 *
 * Replaces the reference's per-launch kernel choice `nnz >= 32 * n_rows`
 * (reference: src/sparse/csr_matvec/csr_matvec.cpp:291-296), which has no
 * persistent object; the reference container is immutable
 * (reference: mlx_sparse/_csr.py:33), so a plan may be cached with it.
 */
msx_status msx_csr_plan_create(msx_itype it, int64_t n_rows, int64_t nnz,
                               const void *indptr, int64_t block_nnz,
                               void *stream, msx_csr_plan **out);

/*
 * Build a plan bound to one matrix's values (`data`, `indices`, `indptr`,
 * all device pointers) on `stream`: the row blocks of msx_csr_plan_create,
 * plus, for scattered gathers, one of two reordered copies of the short
 * rows' values (`opts->slice_mode`; AUTO picks as described at
 * MSX_SLICE_AUTO):
 *   XCD slices - the values of each 256-row block reordered into 8 column
 *     slices; slice s runs on the workgroups the hardware places on XCD s,
 *     so each XCD gathers from one eighth of x, which stays in its L2;
 *     per-slice row sums are added in slice order.
 *   panels - x cut into panels of 128 KB (32768 float32/float16/bfloat16
 *     or 16384 complex64 entries) and the rows into tiles of at most 64 KB
 *     of products plus one word per row.  Pass 1 holds one panel of x in LDS
 *     and streams that panel's values, writing their products; pass 2 loads
 *     one tile's products into LDS by stored position and sums each row in
 *     stored order, so short rows equal the reference CPU kernel bit for bit.
 *     Needs nnz < 2^31 and at most 2048 panels; MSX_SLICE_PANELS on a matrix
 *     outside those limits fails with MSX_EINVAL.
 * Long rows keep the row-block path in every mode.  When x is at least
 * 4 MB and every long row holds sorted columns, the plan also records each
 * long row's 8 column-slice stretches (pieces of at most 1020 values): the
 * pieces of slice s are summed on XCD s, in the same launch as the short
 * blocks, and a fixed-order tree adds a row's pieces.  Every bound plan
 * also records the column window of each 32-row tile (see msx_csr_spmm).
 * `opts` may be NULL (defaults).  Synchronises `stream`.
 *
 * A bound plan reads the matrix from its own copy: msx_csr_spmv must be
 * given the same data/indices/indptr pointers it was built from (other
 * pointers are rejected with MSX_EINVAL).  When the values change, call
 * msx_csr_plan_refresh before the next product; when indices or indptr
 * change, build a new plan.  Replaces, like msx_csr_plan_create, the
 * reference's per-launch kernel choice (reference:
 * src/sparse/csr_matvec/csr_matvec.cpp:291-296).
 */
msx_status msx_csr_plan_create_bound(msx_vtype vt, msx_itype it,
                                     int64_t n_rows, int64_t n_cols,
                                     int64_t nnz, const void *data,
                                     const void *indices, const void *indptr,
                                     const msx_plan_options *opts,
                                     void *stream, msx_csr_plan **out);

/*
 * The values of a bound plan's matrix changed (in place, or copied to a new
 * buffer `data`), its indices and indptr did not: rewrite the plan's own
 * copies of the values (the XCD-sliced or panel copy) from `data` on
 * `stream`, asynchronously, and bind the plan to `data` from now on.  A
 * gather through the layout the plan already holds: O(nnz), no allocation
 * and no re-sort (the headline matrix: one pass over its values instead of
 * the 20 ms build).  Row-block plans hold no values: a no-op.  Calls that
 * share the plan must be ordered after this one (same stream).
 *
 * No reference counterpart: the reference's arrays are immutable
 * (reference: mlx_sparse/_csr.py:33), so its kernels always read the
 * current values; torch tensors are not, and this keeps a cached plan right
 * after an optimizer updates the values in place.
 */
msx_status msx_csr_plan_refresh(msx_csr_plan *plan, const void *data,
                                void *stream);

/* Release a plan (NULL is accepted).  Synchronises the plan's device. */
msx_status msx_csr_plan_destroy(msx_csr_plan *plan);

/* Fill `info` from a plan. */
msx_status msx_csr_plan_info(const msx_csr_plan *plan, msx_plan_info *info);

/*
 * Copy a plan's index arrays to host memory (synchronous), for bit-exact
 * checks of the binning.  Each pointer may be NULL to skip that array.
 *   bounds:          n_bounds + 1 int64: in row order, each row that starts a
 *                    short block or is long, long rows with bit 31 set
 *                    (value row | 2^31), then a sentinel equal to n_rows.  A
 *                    short block spans its entry up to the next entry;
 *   long_rows:       n_long_rows int64 (row ids, ascending);
 *   long_chunk_begin: n_long_rows + 1 int64 (first chunk of each long row,
 *                    then n_chunks).
 */
msx_status msx_csr_plan_export(const msx_csr_plan *plan,
                               int64_t *bounds, int64_t *long_rows,
                               int64_t *long_chunk_begin);

/*
 * Copy a panel plan's layout to host memory (synchronous), for bit-exact
 * checks.  Each pointer may be NULL to skip that array.
 *   tile_begin, tile_end: n_tiles int64 - tile t holds rows
 *                    [tile_begin[t], tile_end[t]), all short; a short row
 *                    starts a tile at r = 0, after a long row, or when
 *                    (indptr[r] + r) / H changes (indptr clamped to
 *                    [0, nnz]), H = 16384 - W (float32, float16, bfloat16)
 *                    or 8192 - W (complex64);
 *   seg_begin:       n_panels * n_tiles + 1 int64 - start of segment
 *                    (panel p, tile t) at index p * n_tiles + t of the
 *                    panel copy, whose values are ordered by (panel, tile,
 *                    stored position), each segment padded to a multiple
 *                    of 4 entries; the last entry is panel_values.
 * MSX_EINVAL when the plan has no panels.  No reference counterpart: a
 * layout check of this library's own plans.
 */
msx_status msx_csr_plan_export_panels(const msx_csr_plan *plan,
                                      int64_t *tile_begin, int64_t *tile_end,
                                      int64_t *seg_begin);

/*
 * y[i] = sum_{p = indptr[i]}^{indptr[i+1]-1} data[p] * x[indices[p]]
 * for i in [0, n_rows).  All pointers are device pointers.  `plan` may be
 * NULL (a plan-free kernel sized from nnz / n_rows is used); a non-NULL plan
 * must have been built from this `indptr` buffer (the same pointer; another
 * buffer is rejected with MSX_EINVAL, whatever it holds).
 *
 * Replaces CSRMatVec::eval_gpu (reference:
 * src/sparse/csr_matvec/csr_matvec.cpp:278-317) and the Metal kernels
 * csr_matvec_* / csr_matvec_vector_* (reference:
 * src/sparse/csr_matvec/csr_matvec.metal:17-123).
 */
msx_status msx_csr_spmv(msx_vtype vt, msx_itype it, int64_t n_rows,
                        int64_t n_cols, int64_t nnz, const void *data,
                        const void *indices, const void *indptr,
                        const void *x, void *y, const msx_csr_plan *plan,
                        void *stream);

/*
 * Y[i, c] = sum_p data[p] * X[indices[p], c] for c in [0, k), with X an
 * n_cols x k row-major matrix of leading dimension ldx (>= k) and Y an
 * n_rows x k row-major matrix of leading dimension ldy (>= k).  Device
 * pointers.  `plan` may be NULL; a bound plan of the matrix lets the SpMM
 * stage each 64-row tile's column window of X in LDS when every window fits
 * (banded matrices), reading X from HBM about once.
 *
 * Replaces CSRMatMul::eval_gpu (reference:
 * src/sparse/csr_matmul/csr_matmul.cpp:260-300) and the Metal kernels
 * csr_matmul_* (reference: src/sparse/csr_matmul/csr_matmul.metal:17-135).
 */
msx_status msx_csr_spmm(msx_vtype vt, msx_itype it, int64_t n_rows,
                        int64_t n_cols, int64_t nnz, const void *data,
                        const void *indices, const void *indptr, int64_t k,
                        const void *X, int64_t ldx, void *Y, int64_t ldy,
                        const msx_csr_plan *plan, void *stream);

/*
 * Batched SpMV on the device: Y[b, :] = A X[b, :] for b < batch, X a
 * batch x n_cols matrix with row stride ldx, Y batch x n_rows with row stride
 * ldy (elements).  Each output is summed from zero in stored order, so
 * float32 results equal the reference's batched CPU kernel bit for bit.  The
 * vectors are transposed into one n_cols x batch operand and multiplied by
 * one SpMM (the matrix is read once), through scratch taken from the
 * stream-ordered allocator of `stream`.
 *
 * Replaces CSRBatchedMatVec::eval_gpu (reference:
 * src/sparse/csr_batched_matvec/csr_batched_matvec.cpp:186-226).
 */
msx_status msx_csr_batched_spmv(msx_vtype vt, msx_itype it, int64_t n_rows,
                                int64_t n_cols, int64_t nnz, const void *data,
                                const void *indices, const void *indptr,
                                int64_t batch, const void *X, int64_t ldx,
                                void *Y, int64_t ldy, void *stream);

/*
 * Batched SpMM on the device: Y[b] = A X[b] for b < batch.  X[b] starts at
 * X + b * x_batch (row-major n_cols x k, row stride ldx), Y[b] at
 * Y + b * y_batch (n_rows x k, row stride ldy); strides in elements.  Summed
 * like msx_csr_spmm.  No scratch.
 *
 * Replaces CSRBatchedMatMul::eval_gpu (reference:
 * src/sparse/csr_batched_matmul/csr_batched_matmul.cpp).
 */
msx_status msx_csr_batched_spmm(msx_vtype vt, msx_itype it, int64_t n_rows,
                                int64_t n_cols, int64_t nnz, const void *data,
                                const void *indices, const void *indptr,
                                int64_t batch, int64_t k, const void *X,
                                int64_t x_batch, int64_t ldx, void *Y,
                                int64_t y_batch, int64_t ldy, void *stream);

/*
 * CSR of A^T (shape n_cols x n_rows, the CSC of A) into caller buffers:
 * t_data and t_indices (nnz entries; t_indices holds row ids) and t_indptr
 * (n_cols + 1).  Each column lists its entries by increasing row, as the
 * reference's counting sort does.  Values with a column outside [0, n_cols)
 * are left out: t_indptr[n_cols] counts the rest, and entries past it are
 * unspecified.  Device: a stable radix sort, asynchronous on `stream`
 * (scratch from its stream-ordered allocator); nnz < 2^31 - 1.
 *
 * Replaces CSRTranspose::eval_gpu / eval_cpu (reference:
 * src/sparse/csr_transpose/csr_transpose.cpp), the structure behind
 * CSRArray.transpose (mlx_sparse/_csr.py:252-275).
 */
msx_status msx_csr_transpose(msx_vtype vt, msx_itype it, int64_t n_rows,
                             int64_t n_cols, int64_t nnz, const void *data,
                             const void *indices, const void *indptr,
                             void *t_data, void *t_indices, void *t_indptr,
                             void *stream);
msx_status msx_csr_transpose_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                 int64_t n_cols, int64_t nnz, const void *data,
                                 const void *indices, const void *indptr,
                                 void *t_data, void *t_indices, void *t_indptr);

/*
 * The structure of A^T (t_indices, t_indptr exactly as msx_csr_transpose
 * writes them) and, per entry i < t_indptr[n_cols], the stored position of
 * A it holds: t_pos[i] (int32); entries past t_indptr[n_cols] (values with
 * a column outside [0, n_cols)) get -1.  Asynchronous on `stream` (scratch
 * from its stream-ordered allocator); nnz < 2^31 - 1.
 *
 * With msx_csr_transpose_values this refreshes a cached transpose after A's
 * values changed in place; no reference counterpart (the reference's arrays
 * are immutable, reference: mlx_sparse/_csr.py:33; the structure is the one
 * of CSRTranspose, src/sparse/csr_transpose/csr_transpose.cpp).
 */
msx_status msx_csr_transpose_positions(msx_itype it, int64_t n_rows,
                                       int64_t n_cols, int64_t nnz,
                                       const void *indices, const void *indptr,
                                       int32_t *t_pos, void *t_indices,
                                       void *t_indptr, void *stream);

/*
 * t_data[i] = data[t_pos[i]] for i < nnz whose t_pos[i] lies in [0, nnz)
 * (complex conjugated when `conjugate` is nonzero and vt is complex64, which
 * gives the values of A^H); other entries get zero bits, as
 * msx_csr_transpose writes them.  Device pointers, asynchronous on
 * `stream`.  One random gather per value.
 */
msx_status msx_csr_transpose_values(msx_vtype vt, int64_t nnz,
                                    const void *data, const int32_t *t_pos,
                                    int conjugate, void *t_data, void *stream);

/*
 * The same regather as msx_csr_transpose_values in two streaming passes,
 * for a transpose whose values are refreshed many times (a training loop):
 *
 * msx_csr_transpose_layout computes, once, from t_pos (as
 * msx_csr_transpose_positions writes it) the layout of the two passes for
 * values of type vt: slot1 (nnz uint16), src1 (nnz uint32), slot2 (nnz
 * uint16).  Scratch from `stream`'s stream-ordered allocator (24 bytes per
 * value).
 *
 * msx_csr_transpose_values_layout then writes t_data exactly as
 * msx_csr_transpose_values would (conjugation, zero bits for dropped
 * entries), with `scratch` nnz values of type vt (overwritten) and a layout
 * built for the same vt and nnz.  Device pointers, asynchronous on
 * `stream`; calls that share `scratch` must not overlap.
 *
 * No reference counterpart (the reference's arrays are immutable,
 * reference: mlx_sparse/_csr.py:33).
 */
msx_status msx_csr_transpose_layout(msx_vtype vt, int64_t nnz,
                                    const int32_t *t_pos, uint16_t *slot1,
                                    uint32_t *src1, uint16_t *slot2,
                                    void *stream);
msx_status msx_csr_transpose_values_layout(msx_vtype vt, int64_t nnz,
                                           const void *data,
                                           const uint16_t *slot1,
                                           const uint32_t *src1,
                                           const uint16_t *slot2, int conjugate,
                                           void *scratch, void *t_data,
                                           void *stream);

/*
 * y = A^T x (x: n_rows, y: n_cols) and Y = A^T X (X: n_rows x k, row stride
 * ldx; Y: n_cols x k, row stride ldy), without a transpose: every stored
 * value adds its product into its column's output with a float atomic, so
 * the order of additions is not fixed (results agree with a sequential sum
 * to rounding).  float16/bfloat16 accumulate in float32 scratch.  For a
 * deterministic result, transpose once (msx_csr_transpose) and multiply
 * with msx_csr_spmv / msx_csr_spmm.
 *
 * Replace CSRMatVecTranspose::eval_gpu and CSRMatMulTranspose::eval_gpu
 * (reference: src/sparse/csr_matvec_transpose/csr_matvec_transpose.metal:27-49,
 * src/sparse/csr_matmul_transpose/); the VJP of csr_matvec / csr_matmul
 * with respect to the dense operand (csr_matvec.cpp:232-259,
 * csr_matmul.cpp:336-363), with conjugated values for complex64.
 */
msx_status msx_csr_spmv_transpose(msx_vtype vt, msx_itype it, int64_t n_rows,
                                  int64_t n_cols, int64_t nnz, const void *data,
                                  const void *indices, const void *indptr,
                                  const void *x, void *y, void *stream);
msx_status msx_csr_spmm_transpose(msx_vtype vt, msx_itype it, int64_t n_rows,
                                  int64_t n_cols, int64_t nnz, const void *data,
                                  const void *indices, const void *indptr,
                                  int64_t k, const void *X, int64_t ldx,
                                  void *Y, int64_t ldy, void *stream);

/*
 * msx_csr_spmv_transpose without any allocation, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  No reference counterpart.
 * Same arguments and results as msx_csr_spmv_transpose; float16/bfloat16
 * accumulate in a fixed float32 scratch array inside the library instead of
 * stream-ordered scratch, so they need n_cols <= 8388608 (32 MiB; larger
 * n_cols fail with MSX_EINVAL).  Each GPU holds its own scratch array from
 * the first such call until the process ends, and every call on that GPU
 * uses it: calls that overlap on one GPU (different streams, or different
 * host threads) race.  float32 and complex64 accumulate in y, as in
 * msx_csr_spmv_transpose, and use no scratch.
 */
msx_status msx_csr_spmv_transpose_noalloc(msx_vtype vt, msx_itype it,
                                          int64_t n_rows, int64_t n_cols,
                                          int64_t nnz, const void *data,
                                          const void *indices,
                                          const void *indptr, const void *x,
                                          void *y, void *stream);

/*
 * Host (CPU) transposed products, contiguous operands, the reference's
 * algorithm: with one worker every output is summed from zero over the rows
 * in order; with W workers, rows are split by row length into W ranges, each
 * accumulates its own partial output from zero, and the partials are added
 * from zero in range order (reference: csr_matvec_transpose.cpp,
 * csr_matvec_transpose_cpu_impl; csr_matmul_transpose.cpp,
 * csr_matmul_transpose_cpu_impl).  Results depend on n_threads, as there.
 */
msx_status msx_csr_spmv_transpose_cpu(msx_vtype vt, msx_itype it,
                                      int64_t n_rows, int64_t n_cols,
                                      int64_t nnz, const void *data,
                                      const void *indices, const void *indptr,
                                      const void *x, void *y, int n_threads);
msx_status msx_csr_spmm_transpose_cpu(msx_vtype vt, msx_itype it,
                                      int64_t n_rows, int64_t n_cols,
                                      int64_t nnz, const void *data,
                                      const void *indices, const void *indptr,
                                      int64_t k, const void *X, void *Y,
                                      int n_threads);

/*
 * Value gradients of y = A x and Y = A X: out[p] = cot[row(p)] * x[col(p)],
 * one rounding; out[p] = sum_q cot[row(p), q] * X[col(p), q], summed from zero
 * in q order (cot: n_rows x k, row stride ldc).  Values with a column outside
 * [0, n_cols) get zero.  For complex64 the caller passes conj(x) / conj(X)
 * (the Hermitian rule of the reference VJPs).
 *
 * msx_csr_spmv_data_vjp takes an optional plan of the matrix (NULL: none;
 * otherwise checked as for msx_csr_spmv, except that a bound plan's values
 * are not compared: the gradient does not read them).  A bound panel plan
 * whose copy holds every value gathers x from LDS panels and uses the plan's
 * product buffer as scratch, so calls that overlap on one plan race, as SpMV
 * calls do.
 *
 * Replace csr_matvec_data_vjp and csr_matmul_data_vjp (reference:
 * src/sparse/csr_matvec_data_vjp/csr_matvec_data_vjp.cpp,
 * src/sparse/csr_matmul_data_vjp/csr_matmul_data_vjp.cpp).
 */
msx_status msx_csr_spmv_data_vjp(msx_vtype vt, msx_itype it, int64_t n_rows,
                                 int64_t n_cols, int64_t nnz, const void *indices,
                                 const void *indptr, const void *x,
                                 const void *cot, void *out,
                                 const msx_csr_plan *plan, void *stream);
msx_status msx_csr_spmm_data_vjp(msx_vtype vt, msx_itype it, int64_t n_rows,
                                 int64_t n_cols, int64_t nnz, const void *indices,
                                 const void *indptr, int64_t k, const void *X,
                                 int64_t ldx, const void *cot, int64_t ldc,
                                 void *out, void *stream);
msx_status msx_csr_spmv_data_vjp_cpu(msx_vtype vt, msx_itype it,
                                     int64_t n_rows, int64_t n_cols,
                                     int64_t nnz, const void *indices,
                                     const void *indptr, const void *x,
                                     const void *cot, void *out, int n_threads);
msx_status msx_csr_spmm_data_vjp_cpu(msx_vtype vt, msx_itype it,
                                     int64_t n_rows, int64_t n_cols,
                                     int64_t nnz, const void *indices,
                                     const void *indptr, int64_t k,
                                     const void *X, const void *cot, void *out,
                                     int n_threads);

/*
 * Result of an iterative solve.  info: 0 converged (||r|| <= max(atol,
 * rtol * ||b||)); > 0 the iteration budget ran out (maxiter, or 1 when
 * maxiter is 0); -1 near-zero denominator; -2 non-positive preconditioned
 * product r.z; -3 non-finite scalar or vector.  residual: norm of the final
 * residual; iterations: completed iterations.
 */
typedef struct msx_solver_result {
  int32_t info;
  int32_t iterations;
  float residual;
  int32_t reserved;
} msx_solver_result;

/*
 * Conjugate gradients for a square symmetric positive-definite float32 CSR
 * matrix (n x n): x from x0 (device pointers; x0 and x may not overlap).
 * Device-wide: the path's SpMV with `plan` (nullable; a plan from
 * msx_csr_plan_create[_bound] for this matrix) and fused vector kernels,
 * scalars kept on the device; the host reads the solver state between
 * batches of iterations, so the call returns when the solve is over
 * (`stream` is synchronised; scratch from its stream-ordered allocator).
 * Dot products are double sums added per workgroup in a fixed order, so
 * results are reproducible run to run; they agree with the sequential CPU
 * loop to rounding.
 *
 * Replaces CSRCG::eval_gpu (reference: src/linalg/cg/cg.cpp:277-327, the
 * single-threadgroup kernel csr_cg in cg.metal) with the arithmetic of
 * csr_cg_cpu_impl (cg.cpp:75-246): float SpMV summed from zero, double dot
 * products and updates, the same tolerance and status rules.
 */
msx_status msx_csr_cg(msx_itype it, int64_t n, int64_t nnz, const float *data,
                      const void *indices, const void *indptr, const float *b,
                      const float *x0, float *x, float rtol, float atol,
                      int64_t maxiter, const msx_csr_plan *plan,
                      msx_solver_result *result, void *stream);

/*
 * Jacobi-preconditioned CG (z = inv_diag * r), float scalars from double
 * sums and float vector updates.  Replaces CSRPCGJacobi::eval_gpu
 * (reference: src/preconditioners/pcg/pcg.cpp, pcg.metal:18) with the
 * arithmetic of csr_pcg_jacobi_cpu_impl (pcg.cpp:71-236).
 */
msx_status msx_csr_pcg_jacobi(msx_itype it, int64_t n, int64_t nnz,
                              const float *data, const void *indices,
                              const void *indptr, const float *b,
                              const float *x0, const float *inv_diag, float *x,
                              float rtol, float atol, int64_t maxiter,
                              const msx_csr_plan *plan,
                              msx_solver_result *result, void *stream);

/*
 * BiCGSTAB for a square float32 CSR matrix (n x n, not necessarily
 * symmetric): x from x0 (device pointers; x0 and x may not overlap).  Runs
 * on the device like msx_csr_cg: per iteration two SpMVs of the path with
 * `plan` (nullable) and fused vector passes; the scalars stay on the device
 * and the host reads the solver state between batches of iterations and
 * when a residual estimate falls under the tolerance (the reference then
 * confirms it on the true residual b - A x, computed here on the device).
 * `stream` is synchronised; scratch comes from its stream-ordered
 * allocator.  Status and residual as msx_solver_result describes
 * (-1: near-zero rho, alpha denominator or omega).
 *
 * Replaces CSRBiCGSTAB::eval_gpu (reference:
 * src/linalg/bicgstab/bicgstab.cpp:388-436, the single-threadgroup kernel
 * of bicgstab.metal:54-320) with the arithmetic of csr_bicgstab_cpu_impl
 * (bicgstab.cpp:80-362).
 */
msx_status msx_csr_bicgstab(msx_itype it, int64_t n, int64_t nnz,
                            const float *data, const void *indices,
                            const void *indptr, const float *b, const float *x0,
                            float *x, float rtol, float atol, int64_t maxiter,
                            const msx_csr_plan *plan, msx_solver_result *result,
                            void *stream);

/*
 * BiCGSTAB with the Jacobi preconditioner M = diag(inv_diag) (inv_diag: n
 * device floats): msx_csr_bicgstab's device loop with x advanced along
 * p_hat = M p and s_hat = M s, which the SpMVs take.  The reference's
 * preconditioned loop differs from the plain one in its edge cases, kept
 * here: ||b|| is rounded to float before its square root; non-finite b or
 * x0, or a non-finite true residual, ends the solve with -3 and the
 * reported residual left as it was (infinity before the first iteration);
 * the reported residual follows ||s|| after the s update.
 *
 * Replaces CSRBiCGSTABJacobi::eval_gpu (reference:
 * src/preconditioners/bicgstab/bicgstab.cpp:548-598, a single-threadgroup
 * kernel of bicgstab.metal) with the arithmetic of
 * left_preconditioned_bicgstab_host (bicgstab.cpp:140-421) and the Jacobi
 * apply of csr_bicgstab_jacobi_cpu_impl (bicgstab.cpp:425-521).
 */
msx_status msx_csr_bicgstab_jacobi(msx_itype it, int64_t n, int64_t nnz,
                                   const float *data, const void *indices,
                                   const void *indptr, const float *b,
                                   const float *x0, const float *inv_diag,
                                   float *x, float rtol, float atol,
                                   int64_t maxiter, const msx_csr_plan *plan,
                                   msx_solver_result *result, void *stream);

/*
 * MINRES for (A - shift I) x = b with A square symmetric (possibly
 * indefinite) float32 CSR: x from x0 (device pointers).  Per iteration two
 * SpMVs (A v for the Lanczos step, A x for the true residual the reference
 * tests every iteration) and fused vector passes; the Givens recurrences
 * run redundantly in every workgroup from the same sums.  `stream` is
 * synchronised; scratch from its stream-ordered allocator.  residual: the
 * true residual ||b - (A - shift I) x||.
 *
 * Replaces CSRMINRES::eval_gpu (reference: src/linalg/minres/minres.cpp,
 * the single-threadgroup kernels of minres.metal:71-140) with the
 * arithmetic of csr_minres_cpu_impl (minres.cpp:93-312).
 */
msx_status msx_csr_minres(msx_itype it, int64_t n, int64_t nnz,
                          const float *data, const void *indices,
                          const void *indptr, const float *b, const float *x0,
                          float *x, float rtol, float atol, int64_t maxiter,
                          float shift, const msx_csr_plan *plan,
                          msx_solver_result *result, void *stream);

/*
 * MINRES with the Jacobi preconditioner M = diag(inv_diag) (inv_diag: n
 * device floats, each > 0): msx_csr_minres's device loop with the Lanczos
 * vectors normalised in the M inner product (y = M r2, beta^2 = r2.y).  As
 * the reference's Jacobi loop: an inverse diagonal entry that is not > 0
 * stops the start with -2 (after the non-finite test, before the
 * convergence test), and a non-finite or non-positive r2.y gives -2.
 *
 * Replaces CSRMINRESJacobi::eval_gpu (reference:
 * src/preconditioners/minres/minres.cpp:359-410, a single-threadgroup
 * kernel of minres.metal) with the arithmetic of csr_minres_jacobi_cpu_impl
 * (minres.cpp:93-330).
 */
msx_status msx_csr_minres_jacobi(msx_itype it, int64_t n, int64_t nnz,
                                 const float *data, const void *indices,
                                 const void *indptr, const float *b,
                                 const float *x0, const float *inv_diag,
                                 float *x, float rtol, float atol,
                                 int64_t maxiter, float shift,
                                 const msx_csr_plan *plan,
                                 msx_solver_result *result, void *stream);

/*
 * Restarted GMRES for a square float32 CSR matrix (n x n, not necessarily
 * symmetric): x from x0 (device pointers; x0 and x may not overlap).
 * Each cycle of at most `restart` Arnoldi steps (and at most the budget
 * left, and n) starts from the true residual; every step is device-wide:
 * one SpMV of the path with `plan` (nullable) and one fused pass per
 * modified Gram-Schmidt column (two sweeps, as the reference's CPU
 * Arnoldi).  The host reads the Hessenberg matrix once per cycle, solves
 * the small least-squares problem in double by Givens rotations, and the
 * device adds V y to x.  `maxiter` counts Arnoldi steps over all cycles;
 * info > 0 is maxiter (1 when maxiter is 0) when the budget ran out; -1 a
 * failed least-squares solve; -3 non-finite values (residual = infinity
 * when the inputs are not finite).  `stream` is synchronised; scratch
 * (restart + 6 vectors of n floats) comes from its stream-ordered
 * allocator.
 *
 * Replaces the GPU path of csr_gmres (reference:
 * src/linalg/gmres/gmres.cpp:58-220, whose Arnoldi step is
 * CSRArnoldi::eval_gpu, src/linalg/arnoldi/arnoldi.cpp:184-225, a
 * single-threadgroup kernel in arnoldi.metal) with the arithmetic of the
 * reference's CPU Arnoldi (arnoldi.cpp:79-159) and restart loop.
 */
msx_status msx_csr_gmres(msx_itype it, int64_t n, int64_t nnz,
                         const float *data, const void *indices,
                         const void *indptr, const float *b, const float *x0,
                         float *x, float rtol, float atol, int64_t restart,
                         int64_t maxiter, const msx_csr_plan *plan,
                         msx_solver_result *result, void *stream);

/*
 * Restarted GMRES with the Jacobi preconditioner M = diag(inv_diag)
 * (inv_diag: n device floats): msx_csr_gmres's device cycles over the
 * Arnoldi basis of M A (each step's w = M (A v_j), folded into the first
 * Gram-Schmidt pass), each cycle started from z0 = M r with the
 * least-squares right-hand side ||z0||.  As the reference's Jacobi loop:
 * ||r|| decides convergence; ||z0|| <= FLT_EPSILON (or not finite) gives
 * -1; a non-finite inverse diagonal entry is a non-finite input (-3,
 * residual infinity); a non-finite new Arnoldi norm ends the cycle with no
 * steps (-1); the least-squares solution is not tested on its own (a
 * non-finite update row ends the solve with -3, the rows before it
 * updated).
 *
 * Replaces the GPU path of csr_gmres_jacobi (reference:
 * src/preconditioners/gmres/gmres.cpp:572-748, whose Arnoldi step is
 * CSRArnoldiJacobi::eval_gpu, gmres.cpp:474-517, gmres.metal) with the
 * arithmetic of csr_arnoldi_jacobi_cpu_impl (gmres.cpp:342-447).
 */
msx_status msx_csr_gmres_jacobi(msx_itype it, int64_t n, int64_t nnz,
                                const float *data, const void *indices,
                                const void *indptr, const float *b,
                                const float *x0, const float *inv_diag,
                                float *x, float rtol, float atol,
                                int64_t restart, int64_t maxiter,
                                const msx_csr_plan *plan,
                                msx_solver_result *result, void *stream);

/*
 * Host (CPU) solvers, host pointers: the reference's sequential loops
 * (csr_cg_cpu_impl, cg.cpp:75-246; csr_pcg_jacobi_cpu_impl,
 * pcg.cpp:71-236), one thread.
 */
msx_status msx_csr_cg_cpu(msx_itype it, int64_t n, int64_t nnz,
                          const float *data, const void *indices,
                          const void *indptr, const float *b, const float *x0,
                          float *x, float rtol, float atol, int64_t maxiter,
                          msx_solver_result *result);
msx_status msx_csr_pcg_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                  const float *data, const void *indices,
                                  const void *indptr, const float *b,
                                  const float *x0, const float *inv_diag,
                                  float *x, float rtol, float atol,
                                  int64_t maxiter, msx_solver_result *result);
/* csr_bicgstab_cpu_impl (bicgstab.cpp:80-362), csr_bicgstab_jacobi_cpu_impl
 * (src/preconditioners/bicgstab/bicgstab.cpp:140-521), csr_minres_cpu_impl
 * (minres.cpp:93-312) and csr_minres_jacobi_cpu_impl
 * (src/preconditioners/minres/minres.cpp:93-330), one thread. */
msx_status msx_csr_bicgstab_cpu(msx_itype it, int64_t n, int64_t nnz,
                                const float *data, const void *indices,
                                const void *indptr, const float *b,
                                const float *x0, float *x, float rtol,
                                float atol, int64_t maxiter,
                                msx_solver_result *result);
msx_status msx_csr_bicgstab_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                       const float *data, const void *indices,
                                       const void *indptr, const float *b,
                                       const float *x0, const float *inv_diag,
                                       float *x, float rtol, float atol,
                                       int64_t maxiter, msx_solver_result *result);
msx_status msx_csr_minres_cpu(msx_itype it, int64_t n, int64_t nnz,
                              const float *data, const void *indices,
                              const void *indptr, const float *b,
                              const float *x0, float *x, float rtol,
                              float atol, int64_t maxiter, float shift,
                              msx_solver_result *result);
msx_status msx_csr_minres_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                     const float *data, const void *indices,
                                     const void *indptr, const float *b,
                                     const float *x0, const float *inv_diag,
                                     float *x, float rtol, float atol,
                                     int64_t maxiter, float shift,
                                     msx_solver_result *result);
/* csr_gmres_impl (gmres.cpp:58-220) over csr_arnoldi_cpu_impl
 * (arnoldi.cpp:79-159), one thread. */
msx_status msx_csr_gmres_cpu(msx_itype it, int64_t n, int64_t nnz,
                             const float *data, const void *indices,
                             const void *indptr, const float *b,
                             const float *x0, float *x, float rtol,
                             float atol, int64_t restart, int64_t maxiter,
                             msx_solver_result *result);
msx_status msx_csr_gmres_jacobi_cpu(msx_itype it, int64_t n, int64_t nnz,
                                    const float *data, const void *indices,
                                    const void *indptr, const float *b,
                                    const float *x0, const float *inv_diag,
                                    float *x, float rtol, float atol,
                                    int64_t restart, int64_t maxiter,
                                    msx_solver_result *result);

/*
 * Matrix Market files (the text format of the SuiteSparse collection).
 * Header fields: format 0 coordinate / 1 array; field 0 real, 1 integer,
 * 2 complex, 3 pattern; symmetry 0 general, 1 symmetric, 2 skew-symmetric,
 * 3 hermitian.  entries: data lines; nnz_bound: stored values after the
 * symmetric kinds are expanded, at most.
 *
 * The reference reads these files with scipy.io.mmread (its tests,
 * tests/test_suitesparse_collection.py:36-47, fixtures
 * tests/fixtures/suitesparse/HB/ with its .mtx files) and builds the array with from_scipy
 * (mlx_sparse/_construct.py:854-975).
 */
typedef struct msx_mm_info {
  int64_t n_rows;
  int64_t n_cols;
  int64_t entries;
  int64_t nnz_bound;
  int32_t format;
  int32_t field;
  int32_t symmetry;
  int32_t reserved;
} msx_mm_info;

msx_status msx_mm_info_read(const char *path, msx_mm_info *info);

/*
 * A coordinate (or array) file as canonical CSR in host buffers of capacity
 * `capacity` values (data, indices) and n_rows + 1 (indptr): symmetric kinds
 * expanded (skew: negated mirror, hermitian: conjugated mirror), rows sorted
 * by column, duplicates summed in double in file order, each value rounded
 * once to `vt` (bfloat16 through float32, as from_scipy does).  *nnz gets
 * the stored values.  Pattern files store 1.  n_threads <= 0: the resolved
 * worker count.
 */
msx_status msx_mm_read_csr(const char *path, msx_vtype vt, msx_itype it,
                           int64_t capacity, void *data, void *indices,
                           void *indptr, int64_t *nnz, int n_threads);

/*
 * A file as a dense row-major n_rows x n_cols array (capacity values):
 * array files directly, coordinate files with zeros elsewhere.
 */
msx_status msx_mm_read_dense(const char *path, msx_vtype vt, int64_t capacity,
                             void *out, int n_threads);

/*
 * Host (CPU) SpMV with host pointers, the `use_cpu()` device: rows are summed
 * sequentially in stored order, rows are split over `n_threads` std::threads
 * in nnz-balanced contiguous ranges (n_threads <= 0: the resolved worker
 * count of msx_cpu_worker_count).  Output is independent of n_threads.
 *
 * Replaces csr_matvec_cpu_impl / CSRMatVec::eval_cpu (reference:
 * src/sparse/csr_matvec/csr_matvec.cpp:79-200).
 */
msx_status msx_csr_spmv_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                            int64_t n_cols, int64_t nnz, const void *data,
                            const void *indices, const void *indptr,
                            const void *x, void *y, int n_threads);

/*
 * Host (CPU) SpMM, contiguous row-major X (n_cols x k) and Y (n_rows x k).
 *
 * Replaces csr_matmul_cpu_impl / CSRMatMul::eval_cpu (reference:
 * src/sparse/csr_matmul/csr_matmul.cpp:83-257).
 */
msx_status msx_csr_spmm_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                            int64_t n_cols, int64_t nnz, const void *data,
                            const void *indices, const void *indptr,
                            int64_t k, const void *X, void *Y, int n_threads);

/*
 * Host (CPU) batched SpMV / SpMM, contiguous operands: X batch x n_cols and
 * Y batch x n_rows (SpMV), X batch x n_cols x k and Y batch x n_rows x k
 * (SpMM).  Work items are (batch, row) pairs split over `n_threads` threads in
 * contiguous ranges balanced by row length (times k); each output is summed
 * from zero in stored order.
 *
 * Replace csr_batched_matvec_cpu_impl (reference:
 * src/sparse/csr_batched_matvec/csr_batched_matvec.cpp:82-146) and
 * csr_batched_matmul_cpu_impl (reference:
 * src/sparse/csr_batched_matmul/csr_batched_matmul.cpp:85-248).
 */
msx_status msx_csr_batched_spmv_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                    int64_t n_cols, int64_t nnz,
                                    const void *data, const void *indices,
                                    const void *indptr, int64_t batch,
                                    const void *X, void *Y, int n_threads);
msx_status msx_csr_batched_spmm_cpu(msx_vtype vt, msx_itype it, int64_t n_rows,
                                    int64_t n_cols, int64_t nnz,
                                    const void *data, const void *indices,
                                    const void *indptr, int64_t batch, int64_t k,
                                    const void *X, void *Y, int n_threads);

/*
 * CPU worker count resolved from the environment: MLX_SPARSE_CPU_THREADS,
 * then MLX_SPARSE_N_THREADS, then OMP_NUM_THREADS, SLURM_CPUS_PER_TASK,
 * PBS_NP, LSB_DJOB_NUMPROC, NSLOTS, then the process affinity mask, then
 * hardware concurrency.
 *
 * Replaces configured_cpu_worker_count (reference:
 * src/common/cpu_parallel.cpp:97-135).
 */
int msx_cpu_worker_count(void);

/*
 * Contiguous row ranges for `n` rows of per-row work `work` over `parts`
 * workers: equal ranges when all rows carry the same work, otherwise
 * work-balanced ranges (ceil targets, each range non-empty).  Writes
 * *n_ranges pairs (begin, end) into `ranges` (capacity 2 * parts int64).
 *
 * Replaces cpu_ranges_for_output_work / equal_cpu_ranges /
 * weighted_cpu_ranges (reference: src/common/cpu_parallel.h:134-164,
 * src/common/cpu_parallel.cpp:183-253).
 */
msx_status msx_cpu_ranges(const int64_t *work, int64_t n, int parts,
                          int64_t *ranges, int64_t *n_ranges);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MSX_SPARSE_H */
