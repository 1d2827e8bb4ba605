// msx_internal.h - host-side internals shared by the library's translation
// units: error state, the plan object, argument checks and launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "msx_sparse.h"

namespace msx {

// Thread-local error text behind msx_last_error().
void set_error(const std::string &msg);
void clear_error();
msx_status fail(msx_status code, const std::string &msg);
msx_status hip_fail(hipError_t err, const char *what);

#define MSX_HIP_TRY(expr)                                 \
  do {                                                    \
    hipError_t _e = (expr);                               \
    if (_e != hipSuccess) return ::msx::hip_fail(_e, #expr); \
  } while (0)

size_t value_bytes(msx_vtype vt);
size_t index_bytes(msx_itype it);
bool valid_vtype(int vt);
bool valid_itype(int it);

// Plan defaults.  W: window of the nnz range that a short block's row starts
// fall in (block nnz < 2W); R: short blocks never cross a multiple of R rows;
// C: chunk length of long rows.
constexpr int64_t kDefaultBlockNnz = 256;
// Default W for rows averaging kWideBlockMean or more values: larger blocks
// keep more bytes in flight per wavefront (banded matrix, 42.6 values per
// row, f32: 103 -> 98 us; bf16: 112 -> 96 us), while short rows lose with
// them (3D Poisson, 7 per row: 35 -> 40 us).
constexpr int64_t kWideBlockNnz = 512;
constexpr int64_t kWideBlockMean = 20;
constexpr int64_t kBlockRows = 256;
constexpr int64_t kChunkNnz = 4096;
// Column slices of a sliced plan: one per XCD.
constexpr int kSlices = 8;

}  // namespace msx

struct msx_csr_plan {
  msx_itype itype;
  int64_t n_rows;
  int64_t nnz;
  int64_t block_nnz;   // W
  int64_t block_rows;  // R
  int64_t chunk_nnz;   // C
  int64_t n_blocks;    // short blocks
  int64_t n_bounds;    // short blocks + long rows
  int64_t n_long;
  int64_t n_chunks;
  int device;
  size_t bytes;
  // Device arrays (rows < 2^31; chunk ids < 2^31 checked at build).
  int32_t *bounds;            // n_bounds + 1: block-start or long row (bit 31), sentinel n
  int64_t *bounds_nnz;        // n_bounds + 1: indptr at each entry
  int32_t *long_rows;         // n_long
  int32_t *long_chunk_begin;  // n_long + 1
  int32_t *chunk_row;         // n_chunks: index into long_rows
  void *partials;             // n_chunks * 8 bytes: long-row chunk sums
  void *base;                 // single allocation holding the arrays above
  // Column slicing (csr_slice.hip); n_slices == 0 when the plan is not sliced.
  msx_vtype vtype;
  int64_t n_cols;
  int slice_mode;
  int n_slices;
  int64_t slice_width;
  int col_bits;
  const void *indptr;         // the row pointers the plan was built from
  bool bound;                 // built by msx_csr_plan_create_bound
  const void *bound_data;     // the buffers a bound plan was built from (data: as last refreshed)
  const void *bound_indices;
  void *s_data;               // values reordered by slice inside each short block
  uint32_t *s_col;            // (row_in_block << col_bits) | column_in_slice
  uint32_t *s_seg;            // per 256-row super-block: kSlices + 1 offsets from its first value
  const void *s_indptr;       // indptr the sliced copy was built from
  void *s_partial;            // kSlices * n_rows accumulators
  void *s_base;
  size_t s_bytes;
  // Column panels (csr_panel.hip, csr_panel_build.hip); n_panels == 0 when
  // the plan has none.  The tiles are built over virtual rows: every short
  // row, and every chunk of block_nnz values of a long row.  Values with a
  // valid column, ordered by (panel, tile, stored position): segment (panel
  // q, tile t) is [pn_seg[q * n_tiles + t], pn_seg[q * n_tiles + t + 1]).
  int64_t n_panels;
  int64_t panel_width;        // columns per panel (LDS-resident in pass 1)
  int64_t n_tiles;
  int64_t tile_words;         // LDS words of a tile: products plus one per row
  int64_t pn_values;          // values in the panel copy
  int64_t pn_chunks;          // pass-1 workgroups
  bool pn_dropped;            // some short-row values had a column outside [0, n_cols)
  int32_t *pn_tile_begin;     // n_tiles
  int32_t *pn_tile_end;       // n_tiles
  uint32_t *pn_seg;           // n_panels * n_tiles + 1
  int64_t *pn_chunk_begin;    // pn_chunks + 1: pass-1 ranges of the panel copy
  int32_t *pn_chunk_panel;    // pn_chunks
  void *pn_data;              // pn_values storage values
  uint16_t *pn_col;           // column within the panel
  uint16_t *pn_dest;          // LDS word of the value in its tile: (p - tile's first value) + (row - tile's first row)
  void *pn_prod;              // pn_values accumulator-type products (pass 1 -> pass 2)
  void *pn_base;              // allocation of pn_data, pn_col, pn_dest, pn_prod
  void *pn_meta;              // allocation of the tile, segment and chunk arrays
  // Virtual rows when the matrix has long rows (all null otherwise: then the
  // virtual rows are the rows, delimited by indptr).  Virtual row v spans
  // values [pn_vstart[v], pn_vstart[v + 1]); pn_vslot[v] is its row when
  // it is a short row, -1 - r for a chunk of long row r, whose sum pass 2
  // writes to pn_partial[v]; long row r owns virtual rows
  // [pn_vbase[r], pn_vbase[r + 1]).
  int64_t pn_vrows;           // virtual rows (n_rows without long rows)
  int64_t pn_tile_rows_max;   // most virtual rows of a tile
  uint32_t *pn_vstart;        // pn_vrows + 1
  int32_t *pn_vslot;          // pn_vrows
  uint32_t *pn_vbase;         // n_rows + 1
  void *pn_partial;           // pn_vrows accumulators
  void *pn_vmeta;             // allocation of the four arrays above
  size_t pn_bytes;
  // Column windows of bound plans (csr_spmm.hip): for row tile t (rows
  // [32t, 32t + 32)), win[2t] and win[2t + 1] are the lowest and highest
  // valid column of its values (1 and 0 when it has none).  win_rows_max is
  // the widest window in rows of X (0 when the plan has no windows);
  // win_nnz_max the most values of a tile.
  int64_t n_win;
  int64_t win_rows_max;
  int64_t win_nnz_max;
  int32_t *win;
  size_t win_bytes;
  // XCD-sliced long rows (csr_long_slice.hip); ls_units == 0 when unused.
  // Bound plans whose long rows all hold sorted columns cut each long row at
  // the kSlices column-slice boundaries into pieces of at most
  // kLongPieceMax values.  Pieces are grouped by slice ([ls_slice_begin[s],
  // ls_slice_begin[s + 1])) and carry the accumulator slot they write;
  // long row li owns slots [ls_row_slot[li], ls_row_slot[li + 1]).
  int64_t ls_units;
  int64_t ls_slice_max;     // most pieces of one slice
  int64_t *ls_begin;        // ls_units: first position of the piece
  int32_t *ls_len;          // ls_units: values in the piece
  int32_t *ls_slot;         // ls_units: accumulator slot of the piece
  int32_t *ls_slice_begin;  // kSlices + 1
  int32_t *ls_row_slot;     // n_long + 1
  void *ls_partial;         // ls_units accumulators
  void *ls_base;
  size_t ls_bytes;
};

namespace msx {

// A plan passed with a matrix must have been built for it (same index type,
// rows, values and indptr buffer; a bound plan also the same data and
// indices buffers, value type and columns) on the current device (capi.hip).
msx_status check_plan(const char *op, const msx_csr_plan *plan, msx_vtype vt, msx_itype it,
                      int64_t n_rows, int64_t n_cols, int64_t nnz, const void *data,
                      const void *indices, const void *indptr);

// Launchers (csr_spmv.hip / csr_spmm.hip).  Arguments are already checked.
msx_status launch_spmv(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz,
                       const void *data, const void *indices, const void *indptr,
                       const void *x, void *y, const msx_csr_plan *plan, hipStream_t stream);

// Sliced plans (csr_slice.hip).
msx_status build_slices(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                        hipStream_t stream);
msx_status launch_spmv_sliced(const msx_csr_plan *p, const void *x, void *y, hipStream_t stream);
// Rewrite the values of a plan's sliced / panel copy from `data` (the
// matrix's values changed; its indices and indptr did not).  Asynchronous.
msx_status refresh_slices(msx_csr_plan *p, const void *data, hipStream_t stream);
msx_status refresh_panels(msx_csr_plan *p, const void *data, hipStream_t stream);
// True when most short blocks have valid columns spread over more than a
// quarter of x (the AUTO rule's test for a reordered copy); also the number
// of values in short blocks.  Synchronises `stream`.
msx_status probe_scattered(const msx_csr_plan *p, const void *indices, hipStream_t stream,
                           bool *scattered, int64_t *short_values);
// Minimum short-row values of an AUTO panel plan: one pass-1 chunk
// (csr_panel_build.hip, kMinChunk) per compute unit of `device`.
int64_t panels_min_values(int device);

// Panel plans (csr_panel_build.hip / csr_panel.hip).
bool panels_eligible(const msx_csr_plan *p);
msx_status build_panels(msx_csr_plan *p, const void *data, const void *indices, const void *indptr,
                        hipStream_t stream);
msx_status launch_spmv_panels(const msx_csr_plan *p, const void *indptr, const void *x, void *y,
                              hipStream_t stream);
// Raises the dynamic-LDS limit of the two panel kernels on the current device.
msx_status prepare_spmv_panels(const msx_csr_plan *p);
// Value gradient of y = A x through a panel plan of A (csr_panel.hip), for
// plans whose copy holds every value and whose widest tile fits the LDS.
bool panel_data_vjp_fits(const msx_csr_plan *p);
msx_status launch_panel_data_vjp(const msx_csr_plan *p, const void *indptr, const void *x,
                                 const void *cot, void *out, hipStream_t stream);

// Y[b] = A X[b] for b < batch: X[b] at X + b * x_batch (row stride ldx),
// Y[b] at Y + b * y_batch (row stride ldy), all in elements.  y_nt: Y is
// stored non-temporally (false when the caller reads it back right away).
msx_status launch_spmm_batched(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                               int64_t nnz, const void *data, const void *indices,
                               const void *indptr, int64_t batch, int64_t k, const void *X,
                               int64_t x_batch, int64_t ldx, void *Y, int64_t y_batch, int64_t ldy,
                               bool y_nt, hipStream_t stream);

// Batched SpMV from transposed vectors (Xt: n_cols x kpad, 16-byte aligned
// rows) into batch-major Y (Y[b * ldy + i], b < batch); *done is false when
// kpad is not a width the kernel takes (nothing is launched then).
msx_status launch_spmv_batch_rows(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols,
                                  int64_t nnz, const void *data, const void *indices,
                                  const void *indptr, const void *Xt, int64_t kpad, void *Y,
                                  int64_t ldy, int64_t batch, hipStream_t stream, bool *done);
msx_status launch_spmm(msx_vtype vt, msx_itype it, int64_t n_rows, int64_t n_cols, int64_t nnz,
                       const void *data, const void *indices, const void *indptr, int64_t k,
                       const void *X, int64_t ldx, void *Y, int64_t ldy, const msx_csr_plan *plan,
                       hipStream_t stream);
// XCD-sliced long rows of a bound plan (csr_long_slice.hip): built when
// x is at least 4 MB and every long row's columns are sorted; otherwise the
// plan keeps ls_units == 0.  Synchronises `stream`.
msx_status build_long_slices(msx_csr_plan *p, const void *indices, const void *indptr,
                             hipStream_t stream);
// Long rows of such a plan: y[row] for every long row.  x_bytes as for the
// short-block kernel (x's size rounded up to a dword, nonzero).
msx_status launch_long_sliced(const msx_csr_plan *p, const void *data, const void *indices,
                              const void *x, void *y, uint32_t x_bytes, bool stream_nt,
                              hipStream_t stream);
// Only the fixup of those long rows, after their pieces were summed by the
// fused short-block kernel (csr_spmv.hip).
msx_status launch_long_sliced_fixup(const msx_csr_plan *p, void *y, hipStream_t stream);
// Column windows of a bound plan (csr_spmm.hip).  Synchronises `stream`.
msx_status build_windows(msx_csr_plan *p, const void *indices, const void *indptr,
                         hipStream_t stream);

}  // namespace msx
