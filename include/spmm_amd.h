/*
 * spmm_amd.h -- C ABI of the MI355X (gfx950) SpMM library libspmm_amd.so.
 *
 * Y = A * X with A sparse (BOO, PBR or CSR), X dense [batch][cols][K] and
 * Y dense [batch][rows][K], both row-major and contiguous.  Every pointer in a
 * descriptor or argument list is a DEVICE pointer unless its name starts with
 * `h_`.  The caller owns every buffer, including Y and the workspace; nothing
 * here allocates device memory.  All work is enqueued on `stream` (a
 * hipStream_t, NULL = the legacy default stream) and is asynchronous with
 * respect to the host.  Entry points keep no global state and are re-entrant;
 * concurrent calls on different streams are safe as long as they do not share
 * Y or workspace.
 *
 * Every entry point returns an spmm_status; on failure spmm_last_error()
 * returns a thread-local message naming the failed check.
 *
 * Reference interfaces these replace (paths relative to the reference root,
 * torch_fast_spdmm/):
 *   spmm_boo_matmul    <- boo_spmm_cuda_{f32,f64} / boo_run_into
 *                         (bindings/bindings_boo.cu:125-313, 34-118, 409-414)
 *                         + launch_boo_spmm (kernels/boo_kernel.cu:668-708)
 *                         + launch_csr_spmm for the remainder (kernels/pbr_kernel.cu:1102-1135)
 *   spmm_pbr_matmul    <- pbr_spmm_cuda_{i32,i64}_{f32,f64} / pbr_run_into
 *                         (bindings/bindings_kernels.cu:91-123, 18-89, 436-439)
 *                         + launch_pbr_spmm (kernels/pbr_kernel.cu:329-390)
 *   spmm_csr_naive     <- spdmm_csr_naive (kernels/csr_kernels.cu:31-53)
 *   spmm_boo_plan_*    <- no single counterpart: the row-group schedule the
 *                         reference never builds because it launches one CTA
 *                         per block and resolves rows with atomics
 *                         (kernels/boo_kernel.cu:574-590).
 */
#ifndef SPMM_AMD_H_
#define SPMM_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum spmm_status {
    SPMM_OK = 0,
    SPMM_EINVAL = 1,       /* bad argument (shape, null pointer, size) */
    SPMM_EUNSUPPORTED = 2, /* valid input this build does not handle  */
    SPMM_ELAUNCH = 3,      /* HIP launch or runtime failure            */
    SPMM_ENOMEM = 4        /* workspace too small                      */
} spmm_status;

typedef enum spmm_dtype { SPMM_F32 = 0, SPMM_F64 = 1 } spmm_dtype;
typedef enum spmm_itype { SPMM_I32 = 0, SPMM_I64 = 1 } spmm_itype;

/* Thread-local description of the last failure in this thread. */
const char* spmm_last_error(void);

/* Library version string, e.g. "spmm_amd 0.1 gfx950". */
const char* spmm_version(void);

/* ---------------------------------------------------------------------------
 * BOO (blocked COO).  Arrays are exactly those csr_to_boo emits
 * (boo_matrix/boo_matrix.hpp:56-138) narrowed to int32, with nz_idx sorted
 * row-major inside every block (nz_order == rowmajor; the host stages a
 * row-major copy for column-major matrices).  The tail of the tail_batch
 * policy is passed merged into the remainder CSR (rem_*), so every row's
 * non-block entries are one CSR row.
 *
 * The schedule (work items) comes from spmm_boo_plan_build: one item is one
 * row group, or a contiguous slice of a heavy row group's blocks.  The first
 * item of a row group (slot < 0) owns its rows: it adds the remainder and
 * stores Y directly.  The other items of a split row group write partial sums
 * to workspace slots, and a second pass adds them into Y in slot order, so the
 * result does not depend on scheduling.  Remainder rows longer than
 * long_threshold are left out of the owner item and summed by a split-row pass
 * that runs last.
 * ------------------------------------------------------------------------- */
typedef struct spmm_boo_desc {
    int32_t rows, cols;
    int32_t n_row_groups, n_col_groups, num_blocks;
    int32_t max_nr, max_nc, max_nnz_blk;
    const int32_t* row_grp_ptr; /* [n_row_groups+1] */
    const int32_t* row_ids;     /* [rows] */
    const int32_t* col_grp_ptr; /* [n_col_groups+1] */
    const int32_t* col_ids;     /* [cols] */
    const int32_t* blk_col_grp; /* [num_blocks] */
    const int32_t* blk_nz_ptr;  /* [num_blocks+1] */
    const uint8_t* blk_shift;   /* [num_blocks] */
    const uint16_t* nz_idx;     /* [compressed_nnz], row-major per block */
    const void* nz_val;         /* [compressed_nnz] float or double */
    const int32_t* rem_indptr;  /* [rows+1] */
    const int32_t* rem_col_ind; /* [remainder_nnz] */
    const void* rem_vals;       /* [remainder_nnz] */
    /* schedule from spmm_boo_plan_build, copied to the device */
    int32_t n_items;
    const int32_t* items;       /* [n_items*4]: row_group, blk_begin, blk_end, slot */
    int32_t n_slots;            /* partial-sum slots (0 when no row group is split) */
    int32_t n_splits;           /* row groups split over more than one item */
    const int32_t* splits;      /* [n_splits*3]: row_group, slot_begin, slot_end */
    int32_t n_long;             /* rows whose remainder is longer than long_threshold */
    const int32_t* long_rows;   /* [n_long] */
    int32_t long_threshold;
} spmm_boo_desc;

/* Host-side schedule builder (no device work).  Reads host copies of
 * row_grp_ptr, blk_row_grp (blocks sorted by row group, as csr_to_boo emits
 * them), blk_nz_ptr and rem_indptr.  Writes h_items (capacity item_cap*4
 * ints), h_splits (capacity item_cap*3 ints) and h_long_rows (capacity rows),
 * and the counts through n_items/n_slots/n_splits/n_long.  A row group whose
 * blocks hold more than max_item_nnz nonzeros, or that has more than 64
 * blocks, is cut at block boundaries into items within both limits (an item
 * always holds at least one block).  Call with h_items == NULL first: only n_items is
 * computed, and item_cap must then be at least that. */
int spmm_boo_plan_build(int32_t rows, int32_t n_row_groups, int32_t num_blocks,
                        const int32_t* h_row_grp_ptr, const int32_t* h_blk_row_grp,
                        const int32_t* h_blk_nz_ptr, const int32_t* h_rem_indptr,
                        int32_t max_item_nnz, int32_t long_threshold,
                        int32_t* h_items, int32_t* h_splits, int32_t item_cap,
                        int32_t* h_long_rows,
                        int32_t* n_items, int32_t* n_slots, int32_t* n_splits,
                        int32_t* n_long);

/* Workspace bytes spmm_boo_matmul needs for this schedule and shape. */
size_t spmm_boo_workspace_bytes(const spmm_boo_desc* A, spmm_dtype dtype, int64_t batch, int64_t K);

/* Y[b] = A X[b] for b < batch.  X: [batch][A->cols][K], Y: [batch][A->rows][K].
 * Y needs no initialisation: every element is produced by plain stores (no
 * memset, no atomics), so results are the same from run to run. */
int spmm_boo_matmul(const spmm_boo_desc* A, spmm_dtype dtype,
                    const void* X, void* Y, int64_t batch, int64_t K,
                    void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * PBR (packed block rows).  Arrays are those csr_to_pbr emits
 * (pbr_matrix/pbr_matrix.hpp:98-167): codes as the 64-bit bitset pattern,
 * coords interleaved (row, col) pairs, offsets[num_blocks+1], data packed in
 * bit order per block; the remainder is CSR.  Index arrays are int32 or int64
 * (itype), as the reference stages them (torch_fast_spdmm/__init__.py:17-40).
 * stripe_ptr [n_stripes+1] (n_stripes = ceil(rows/block_rows)) delimits each
 * block row's blocks, which csr_to_pbr emits contiguously.
 * ------------------------------------------------------------------------- */
typedef struct spmm_pbr_desc {
    int64_t rows, cols;
    int32_t block_rows, block_cols;  /* 2x2, 4x4 or 8x8 */
    int64_t num_blocks;
    spmm_itype itype;
    const int64_t* codes;        /* [num_blocks] */
    const void* coords;          /* [num_blocks*2] */
    const void* offsets;         /* [num_blocks+1] */
    const void* data;            /* [compressed_nnz] */
    const void* rem_indptr;      /* [rows+1] */
    const void* rem_col_ind;
    const void* rem_vals;
    const int32_t* stripe_ptr;   /* [n_stripes+1] */
    int32_t n_long;              /* rows whose remainder exceeds long_threshold */
    const int32_t* long_rows;
    int32_t long_threshold;
} spmm_pbr_desc;

int spmm_pbr_matmul(const spmm_pbr_desc* A, spmm_dtype dtype,
                    const void* X, void* Y, int64_t batch, int64_t K, void* stream);

/* ---------------------------------------------------------------------------
 * Naive CSR baseline: Y[r][f] = sum_j val[j] * X[col[j]][f], one thread per
 * output element, plain stores (kernels/csr_kernels.cu:5-29 semantics).
 * ------------------------------------------------------------------------- */
int spmm_csr_naive(const void* indptr, const void* col_ind, const void* vals,
                   spmm_itype itype, spmm_dtype dtype, int64_t rows, int64_t cols,
                   const void* X, void* Y, int64_t K, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SPMM_AMD_H_ */
