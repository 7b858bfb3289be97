/*
 * spmm_amd.h -- C ABI of the MI355X (gfx950) SpMM library libspmm_amd.so.
 *
 * Y = A * X with A sparse (BOO, PBR or CSR), X dense [batch][cols][K] and
 * Y dense [batch][rows][K], both row-major and contiguous.  Every pointer in a
 * descriptor or argument list is a DEVICE pointer unless its name starts with
 * `h_`.  The caller owns every buffer, including Y and the workspace; nothing
 * here allocates device memory.  All work is enqueued on `stream` (a
 * hipStream_t, NULL = the legacy default stream) and is asynchronous with
 * respect to the host.  Entry points are re-entrant; concurrent calls on
 * different streams are safe as long as they do not share Y or workspace.
 * The only process-wide state is the PBR launch knob
 * (spmm_pbr_set_slab_bytes) and the per-GPU scratch array of
 * spmm_boo_matmul_noalloc.
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
 *   spmm_boo_stage_*   <- the staging of _boo_to_method (torch_fast_spdmm/boo.py:54-96)
 *                         and prepare_boo_cuda's precomputed row tables
 *                         (torch_fast_spdmm/boo_plan.py:84-123); the tile stream
 *                         replaces the reference's one-CTA-per-block launch with
 *                         row merging by atomics (kernels/boo_kernel.cu:574-590).
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
 * BOO (blocked COO).
 *
 * The device-side BOO operand is a tile stream staged once on the host from
 * the arrays csr_to_boo emits (boo_matrix/boo_matrix.hpp:56-138; the
 * reference stages its own GPU copy in torch_fast_spdmm/boo.py:54-96 and,
 * for its plan mode, precomputed row tables in boo_plan.py:84-123):
 *
 *   spmm_boo_stage_create   host BOO arrays -> opaque staging (host memory)
 *   spmm_boo_stage_sizes    array lengths, so the caller can allocate
 *   spmm_boo_stage_copy     copy the arrays out (host pointers)
 *   spmm_boo_stage_destroy
 *
 * The caller copies the arrays to the device and fills spmm_boo_desc.
 * Every row group is cut into 32-row slices; each slice's work becomes tiles
 * of <= 32 rows x <= 32 columns with <= 96 entries (block entries keep the
 * block's row-major order; the slice's remainder rows with <= long_threshold
 * entries become tiles over their distinct columns; longer remainder rows are
 * listed in long_rows and summed by a split-row pass).  A slice heavier than
 * max_item_nnz is cut into several items: the first stores Y, the others
 * write partial sums to workspace slots that a fixup pass adds in slot order,
 * so results do not depend on scheduling.  Groups of slices (see group
 * below) are dealt to workgroups as contiguous ranges of near-equal cost.
 * Empty slices, and slices whose nonzeros use each distinct column fewer than
 * min_reuse times on average (scattered columns, where staging X tiles cannot
 * pay), leave the tile stream: their rows become a CSR with global columns that a
 * row-wise gather pass computes and stores whole.
 * ------------------------------------------------------------------------- */

/* Host copies of csr_to_boo's arrays, int32 indices, nz_idx row-major inside
 * every block (a column-major matrix needs a row-major copy). */
typedef struct spmm_boo_host {
    int32_t rows, cols, n_row_groups, n_col_groups, num_blocks;
    spmm_dtype dtype;
    const int32_t* row_grp_ptr;  /* [n_row_groups+1] */
    const int32_t* row_ids;      /* [rows] */
    const int32_t* col_grp_ptr;  /* [n_col_groups+1] */
    const int32_t* col_ids;      /* [cols] */
    const int32_t* blk_row_grp;  /* [num_blocks], nondecreasing */
    const int32_t* blk_col_grp;  /* [num_blocks] */
    const int32_t* blk_nz_ptr;   /* [num_blocks+1] */
    const uint8_t* blk_shift;    /* [num_blocks] */
    const uint16_t* nz_idx;      /* [compressed_nnz] */
    const void* nz_val;          /* [compressed_nnz] float or double */
    const int32_t* rem_indptr;   /* [rows+1]; the tail, if any, merged in */
    const int32_t* rem_col_ind;
    const void* rem_vals;
} spmm_boo_host;

typedef struct spmm_boo_stage spmm_boo_stage;  /* opaque, host memory */

typedef struct spmm_boo_stage_info {
    int64_t n_tiles, n_ent, n_tcols, n_splits, n_long, n_crow, n_cnz, n_gtask;
    int32_t n_slots, n_waves, group, n_crow_long;
    int32_t n_stream_rows;       /* rows the tile stream stores; n_stream_rows + n_crow == rows */
    int64_t n_blob16;            /* record stream length in 16-byte units (0: none) */
    int64_t n_gtask_order;       /* chunk-task launch order length: 0 (task order) or n_gtask */
} spmm_boo_stage_info;

/* group (1, 2 or 4): slices that share column chunks are put together, up to
 * group of them, and walk one tile stream in lockstep -- the waves of one
 * workgroup, each owning one slice, load each X tile once between them.
 * n_waves is rounded down to a multiple of group.  min_reuse: slices whose
 * nonzeros use each distinct column fewer than min_reuse times on average,
 * and empty slices, go to the gather pass (0: none does; 1.5 is the default
 * of the Python layer). */
int spmm_boo_stage_create(const spmm_boo_host* H, int32_t max_item_nnz, int32_t long_threshold,
                          int32_t n_waves, int32_t group, float min_reuse, spmm_boo_stage** out);
int spmm_boo_stage_sizes(const spmm_boo_stage* st, spmm_boo_stage_info* info);
/* Host output arrays, sized from spmm_boo_stage_sizes:
 *   tiles [n_tiles*8] int32: ent_off, nnz | nc<<8 | nr<<16 | flags<<24, cid_off, row_off,
 *                            slot (-1: the item stores Y, else its partial slot), 0, 0, 0
 *   tile_rs [n_tiles*33] uint8, ent_val [n_ent] (dtype), ent_col [n_ent] uint8,
 *   tcols [n_tcols] int32, splits [n_splits*4] int32, long_rows [n_long] int32,
 *   wave_tiles [n_waves+1] int32,
 *   crow_ptr [n_crow+1] int32, crow_id [n_crow] int32, ccol [n_cnz] int32, cval [n_cnz] (dtype):
 *   the rows of the gather pass (Y row ids, their entries with global columns);
 *   the last n_crow_long of them are longer than long_threshold (than
 *   min(long_threshold, 32) when the gather rows' lengths have a standard
 *   deviation above their mean) and are summed in
 *   chunk tasks: gtask [n_gtask*2] int32 (entry begin, end), gtask_ptr [n_crow_long+1]
 *   int32 (long row i owns tasks gtask_ptr[i] .. gtask_ptr[i+1]).
 * Every tile's entries start at an even index (odd tiles are followed by a
 * zero entry). */
int spmm_boo_stage_copy(const spmm_boo_stage* st, int32_t* tiles, uint8_t* tile_rs,
                        void* ent_val, uint8_t* ent_col, int32_t* tcols, int32_t* splits,
                        int32_t* long_rows, int32_t* wave_tiles, int32_t* crow_ptr,
                        int32_t* crow_id, int32_t* ccol, void* cval, int32_t* gtask,
                        int32_t* gtask_ptr);
/* The record stream of a float matrix staged with group 4 (n_blob16 > 0): the
 * same tiles as above, one contiguous 16-byte aligned record per wave and
 * step (that step's entries, row starts and the slice's first row), so that
 * a kernel moves a whole step into LDS with one DMA instruction, and beside
 * it the ids of the X rows each wave stages at each step.
 *   blobs [n_blob16*16] bytes, blob_first [n_waves*8] uint32 (per wave: the
 *   offsets of its first 4 records, their sizes, its step count, its first
 *   tile), blob_xid [n_tiles*8] uint32.
 * Optional: a descriptor without it runs the same tiles through the other
 * kernels (same results within the stated tolerance). */
int spmm_boo_stage_copy_blobs(const spmm_boo_stage* st, void* blobs, uint32_t* blob_first, uint32_t* blob_xid);
/* The launch order of the chunk tasks when it is not task order
 * (n_gtask_order = n_gtask > 0): gtask_order [n_gtask] int32, a permutation of
 * the task ids.  A power-law matrix's long rows are split into tasks over
 * their entries in the most used columns and tasks over the rest, and every
 * task of the first kind runs first, so those columns' X rows stay in L2.
 * Optional: a descriptor without it runs the tasks in task order (same
 * results: each row's partial rows are added in task order either way). */
int spmm_boo_stage_copy_gtask_order(const spmm_boo_stage* st, int32_t* gtask_order);
void spmm_boo_stage_destroy(spmm_boo_stage* st);

/* Device descriptor: the staged arrays plus row_ids and the remainder CSR
 * (read only for long_rows).  Every row of Y is stored either by the tile
 * stream (n_stream_rows of them) or by the gather pass (n_crow), never both;
 * spmm_boo_matmul returns SPMM_EINVAL unless n_stream_rows + n_crow == rows,
 * so a descriptor that leaves either part unset cannot leave Y rows
 * unwritten.  Copy both counts from spmm_boo_stage_info. */
typedef struct spmm_boo_desc {
    int32_t rows, cols;
    int32_t n_stream_rows;       /* rows stored by the tile stream (spmm_boo_stage_info) */
    const int32_t* row_ids;      /* [rows] */
    int32_t n_tiles;
    const int32_t* tiles;        /* [n_tiles*8] */
    const uint8_t* tile_rs;      /* [n_tiles*33] */
    const void* ent_val;         /* [n_ent] */
    const uint8_t* ent_col;      /* [n_ent] */
    const int32_t* tcols;        /* [n_tcols] */
    int32_t n_waves;             /* a multiple of group */
    int32_t group;               /* waves per workgroup walking one stream in lockstep */
    const int32_t* wave_tiles;   /* [n_waves+1]: equal lengths within each group of waves */
    int32_t n_slots;             /* partial-sum slots (0 when no slice is split) */
    int32_t n_splits;
    const int32_t* splits;       /* [n_splits*4]: row_off, nr, slot_begin, slot_end */
    int32_t n_long;
    const int32_t* long_rows;    /* [n_long] */
    int32_t n_crow;              /* rows of the gather pass (0: none) */
    const int32_t* crow_ptr;     /* [n_crow+1] */
    const int32_t* crow_id;      /* [n_crow] */
    const int32_t* ccol;         /* [n_cnz] (may be null when n_cnz is 0) */
    const void* cval;            /* [n_cnz] (may be null when n_cnz is 0) */
    int32_t n_crow_long;         /* the last n_crow_long gather rows are summed in chunk tasks */
    int32_t n_gtask;
    const int32_t* gtask;        /* [n_gtask*2] */
    const int32_t* gtask_ptr;    /* [n_crow_long+1] */
    const int32_t* rem_indptr;   /* [rows+1] */
    const int32_t* rem_col_ind;
    const void* rem_vals;
    int64_t n_blob16;            /* record stream (spmm_boo_stage_copy_blobs); 0 and NULLs: none */
    const void* blobs;           /* [n_blob16*16] bytes */
    const uint32_t* blob_first;  /* [n_waves*8] */
    const uint32_t* blob_xid;    /* [n_tiles*8] */
    const int32_t* gtask_order;  /* [n_gtask] launch order of the chunk tasks, or NULL: task order */
} spmm_boo_desc;

/* Workspace bytes spmm_boo_matmul needs for this staging and shape: the
 * partial slots of split slices and the partial rows of chunk tasks. */
size_t spmm_boo_workspace_bytes(const spmm_boo_desc* A, spmm_dtype dtype, int64_t batch, int64_t K);

/* Y[b] = A X[b] for b < batch.  X: [batch][A->cols][K], Y: [batch][A->rows][K].
 * Y needs no initialisation: every element is produced by plain stores (no
 * memset, no atomics), so results are the same from run to run. */
int spmm_boo_matmul(const spmm_boo_desc* A, spmm_dtype dtype,
                    const void* X, void* Y, int64_t batch, int64_t K,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Y = A X like spmm_boo_matmul, but allocating nothing and taking no
 * workspace: for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The workspace lives in a fixed 64 MiB
 * device array of the library (one per GPU, held until the process ends;
 * its address is looked up once per device on the first call there).
 * Returns SPMM_ENOMEM when spmm_boo_workspace_bytes exceeds 64 MiB (no work
 * is enqueued).  Calls on one GPU share that array: calls that overlap on one
 * GPU (different streams, or host threads) race and must be serialised by
 * the caller.  Every byte of workspace a call reads it has written itself
 * earlier in the same call, so no clearing is needed between calls. */
int spmm_boo_matmul_noalloc(const spmm_boo_desc* A, spmm_dtype dtype,
                            const void* X, void* Y, int64_t batch, int64_t K, void* stream);

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

/* Launch knob of the PBR multiply, in the manner of the reference's
 * set_boo_feat_block / set_boo_rowseg_fpt (bindings/bindings_boo.cu:409-420):
 * process-wide, read at each call.  When one batch's X is larger than
 * `bytes` (0, the default: never), the stripe kernel runs its feature tiles
 * one launch after another at the small tile width (64 float / 32 double
 * features), so one tile's X columns can stay in the last-level cache while
 * every stripe reads them; otherwise one launch covers every tile.  Results
 * are the same either way. */
int spmm_pbr_set_slab_bytes(int64_t bytes);
int64_t spmm_pbr_get_slab_bytes(void);

/* ---------------------------------------------------------------------------
 * Naive CSR baseline: Y[r][f] = sum_j val[j] * X[col[j]][f], one thread per
 * output element, plain stores (kernels/csr_kernels.cu:5-29 semantics).
 * ------------------------------------------------------------------------- */
int spmm_csr_naive(const void* indptr, const void* col_ind, const void* vals,
                   spmm_itype itype, spmm_dtype dtype, int64_t rows, int64_t cols,
                   const void* X, void* Y, int64_t K, void* stream);

/* ---------------------------------------------------------------------------
 * Launch introspection.  Replaces boo_rowseg_launch_info and
 * boo_nnzflat_launch_info (kernels/boo_kernel.cu:710-797, bound at
 * bindings/bindings_boo.cu:421-475): the kernel the reference's launcher
 * would select, with registers, local bytes, static shared memory and
 * resident blocks per SM from the runtime.  Here the multiply's own dispatch
 * runs with every launch recorded instead of enqueued, so each entry is a
 * kernel the same call of spmm_boo_matmul / spmm_pbr_matmul launches, in
 * launch order, with the runtime's attributes of that instance
 * (hipFuncGetAttributes) and its resident workgroups per CU at its block size
 * (hipOccupancyMaxActiveBlocksPerMultiprocessor).  X and Y are used only for
 * their alignment, which steers the dispatch (NULL: 16-byte aligned).  Up to
 * cap entries are written; *n_out is the number of launches.  Errors are
 * those of the multiply.  Needs a GPU (the runtime's attribute queries).
 * ------------------------------------------------------------------------- */
typedef struct spmm_launch_info {
    const char* kernel;          /* kernel family name (static string) */
    uint32_t grid[3];            /* workgroups in x, y, z */
    uint32_t block;              /* threads per workgroup */
    int32_t registers;           /* hipFuncAttributes.numRegs: VGPRs per lane */
    int32_t scratch_bytes;       /* localSizeBytes: private (spill) bytes per lane */
    int32_t lds_bytes;           /* sharedSizeBytes: static LDS per workgroup */
    int32_t max_threads;         /* maxThreadsPerBlock (the launch bound) */
    int32_t wgs_per_cu;          /* resident workgroups per CU at this block size */
} spmm_launch_info;

int spmm_boo_launch_info(const spmm_boo_desc* A, spmm_dtype dtype, const void* X, const void* Y,
                         int64_t batch, int64_t K, spmm_launch_info* out, int32_t cap, int32_t* n_out);
int spmm_pbr_launch_info(const spmm_pbr_desc* A, spmm_dtype dtype, const void* X, const void* Y,
                         int64_t batch, int64_t K, spmm_launch_info* out, int32_t cap, int32_t* n_out);

/* ---------------------------------------------------------------------------
 * Measurement adjuncts.
 *
 * C++-timed runs: a timer holds an event pair; a *_timed call records the
 * start on `stream`, makes exactly the product call named, records the end
 * and waits for it, and returns the GPU time between the records in *ms --
 * no host work of the caller's falls inside the interval.  Replaces the
 * timed_run of the reference's BOOTimedSpMM (bindings/bindings_boo_timed.cu:
 * 254-270), PBRTimedSpMM (bindings/bindings_pbr_timed.cu:160-180) and
 * DirectSpMM (bindings/bindings_cusparse.cu:122-134).  A timer serves one
 * host thread at a time.
 * ------------------------------------------------------------------------- */
typedef struct spmm_timer spmm_timer;  /* opaque */

int spmm_timer_create(spmm_timer** out);     /* events created and recorded once */
void spmm_timer_destroy(spmm_timer* t);

int spmm_boo_matmul_timed(const spmm_boo_desc* A, spmm_dtype dtype,
                          const void* X, void* Y, int64_t batch, int64_t K,
                          void* workspace, size_t workspace_bytes, void* stream,
                          spmm_timer* timer, float* ms);
int spmm_pbr_matmul_timed(const spmm_pbr_desc* A, spmm_dtype dtype,
                          const void* X, void* Y, int64_t batch, int64_t K, void* stream,
                          spmm_timer* timer, float* ms);

/* Vendor baseline: a persistent rocSPARSE generic-SpMM plan, Y = A X with A a
 * CSR matrix (int32 indices, fp32 values, base 0), X [cols][K] and Y [rows][K]
 * row-major, alpha 1 and beta 0 (the library writes every element of Y).
 * Replaces the reference's DirectSpMM over cuSPARSE
 * (bindings/bindings_cusparse.cu:21-160).  The plan keeps the pointers it is
 * given; `stream` is its construction stream and the only one run() accepts.
 * librocsparse is loaded on the first create (SPMM_EUNSUPPORTED when it is
 * absent).  The workspace (info.workspace_bytes) is the caller's, passed to
 * preprocess() and kept until destroy(). */
typedef struct spmm_vendor_spmm spmm_vendor_spmm;  /* opaque */

typedef enum spmm_vendor_alg {
    SPMM_VENDOR_ALG_DEFAULT = 0,         /* rocsparse_spmm_alg_default */
    SPMM_VENDOR_ALG_CSR = 1,             /* rocsparse_spmm_alg_csr */
    SPMM_VENDOR_ALG_CSR_ROW_SPLIT = 2,   /* rocsparse_spmm_alg_csr_row_split */
    SPMM_VENDOR_ALG_CSR_NNZ_SPLIT = 3,   /* rocsparse_spmm_alg_csr_nnz_split */
    SPMM_VENDOR_ALG_CSR_MERGE_PATH = 4   /* rocsparse_spmm_alg_csr_merge_path */
} spmm_vendor_alg;

typedef struct spmm_vendor_info {
    int32_t version;            /* rocsparse_get_version of the loaded library */
    int32_t header_version;     /* major*100000 + minor*100 + patch of the headers built against */
    size_t workspace_bytes;
    int32_t supported;          /* 0: the library does not implement this SpMM; run() refuses */
    int32_t preprocess_status;  /* rocsparse_status of the preprocess stage, -1 before it */
} spmm_vendor_info;

int spmm_vendor_spmm_create(int64_t rows, int64_t cols, int64_t nnz, const int32_t* crow,
                            const int32_t* col, const float* val, const float* X, int64_t K,
                            float* Y, int32_t alg, void* stream, spmm_vendor_spmm** out);
int spmm_vendor_spmm_info(const spmm_vendor_spmm* plan, spmm_vendor_info* info);
int spmm_vendor_spmm_preprocess(spmm_vendor_spmm* plan, void* workspace, size_t workspace_bytes);
int spmm_vendor_spmm_run(spmm_vendor_spmm* plan, void* stream);
int spmm_vendor_spmm_run_timed(spmm_vendor_spmm* plan, void* stream, spmm_timer* timer, float* ms);
void spmm_vendor_spmm_destroy(spmm_vendor_spmm* plan);

#ifdef __cplusplus
}
#endif

#endif /* SPMM_AMD_H_ */
