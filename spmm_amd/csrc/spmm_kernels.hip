// libspmm_amd: SpMM kernels for MI355X (gfx950, CDNA4) behind the C ABI of
// include/spmm_amd.h.
//
// Design (one paragraph per kernel; the reference's own kernels launch one CTA
// per sparse block and merge rows with global atomics into a memset Y --
// kernels/boo_kernel.cu:410-595, kernels/pbr_kernel.cu:159-326):
//
//  * boo_items_kernel -- one wave64 owns one row group (a work item) for one
//    feature tile.  Lane (r, h) accumulates local row r for half h of the tile
//    in registers across all of the row group's blocks, then adds the row's
//    CSR remainder and stores Y once.  For each block the wave builds the
//    block's row-start table in LDS from nz_idx (sorted row-major, so row r is
//    the run of entries whose idx >> shift == r) and, when the block reuses
//    its columns enough, stages the block's gathered X column tile in LDS with
//    16-byte loads along K.  The LDS row stride is padded by 32 bytes so the
//    lanes of a wave, which read neighbouring columns, hit distinct banks.
//  * boo_fixup_kernel -- for row groups too heavy for one item, adds the
//    partial sums of the extra items into Y in slot order (deterministic).
//  * rows_long_kernel -- remainder rows longer than the long-row threshold:
//    one workgroup per row, 16 nonzero slots x 16 feature lanes, reduced in a
//    fixed order through LDS and added into Y.
//  * pbr_stripe_kernel -- one wave owns one stripe (block row).  Lane (r, l)
//    holds row r of the stripe; for each 64-bit block code it extracts its row
//    bits, finds its first value with a popcount of the code's lower rows, and
//    walks its set bits with ctz, reading the block's X tile (BC consecutive X
//    rows, staged in LDS).  Dense blocks are never formed.
//  * csr_naive_kernel -- the baseline: one thread per output element.
//
// Workgroup ids are remapped so each of the 8 XCDs gets a contiguous range of
// row groups / stripes: neighbouring row groups share X rows, and each XCD has
// its own L2.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "spmm_amd.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return fail(SPMM_ELAUNCH, "HIP launch of %s failed: %s", what, hipGetErrorString(e));
    }
    return SPMM_OK;
}

// ---------------------------------------------------------------------------
// small device helpers
// ---------------------------------------------------------------------------

template <typename T, int VEC> struct Vec;
template <> struct Vec<float, 1> { typedef float type; };
template <> struct Vec<float, 2> { typedef float type __attribute__((ext_vector_type(2))); };
template <> struct Vec<float, 4> { typedef float type __attribute__((ext_vector_type(4))); };
template <> struct Vec<double, 1> { typedef double type; };
template <> struct Vec<double, 2> { typedef double type __attribute__((ext_vector_type(2))); };

template <typename T, int VEC>
__device__ __forceinline__ void load_vec(const T* p, T (&out)[VEC]) {
    typedef typename Vec<T, VEC>::type V;
    V v = *reinterpret_cast<const V*>(p);
    if constexpr (VEC == 1) {
        out[0] = v;
    } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) out[e] = v[e];
    }
}

template <typename T, int VEC>
__device__ __forceinline__ void store_vec(T* p, const T (&in)[VEC]) {
    typedef typename Vec<T, VEC>::type V;
    V v;
    if constexpr (VEC == 1) {
        v = in[0];
    } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = in[e];
    }
    *reinterpret_cast<V*>(p) = v;
}

// Workgroups are handed out round-robin over the XCDs; grid is a multiple of
// 8.  Give XCD j the contiguous logical range [j*per, (j+1)*per).  This is a
// bijection on [0, grid), so it is correct for any XCD count.
__device__ __forceinline__ int xcd_remap(int bid, int grid) {
    const int per = grid >> 3;
    return (bid & 7) * per + (bid >> 3);
}

inline int round_up8(long long n) { return (int)((n + 7) / 8 * 8); }

// ---------------------------------------------------------------------------
// BOO: row-group items
// ---------------------------------------------------------------------------

constexpr int BOO_TILE_COLS = 32;   // widest column group staged in LDS
constexpr int BOO_ROWS_PER_WAVE = 32;

template <typename T>
struct BooArgs {
    int rows, cols, K, batch, n_items, max_nr, long_threshold;
    const int* row_grp_ptr;
    const int* row_ids;
    const int* col_grp_ptr;
    const int* col_ids;
    const int* blk_col_grp;
    const int* blk_nz_ptr;
    const uint8_t* blk_shift;
    const uint16_t* nz_idx;
    const T* nz_val;
    const int* rem_indptr;
    const int* rem_col_ind;
    const T* rem_vals;
    const int* items;
    const T* X;
    T* Y;
    T* P;
};

// &Xb[row*K + f].  A32: the X slab of one batch is under 4 GiB, so the byte
// offset is formed in 32 bits and the load uses a scalar base + 32-bit vector
// offset (one full-rate integer op instead of a 64-bit multiply-add).
template <typename T, bool A32>
__device__ __forceinline__ const T* xaddr(const T* Xb, int row, int K, int f) {
    if constexpr (A32) {
        const uint32_t off = ((uint32_t)row * (uint32_t)K + (uint32_t)f) * (uint32_t)sizeof(T);
        return reinterpret_cast<const T*>(reinterpret_cast<const char*>(Xb) + (size_t)off);
    } else {
        return Xb + (size_t)row * K + f;
    }
}

// LDS copy of one block nonzero: local index and value read by one ds_read.
template <typename T> struct alignas(2 * sizeof(T) > 8 ? 16 : 8) NzEntry {
    uint32_t idx;
    T val;
};

// Feature tile geometry: lane half h owns the VEC-element chunks 2q+h of the
// tile, q < NQ.  Interleaving the halves keeps the two lanes of a row on
// different LDS banks.
template <typename T, int F, int VEC>
struct BooGeom {
    static constexpr int KT = 2 * F;              // features per tile
    static constexpr int CHUNKS = KT / VEC;       // VEC-chunks per X row slice
    static constexpr int NQ = F / VEC;            // chunks per lane
    static constexpr int STRIDE = KT + 32 / (int)sizeof(T);  // LDS row stride (elements)
    static constexpr int CPI = 64 / CHUNKS;       // columns staged per wave instruction
    static_assert(CHUNKS <= 64 && 64 % CHUNKS == 0, "tile too wide for one wave");
};

// Accumulate nonzeros [j, e) of one block for this lane's row into acc.
// FAST: nonzeros from the LDS copy (nzp, block-relative) and X rows from
// the LDS tile, so the loop waits only on LDS; otherwise both come from global
// memory.  The two are separate loops, run by separate block passes, so a
// fast loop never waits on the vector-memory counter (and so never on the
// next block's prefetch).
template <typename T, int F, int VEC, bool FULL, bool A32, bool FAST>
__device__ __forceinline__ void boo_row_block(
    T (&acc)[F / VEC][VEC], int j, int e, int nz0, uint32_t mask,
    const uint16_t* __restrict__ nz_idx, const T* __restrict__ nz_val,
    const NzEntry<T>* __restrict__ nzp,
    const int* __restrict__ col_ids, int c0, const T* __restrict__ tile,
    const T* __restrict__ Xb, int K, int fbase, int h) {
    typedef BooGeom<T, F, VEC> G;
#pragma nounroll
    for (; j < e; ++j) {
        T v;
        const T* xr;
        if constexpr (FAST) {
            const NzEntry<T> ent = nzp[j];
            const uint32_t c = ent.idx & mask;
            v = ent.val;
            xr = tile + c * G::STRIDE + h * VEC;
        } else {
            const uint32_t c = (uint32_t)nz_idx[nz0 + j] & mask;
            v = nz_val[nz0 + j];
            xr = xaddr<T, A32>(Xb, col_ids[c0 + c], K, fbase + h * VEC);
        }
        T x[G::NQ][VEC];
#pragma unroll
        for (int q = 0; q < G::NQ; ++q)
            if (FULL || fbase + (2 * q + h) * VEC < K) load_vec<T, VEC>(xr + 2 * q * VEC, x[q]);
#pragma unroll
        for (int q = 0; q < G::NQ; ++q) {
            if (FULL || fbase + (2 * q + h) * VEC < K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u) acc[q][u] += v * x[q][u];
            }
        }
    }
}

// One CSR row (the remainder) into acc; entries are fetched four at a time so
// their X loads are in flight together.
template <typename T, int F, int VEC, bool FULL, bool A32>
__device__ __forceinline__ void csr_row_accumulate(
    T (&acc)[F / VEC][VEC], int rs, int re, const int* __restrict__ col_ind,
    const T* __restrict__ vals, const T* __restrict__ Xb, int K, int fbase, int h) {
    typedef BooGeom<T, F, VEC> G;
#pragma nounroll
    for (int j = rs; j < re; j += 4) {
        int col[4];
        T v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int jj = min(j + u, re - 1);   // in bounds; surplus entries get v = 0
            col[u] = col_ind[jj];
            v[u] = j + u < re ? vals[jj] : T(0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const T* xr = xaddr<T, A32>(Xb, col[u], K, fbase + h * VEC);
#pragma unroll
            for (int q = 0; q < G::NQ; ++q) {
                if (FULL || fbase + (2 * q + h) * VEC < K) {
                    T x[VEC];
                    load_vec<T, VEC>(xr + 2 * q * VEC, x);
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[q][e] += v[u] * x[e];
                }
            }
        }
    }
}

// Few rows with remainder entries: the whole wave takes them one row at a time,
// lanes along the tile's features, and hands each row's sum to its lane pair
// through LDS.  This keeps a wave whose remainder sits in 2 of 32 rows from
// running 30 idle lane pairs through every entry.
template <typename T, int F, int VEC, bool FULL, bool A32>
__device__ __forceinline__ void boo_rem_row_serial(
    T (&acc)[F / VEC][VEC], uint64_t rows, int rem_s, int rem_e,
    const int* __restrict__ col_ind, const T* __restrict__ vals, const T* __restrict__ Xb,
    int K, int fbase, int h, T* scratch) {
    typedef BooGeom<T, F, VEC> G;
    const int lane = threadIdx.x;
    const bool fok = lane < G::KT && fbase + lane < K;
    while (rows) {
        const int l2 = __builtin_ctzll(rows);      // lane 2r of row r
        rows &= rows - 1;
        const int rs = __builtin_amdgcn_readlane(rem_s, l2);
        const int re = __builtin_amdgcn_readlane(rem_e, l2);
        T s0 = T(0), s1 = T(0), s2 = T(0), s3 = T(0);
        int j = rs;
        for (; j + 4 <= re; j += 4) {
            const int c0 = col_ind[j], c1 = col_ind[j + 1], c2 = col_ind[j + 2], c3 = col_ind[j + 3];
            const T v0 = vals[j], v1 = vals[j + 1], v2 = vals[j + 2], v3 = vals[j + 3];
            if (fok) {
                s0 += v0 * *xaddr<T, A32>(Xb, c0, K, fbase + lane);
                s1 += v1 * *xaddr<T, A32>(Xb, c1, K, fbase + lane);
                s2 += v2 * *xaddr<T, A32>(Xb, c2, K, fbase + lane);
                s3 += v3 * *xaddr<T, A32>(Xb, c3, K, fbase + lane);
            }
        }
        for (; j < re; ++j) {
            const int c0 = col_ind[j];
            const T v0 = vals[j];
            if (fok) s0 += v0 * *xaddr<T, A32>(Xb, c0, K, fbase + lane);
        }
        __syncthreads();
        if (lane < G::KT) scratch[lane] = (s0 + s1) + (s2 + s3);
        __syncthreads();
        if ((lane & ~1) == l2) {
#pragma unroll
            for (int q = 0; q < G::NQ; ++q) {
                if (FULL || fbase + (2 * q + h) * VEC < K) {
                    T x[VEC];
                    load_vec<T, VEC>(scratch + (2 * q + h) * VEC, x);
#pragma unroll
                    for (int u = 0; u < VEC; ++u) acc[q][u] += x[u];
                }
            }
        }
    }
}

constexpr int BOO_ROW_SERIAL_MAX = 8;   // remainder rows per wave taken one at a time
constexpr int BOO_NZ_CAP = 128;         // nonzeros of a block staged in LDS
constexpr int BOO_MAX_ITEM_BLOCKS = 64;  // blocks per work item (one per lane)

// Register state prefetched for one block while the previous one computes.
template <typename T, int F, int VEC>
struct BooStage {
    static constexpr int NST = BOO_TILE_COLS / BooGeom<T, F, VEC>::CPI;
    T x[NST][VEC];
    uint32_t idx[2];
    T val[2];
};

// Loads for one fast block.  X: instruction m brings columns
// [m*CPI, (m+1)*CPI), their ids read from the LDS copy colbuf, which holds 0
// past nc, so every instruction reads valid memory (rows past nc are never
// read back) and none needs a branch.  Nonzeros: entries lane and lane+64,
// clamped into the block.  Nothing here waits on an earlier global load.
template <typename T, int F, int VEC, bool FULL, bool A32>
__device__ __forceinline__ void boo_prefetch(BooStage<T, F, VEC>& st, int nz0, int nnz, int nc,
                                             const int* colbuf, const BooArgs<T>& a,
                                             const T* __restrict__ Xb, int fbase) {
    typedef BooGeom<T, F, VEC> G;
    const int lane = threadIdx.x;
    const int ch = lane % G::CHUNKS;
    const int f = fbase + ch * VEC;
    int gcol[BooStage<T, F, VEC>::NST];
#pragma unroll
    for (int m = 0; m < BooStage<T, F, VEC>::NST; ++m) gcol[m] = colbuf[m * G::CPI + lane / G::CHUNKS];
#pragma unroll
    for (int m = 0; m < BooStage<T, F, VEC>::NST; ++m)
        if (FULL || f < a.K) load_vec<T, VEC>(xaddr<T, A32>(Xb, gcol[m], a.K, f), st.x[m]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int k = nz0 + min(lane + 64 * c, nnz - 1);
        st.idx[c] = a.nz_idx[k];
        st.val[c] = a.nz_val[k];
    }
}

// Row-start table of local rows [s0, s0+32] for a block whose first entries
// are in registers (lane k: idx[0] = entry k, idx[1] = entry k+64; nnz < 128):
// entry k starts the rows in (row(k-1), row(k)], row(-1) = -1, row(nnz) = +inf.
__device__ __forceinline__ void boo_rowtab_regs(const uint32_t (&idx)[2], int nnz, uint32_t shift,
                                                int s0, int* rowtab) {
    const int lane = threadIdx.x;
    int rk[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) rk[c] = lane + 64 * c < nnz ? (int)(idx[c] >> shift) : 0x7fffffff;
    const int last0 = __builtin_amdgcn_readlane(rk[0], 63);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        const int k = lane + 64 * c;
        int rp = __shfl_up(rk[c], 1);
        if (lane == 0) rp = (c == 0) ? -1 : last0;
        if (k <= nnz) {
            const int lo = max(rp + 1, s0);
            const int hi = min(rk[c], s0 + BOO_ROWS_PER_WAVE);
            for (int r = lo; r <= hi; ++r) rowtab[r - s0] = k;
        }
    }
}

// Same table read straight from global memory (blocks of any size).
__device__ __forceinline__ void boo_rowtab_global(const uint16_t* __restrict__ nz_idx, int nz0,
                                                  int nnz, uint32_t shift, int s0, int* rowtab) {
    for (int k = threadIdx.x; k <= nnz; k += 64) {
        const int rk = k < nnz ? (int)((uint32_t)nz_idx[nz0 + k] >> shift) : 0x7fffffff;
        const int rp = k > 0 ? (int)((uint32_t)nz_idx[nz0 + k - 1] >> shift) : -1;
        const int lo = max(rp + 1, s0);
        const int hi = min(rk, s0 + BOO_ROWS_PER_WAVE);
        for (int r = lo; r <= hi; ++r) rowtab[r - s0] = k;
    }
}

template <typename T, int F, int VEC, bool FULL, bool A32>
__device__ __forceinline__ void boo_item_body(const BooArgs<T>& a, int item, int kt, int b,
                                              T* tile, NzEntry<T>* nzp, int* rowtab,
                                              int* colbuf) {
    typedef BooGeom<T, F, VEC> G;
    const int lane = threadIdx.x;
    const int h = lane & 1;
    const int lr_in = lane >> 1;
    const int4 it = reinterpret_cast<const int4*>(a.items)[item];
    const int rg = it.x, b0 = it.y, nblk = it.z - it.y, slot = it.w;
    const int r0 = a.row_grp_ptr[rg];
    const int nr = a.row_grp_ptr[rg + 1] - r0;
    const int K = a.K;
    const int fbase = kt * G::KT;
    const T* Xb = a.X + (size_t)b * a.cols * K;

    // Block metadata, lane i for block b0+i (an item has at most 64 blocks).
    int m_nz0 = 0, m_nnz = 0, m_sh = 0, m_c0 = 0, m_nc = 0;
    if (lane < nblk) {
        const int blk = b0 + lane;
        const int cg = a.blk_col_grp[blk];
        m_nz0 = a.blk_nz_ptr[blk];
        m_nnz = a.blk_nz_ptr[blk + 1] - m_nz0;
        m_sh = a.blk_shift[blk];
        m_c0 = a.col_grp_ptr[cg];
        m_nc = a.col_grp_ptr[cg + 1] - m_c0;
    }
    // Fast blocks: the column group fits the LDS tile, the block reuses its
    // columns (>= 1.5 entries per column) and its entries fit the LDS copy.
    const bool m_fast = lane < nblk && m_nc <= BOO_TILE_COLS && 2 * m_nnz >= 3 * m_nc &&
                        m_nnz < BOO_NZ_CAP;
    const uint64_t fast_set = __ballot(m_fast);
    const uint64_t slow_set = __ballot(lane < nblk && !m_fast);
    auto next_of = [](uint64_t set, int after) -> int {  // first member > after, or 64
        const uint64_t rest = after >= 63 ? 0ull : (set & (~0ull << (after + 1)));
        return rest ? __builtin_ctzll(rest) : 64;
    };
    auto colids_of = [&](int j) -> int {  // lane c: column id c of block j (0 past nc)
        if (j >= 64) return 0;
        const int c0 = __builtin_amdgcn_readlane(m_c0, j), nc = __builtin_amdgcn_readlane(m_nc, j);
        return lane < nc ? a.col_ids[c0 + lane] : 0;
    };

    for (int s0 = 0; s0 < nr; s0 += BOO_ROWS_PER_WAVE) {
        const int lr = s0 + lr_in;
        const bool active = lr < nr;
        const int row = a.row_ids[r0 + min(lr, nr - 1)];
        int rem_s = 0, rem_e = 0;
        if (slot < 0) {
            rem_s = a.rem_indptr[row];
            rem_e = a.rem_indptr[row + 1];
        }
        T acc[G::NQ][VEC];
#pragma unroll
        for (int q = 0; q < G::NQ; ++q)
#pragma unroll
            for (int u = 0; u < VEC; ++u) acc[q][u] = T(0);

        // ---- pass 1: fast blocks, software-pipelined one block ahead.  The
        // block's column ids travel through colbuf (LDS) so the prefetch's
        // address math waits only on LDS, never on outstanding global loads.
        BooStage<T, F, VEC> st;
        int j = next_of(fast_set, -1);
        int jn = next_of(fast_set, j);
        int colv = 0;
        if (j < 64) {
            colv = colids_of(j);
            __syncthreads();
            if (lane < BOO_TILE_COLS) colbuf[lane] = colv;
            __syncthreads();
            boo_prefetch<T, F, VEC, FULL, A32>(st, __builtin_amdgcn_readlane(m_nz0, j),
                                          __builtin_amdgcn_readlane(m_nnz, j),
                                          __builtin_amdgcn_readlane(m_nc, j), colbuf, a, Xb, fbase);
            colv = colids_of(jn);
        }
        while (j < 64) {
            const int nnz = __builtin_amdgcn_readlane(m_nnz, j);
            const uint32_t shift = __builtin_amdgcn_readlane(m_sh, j);
            const int nc = __builtin_amdgcn_readlane(m_nc, j);
            const uint32_t mask = (1u << shift) - 1u;

            __syncthreads();  // the previous block's readers of LDS are done
            {
                const int ch = lane % G::CHUNKS;
#pragma unroll
                for (int m = 0; m < BooStage<T, F, VEC>::NST; ++m) {
                    if (FULL || fbase + ch * VEC < K)
                        store_vec<T, VEC>(tile + (m * G::CPI + lane / G::CHUNKS) * G::STRIDE + ch * VEC,
                                          st.x[m]);
                }
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int k = lane + 64 * c;
                    if (k < nnz) nzp[k] = NzEntry<T>{st.idx[c], st.val[c]};
                }
                if (lane < BOO_TILE_COLS) colbuf[lane] = colv;  // ids of block jn
            }
            boo_rowtab_regs(st.idx, nnz, shift, s0, rowtab);
            __syncthreads();
            // Issue the next fast block's loads; they land while this one computes.
            const int jnn = next_of(fast_set, jn);
            if (jn < 64) {
                boo_prefetch<T, F, VEC, FULL, A32>(st, __builtin_amdgcn_readlane(m_nz0, jn),
                                              __builtin_amdgcn_readlane(m_nnz, jn),
                                              __builtin_amdgcn_readlane(m_nc, jn), colbuf, a, Xb,
                                              fbase);
                colv = colids_of(jnn);
            }
            if (active)
                boo_row_block<T, F, VEC, FULL, A32, true>(acc, rowtab[lr_in], rowtab[lr_in + 1], 0, mask,
                                                     a.nz_idx, a.nz_val, nzp, a.col_ids, 0,
                                                     tile, Xb, K, fbase, h);
            j = jn;
            jn = jnn;
        }

        // ---- pass 2: the other blocks, straight from global memory
        for (int js = next_of(slow_set, -1); js < 64; js = next_of(slow_set, js)) {
            const int nz0 = __builtin_amdgcn_readlane(m_nz0, js);
            const int nnz = __builtin_amdgcn_readlane(m_nnz, js);
            const uint32_t shift = __builtin_amdgcn_readlane(m_sh, js);
            const int c0 = __builtin_amdgcn_readlane(m_c0, js);
            __syncthreads();
            boo_rowtab_global(a.nz_idx, nz0, nnz, shift, s0, rowtab);
            __syncthreads();
            if (active)
                boo_row_block<T, F, VEC, FULL, A32, false>(acc, rowtab[lr_in], rowtab[lr_in + 1], nz0,
                                                      (1u << shift) - 1u, a.nz_idx, a.nz_val, nzp,
                                                      a.col_ids, c0, tile, Xb, K, fbase, h);
        }

        // ---- remainder rows (short ones; longer rows go to the split-row pass)
        const bool has_rem = active && slot < 0 && rem_e > rem_s && rem_e - rem_s <= a.long_threshold;
        const uint64_t rem_rows = __ballot(has_rem && h == 0);
        if (__popcll(rem_rows) > BOO_ROW_SERIAL_MAX) {
            // many rows have entries: every lane pair walks its own row
            if (has_rem)
                csr_row_accumulate<T, F, VEC, FULL, A32>(acc, rem_s, rem_e, a.rem_col_ind, a.rem_vals,
                                                    Xb, K, fbase, h);
        } else if (rem_rows) {
            boo_rem_row_serial<T, F, VEC, FULL, A32>(acc, rem_rows, rem_s, rem_e, a.rem_col_ind,
                                                a.rem_vals, Xb, K, fbase, h, tile);
        }
        if (!active) continue;
        T* out;
        if (slot < 0) {
            out = a.Y + ((size_t)b * a.rows + row) * K + fbase + h * VEC;
        } else {
            out = a.P + (((size_t)slot * a.batch + b) * a.max_nr + lr) * K + fbase + h * VEC;
        }
#pragma unroll
        for (int q = 0; q < G::NQ; ++q) {
            if (FULL || fbase + (2 * q + h) * VEC < K) store_vec<T, VEC>(out + 2 * q * VEC, acc[q]);
        }
    }
}

template <typename T, int F, int VEC, bool FULL, bool A32>
__global__ void __launch_bounds__(64) boo_items_kernel(BooArgs<T> a, int kt0) {
    typedef BooGeom<T, F, VEC> G;
    __shared__ __attribute__((aligned(16))) T tile[BOO_TILE_COLS * G::STRIDE];
    __shared__ NzEntry<T> nzp[BOO_NZ_CAP];
    __shared__ int rowtab[BOO_ROWS_PER_WAVE + 1];
    __shared__ int colbuf[BOO_TILE_COLS];
    const int item = xcd_remap(blockIdx.x, gridDim.x);
    if (item >= a.n_items) return;
    boo_item_body<T, F, VEC, FULL, A32>(a, item, kt0 + (int)blockIdx.y, blockIdx.z, tile, nzp, rowtab,
                                        colbuf);
}

template <typename T>
__global__ void __launch_bounds__(256) boo_fixup_kernel(const int* __restrict__ splits,
                                                        const int* __restrict__ row_grp_ptr,
                                                        const int* __restrict__ row_ids,
                                                        const T* __restrict__ P, T* __restrict__ Y,
                                                        int rows, int K, int batch, int max_nr) {
    const int s = blockIdx.x;
    const int b = blockIdx.z;
    const int rg = splits[3 * s], sb = splits[3 * s + 1], se = splits[3 * s + 2];
    const int r0 = row_grp_ptr[rg];
    const int nr = row_grp_ptr[rg + 1] - r0;
    const long long total = (long long)nr * K;
    for (long long e = threadIdx.x; e < total; e += blockDim.x) {
        const int lr = (int)(e / K);
        const int f = (int)(e % K);
        T* y = Y + ((size_t)b * rows + row_ids[r0 + lr]) * K + f;
        T acc = *y;
        for (int sl = sb; sl < se; ++sl) acc += P[(((size_t)sl * batch + b) * max_nr + lr) * K + f];
        *y = acc;
    }
}

// ---------------------------------------------------------------------------
// Long remainder rows (BOO and PBR): Y[row] += sum over the row's CSR entries.
// 256 threads = 16 nonzero slots x 16 lanes of VEC features.
// ---------------------------------------------------------------------------

template <typename T, typename I, int VEC>
__global__ void __launch_bounds__(256) rows_long_kernel(const int* __restrict__ long_rows,
                                                        const I* __restrict__ indptr,
                                                        const I* __restrict__ col_ind,
                                                        const T* __restrict__ vals,
                                                        const T* __restrict__ X, T* __restrict__ Y,
                                                        long long rows, long long cols, int K) {
    constexpr int LANES = 16, SLOTS = 16, KT = LANES * VEC;
    __shared__ T red[SLOTS][KT];
    const int row = long_rows[blockIdx.x];
    const int kt = blockIdx.y;
    const int b = blockIdx.z;
    const int slot = threadIdx.x / LANES;
    const int ch = threadIdx.x % LANES;
    const int f = kt * KT + ch * VEC;
    const bool fok = f < K;
    const T* Xb = X + (size_t)b * cols * K;
    T acc[VEC];
#pragma unroll
    for (int u = 0; u < VEC; ++u) acc[u] = T(0);
    const long long rs = (long long)indptr[row], re = (long long)indptr[row + 1];
    if (fok) {
        for (long long j = rs + slot; j < re; j += SLOTS) {
            const T v = vals[j];
            T x[VEC];
            load_vec<T, VEC>(Xb + (size_t)col_ind[j] * K + f, x);
#pragma unroll
            for (int u = 0; u < VEC; ++u) acc[u] += v * x[u];
        }
    }
#pragma unroll
    for (int u = 0; u < VEC; ++u) red[slot][ch * VEC + u] = acc[u];
    __syncthreads();
    if (threadIdx.x < KT) {
        const int fe = kt * KT + threadIdx.x;
        if (fe < K) {
            T s = T(0);
#pragma unroll
            for (int sl = 0; sl < SLOTS; ++sl) s += red[sl][threadIdx.x];
            T* y = Y + ((size_t)b * rows + row) * K + fe;
            *y += s;
        }
    }
}

// ---------------------------------------------------------------------------
// PBR: stripe owner
// ---------------------------------------------------------------------------

template <typename T, typename I>
struct PbrArgs {
    long long rows, cols;
    int K, n_stripes, long_threshold;
    const int64_t* codes;
    const I* coords;
    const I* offsets;
    const T* data;
    const I* rem_indptr;
    const I* rem_col_ind;
    const T* rem_vals;
    const int* stripe_ptr;
    const T* X;
    T* Y;
};

// BR x BR blocks.  LPR = 64/BR lanes per stripe row; lane l of a row owns the
// VEC-chunks q*LPR + l of the tile (q < NQ), so a row's lanes read one
// contiguous run per instruction.
template <typename T, int BR, int KT, int VEC>
struct PbrGeom {
    static constexpr int LPR = 64 / BR;
    static constexpr int F = KT / LPR;
    static constexpr int NQ = F / VEC;
    static constexpr int CHUNKS = KT / VEC;
    static constexpr int STRIDE = KT + 32 / (int)sizeof(T);
    static constexpr int STAGE_ITERS = (BR * CHUNKS + 63) / 64;
    static_assert(F % VEC == 0 && NQ >= 1, "bad PBR tile");
};

template <typename T, typename I, int BR, int KT, int VEC, bool FULL>
__device__ __forceinline__ void pbr_stripe_body(const PbrArgs<T, I>& a, int stripe, int kt, int b,
                                                T* tile) {
    typedef PbrGeom<T, BR, KT, VEC> G;
    const int lane = threadIdx.x;
    const int r = lane / G::LPR;
    const int l = lane % G::LPR;
    const long long row = (long long)stripe * BR + r;
    const bool active = row < a.rows;
    const int K = a.K;
    const int fbase = kt * KT;
    const T* Xb = a.X + (size_t)b * a.cols * K;
    constexpr uint64_t rowbits = (BR == 8) ? 0xffull : ((1ull << BR) - 1ull);

    T acc[G::NQ][VEC];
#pragma unroll
    for (int q = 0; q < G::NQ; ++q)
#pragma unroll
        for (int u = 0; u < VEC; ++u) acc[q][u] = T(0);

    const int p0 = a.stripe_ptr[stripe], p1 = a.stripe_ptr[stripe + 1];
    for (int blk = p0; blk < p1; ++blk) {
        const uint64_t code = (uint64_t)a.codes[blk];
        const long long col0 = (long long)a.coords[2 * (size_t)blk + 1];
        const long long off = (long long)a.offsets[blk];
        __syncthreads();
#pragma unroll
        for (int m = 0; m < G::STAGE_ITERS; ++m) {
            const int idx = m * 64 + lane;
            const int c = idx / G::CHUNKS;
            const int ch = idx % G::CHUNKS;
            const int f = fbase + ch * VEC;
            if (c < BR && col0 + c < a.cols && (FULL || f < K)) {
                T x[VEC];
                load_vec<T, VEC>(Xb + (size_t)(col0 + c) * K + f, x);
                store_vec<T, VEC>(tile + c * G::STRIDE + ch * VEC, x);
            }
        }
        __syncthreads();
        if (active) {
            uint32_t rb = (uint32_t)((code >> (BR * r)) & rowbits);
            const uint64_t below = (r == 0) ? 0ull : (code & ((1ull << (BR * r)) - 1ull));
            const T* dp = a.data + off + __popcll(below);
            while (rb) {
                const int c = __builtin_ctz(rb);
                rb &= rb - 1u;
                const T v = *dp++;
                const T* xr = tile + c * G::STRIDE + l * VEC;
#pragma unroll
                for (int q = 0; q < G::NQ; ++q) {
                    if (FULL || fbase + (q * G::LPR + l) * VEC < K) {
                        T x[VEC];
                        load_vec<T, VEC>(xr + q * G::LPR * VEC, x);
#pragma unroll
                        for (int u = 0; u < VEC; ++u) acc[q][u] += v * x[u];
                    }
                }
            }
        }
    }
    if (!active) return;
    const long long rs = (long long)a.rem_indptr[row], re = (long long)a.rem_indptr[row + 1];
    if (re - rs <= a.long_threshold) {
        for (long long j = rs; j < re; ++j) {
            const T v = a.rem_vals[j];
            const T* xr = Xb + (size_t)a.rem_col_ind[j] * K + fbase + l * VEC;
#pragma unroll
            for (int q = 0; q < G::NQ; ++q) {
                if (FULL || fbase + (q * G::LPR + l) * VEC < K) {
                    T x[VEC];
                    load_vec<T, VEC>(xr + q * G::LPR * VEC, x);
#pragma unroll
                    for (int u = 0; u < VEC; ++u) acc[q][u] += v * x[u];
                }
            }
        }
    }
    T* out = a.Y + ((size_t)b * a.rows + row) * K + fbase + l * VEC;
#pragma unroll
    for (int q = 0; q < G::NQ; ++q) {
        if (FULL || fbase + (q * G::LPR + l) * VEC < K) store_vec<T, VEC>(out + q * G::LPR * VEC, acc[q]);
    }
}

template <typename T, typename I, int BR, int KT, int VEC>
__global__ void __launch_bounds__(64) pbr_stripe_kernel(PbrArgs<T, I> a) {
    typedef PbrGeom<T, BR, KT, VEC> G;
    __shared__ __attribute__((aligned(16))) T tile[BR * G::STRIDE];
    const int stripe = xcd_remap(blockIdx.x, gridDim.x);
    if (stripe >= a.n_stripes) return;
    const int kt = blockIdx.y;
    const int b = blockIdx.z;
    if ((kt + 1) * KT <= a.K) {
        pbr_stripe_body<T, I, BR, KT, VEC, true>(a, stripe, kt, b, tile);
    } else {
        pbr_stripe_body<T, I, BR, KT, VEC, false>(a, stripe, kt, b, tile);
    }
}

// ---------------------------------------------------------------------------
// Naive CSR baseline (kernels/csr_kernels.cu:5-29 semantics)
// ---------------------------------------------------------------------------

template <typename T, typename I>
__global__ void __launch_bounds__(256) csr_naive_kernel(const I* __restrict__ indptr,
                                                        const I* __restrict__ col_ind,
                                                        const T* __restrict__ vals,
                                                        const T* __restrict__ X, T* __restrict__ Y,
                                                        long long rows, int K) {
    const long long row = (long long)blockIdx.x * 4 + threadIdx.y;
    const int f = blockIdx.y * 64 + threadIdx.x;
    if (row >= rows || f >= K) return;
    T acc = T(0);
    const long long rs = (long long)indptr[row], re = (long long)indptr[row + 1];
    for (long long j = rs; j < re; ++j) acc += vals[j] * X[(size_t)col_ind[j] * K + f];
    Y[(size_t)row * K + f] = acc;
}

// ---------------------------------------------------------------------------
// host-side dispatch
// ---------------------------------------------------------------------------

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Elements per vector load: 16 bytes when rows and bases allow it.
template <typename T>
int pick_vec(int K, int F, const void* X, const void* Y) {
    const int full = 16 / (int)sizeof(T);
    if (F >= full && K % full == 0 && aligned16(X) && aligned16(Y)) return full;
    if (sizeof(T) == 4 && F >= 2 && K % 2 == 0 && ((uintptr_t)X & 7u) == 0 && ((uintptr_t)Y & 7u) == 0)
        return 2;
    return 1;
}

// F (features per lane, 2 lanes per row) for a BOO feature tile: the tile is
// 2F wide, at most 256 bytes.
template <typename T>
int boo_pick_f(int K) {
    const int fmax = 128 / (int)sizeof(T);  // 32 floats / 16 doubles
    int f = 1;
    while (f < fmax && 2 * f < K) f *= 2;
    return f;
}

// Full feature tiles in one launch, a partial last tile (K % 2F != 0) in a
// second one compiled with the per-chunk feature guards.
template <typename T, int F, int VEC, bool A32>
int launch_boo_items_a(const BooArgs<T>& a, hipStream_t s) {
    const int full = a.K / (2 * F);
    if (full > 0) {
        const dim3 grid(round_up8(a.n_items), full, a.batch);
        hipLaunchKernelGGL((boo_items_kernel<T, F, VEC, true, A32>), grid, dim3(64), 0, s, a, 0);
        if (int rc = check_launch("boo_items_kernel")) return rc;
    }
    if (a.K % (2 * F)) {
        const dim3 grid(round_up8(a.n_items), 1, a.batch);
        hipLaunchKernelGGL((boo_items_kernel<T, F, VEC, false, A32>), grid, dim3(64), 0, s, a, full);
        return check_launch("boo_items_kernel");
    }
    return SPMM_OK;
}

// 32-bit X addressing when one batch's X slab is under 4 GiB.
template <typename T, int F, int VEC>
int launch_boo_items(const BooArgs<T>& a, hipStream_t s) {
    if ((uint64_t)a.cols * (uint64_t)a.K * sizeof(T) < (1ull << 32))
        return launch_boo_items_a<T, F, VEC, true>(a, s);
    return launch_boo_items_a<T, F, VEC, false>(a, s);
}

template <typename T>
int boo_dispatch(const BooArgs<T>& a, hipStream_t s) {
    const int F = boo_pick_f<T>(a.K);
    const int VEC = pick_vec<T>(a.K, F, a.X, a.Y);
#define SPMM_BOO_CASE(FF, VV) \
    if (F == FF && VEC == VV) return launch_boo_items<T, FF, VV>(a, s);
    if constexpr (sizeof(T) == 4) {
        SPMM_BOO_CASE(32, 4) SPMM_BOO_CASE(32, 2) SPMM_BOO_CASE(32, 1)
        SPMM_BOO_CASE(16, 4) SPMM_BOO_CASE(16, 2) SPMM_BOO_CASE(16, 1)
        SPMM_BOO_CASE(8, 4) SPMM_BOO_CASE(8, 2) SPMM_BOO_CASE(8, 1)
        SPMM_BOO_CASE(4, 4) SPMM_BOO_CASE(4, 2) SPMM_BOO_CASE(4, 1)
        SPMM_BOO_CASE(2, 2) SPMM_BOO_CASE(2, 1)
        SPMM_BOO_CASE(1, 1)
    } else {
        SPMM_BOO_CASE(16, 2) SPMM_BOO_CASE(16, 1)
        SPMM_BOO_CASE(8, 2) SPMM_BOO_CASE(8, 1)
        SPMM_BOO_CASE(4, 2) SPMM_BOO_CASE(4, 1)
        SPMM_BOO_CASE(2, 2) SPMM_BOO_CASE(2, 1)
        SPMM_BOO_CASE(1, 1)
    }
#undef SPMM_BOO_CASE
    return fail(SPMM_EUNSUPPORTED, "no BOO kernel for F=%d VEC=%d", F, VEC);
}

template <typename T, typename I>
int launch_long_rows(const int* long_rows, int n_long, const I* indptr, const I* col_ind,
                     const T* vals, const T* X, T* Y, long long rows, long long cols, int K,
                     int batch, hipStream_t s) {
    if (n_long == 0 || K == 0 || batch == 0) return SPMM_OK;
    const int full = 16 / (int)sizeof(T);
    const bool vec = (K % full == 0) && aligned16(X) && aligned16(Y);
    if (vec) {
        constexpr int V = 16 / sizeof(T);
        const dim3 grid(n_long, (K + 16 * V - 1) / (16 * V), batch);
        hipLaunchKernelGGL((rows_long_kernel<T, I, V>), grid, dim3(256), 0, s, long_rows, indptr,
                           col_ind, vals, X, Y, rows, cols, K);
    } else {
        const dim3 grid(n_long, (K + 15) / 16, batch);
        hipLaunchKernelGGL((rows_long_kernel<T, I, 1>), grid, dim3(256), 0, s, long_rows, indptr,
                           col_ind, vals, X, Y, rows, cols, K);
    }
    return check_launch("rows_long_kernel");
}

template <typename T>
int boo_matmul_t(const spmm_boo_desc* A, const void* Xv, void* Yv, int64_t batch, int64_t K,
                 void* ws, size_t ws_bytes, hipStream_t s) {
    const T* X = static_cast<const T*>(Xv);
    T* Y = static_cast<T*>(Yv);
    if (A->rows == 0 || K == 0 || batch == 0) return SPMM_OK;
    if (A->n_items <= 0 || !A->items) return fail(SPMM_EINVAL, "BOO schedule is empty; build it with spmm_boo_plan_build");
    if (A->cols > 0 && !X) return fail(SPMM_EINVAL, "X is null");
    if (!Y) return fail(SPMM_EINVAL, "Y is null");
    const size_t need = spmm_boo_workspace_bytes(A, sizeof(T) == 4 ? SPMM_F32 : SPMM_F64, batch, K);
    if (need > ws_bytes || (need && !ws))
        return fail(SPMM_ENOMEM, "BOO workspace too small: need %zu bytes, got %zu", need, ws_bytes);

    BooArgs<T> a;
    a.rows = A->rows;
    a.cols = A->cols;
    a.K = (int)K;
    a.batch = (int)batch;
    a.n_items = A->n_items;
    a.max_nr = A->max_nr;
    a.long_threshold = A->long_threshold;
    a.row_grp_ptr = A->row_grp_ptr;
    a.row_ids = A->row_ids;
    a.col_grp_ptr = A->col_grp_ptr;
    a.col_ids = A->col_ids;
    a.blk_col_grp = A->blk_col_grp;
    a.blk_nz_ptr = A->blk_nz_ptr;
    a.blk_shift = A->blk_shift;
    a.nz_idx = A->nz_idx;
    a.nz_val = static_cast<const T*>(A->nz_val);
    a.rem_indptr = A->rem_indptr;
    a.rem_col_ind = A->rem_col_ind;
    a.rem_vals = static_cast<const T*>(A->rem_vals);
    a.items = A->items;
    a.X = X;
    a.Y = Y;
    a.P = static_cast<T*>(ws);
    int rc = boo_dispatch<T>(a, s);
    if (rc) return rc;
    if (A->n_splits > 0) {
        const dim3 grid(A->n_splits, 1, (unsigned)batch);
        hipLaunchKernelGGL((boo_fixup_kernel<T>), grid, dim3(256), 0, s, A->splits, A->row_grp_ptr,
                           A->row_ids, (const T*)ws, Y, A->rows, (int)K, (int)batch, A->max_nr);
        rc = check_launch("boo_fixup_kernel");
        if (rc) return rc;
    }
    return launch_long_rows<T, int>(A->long_rows, A->n_long, A->rem_indptr, A->rem_col_ind,
                                    static_cast<const T*>(A->rem_vals), X, Y, A->rows, A->cols,
                                    (int)K, (int)batch, s);
}

template <typename T, typename I, int BR, int KT, int VEC>
int launch_pbr(const PbrArgs<T, I>& a, int batch, hipStream_t s) {
    const dim3 grid(round_up8(a.n_stripes), (a.K + KT - 1) / KT, batch);
    hipLaunchKernelGGL((pbr_stripe_kernel<T, I, BR, KT, VEC>), grid, dim3(64), 0, s, a);
    return check_launch("pbr_stripe_kernel");
}

// KT (tile features) is 64 or 256 (float) / 32 or 128 (double); VEC is the
// widest load the lane's run of F features and the buffers allow.
template <typename T, typename I, int BR>
int pbr_dispatch_br(const PbrArgs<T, I>& a, int batch, hipStream_t s) {
    constexpr int small_kt = 256 / (int)sizeof(T);
    constexpr int big_kt = 1024 / (int)sizeof(T);
    const bool big = a.K >= big_kt;
    const int F = (big ? big_kt : small_kt) / (64 / BR);
    const int full = 16 / (int)sizeof(T);
    int vec = 1;
    if (F % full == 0 && a.K % full == 0 && aligned16(a.X) && aligned16(a.Y)) vec = full;
    if (big) {
        if (vec > 1) return launch_pbr<T, I, BR, big_kt, 16 / sizeof(T)>(a, batch, s);
        return launch_pbr<T, I, BR, big_kt, 1>(a, batch, s);
    }
    if constexpr ((small_kt / (64 / BR)) % (16 / sizeof(T)) == 0) {
        if (vec > 1) return launch_pbr<T, I, BR, small_kt, 16 / sizeof(T)>(a, batch, s);
    }
    return launch_pbr<T, I, BR, small_kt, 1>(a, batch, s);
}

template <typename T, typename I>
int pbr_matmul_t(const spmm_pbr_desc* A, const void* Xv, void* Yv, int64_t batch, int64_t K,
                 hipStream_t s) {
    if (A->rows == 0 || K == 0 || batch == 0) return SPMM_OK;
    if (A->block_rows != A->block_cols ||
        (A->block_rows != 2 && A->block_rows != 4 && A->block_rows != 8))
        return fail(SPMM_EUNSUPPORTED,
                    "Unsupported block size for PBR SpMM. Only 2x2, 4x4, and 8x8 are supported.");
    if (!A->stripe_ptr) return fail(SPMM_EINVAL, "PBR stripe_ptr is null");
    const long long n_stripes = (A->rows + A->block_rows - 1) / A->block_rows;
    if (n_stripes > 0x7fffff00LL) return fail(SPMM_EUNSUPPORTED, "too many PBR stripes");
    PbrArgs<T, I> a;
    a.rows = A->rows;
    a.cols = A->cols;
    a.K = (int)K;
    a.n_stripes = (int)n_stripes;
    a.long_threshold = A->long_threshold;
    a.codes = A->codes;
    a.coords = static_cast<const I*>(A->coords);
    a.offsets = static_cast<const I*>(A->offsets);
    a.data = static_cast<const T*>(A->data);
    a.rem_indptr = static_cast<const I*>(A->rem_indptr);
    a.rem_col_ind = static_cast<const I*>(A->rem_col_ind);
    a.rem_vals = static_cast<const T*>(A->rem_vals);
    a.stripe_ptr = A->stripe_ptr;
    a.X = static_cast<const T*>(Xv);
    a.Y = static_cast<T*>(Yv);
    int rc;
    switch (A->block_rows) {
        case 2: rc = pbr_dispatch_br<T, I, 2>(a, (int)batch, s); break;
        case 4: rc = pbr_dispatch_br<T, I, 4>(a, (int)batch, s); break;
        default: rc = pbr_dispatch_br<T, I, 8>(a, (int)batch, s); break;
    }
    if (rc) return rc;
    return launch_long_rows<T, I>(A->long_rows, A->n_long, a.rem_indptr, a.rem_col_ind, a.rem_vals,
                                  a.X, a.Y, A->rows, A->cols, (int)K, (int)batch, s);
}

int check_shape(int64_t batch, int64_t K) {
    if (batch < 0 || K < 0) return fail(SPMM_EINVAL, "negative batch or K");
    if (batch > 65535) return fail(SPMM_EUNSUPPORTED, "batch %lld exceeds 65535", (long long)batch);
    if (K > 0x7fffffffLL) return fail(SPMM_EUNSUPPORTED, "K too large");
    return SPMM_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

const char* spmm_last_error(void) { return g_last_error.c_str(); }

const char* spmm_version(void) { return "spmm_amd 0.1 gfx950"; }

int spmm_boo_plan_build(int32_t rows, int32_t n_row_groups, int32_t num_blocks,
                        const int32_t* h_row_grp_ptr, const int32_t* h_blk_row_grp,
                        const int32_t* h_blk_nz_ptr, const int32_t* h_rem_indptr,
                        int32_t max_item_nnz, int32_t long_threshold, int32_t* h_items,
                        int32_t* h_splits, int32_t item_cap, int32_t* h_long_rows,
                        int32_t* n_items, int32_t* n_slots, int32_t* n_splits, int32_t* n_long) {
    if (rows < 0 || n_row_groups < 0 || num_blocks < 0) return fail(SPMM_EINVAL, "negative sizes");
    if (!h_row_grp_ptr || (num_blocks > 0 && (!h_blk_row_grp || !h_blk_nz_ptr)) || !n_items)
        return fail(SPMM_EINVAL, "null plan input");
    if (max_item_nnz < 1) return fail(SPMM_EINVAL, "max_item_nnz must be positive");
    int items = 0, slots = 0, splits = 0;
    int blk = 0;
    for (int rg = 0; rg < n_row_groups; ++rg) {
        const int bb = blk;
        while (blk < num_blocks && h_blk_row_grp[blk] == rg) ++blk;
        if (blk < num_blocks && h_blk_row_grp[blk] < rg)
            return fail(SPMM_EINVAL, "blocks are not sorted by row group");
        const int be = blk;
        // cut [bb, be) into runs of at most max_item_nnz nonzeros (at least one block each)
        int start = bb;
        int first = 1;
        const int slot_begin = slots;
        do {
            int end = start;
            long long acc = 0;
            while (end < be && end - start < BOO_MAX_ITEM_BLOCKS) {
                const long long w = (long long)h_blk_nz_ptr[end + 1] - h_blk_nz_ptr[end];
                if (end > start && acc + w > max_item_nnz) break;
                acc += w;
                ++end;
            }
            if (h_items) {
                if (items >= item_cap) return fail(SPMM_EINVAL, "item_cap too small");
                h_items[4 * items + 0] = rg;
                h_items[4 * items + 1] = start;
                h_items[4 * items + 2] = end;
                h_items[4 * items + 3] = first ? -1 : slots;
            }
            if (!first) ++slots;
            ++items;
            first = 0;
            start = end;
        } while (start < be);
        if (slots > slot_begin) {
            if (h_items && h_splits) {
                h_splits[3 * splits + 0] = rg;
                h_splits[3 * splits + 1] = slot_begin;
                h_splits[3 * splits + 2] = slots;
            }
            ++splits;
        }
    }
    if (blk != num_blocks) return fail(SPMM_EINVAL, "block row groups out of range");
    *n_items = items;
    if (n_slots) *n_slots = slots;
    if (n_splits) *n_splits = splits;
    if (h_items) {
        int nl = 0;
        if (h_rem_indptr && h_long_rows) {
            for (int r = 0; r < rows; ++r)
                if (h_rem_indptr[r + 1] - h_rem_indptr[r] > long_threshold) h_long_rows[nl++] = r;
        }
        if (n_long) *n_long = nl;
    }
    return SPMM_OK;
}

size_t spmm_boo_workspace_bytes(const spmm_boo_desc* A, spmm_dtype dtype, int64_t batch, int64_t K) {
    if (!A || A->n_slots <= 0 || batch <= 0 || K <= 0) return 0;
    const size_t es = dtype == SPMM_F64 ? 8 : 4;
    return (size_t)A->n_slots * (size_t)batch * (size_t)std::max(A->max_nr, 1) * (size_t)K * es;
}

int spmm_boo_matmul(const spmm_boo_desc* A, spmm_dtype dtype, const void* X, void* Y,
                    int64_t batch, int64_t K, void* workspace, size_t workspace_bytes,
                    void* stream) {
    if (!A) return fail(SPMM_EINVAL, "null BOO descriptor");
    int rc = check_shape(batch, K);
    if (rc) return rc;
    if (A->rows < 0 || A->cols < 0) return fail(SPMM_EINVAL, "negative BOO dims");
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == SPMM_F32) return boo_matmul_t<float>(A, X, Y, batch, K, workspace, workspace_bytes, s);
    if (dtype == SPMM_F64) return boo_matmul_t<double>(A, X, Y, batch, K, workspace, workspace_bytes, s);
    return fail(SPMM_EINVAL, "unknown dtype %d", (int)dtype);
}

int spmm_pbr_matmul(const spmm_pbr_desc* A, spmm_dtype dtype, const void* X, void* Y,
                    int64_t batch, int64_t K, void* stream) {
    if (!A) return fail(SPMM_EINVAL, "null PBR descriptor");
    int rc = check_shape(batch, K);
    if (rc) return rc;
    if (A->rows < 0 || A->cols < 0) return fail(SPMM_EINVAL, "negative PBR dims");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool i64 = A->itype == SPMM_I64;
    if (dtype == SPMM_F32)
        return i64 ? pbr_matmul_t<float, int64_t>(A, X, Y, batch, K, s)
                   : pbr_matmul_t<float, int32_t>(A, X, Y, batch, K, s);
    if (dtype == SPMM_F64)
        return i64 ? pbr_matmul_t<double, int64_t>(A, X, Y, batch, K, s)
                   : pbr_matmul_t<double, int32_t>(A, X, Y, batch, K, s);
    return fail(SPMM_EINVAL, "unknown dtype %d", (int)dtype);
}

int spmm_csr_naive(const void* indptr, const void* col_ind, const void* vals, spmm_itype itype,
                   spmm_dtype dtype, int64_t rows, int64_t cols, const void* X, void* Y, int64_t K,
                   void* stream) {
    (void)cols;
    if (rows < 0 || K < 0) return fail(SPMM_EINVAL, "negative CSR dims");
    if (rows == 0 || K == 0) return SPMM_OK;
    if (K > 64LL * 65535) return fail(SPMM_EUNSUPPORTED, "K too large for the naive kernel");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)((rows + 3) / 4), (unsigned)((K + 63) / 64));
    const dim3 block(64, 4);
#define SPMM_NAIVE(TT, II)                                                                       \
    hipLaunchKernelGGL((csr_naive_kernel<TT, II>), grid, block, 0, s,                          \
                       static_cast<const II*>(indptr), static_cast<const II*>(col_ind),        \
                       static_cast<const TT*>(vals), static_cast<const TT*>(X),                \
                       static_cast<TT*>(Y), (long long)rows, (int)K)
    if (dtype == SPMM_F32) {
        if (itype == SPMM_I64) SPMM_NAIVE(float, int64_t); else SPMM_NAIVE(float, int32_t);
    } else if (dtype == SPMM_F64) {
        if (itype == SPMM_I64) SPMM_NAIVE(double, int64_t); else SPMM_NAIVE(double, int32_t);
    } else {
        return fail(SPMM_EINVAL, "unknown dtype %d", (int)dtype);
    }
#undef SPMM_NAIVE
    return check_launch("csr_naive_kernel");
}

}  // extern "C"
