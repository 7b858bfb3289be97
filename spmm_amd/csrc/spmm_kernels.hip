// libspmm_amd: SpMM kernels for MI355X (gfx950, CDNA4) behind the C ABI of
// include/spmm_amd.h.
//
// Design (one paragraph per kernel; the reference's own kernels launch one CTA
// per sparse block and merge rows with global atomics into a memset Y --
// kernels/boo_kernel.cu:410-595, kernels/pbr_kernel.cu:159-326):
//
//  * boo_stream_kernel -- persistent workgroups of WG waves.  The matrix is
//    staged on the host into tile streams (<= 32 rows x 32 columns, <= 128
//    entries, row starts precomputed; see boo_stage.hpp): one stream per
//    wave, the WG streams of a workgroup in lock step, step s of every member
//    using the same 32 X columns.  Lane (r, h) of a wave accumulates row r of
//    its 32-row slice for half h of a 64-feature tile in registers across the
//    slice's tiles (the BOO blocks, then the short remainder rows) and stores
//    Y once.  Each wave loads 32/WG of the step's X rows D steps ahead, and
//    its tile's entries, row range and the column ids of the tile D steps
//    later DF steps ahead, so a step never waits on a load issued in the
//    same step; the X tile is then assembled in LDS (row stride padded by
//    32 bytes so neighbouring columns fall in distinct banks), one barrier
//    publishes it, and every member reads the columns its rows use.
//  * boo_stream_dma_kernel -- the same walk for float 64-feature tiles, with
//    each wave's share of the next X tile copied from memory straight into
//    LDS by global_load_lds_dwordx4 (no staging registers), whole X rows per
//    instruction.  Both stream kernels store an item's Y rows 4 lanes per row
//    (64-byte runs) after a DPP exchange inside each quad of lanes.
//  * boo_rows_kernel, gather_chunk_kernel, gather_fix_kernel -- the gather
//    pass: rows whose columns are too scattered for X tiles, a lane group per
//    row gathering X rows directly; rows over the long-row threshold in
//    chunk tasks whose partial rows are added in order.
//  * boo_fixup_kernel -- for row slices too heavy for one item, adds the
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
#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <type_traits>
#include <string>
#include <vector>

#include "spmm_amd.h"
#include "boo_stage.hpp"
#include "internal.hpp"

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

}  // namespace

namespace spmm_internal {
int set_error(int code, const char* msg) {
    g_last_error = msg;
    return code;
}
}  // namespace spmm_internal

namespace {

int check_launch(const char* what) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        return fail(SPMM_ELAUNCH, "HIP launch of %s failed: %s", what, hipGetErrorString(e));
    }
    return SPMM_OK;
}

// Launch recorder.  While t_record is set (on this thread), launch() appends
// the kernel, its grid and its block to it instead of launching: the
// *_launch_info entry points run the multiply's own dispatch code this way,
// so what they report is exactly what the multiply launches.
struct LaunchRec {
    const void* fn;
    const char* name;
    dim3 grid, block;
};
thread_local std::vector<LaunchRec>* t_record = nullptr;

template <typename... P, typename... Args>
int launch(const char* name, void (*kern)(P...), dim3 grid, dim3 block, hipStream_t s, Args&&... args) {
    if (t_record) {
        t_record->push_back({reinterpret_cast<const void*>(kern), name, grid, block});
        return SPMM_OK;
    }
    hipLaunchKernelGGL(kern, grid, block, 0, s, std::forward<Args>(args)...);
    return check_launch(name);
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

// store_vec through a global (address space 1) pointer: a global store,
// tracked by the vector-memory counter alone.  A flat store -- what a generic
// pointer the compiler cannot trace to a kernel argument becomes -- also
// holds the LDS counter until it is acknowledged, so the next wait for an
// LDS read would wait for the store too.
template <typename T, int VEC>
__device__ __forceinline__ void store_vec_global(T* p, const T (&in)[VEC]) {
    typedef typename Vec<T, VEC>::type V;
    typedef __attribute__((address_space(1))) V gV;
    V v;
    if constexpr (VEC == 1) {
        v = in[0];
    } else {
#pragma unroll
        for (int e = 0; e < VEC; ++e) v[e] = in[e];
    }
    *(gV*)(p) = v;
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
// BOO: persistent tile stream
// ---------------------------------------------------------------------------

constexpr int ST_ROWS = 32;   // rows of a tile / an item slice (2 lanes per row)
constexpr int ST_COLS = 32;   // columns (X rows) of a tile
constexpr int ST_ENT = 96;    // entries of a tile
constexpr int ST_RS = 33;     // row-start table length
constexpr int ST_WORDS = 8;   // metadata words per tile
constexpr int ST_FLAG_LAST = 1;     // last tile of its item: store the rows
constexpr int ST_FLAG_SERIAL = 2;   // few busy rows: walk them one at a time, lanes along K

template <typename T>
struct StreamArgs {
    int rows, cols, K, batch, n_waves, n_tiles, group;
    const int* tiles;           // 8 words: ent_off, nnz | nc<<8 | nr<<16 | flags<<24, cid_off, row_off, slot
    const uint8_t* tile_rs;
    const T* ent_val;
    const uint8_t* ent_col;
    const int* tcols;
    const int* row_ids;
    const int* wave_tiles;
    const T* X;
    T* Y;
    T* P;
    const uint32_t* blobs;       // record stream (float, group 4), or null
    const uint32_t* blob_first;
    const uint32_t* blob_xid;
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

// LDS copy of one tile entry: local column and value read by one ds_read.
template <typename T> struct alignas(2 * sizeof(T) > 8 ? 16 : 8) NzEntry {
    uint32_t col;
    T val;
};

// Feature tile geometry: lane half h owns the VEC-element chunks 2q+h of the
// tile, q < NQ.  Interleaving the halves keeps the two lanes of a row on
// different LDS banks.  The LDS row stride is padded by 32 bytes so the lanes
// of a wave, which read neighbouring columns, hit distinct banks.
template <typename T, int F, int VEC>
struct BooGeom {
    static constexpr int KT = 2 * F;              // features per tile
    static constexpr int CHUNKS = KT / VEC;       // VEC-chunks per X row slice
    static constexpr int NQ = F / VEC;            // chunks per lane
    static constexpr int STRIDE = KT + 32 / (int)sizeof(T);  // LDS row stride (elements)
    static constexpr int CPI = 64 / CHUNKS;       // columns staged per wave instruction
    static constexpr int NST = ST_COLS / CPI;     // staging instructions per tile
    static_assert(CHUNKS <= 64 && 64 % CHUNKS == 0, "tile too wide for one wave");
};

// Prefetch state of one tile, in two parts with different lead times.
// Far part: the tile's small streaming arrays (entries, row range, row id,
// slot), the column ids, and one word of the metadata of a later tile --
// loaded DF steps ahead, since they come straight from HBM.  Near part: the
// tile's X column tile, gathered from rows that neighbouring tiles share and
// so mostly served by L2 -- loaded D steps ahead, once the column ids are in.
template <typename T> struct Pair;
template <> struct Pair<float> { typedef float type __attribute__((ext_vector_type(2))); };
template <> struct Pair<double> { typedef double type __attribute__((ext_vector_type(2))); };

template <typename T>
struct StFar {
    typename Pair<T>::type v;  // entries 2*lane, 2*lane+1
    uint32_t c;                // their local columns (low byte, next byte)
    int rs0;                   // first entry of this lane's row (the row's end comes from lane+2)
    int row;                   // this lane's row id
    int cid;                   // column id of the column this lane stages in the tile D steps later (clamped to its last)
    int meta;                  // lanes 0-7: metadata word (lane) of the tile DF+D steps later
    int4 m;                    // this tile's metadata words 0-3 (uniform)
    int slot;                  // its word 4: the item's partial slot, -1 for the owner (uniform)
};

template <typename T, int F, int VEC, int NW>
struct StNear {
    T x[NW][VEC];  // this wave's X instructions: instruction i holds column g*NST + i0 + i, g = lane / CHUNKS
};

// Orders this wave's LDS writes before its later LDS reads by other lanes.
// The LDS executes one wave's instructions in order; this only stops the
// compiler from moving memory operations across the point.
__device__ __forceinline__ void wave_lds_fence() {
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ int opaque_copy(int v) {
    int r;
    asm volatile("v_mov_b32 %0, %1" : "=v"(r) : "v"(v));
    return r;
}

// A uniform pointer the compiler cannot trace back to the kernel argument it
// was read from.  Selecting between two such fields (Y or a partial slot)
// otherwise becomes a load through a selected field address, which keeps a
// private copy of the whole argument struct in scratch.
template <typename P>
__device__ __forceinline__ P* opaque_ptr(P* p) {
    asm volatile("" : "+s"(p));
    return p;
}


struct TileMeta {
    int4 m;     // ent_off, nnz | nc<<8 | nr<<16 | flags<<24, cid_off, row_off
    int slot;
};

// The metadata of the tile whose 8 words lanes 8k..8k+7 hold in v.
__device__ __forceinline__ TileMeta meta_of(int v, int k = 0) {
    TileMeta t;
    t.m = make_int4(__builtin_amdgcn_readlane(v, 8 * k), __builtin_amdgcn_readlane(v, 8 * k + 1),
                    __builtin_amdgcn_readlane(v, 8 * k + 2), __builtin_amdgcn_readlane(v, 8 * k + 3));
    t.slot = __builtin_amdgcn_readlane(v, 8 * k + 4);
    return t;
}

// base[idx] with a 32-bit element index: a scalar base plus a 32-bit vector
// offset, so the address costs one integer op.
template <typename V>
__device__ __forceinline__ V ld32(const V* base, uint32_t idx) {
    return *reinterpret_cast<const V*>(reinterpret_cast<const char*>(base) + (size_t)(idx * (uint32_t)sizeof(V)));
}

// Far loads of tile t (metadata tm), the id of column cl of tile tc (metadata
// mc; each lane names the column it stages) and the metadata words of tile
// tn: six vector loads, the same six whatever
// the tiles hold (indices are clamped into valid memory instead of
// branching), so the compiler can count them.
template <typename T, bool SKIP = false>
__device__ __forceinline__ void st_issue_far(StFar<T>& fr, const StreamArgs<T>& a, const TileMeta& tm,
                                             int t, const TileMeta& mc, int tn, int cl) {
    const int lane = threadIdx.x & 63;
    fr.m = tm.m;
    fr.slot = tm.slot;
    const int nnz = tm.m.y & 0xff, nr = (tm.m.y >> 16) & 0xff;
    const int nc = (mc.m.y >> 8) & 0xff;
    const int lr = lane >> 1;
    // entries 2*lane, 2*lane+1 (tiles start at even entries; past nnz: padding)
    const uint32_t k = (uint32_t)(tm.m.x + 2 * min(lane, max((nnz - 1) >> 1, 0)));
    // SKIP (for a kernel that waits for all its loads at every step rather
    // than counting them): no entries or row starts for an empty tile, row ids
    // only for the tile that stores its rows -- uniform branches
    if (!SKIP || nnz > 0) {
        fr.v = *reinterpret_cast<const typename Pair<T>::type*>(
            reinterpret_cast<const char*>(a.ent_val) + (size_t)(k * (uint32_t)sizeof(T)));
        fr.c = ld32(reinterpret_cast<const uint16_t*>(a.ent_col), k >> 1);
        fr.rs0 = ld32(a.tile_rs, (uint32_t)t * ST_RS + (uint32_t)lr);
    } else {
        fr.rs0 = 0;
    }
    if (!SKIP || ((tm.m.y >> 24) & ST_FLAG_LAST))
        fr.row = ld32(a.row_ids, (uint32_t)(tm.m.w + min(lr, max(nr - 1, 0))));
    else
        fr.row = 0;
    fr.cid = ld32(a.tcols, (uint32_t)(mc.m.z + min(cl, max(nc - 1, 0))));
    fr.meta = ld32(a.tiles, (uint32_t)ST_WORDS * (uint32_t)tn + (uint32_t)(lane & 7));
}

// Near loads: this wave's share (NW staging instructions starting at i0) of
// the X column tile whose column ids are in colbuf (all 32 entries hold valid
// ids, so no load is predicated).
template <typename T, int F, int VEC, int NW, bool FULL, bool A32>
__device__ __forceinline__ void st_issue_near(StNear<T, F, VEC, NW>& nr, const StreamArgs<T>& a,
                                              const int* colbuf, int i0, const T* __restrict__ Xb,
                                              int fbase) {
    typedef BooGeom<T, F, VEC> G;
    const int lane = threadIdx.x & 63;
    const int g = lane / G::CHUNKS;
    const int ch = lane % G::CHUNKS;
    const int f = FULL ? fbase + ch * VEC : min(fbase + ch * VEC, a.K - VEC);
    int col[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) col[i] = colbuf[g * G::NST + i0 + i];
    if constexpr (A32) {
        const uint32_t rowb = (uint32_t)a.K * (uint32_t)sizeof(T);
        const uint32_t fb = (uint32_t)f * (uint32_t)sizeof(T);
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const uint32_t off = __umul24((uint32_t)col[i], rowb) + fb;
            load_vec<T, VEC>(reinterpret_cast<const T*>(reinterpret_cast<const char*>(Xb) + (size_t)off), nr.x[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NW; ++i) load_vec<T, VEC>(Xb + (size_t)col[i] * a.K + f, nr.x[i]);
    }
}

// Accumulate entries [j, e) of the LDS tile into this lane's row.  The next
// entry is read while the current one's X row is read and used, so each
// iteration waits on one LDS round trip, not two.  The read-ahead reaches
// nzp[e] at most, which is inside the workgroup's LDS (e <= ST_ENT + ST_SYN,
// and nzp is followed by colbuf).  Addresses are formed in 32 bits in the
// LDS address space (one 24-bit multiply-add per entry).
template <typename T, int F, int VEC, bool FULL>
__device__ __forceinline__ void st_row(T (&acc)[F / VEC][VEC], int j, int e, const NzEntry<T>* nzp,
                                       const T* __restrict__ tile, int K, int fbase, int h) {
    typedef BooGeom<T, F, VEC> G;
    if (j >= e) return;
    typedef __attribute__((address_space(3))) const char lds_char;
    typedef __attribute__((address_space(3))) const T lds_t;
    lds_char* tb = (lds_char*)(tile) + h * VEC * (int)sizeof(T);
    auto entry = [&](const NzEntry<T>& ent) {
        const T* xr = (const T*)(lds_t*)(tb + __umul24(ent.col, (uint32_t)(G::STRIDE * sizeof(T))));
        T x[G::NQ][VEC];
#pragma unroll
        for (int q = 0; q < G::NQ; ++q)
            if (FULL || fbase + (2 * q + h) * VEC < K) load_vec<T, VEC>(xr + 2 * q * VEC, x[q]);
#pragma unroll
        for (int q = 0; q < G::NQ; ++q) {
            if (FULL || fbase + (2 * q + h) * VEC < K) {
#pragma unroll
                for (int u = 0; u < VEC; ++u) acc[q][u] += ent.val * x[q][u];
            }
        }
    };
    NzEntry<T> ent = nzp[j];
#pragma nounroll
    for (; j < e; ++j) {
        const NzEntry<T> nxt = nzp[j + 1];
        __builtin_amdgcn_sched_barrier(0);
        entry(ent);
        ent = nxt;
    }
}

constexpr int ST_SYN = 4;   // busy rows a serial tile may have

// A tile whose entries sit in a few busy rows: the whole wave takes one busy
// row at a time with lanes along the tile's features, and leaves the row's
// sums in LDS as row k of syn with a matching entry {k, 1} (nzp[ST_ENT + k]);
// the row's lanes get that one entry as their range, so the ordinary row pass
// over syn adds the sums (multiplying by 1 is exact).  busy: bit 2r set for
// each busy row r; rs: this lane's row range (lane 2r holds row r's),
// replaced for the busy rows' lanes.
template <typename T, int F, int VEC, bool FULL>
__device__ __forceinline__ void st_serial(uint64_t busy, int& rs0, int& rs1, NzEntry<T>* __restrict__ nzp,
                                          const T* __restrict__ tile, T* __restrict__ syn, int K,
                                          int fbase) {
    typedef BooGeom<T, F, VEC> G;
    const int lane = threadIdx.x & 63;
    const bool fok = lane < G::KT && (FULL || fbase + lane < K);
    const T* xc = tile + (lane < G::KT ? lane : 0);
    const int in0 = rs0, in1 = rs1;
    for (int k = 0; busy; ++k) {
        const int l2 = __builtin_ctzll(busy);
        busy &= busy - 1;
        int j = __builtin_amdgcn_readlane(in0, l2);
        const int e = __builtin_amdgcn_readlane(in1, l2);
        T s0 = T(0), s1 = T(0);
        for (; j + 2 <= e; j += 2) {
            const NzEntry<T> a0 = nzp[j], a1 = nzp[j + 1];
            s0 += a0.val * xc[a0.col * G::STRIDE];
            s1 += a1.val * xc[a1.col * G::STRIDE];
        }
        if (j < e) {
            const NzEntry<T> a0 = nzp[j];
            s0 += a0.val * xc[a0.col * G::STRIDE];
        }
        if (lane < G::KT) syn[k * G::STRIDE + lane] = fok ? s0 + s1 : T(0);
        if (lane == 0) nzp[ST_ENT + k] = NzEntry<T>{(uint32_t)k, T(1)};
        if ((lane & ~1) == l2) {
            rs0 = ST_ENT + k;
            rs1 = ST_ENT + k + 1;
        }
    }
}

// Store an item's rows: lane (r, h) writes its half of row r (to Y, or to the
// row of a partial slot).
template <typename T, int F, int VEC, bool FULL>
__device__ __forceinline__ void st_store(const StreamArgs<T>& a, const T (&acc)[F / VEC][VEC], int row,
                                         int slot, int nrow, int b, int fbase) {
    typedef BooGeom<T, F, VEC> G;
    const int lane = threadIdx.x & 63;
    const int h = lane & 1;
    const int lr = lane >> 1;
    const int K = a.K;
    if (lr < nrow) {
        T* out = slot < 0 ? opaque_ptr(a.Y) + ((size_t)b * a.rows + row) * K + fbase + h * VEC
                          : opaque_ptr(a.P) + (((size_t)slot * a.batch + b) * ST_ROWS + lr) * K + fbase + h * VEC;
#pragma unroll
        for (int q = 0; q < G::NQ; ++q)
            if (FULL || fbase + (2 * q + h) * VEC < K) store_vec_global<T, VEC>(out + 2 * q * VEC, acc[q]);
    }
}

// One element moved from lane i ^ 2 of its quad (DPP quad_perm(2,3,0,1)),
// 32 bits at a time.
__device__ __forceinline__ float quad_xor2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ double quad_xor2(double v) {
    const long long w = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_mov_dpp((int)(unsigned)(w & 0xffffffffll), 0x4E, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_mov_dpp((int)(w >> 32), 0x4E, 0xF, 0xF, false);
    return __builtin_bit_cast(double, ((long long)hi << 32) | (long long)(unsigned)lo);
}

// st_store with 4 lanes per row, for 16-byte chunks (VEC * sizeof(T) = 16)
// and an even number of chunks per lane.  Lane 2r + h holds chunks 2q + h of
// row r, so plain stores write 32 bytes to each of 32 rows per instruction.
// The quad of lanes 4m .. 4m+3 holds rows 2m and 2m+1; swapping one chunk of
// each pair (2s, 2s + 1) between lanes i and i ^ 2 (DPP quad_perm) gives lane
// i chunk 4s + i of row 2m (store 2s) and of row 2m + 1 (store 2s + 1), so
// every store instruction writes 64 contiguous bytes to each of 16 rows: half
// the write requests (config 2 62.8 -> 61.1 us, config 1 18.3 -> 16.9 us).  A
// second exchange between lanes j and j ^ 4 for whole 128-byte lines cost
// more than it saved (61.5 and 17.3 us).
template <typename T, int F, int VEC, bool FULL>
__device__ __forceinline__ void st_store_quad(const StreamArgs<T>& a, const T (&acc)[F / VEC][VEC], int row,
                                              int slot, int nrow, int b, int fbase) {
    static_assert(VEC * sizeof(T) == 16 && (F / VEC) % 2 == 0, "16-byte chunks, an even number per lane");
    constexpr int NQ = F / VEC;
    const int lane = threadIdx.x & 63;
    const int i = lane & 3;
    const bool hi = (lane & 2) != 0;
    const int m2 = (lane >> 2) * 2;                                         // the quad's first local row
    const int ra = __builtin_amdgcn_mov_dpp(row, 0x00, 0xF, 0xF, false);   // row 2m's id (quad lane 0)
    const int rb = __builtin_amdgcn_mov_dpp(row, 0xAA, 0xF, 0xF, false);   // row 2m+1's id (quad lane 2)
    const int K = a.K;
    T* oa;
    T* ob;
    if (slot < 0) {
        oa = opaque_ptr(a.Y) + ((size_t)b * a.rows + ra) * K + fbase + i * VEC;
        ob = opaque_ptr(a.Y) + ((size_t)b * a.rows + rb) * K + fbase + i * VEC;
    } else {
        oa = opaque_ptr(a.P) + (((size_t)slot * a.batch + b) * ST_ROWS + m2) * K + fbase + i * VEC;
        ob = oa + K;
    }
    const bool wa = m2 < nrow, wb = m2 + 1 < nrow;
#pragma unroll
    for (int s = 0; s < NQ / 2; ++s) {
        T own[VEC], rcv[VEC], da[VEC], db[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) {
            own[u] = hi ? acc[2 * s + 1][u] : acc[2 * s][u];
            rcv[u] = quad_xor2(hi ? acc[2 * s][u] : acc[2 * s + 1][u]);
            da[u] = hi ? rcv[u] : own[u];   // chunk 4s + i of row 2m
            db[u] = hi ? own[u] : rcv[u];   // chunk 4s + i of row 2m + 1
        }
        if (!FULL && fbase + (4 * s + i) * VEC >= K) continue;
        if (wa) store_vec_global<T, VEC>(oa + 4 * s * VEC, da);
        if (wb) store_vec_global<T, VEC>(ob + 4 * s * VEC, db);
    }
}

// LDS of one workgroup of WG waves: the shared X tile, double-buffered, and
// per wave its entries, its serial-row sums and its column ids.
template <typename T, int F, int VEC, int WG>
struct StLds {
    typedef BooGeom<T, F, VEC> G;
    T tile[2][ST_COLS * G::STRIDE];
    T syn[WG][ST_SYN * G::STRIDE];
    NzEntry<T> nzp[WG][ST_ENT + ST_SYN];
    int colbuf[WG][ST_COLS];
};

// Every wave of the workgroup has written its share of the X tile.  Only LDS
// writes need to be complete (lgkmcnt), never the loads still in flight.
template <int WG>
__device__ __forceinline__ void group_sync() {
    if constexpr (WG > 1) {
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
        wave_lds_fence();
    }
}

// Workgroups of WG waves; wave v of workgroup b streams the tiles
// [wave_tiles[b*WG+v], wave_tiles[b*WG+v+1]) of its items for one feature
// tile.  The WG streams of a workgroup have equal lengths and, step by step,
// the same X tile (column chunk), so each wave loads 1/WG of it and the
// workgroup shares it in LDS (double-buffered: one barrier per step).  A
// tile's far loads (entries, row range, row id) are issued DF steps before it
// is computed, together with the column ids of the tile D steps after it and
// the metadata of the tile DF+D steps after it; its X loads are issued D
// steps before it is computed.  So every wait is for loads issued at least D
// steps earlier, and every step issues the same loads, which lets the
// compiler count them.  Lane (r, h) keeps F accumulators of row r across the
// item's tiles and stores them once, at the item's last tile (to Y, or to a
// partial slot of a split item).  Steps past the end of the stream load its
// last tile (the data is never used) and store nothing.
// Waves per SIMD the kernel is compiled for, as many as its registers allow
// without spilling: fp64 with 16 features per lane 2 (the 64 accumulators and
// the X staging registers), with 8 features 3; a one-wave workgroup of float
// 64-feature tiles stages all 32 X columns itself, 2.
template <typename T, int F, int VEC, int WG>
constexpr int stream_occupancy() {
    if (sizeof(T) == 8) return F >= 16 ? 2 : F >= 8 ? 3 : 4;
    return F >= 32 && WG == 1 ? 2 : 4;
}

template <typename T, int F, int VEC, int D, int DF, int WG, bool FULL, bool A32>
__global__ void __launch_bounds__(64 * WG, (stream_occupancy<T, F, VEC, WG>())) boo_stream_kernel(StreamArgs<T> a,
                                                                                                  int kt0) {
    typedef BooGeom<T, F, VEC> G;
    constexpr int NW = G::NST / WG;   // X staging instructions per wave
    static_assert(G::NST % WG == 0, "X tile does not split over the workgroup");
    static_assert(DF % D == 0 && DF > D && ST_WORDS * (DF + D) <= 64, "bad prefetch depths");
    __shared__ __attribute__((aligned(16))) StLds<T, F, VEC, WG> L;
    const int wv = threadIdx.x >> 6;
    const int w = xcd_remap(blockIdx.x, gridDim.x) * WG + wv;
    if (w >= a.n_waves) return;  // uniform per workgroup: n_waves is a multiple of WG
    const int lane = threadIdx.x & 63;
    const int h = lane & 1;
    const int lr = lane >> 1;
    const int K = a.K;
    const int fbase = (kt0 + (int)blockIdx.y) * G::KT;
    const int b = blockIdx.z;
    const T* Xb = a.X + (size_t)b * a.cols * K;
    const int t0 = a.wave_tiles[w], t1 = a.wave_tiles[w + 1];
    if (t0 >= t1) return;  // uniform per workgroup: its streams have equal lengths
    const int tl = t1 - 1;
    auto cl = [tl](int t) { return min(t, tl); };
    int* colbuf = L.colbuf[wv];
    NzEntry<T>* nzp = L.nzp[wv];
    T* syn = L.syn[wv];
    const int i0 = wv * NW;           // first staging instruction of this wave

    StFar<T> fr[DF];
    StNear<T, F, VEC, NW> nr[D];
    TileMeta msave[DF];   // msave[(t - t0) % DF]: metadata of tile t+DF+D, kept D steps
    {
        // metadata of tiles t0 .. t0+DF+D-1 (lanes 8k..8k+7: tile t0+k)
        const int mw = ld32(a.tiles, (uint32_t)ST_WORDS * (uint32_t)cl(t0 + (lane >> 3)) + (uint32_t)(lane & 7));
        // column ids of tiles t0 .. t0+D-1
        int cid0[D];
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int4 m = meta_of(mw, j).m;
            cid0[j] = ld32(a.tcols, (uint32_t)(m.z + min(lane & 31, max(((m.y >> 8) & 0xff) - 1, 0))));
        }
        // The far loads of tiles t0 .. t0+DF-1 and the X loads of t0 ..
        // t0+D-1, issued in the order the DF steps before t0 would have
        // issued them (X of tile u at step u-D, far of tile u at step u-DF),
        // so the waits the compiler derives for the loop hold from its first
        // step on.
#pragma unroll
        for (int j = 0; j < DF; ++j) {
            if (j >= DF - D) {
                const int u = j - (DF - D);
                if (lane < ST_COLS) colbuf[lane] = cid0[u];
                wave_lds_fence();
                st_issue_near<T, F, VEC, NW, FULL, A32>(nr[u], a, colbuf, i0, Xb, fbase);
                wave_lds_fence();
            }
            st_issue_far<T>(fr[j], a, meta_of(mw, j), cl(t0 + j), meta_of(mw, j + D), cl(t0 + j + DF + D),
                            lane & 31);
        }
#pragma unroll
        for (int j = 0; j < D; ++j) msave[(DF - D + j) % DF] = meta_of(mw, DF + j);
    }

    T acc[G::NQ][VEC];
#pragma unroll
    for (int q = 0; q < G::NQ; ++q)
#pragma unroll
        for (int u = 0; u < VEC; ++u) acc[q][u] = T(0);

    // One step: tile t (step n of the stream), whose far loads are in FR and
    // X loads in NR.  MS is msave[s]; MP is msave[(s - D) mod DF], the
    // metadata of tile t+DF.
    auto step = [&](StFar<T>& FR, StNear<T, F, VEC, NW>& NR, TileMeta& MS, const TileMeta& MP, int t,
                    int n, bool real) {
        const int4 mt = FR.m;
        const int nnz = mt.y & 0xff;
        T* tile = L.tile[n & 1];
        // (1) this wave's share of X tile t to LDS; entries; column ids of
        // tile t+D to colbuf
        {
            const int g = lane / G::CHUNKS, ch = lane % G::CHUNKS;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                if (FULL || fbase + ch * VEC < K)
                    store_vec<T, VEC>(tile + (g * G::NST + i0 + i) * G::STRIDE + ch * VEC, NR.x[i]);
            }
            if (2 * lane < nnz) {
                NzEntry<T>* e = nzp + 2 * lane;
                e[0] = NzEntry<T>{FR.c & 0xffu, FR.v.x};
                e[1] = NzEntry<T>{(FR.c >> 8) & 0xffu, FR.v.y};
            }
            if (lane < ST_COLS) colbuf[lane] = FR.cid;
        }
        // Copies of what this step still needs from FR after FR is refilled.
        // The copies are opaque to the compiler, so the refill can reuse FR's
        // registers instead of loading into fresh ones that would then be
        // copied (and waited for) at the loop back-edge.
        int rs0 = opaque_copy(FR.rs0);
        int rs1 = __shfl_down(rs0, 2);          // the next row's start
        if (lr == ST_ROWS - 1) rs1 = nnz;
        const int row = opaque_copy(FR.row);
        const int slot = FR.slot;
        const TileMeta mfar = MP;                  // tile t+DF
        const TileMeta mnew = meta_of(FR.meta);    // tile t+DF+D
        MS = mnew;
        group_sync<WG>();
        __builtin_amdgcn_sched_barrier(0);
        // (2) X loads of tile t+D; far loads of tile t+DF
        st_issue_near<T, F, VEC, NW, FULL, A32>(NR, a, colbuf, i0, Xb, fbase);
        st_issue_far<T>(FR, a, mfar, cl(t + DF), mnew, cl(t + 2 * DF + D), lane & 31);
        __builtin_amdgcn_sched_barrier(0);
        // (3) tile t (a step past the range recomputes the last tile into an
        // accumulator that is never stored again)
        const T* src = tile;
        if ((mt.y >> 24) & ST_FLAG_SERIAL) {
            const uint64_t busy = __ballot(h == 0 && rs0 != rs1);
            st_serial<T, F, VEC, FULL>(busy, rs0, rs1, nzp, tile, syn, K, fbase);
            wave_lds_fence();
            src = syn;
        }
        st_row<T, F, VEC, FULL>(acc, rs0, rs1, nzp, src, K, fbase, h);
        wave_lds_fence();
        // (4) end of the item: store its rows
        if (real && ((mt.y >> 24) & ST_FLAG_LAST)) {
            const int nrow = (mt.y >> 16) & 0xff;
            if constexpr (VEC * sizeof(T) == 16 && (F / VEC) % 2 == 0)
                st_store_quad<T, F, VEC, FULL>(a, acc, row, slot, nrow, b, fbase);
            else
                st_store<T, F, VEC, FULL>(a, acc, row, slot, nrow, b, fbase);
#pragma unroll
            for (int q = 0; q < G::NQ; ++q)
#pragma unroll
                for (int u = 0; u < VEC; ++u) acc[q][u] = T(0);
        }
    };

    for (int tb = t0; tb < t1; tb += DF) {
#pragma unroll
        for (int s = 0; s < DF; ++s)
            step(fr[s], nr[s % D], msave[s], msave[(s + DF - D) % DF], tb + s, tb + s - t0, tb + s < t1);
    }
}

// ---------------------------------------------------------------------------
// BOO tile stream, float, 64-feature tiles: X tiles staged by LDS DMA.
//
// The same stream, steps and barriers as boo_stream_kernel (WG = 4), but each
// wave's share of the next X tile goes from memory straight to LDS with two
// global_load_lds_dwordx4 (no registers, no LDS writes), issued last in a
// step; the next step's s_waitcnt vmcnt(0) before its barrier is then the
// only wait for it, and counting nothing is needed to be correct.  DMA
// instruction I (of 8) stages columns I, I+8, I+16 and I+24 as whole 256-byte
// feature rows, 16 neighbouring lanes per row, so it reads 8 whole lines; its
// 1 KiB block starts at I * DMA_BLK, and the 32 bytes of padding per block put
// columns that differ mod 8 on distinct banks.  Lane (r, h) reads the 8
// chunks 2m+h of a column at one base plus 32-byte immediates.  Y rows leave
// through st_store_quad (4 lanes per row).
// ---------------------------------------------------------------------------

#ifndef SPMM_BOO_DMA_HALVES
#define SPMM_BOO_DMA_HALVES 1   // parts an entry's X row is read in by the LDS-DMA kernel's walk
#endif
#ifndef SPMM_BOO_DMA_OCC
#define SPMM_BOO_DMA_OCC 4      // waves per SIMD the LDS-DMA kernel is compiled for
#endif
constexpr int DMA_BLK = 1056;  // bytes between DMA instruction blocks (1 KiB + 32)
template <int WG>
struct StDmaLds {
    float tile[2][8 * DMA_BLK / 4];
    float syn[WG * ST_SYN * 64];                // wave w's serial row k: 256-byte row ST_SYN w + k
    NzEntry<float> nzp[WG][ST_ENT + ST_SYN];
    int spare[4];                               // the row pass reads one entry past its range
};

// LDS byte offset of column c of a tile: DMA instruction I = c % 8 holds
// columns I, I+8, I+16, I+24, each as a whole 256-byte feature row (16
// neighbouring lanes per row: whole lines), blocks DMA_BLK apart.
__device__ __forceinline__ uint32_t dma_col_off(uint32_t c) { return (c & 7u) * (uint32_t)DMA_BLK + ((c >> 3) << 8); }

// Low 32 bits of a generic pointer into LDS: the LDS byte address.
__device__ __forceinline__ uint32_t lds_u32(const void* p) { return (uint32_t)(uintptr_t)p; }

// 64 lanes x 16 bytes from gbase + voff (per lane) to LDS [ldsa, ldsa + 1 KiB),
// lane i at ldsa + 16 i.
__device__ __forceinline__ void dma16(const float* gbase, uint32_t voff, uint32_t ldsa) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(gbase), "s"(ldsa)
                 : "memory", "m0");
}

// st_row for the DMA tile: entries carry their column's LDS byte offset.
__device__ __forceinline__ void dma_row(float (&acc)[8][4], int j, int e, const NzEntry<float>* nzp,
                                        const float* tile, int h) {
    if (j >= e) return;
    typedef __attribute__((address_space(3))) const char lds_char;
    lds_char* tb = (lds_char*)(tile) + h * 16;
    NzEntry<float> ent = nzp[j];
#pragma nounroll
    for (; j < e; ++j) {
        const NzEntry<float> nxt = nzp[j + 1];
        __builtin_amdgcn_sched_barrier(0);
        const float* xr = (const float*)(lds_char*)(tb + ent.col);
        // the row's 32 features in SPMM_BOO_DMA_HALVES parts, each read and
        // used before the next is read (fewer registers in flight)
        constexpr int QP = 8 / SPMM_BOO_DMA_HALVES;
#pragma unroll
        for (int p = 0; p < SPMM_BOO_DMA_HALVES; ++p) {
            float x[QP][4];
#pragma unroll
            for (int q = 0; q < QP; ++q) load_vec<float, 4>(xr + (p * QP + q) * 8, x[q]);
#pragma unroll
            for (int q = 0; q < QP; ++q)
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[p * QP + q][u] += ent.val * x[q][u];
            if (p + 1 < SPMM_BOO_DMA_HALVES) __builtin_amdgcn_sched_barrier(0);
        }
        ent = nxt;
    }
}

// st_serial for the DMA tile: lane f takes feature f; busy row k's
// sums become row ST_SYN wv + k of the syn rows (256 bytes each).
__device__ __forceinline__ void dma_serial(uint64_t busy, int& rs0, int& rs1, NzEntry<float>* nzp,
                                           const float* tile, float* syn, int wv) {
    const int lane = threadIdx.x & 63;
    const int fo = lane;  // feature lane's offset (floats) inside a column's row
    const float* xc = tile + fo;
    const int in0 = rs0, in1 = rs1;
    for (int k = 0; busy; ++k) {
        const int l2 = __builtin_ctzll(busy);
        busy &= busy - 1;
        int j = __builtin_amdgcn_readlane(in0, l2);
        const int e = __builtin_amdgcn_readlane(in1, l2);
        float s0 = 0.f, s1 = 0.f;
        for (; j + 2 <= e; j += 2) {
            const NzEntry<float> a0 = nzp[j], a1 = nzp[j + 1];
            s0 += a0.val * xc[a0.col >> 2];
            s1 += a1.val * xc[a1.col >> 2];
        }
        if (j < e) {
            const NzEntry<float> a0 = nzp[j];
            s0 += a0.val * xc[a0.col >> 2];
        }
        const uint32_t col = (uint32_t)(ST_SYN * wv + k) * 256u;
        syn[fo + (col >> 2)] = s0 + s1;
        if (lane == 0) nzp[ST_ENT + k] = NzEntry<float>{col, 1.f};
        if ((lane & ~1) == l2) {
            rs0 = ST_ENT + k;
            rs1 = ST_ENT + k + 1;
        }
    }
}

// WG waves (2 or 4) share each X tile: the tile's 8 DMA instructions are
// split 8/WG per wave.
template <int DF, int WG>
__global__ void __launch_bounds__(64 * WG, SPMM_BOO_DMA_OCC) boo_stream_dma_kernel(StreamArgs<float> a, int kt0) {
    constexpr int D = 1;
    constexpr int NI = 8 / WG;  // DMA instructions per wave and tile
    static_assert(DF > D && ST_WORDS * (DF + D) <= 64, "bad prefetch depth");
    static_assert(WG == 2 || WG == 4, "the X tile splits over 2 or 4 waves");
    __shared__ __attribute__((aligned(16))) StDmaLds<WG> L;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int w = xcd_remap(blockIdx.x, gridDim.x) * WG + wv;
    if (w >= a.n_waves) return;  // uniform per workgroup: n_waves is a multiple of WG
    const int lane = threadIdx.x & 63;
    const int h = lane & 1;
    const int lr = lane >> 1;
    const int fbase = (kt0 + (int)blockIdx.y) * 64;
    const int b = blockIdx.z;
    const float* Xb = a.X + (size_t)b * a.cols * a.K;
    const int t0 = a.wave_tiles[w], t1 = a.wave_tiles[w + 1];
    if (t0 >= t1) return;  // uniform per workgroup: its streams have equal lengths
    const int tl = t1 - 1;
    auto cl = [tl](int t) { return min(t, tl); };
    NzEntry<float>* nzp = L.nzp[wv];
    const uint32_t rowb = (uint32_t)a.K * 4u;
    // this wave's DMA instructions I = NI wv + k (k < NI) stage columns
    // I + 8 (lane / 16), chunk lane % 16.  A lane loads the column id of one
    // of its NI columns (scol) and takes the others from the lanes next to it:
    // NI = 2, from lane ^ 1; NI = 4, by broadcast inside its group of four.
    const int scol = NI * wv + 8 * (lane >> 4) + (lane & (NI - 1));
    const uint32_t lane_off = (uint32_t)fbase * 4u + (uint32_t)(lane & 15) * 16u;
    const bool odd = (lane & 1) != 0;
    auto issue_dma = [&](int cid, int buf) {
        const uint32_t l0 = lds_u32(&L.tile[buf][0]) + (uint32_t)(NI * wv) * (uint32_t)DMA_BLK;
        if constexpr (NI == 2) {
            const int oth = __builtin_amdgcn_mov_dpp(cid, 0xB1, 0xF, 0xF, false);  // lane ^ 1
            const uint32_t c0 = (uint32_t)(odd ? oth : cid), c1 = (uint32_t)(odd ? cid : oth);
            dma16(Xb, __umul24(c0, rowb) + lane_off, l0);
            dma16(Xb, __umul24(c1, rowb) + lane_off, l0 + (uint32_t)DMA_BLK);
        } else {
            // quad_perm(k, k, k, k): every lane of a group of four takes lane k's id
            const uint32_t c0 = (uint32_t)__builtin_amdgcn_mov_dpp(cid, 0x00, 0xF, 0xF, false);
            const uint32_t c1 = (uint32_t)__builtin_amdgcn_mov_dpp(cid, 0x55, 0xF, 0xF, false);
            const uint32_t c2 = (uint32_t)__builtin_amdgcn_mov_dpp(cid, 0xAA, 0xF, 0xF, false);
            const uint32_t c3 = (uint32_t)__builtin_amdgcn_mov_dpp(cid, 0xFF, 0xF, 0xF, false);
            dma16(Xb, __umul24(c0, rowb) + lane_off, l0);
            dma16(Xb, __umul24(c1, rowb) + lane_off, l0 + (uint32_t)DMA_BLK);
            dma16(Xb, __umul24(c2, rowb) + lane_off, l0 + 2u * (uint32_t)DMA_BLK);
            dma16(Xb, __umul24(c3, rowb) + lane_off, l0 + 3u * (uint32_t)DMA_BLK);
        }
    };

    StFar<float> fr[DF];
    TileMeta msave[DF];
    {
        const int mw = ld32(a.tiles, (uint32_t)ST_WORDS * (uint32_t)cl(t0 + (lane >> 3)) + (uint32_t)(lane & 7));
        const int4 m0 = meta_of(mw, 0).m;
        const int cid0 = ld32(a.tcols, (uint32_t)(m0.z + min(scol, max(((m0.y >> 8) & 0xff) - 1, 0))));
#pragma unroll
        for (int j = 0; j < DF; ++j)
            st_issue_far<float, true>(fr[j], a, meta_of(mw, j), cl(t0 + j), meta_of(mw, j + D),
                                      cl(t0 + j + DF + D), scol);
        issue_dma(cid0, 0);
        msave[DF - D] = meta_of(mw, DF);
    }

    float acc[8][4];
#pragma unroll
    for (int q = 0; q < 8; ++q)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[q][u] = 0.f;

    auto step = [&](StFar<float>& FR, TileMeta& MS, const TileMeta& MP, int t, int n, bool real) {
        const int4 mt = FR.m;
        const int nnz = mt.y & 0xff;
        const float* tile = L.tile[n & 1];
        if (2 * lane < nnz) {
            NzEntry<float>* e = nzp + 2 * lane;
            e[0] = NzEntry<float>{dma_col_off(FR.c & 0xffu), FR.v.x};
            e[1] = NzEntry<float>{dma_col_off((FR.c >> 8) & 0xffu), FR.v.y};
        }
        int rs0 = opaque_copy(FR.rs0);
        int rs1 = __shfl_down(rs0, 2);          // the next row's start
        if (lr == ST_ROWS - 1) rs1 = nnz;
        const int row = opaque_copy(FR.row);
        const int cidn = opaque_copy(FR.cid);
        const int slot = FR.slot;
        const TileMeta mfar = MP;                  // tile t+DF
        const TileMeta mnew = meta_of(FR.meta);    // tile t+DF+D
        MS = mnew;
        __builtin_amdgcn_sched_barrier(0);
        // every load of the last step has landed (this wave's DMA share of
        // tile t among them); the barrier publishes the whole tile
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        st_issue_far<float, true>(FR, a, mfar, cl(t + DF), mnew, cl(t + 2 * DF + D), scol);
        __builtin_amdgcn_sched_barrier(0);
        issue_dma(cidn, (n + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        const float* src = tile;
        if ((mt.y >> 24) & ST_FLAG_SERIAL) {
            const uint64_t busy = __ballot(h == 0 && rs0 != rs1);
            dma_serial(busy, rs0, rs1, nzp, tile, L.syn, wv);
            wave_lds_fence();
            src = L.syn;
        }
        dma_row(acc, rs0, rs1, nzp, src, h);
        wave_lds_fence();
        if (real && ((mt.y >> 24) & ST_FLAG_LAST)) {
            const int nrow = (mt.y >> 16) & 0xff;
            st_store_quad<float, 32, 4, true>(a, acc, row, slot, nrow, b, fbase);
#pragma unroll
            for (int q = 0; q < 8; ++q)
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[q][u] = 0.f;
        }
    };

    for (int tb = t0; tb < t1; tb += DF) {
#pragma unroll
        for (int s = 0; s < DF; ++s)
            step(fr[s], msave[s], msave[(s + DF - D) % DF], tb + s, tb + s - t0, tb + s < t1);
    }
    // the last step's DMA lands before the workgroup's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// ---------------------------------------------------------------------------
// BOO tile stream, float, 64-feature tiles, every load a DMA into LDS.
//
// The same groups and lock step as boo_stream_dma_kernel, but no load lands
// in a register, so every wait is explicit and counted, and every wait is for
// loads issued two or more steps earlier.  Three streams per wave, all moved
// into LDS by global_load_lds:
//   * records (boo_stage.hpp): a step's entries and row starts, one DMA
//     instruction each, BLOB_LOOKAHEAD = 4 steps ahead;
//   * X ids: the 8 X rows the wave stages for a step, 32 bytes, XID_AHEAD = 5
//     steps ahead (they only address the X tile, so they never wait for a
//     record);
//   * X tiles: the wave's 2 of the tile's 8 DMA instructions, DX = 2 steps
//     ahead, into a ring of 3 tiles shared by the workgroup.
// Per step a wave issues, in this order: X(n + 2) (top, right after the
// barrier), then at the bottom its Y stores (8, at an item's end), record
// n + 4 and X ids n + 5.  At the top of step n it needs X(n) from every wave,
// record n and X ids n + 2; in issue order everything after X(n) may still be
// in flight: 6 operations plus the stores of steps n - 2 and n - 1.  Y rows
// are written by inline-asm stores so that their count is known exactly.
// ---------------------------------------------------------------------------

constexpr int BLOB_BUF = 544;    // LDS bytes per record buffer (the largest record, 528, + read-ahead)
constexpr uint32_t BL_LAST = 1u, BL_SERIAL = 2u, BL_ROWCONTIG = 4u;
constexpr int SYN_STRIDE = 272;  // bytes per serial-row sum (64 floats + 16)
constexpr int XID_RING = 8;      // X-id slots per wave (32 bytes each)
constexpr int XID_AHEAD = 5;

// DX + 1 X tiles + 16 serial rows + 16 records + 32 X-id slots: 39,424
// bytes at DX = 2 (four workgroups, 16 waves, per CU), 30,976 at DX = 1
// (five workgroups, 20 waves).
template <int DX>
struct StBlobLds {
    float xt[DX + 1][8 * DMA_BLK / 4];         // X tile ring
    float syn[4 * ST_SYN * SYN_STRIDE / 4];    // serial rows: wave w's are rows ST_SYN w ..
    uint8_t rec[4][4][BLOB_BUF];               // [wave][step mod 4] records
    uint32_t xid[4][XID_RING][8];              // [wave][step mod 8] X ids
};

struct BlobArgs {
    int rows, cols, K, batch, n_waves;
    const uint32_t* blobs;   // records, 16-byte units
    const uint32_t* first;   // [n_waves][8]
    const uint32_t* xid;     // [n_tiles][8]
    const int* row_ids;
    const float* X;
    float* Y;
    float* P;
};

template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

typedef float f4_t __attribute__((ext_vector_type(4)));

// 8 x 16-byte stores of one lane's 32 features (chunks 32 bytes apart).
__device__ __forceinline__ void store8(float* p, const f4_t (&d)[8]) {
    asm volatile(
        "global_store_dwordx4 %0, %1, off\n\t"
        "global_store_dwordx4 %0, %2, off offset:32\n\t"
        "global_store_dwordx4 %0, %3, off offset:64\n\t"
        "global_store_dwordx4 %0, %4, off offset:96\n\t"
        "global_store_dwordx4 %0, %5, off offset:128\n\t"
        "global_store_dwordx4 %0, %6, off offset:160\n\t"
        "global_store_dwordx4 %0, %7, off offset:192\n\t"
        "global_store_dwordx4 %0, %8, off offset:224" ::"v"(p),
        "v"(d[0]), "v"(d[1]), "v"(d[2]), "v"(d[3]), "v"(d[4]), "v"(d[5]), "v"(d[6]), "v"(d[7])
        : "memory");
}

template <int DX>
__global__ void __launch_bounds__(256, DX == 1 ? 5 : 4) boo_blob_kernel(BlobArgs a, int kt0) {
    static_assert(DX == 1 || DX == 2, "X tiles are staged 1 or 2 steps ahead");
    __shared__ __attribute__((aligned(16))) StBlobLds<DX> L;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int w = xcd_remap(blockIdx.x, gridDim.x) * 4 + wv;
    if (w >= a.n_waves) return;  // uniform per workgroup: n_waves is a multiple of 4
    // the wave's 8 words, held in SGPRs before any DMA: a vector load here
    // would enter the counted waits below
    const uint32_t* F = a.first + 8 * (size_t)w;
    uint32_t fw[7];
#pragma unroll
    for (int k = 0; k < 7; ++k) fw[k] = (uint32_t)__builtin_amdgcn_readfirstlane((int)F[k]);
    asm volatile("" ::"s"(fw[0]), "s"(fw[1]), "s"(fw[2]), "s"(fw[3]), "s"(fw[4]), "s"(fw[5]), "s"(fw[6]));
    const int nsteps = (int)fw[5];
    if (nsteps <= 0) return;     // uniform per workgroup: its streams have equal lengths
    const uint32_t t0 = fw[6];
    const int lane = threadIdx.x & 63;
    const int h = lane & 1;
    const int lr = lane >> 1;
    const int fbase = (kt0 + (int)blockIdx.y) * 64;
    const int b = blockIdx.z;
    const int K = a.K;
    const float* Xb = a.X + (size_t)b * a.cols * K;
    const uint32_t rowb = (uint32_t)K * 4u;
    const uint32_t lane_x = (uint32_t)fbase * 4u + (uint32_t)(lane & 15) * 16u;
    const int kq = lane >> 4;  // column I + 8 kq of DMA instruction I
    const uint32_t x_lds = lds_u32(&L.xt[0][0]) + (uint32_t)(2 * wv) * DMA_BLK;
    const uint32_t rec_lds = lds_u32(&L.rec[wv][0][0]);
    const uint32_t xid_lds = lds_u32(&L.xid[wv][0][0]);
    const int last = nsteps - 1;

    auto issue_rec = [&](uint32_t off16, uint32_t nvec, int n) {
        if ((uint32_t)lane < nvec)
            dma16(reinterpret_cast<const float*>(a.blobs), off16 * 16u + (uint32_t)lane * 16u,
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(rec_lds + (uint32_t)(n & 3) * BLOB_BUF)));
    };
    // X ids of step n (clamped to the last): 32 bytes, lanes 0 and 1
    auto issue_xid = [&](int n) {
        const uint32_t t = t0 + (uint32_t)min(n, last);
        if (lane < 2)
            dma16(reinterpret_cast<const float*>(a.xid), t * 32u + (uint32_t)lane * 16u,
                  (uint32_t)__builtin_amdgcn_readfirstlane((int)(xid_lds + (uint32_t)(n & (XID_RING - 1)) * 32u)));
    };
    // this wave's two DMA instructions (2 wv, 2 wv + 1) of X tile n
    auto issue_x = [&](int n) {
        const uint32_t* ids = &L.xid[wv][n & (XID_RING - 1)][0];
        const uint32_t id0 = ids[kq], id1 = ids[4 + kq];
        const uint32_t l0 = x_lds + (uint32_t)(n % (DX + 1)) * (8u * DMA_BLK);
        dma16(Xb, __umul24(id0, rowb) + lane_x, l0);
        dma16(Xb, __umul24(id1, rowb) + lane_x, l0 + (uint32_t)DMA_BLK);
    };

    // prologue: the operations before step 0 are laid out as the steady
    // state leaves them (after X(0): record 2, ids 3, X(1), record 3, ids 4),
    // so step 0 waits like any other step
    {
        const uint32_t nv = fw[4];
        if constexpr (DX == 2) {
            // after X(0): record 2, ids 3, X(1), record 3, ids 4
            issue_xid(0);
            issue_xid(1);
            issue_xid(2);
            issue_rec(fw[0], nv & 0xffu, 0);
            issue_rec(fw[1], (nv >> 8) & 0xffu, 1);
            wait_vm<4>();                       // ids 0
            issue_x(0);
            issue_rec(fw[2], (nv >> 16) & 0xffu, 2);
            issue_xid(3);
            wait_vm<7>();                       // ids 1
            issue_x(1);
            issue_rec(fw[3], nv >> 24, 3);
            issue_xid(4);
        } else {
            // after X(0): record 3, ids 4
            issue_xid(0);
            issue_xid(1);
            issue_xid(2);
            issue_rec(fw[0], nv & 0xffu, 0);
            issue_rec(fw[1], (nv >> 8) & 0xffu, 1);
            issue_rec(fw[2], (nv >> 16) & 0xffu, 2);
            issue_xid(3);
            wait_vm<6>();                       // ids 0
            issue_x(0);
            issue_rec(fw[3], nv >> 24, 3);
            issue_xid(4);
        }
    }

    f4_t acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = f4_t{0.f, 0.f, 0.f, 0.f};

    typedef __attribute__((address_space(3))) const char lds_char;
    int st1 = 0, st2 = 0;   // stores issued by steps n - 1 and n - 2 (0 or 8 each)
    for (int n = 0; n < nsteps; ++n) {
        // (1) X tile n (every wave's share), record n and ids n + 2 are in
        // LDS; the barrier publishes the tile
        if constexpr (DX == 2) {
            // after X(n): ops of steps n - 2 (bottom) and n - 1
            const int pend = st1 + st2;
            if (pend == 0) asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            else if (pend == 8) asm volatile("s_waitcnt vmcnt(14) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(22) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        } else {
            // after X(n): the bottom of step n - 1
            if (st1 == 0) asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            else asm volatile("s_waitcnt vmcnt(10) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        }
        __builtin_amdgcn_sched_barrier(0);
        // (2) X tile n + DX into the buffer tile n - 1 used
        issue_x(n + DX);
        __builtin_amdgcn_sched_barrier(0);
        // (3) record n
        const uint8_t* rp = &L.rec[wv][n & 3][0];
        const uint4 hd = *reinterpret_cast<const uint4*>(rp);
        const uint32_t w0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)hd.x);
        const int slot = __builtin_amdgcn_readfirstlane((int)hd.y);
        const uint32_t next_off = (uint32_t)__builtin_amdgcn_readfirstlane((int)hd.z);
        const int rbase = __builtin_amdgcn_readfirstlane((int)hd.w);
        const int nnz = (int)(w0 & 0xffu);
        const int nr = (int)((w0 >> 8) & 63u);
        const uint32_t fl = (w0 >> 20) & 15u;
        const uint32_t next_nvec = w0 >> 24;
        const int p_cols = nnz > 0 ? 48 : 16;
        const uint8_t* cols = rp + p_cols;
        const float* vals = reinterpret_cast<const float*>(rp + p_cols + ((nnz + 3) & ~3));
        int rs0 = 0, rs1 = 0;
        if (nnz > 0) {
            rs0 = rp[16 + lr];
            rs1 = lr == ST_ROWS - 1 ? nnz : (int)rp[16 + lr + 1];
        }
        const float* tile = &L.xt[n % (DX + 1)][0];
        // (4) the walk
        if (fl & BL_SERIAL) {
            // few busy rows: the whole wave takes one busy row at a time,
            // lane f on feature f, and leaves its sums in syn for the row's lanes
            uint64_t busy = __ballot(h == 0 && rs0 != rs1);
            int mine = -1;
            const char* xc = reinterpret_cast<const char*>(tile) + lane * 4;
            for (int k = 0; busy; ++k) {
                const int l2 = __builtin_ctzll(busy);
                busy &= busy - 1;
                int j = __builtin_amdgcn_readlane(rs0, l2);
                const int e = __builtin_amdgcn_readlane(rs1, l2);
                float s0 = 0.f, s1 = 0.f;
                for (; j + 2 <= e; j += 2) {
                    const uint32_t c0 = cols[j], c1 = cols[j + 1];
                    s0 += vals[j] * *reinterpret_cast<const float*>(xc + dma_col_off(c0));
                    s1 += vals[j + 1] * *reinterpret_cast<const float*>(xc + dma_col_off(c1));
                }
                if (j < e) s0 += vals[j] * *reinterpret_cast<const float*>(xc + dma_col_off(cols[j]));
                *reinterpret_cast<float*>(reinterpret_cast<char*>(L.syn) + (ST_SYN * wv + k) * SYN_STRIDE +
                                          lane * 4) = s0 + s1;
                if ((lane & ~1) == l2) mine = k;
            }
            wave_lds_fence();
            if (mine >= 0) {
                lds_char* sr = (lds_char*)(L.syn) + (ST_SYN * wv + mine) * SYN_STRIDE + h * 16;
                const f4_t* xr = (const f4_t*)sr;
                f4_t x[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = xr[2 * q];
#pragma unroll
                for (int q = 0; q < 8; ++q) acc[q] += x[q];
            }
        } else if (rs0 < rs1) {
            lds_char* tb = (lds_char*)(tile) + h * 16;
            int j = rs0;
            uint32_t c = cols[j];
            float v = vals[j];
#pragma nounroll
            for (; j < rs1; ++j) {
                const uint32_t cn = cols[j + 1];
                const float vn = vals[j + 1];
                __builtin_amdgcn_sched_barrier(0);
                const f4_t* xr = (const f4_t*)(lds_char*)(tb + dma_col_off(c));
                f4_t x[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) x[q] = xr[2 * q];
                const f4_t vv = f4_t{v, v, v, v};
#pragma unroll
                for (int q = 0; q < 8; ++q) acc[q] = __builtin_elementwise_fma(vv, x[q], acc[q]);
                c = cn;
                v = vn;
            }
        }
        wave_lds_fence();
        // (5) end of the item: store its rows
        st2 = st1;
        st1 = 0;
        if ((fl & BL_LAST) && nr > 0) {
            if (lr < nr) {
                float* out;
                if (slot < 0) {
                    // row ids not consecutive: a plain load, waited for at once
                    // (the compiler's wait also drains this wave's DMAs, so
                    // the counts below only get more conservative)
                    const int row = (fl & BL_ROWCONTIG) ? rbase + lr : a.row_ids[rbase + lr];
                    out = a.Y + ((size_t)b * a.rows + row) * K + fbase + h * 4;
                } else {
                    out = a.P + (((size_t)slot * a.batch + b) * ST_ROWS + lr) * K + fbase + h * 4;
                }
                store8(out, acc);
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) acc[q] = f4_t{0.f, 0.f, 0.f, 0.f};
            st1 = 8;
        }
        // (6) record n + 4 into this record's buffer once its reads are done,
        // then the X ids of step n + 5
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        issue_rec(next_off, next_nvec, n);
        issue_xid(n + XID_AHEAD);
        __builtin_amdgcn_sched_barrier(0);
    }
    // the last DMAs land before the workgroup's LDS is released
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <typename T>
__global__ void __launch_bounds__(256) fill_zero_kernel(T* __restrict__ Y, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) Y[i] = T(0);
}

// Split items: Y[row] += partial slots [slot_begin, slot_end) in slot order.
template <typename T>
__global__ void __launch_bounds__(256) boo_fixup_kernel(const int* __restrict__ splits,
                                                        const int* __restrict__ row_ids,
                                                        const T* __restrict__ P, T* __restrict__ Y,
                                                        int rows, int K, int batch) {
    const int s = blockIdx.x;
    const int b = blockIdx.z;
    const int row_off = splits[4 * s], nr = splits[4 * s + 1];
    const int sb = splits[4 * s + 2], se = splits[4 * s + 3];
    const long long total = (long long)nr * K;
    for (long long e = threadIdx.x; e < total; e += blockDim.x) {
        const int lr = (int)(e / K);
        const int f = (int)(e % K);
        T* y = Y + ((size_t)b * rows + row_ids[row_off + lr]) * K + f;
        T acc = *y;
        for (int sl = sb; sl < se; ++sl) acc += P[(((size_t)sl * batch + b) * ST_ROWS + lr) * K + f];
        *y = acc;
    }
}

// ---------------------------------------------------------------------------
// BOO gather pass: the rows of slices whose columns are too scattered for X
// tiles to pay (each column used about once).  LPR lanes per row, VEC features
// each (blockIdx.y picks the feature tile); a workgroup of 256 threads covers
// 256 / LPR rows.  The row's entries are read LPR at a time, one per lane
// (coalesced), and handed to the row's lanes by a shuffle; each entry's slice
// of its X row is then gathered straight from memory, U entries at a time so
// that U gathers are in flight.  The row is stored once (plain stores).
// ---------------------------------------------------------------------------

template <typename T, int VEC, int LPR>
__global__ void __launch_bounds__(256) boo_rows_kernel(const int* __restrict__ crow_ptr,
                                                       const int* __restrict__ crow_id,
                                                       const int* __restrict__ ccol,
                                                       const T* __restrict__ cval, int n_crow,
                                                       const T* __restrict__ X, T* __restrict__ Y,
                                                       int rows, int cols, int K) {
    constexpr int RPB = 256 / LPR;
    constexpr int U = 8;
    static_assert(LPR >= 1 && LPR <= 64 && (LPR & (LPR - 1)) == 0, "LPR must be a power of two <= 64");
    const int r = xcd_remap(blockIdx.x, gridDim.x) * RPB + (int)threadIdx.x / LPR;
    if (r >= n_crow) return;  // no barriers below
    const int l = threadIdx.x % LPR;
    const int gbase = (threadIdx.x & 63) & ~(LPR - 1);  // first lane of this row in the wave
    const int f = (int)blockIdx.y * (LPR * VEC) + l * VEC;
    const bool fok = f < K;  // K is a multiple of VEC
    const int b = blockIdx.z;
    const T* Xb = X + (size_t)b * cols * K;
    const int p0 = crow_ptr[r], p1 = crow_ptr[r + 1];
    T acc[VEC];
#pragma unroll
    for (int u = 0; u < VEC; ++u) acc[u] = T(0);
    // lanes past the row's end repeat the chunk's first entry with value 0;
    // the next chunk's entries are fetched behind this chunk's gathers
    auto fetch = [&](int p, int& c, T& v) {
        const int n = min(LPR, p1 - p);
        c = p < p1 ? ccol[p + (l < n ? l : 0)] : 0;
        v = p < p1 && l < n ? cval[p + l] : T(0);
    };
    int cn;
    T vn;
    fetch(p0, cn, vn);
    for (int p = p0; p < p1; p += LPR) {
        const int n = min(LPR, p1 - p);
        const int c = cn;
        const T v = vn;
        fetch(p + LPR, cn, vn);
        for (int i0 = 0; i0 < n; i0 += U) {
            int ci[U];
            T vi[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int src = gbase + min(i0 + u, LPR - 1);
                ci[u] = __shfl(c, src);
                vi[u] = i0 + u < n ? __shfl(v, src) : T(0);
            }
            if (fok) {
                T x[U][VEC];
#pragma unroll
                for (int u = 0; u < U; ++u) load_vec<T, VEC>(Xb + (size_t)ci[u] * K + f, x[u]);
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int e = 0; e < VEC; ++e) acc[e] += vi[u] * x[u][e];
            }
        }
    }
    if (fok) store_vec<T, VEC>(Y + ((size_t)b * rows + crow_id[r]) * K + f, acc);
}

// Long gather rows: one workgroup per chunk task (at most a fixed number of
// one row's entries), 16 entry slots x 16 lanes of VEC features, U entries per
// slot in flight; the slots' sums are reduced in a fixed order through LDS
// into the task's partial row P[task][b][:].  Workgroup x of a feature slab
// runs task order[x] (null: task x): the staging puts the tasks over a
// power-law matrix's most used columns first, and the workgroups are
// dispatched x first, so within each feature slab those tasks run together
// while their X rows fit in L2.
template <typename T, int VEC>
__global__ void __launch_bounds__(256) gather_chunk_kernel(const int* __restrict__ gtask,
                                                           const int* __restrict__ order,
                                                           const int* __restrict__ ccol,
                                                           const T* __restrict__ cval,
                                                           const T* __restrict__ X, T* __restrict__ P,
                                                           int cols, int K, int batch) {
    constexpr int LANES = 16, SLOTS = 16, KT = LANES * VEC, U = 4;
    __shared__ T red[SLOTS][KT];
    const int t = order ? order[blockIdx.x] : (int)blockIdx.x;  // launch position -> task
    const int b = blockIdx.z;
    const int slot = threadIdx.x / LANES;
    const int ch = threadIdx.x % LANES;
    const int f = (int)blockIdx.y * KT + ch * VEC;
    const bool fok = f < K;  // K is a multiple of VEC
    const T* Xb = X + (size_t)b * cols * K;
    T acc[VEC];
#pragma unroll
    for (int u = 0; u < VEC; ++u) acc[u] = T(0);
    const int e0 = gtask[2 * t], e1 = gtask[2 * t + 1];
    if (fok) {
        int j = e0 + slot;
        for (; j + (U - 1) * SLOTS < e1; j += U * SLOTS) {
            int c[U];
            T v[U], x[U][VEC];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                c[u] = ccol[j + u * SLOTS];
                v[u] = cval[j + u * SLOTS];
            }
#pragma unroll
            for (int u = 0; u < U; ++u) load_vec<T, VEC>(Xb + (size_t)c[u] * K + f, x[u]);
#pragma unroll
            for (int u = 0; u < U; ++u)
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[e] += v[u] * x[u][e];
        }
        if (j < e1) {
            // the last (partial) round: every slot's remaining entries in
            // flight at once; entries past the task's end repeat its first
            // column (an L1 hit) with value 0
            int c[U - 1];
            T v[U - 1], x[U - 1][VEC];
#pragma unroll
            for (int u = 0; u < U - 1; ++u) {
                const int jj = j + u * SLOTS;
                c[u] = ccol[jj < e1 ? jj : e0];
                v[u] = jj < e1 ? cval[jj] : T(0);
            }
#pragma unroll
            for (int u = 0; u < U - 1; ++u) load_vec<T, VEC>(Xb + (size_t)c[u] * K + f, x[u]);
#pragma unroll
            for (int u = 0; u < U - 1; ++u)
#pragma unroll
                for (int e = 0; e < VEC; ++e) acc[e] += v[u] * x[u][e];
        }
    }
#pragma unroll
    for (int u = 0; u < VEC; ++u) red[slot][ch * VEC + u] = acc[u];
    __syncthreads();
    if (threadIdx.x < KT) {
        const int fe = (int)blockIdx.y * KT + (int)threadIdx.x;
        if (fe < K) {
            T sum = T(0);
#pragma unroll
            for (int sl = 0; sl < SLOTS; ++sl) sum += red[sl][threadIdx.x];
            P[((size_t)t * batch + b) * K + fe] = sum;
        }
    }
}

// Long gather row i: Y[crow_id[r0 + i]] = sum of its tasks' partial rows, in
// task order (deterministic).  LPR lanes per row, VEC features per lane,
// 256 / LPR rows per workgroup; rows wider than LPR * VEC features loop.
template <typename T, int VEC, int LPR>
__global__ void __launch_bounds__(256) gather_fix_kernel(const int* __restrict__ gtask_ptr,
                                                         const int* __restrict__ crow_id, int r0, int n_long,
                                                         const T* __restrict__ P, T* __restrict__ Y,
                                                         int rows, int K, int batch) {
    constexpr int RPB = 256 / LPR;
    const int i = (int)blockIdx.x * RPB + (int)threadIdx.x / LPR;
    if (i >= n_long) return;  // no barriers below
    const int l = threadIdx.x % LPR;
    const int b = blockIdx.z;
    const int yrow = crow_id[r0 + i];
    const int t0 = gtask_ptr[i], t1 = gtask_ptr[i + 1];
    for (int f = l * VEC; f < K; f += LPR * VEC) {  // K is a multiple of VEC
        T sum[VEC];
#pragma unroll
        for (int u = 0; u < VEC; ++u) sum[u] = T(0);
        for (int t = t0; t < t1; ++t) {
            T p[VEC];
            load_vec<T, VEC>(P + ((size_t)t * batch + b) * K + f, p);
#pragma unroll
            for (int u = 0; u < VEC; ++u) sum[u] += p[u];
        }
        store_vec<T, VEC>(Y + ((size_t)b * rows + yrow) * K + f, sum);
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

// &Xb[col][f] (row length K): a 32-bit byte offset (A32: one batch's X is
// under 4 GiB) or a 64-bit element offset.
template <typename T, bool A32>
__device__ __forceinline__ const T* x_at(const T* Xb, long long col, int K, int f) {
    if constexpr (A32) {
        const uint32_t off = (uint32_t)col * ((uint32_t)K * (uint32_t)sizeof(T)) + (uint32_t)f * (uint32_t)sizeof(T);
        return reinterpret_cast<const T*>(reinterpret_cast<const char*>(Xb) + off);
    } else {
        return Xb + (size_t)col * K + f;
    }
}

template <typename T, typename I>
struct PbrArgs {
    long long rows, cols;
    int K, n_stripes, long_threshold;
    int kt0;                   // first feature tile of this launch
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
// 8x8 blocks put two stripe rows in each 16-lane group of an LDS read.  A
// row's LPR lanes read LPR * VEC * sizeof(T) = 128 contiguous bytes per chunk
// q (32 banks); rows r and r+1 read random columns.  With the row stride a
// multiple of 256 bytes and odd rows walking their chunks in the order q ^ 1
// (SWAP), the two rows of a group always read opposite halves of the 64
// banks, so the walk is free of bank conflicts whatever the columns.
// Otherwise the stride is padded by 32 bytes.
template <typename T, int BR, int KT, int VEC>
struct PbrGeom {
    static constexpr int LPR = 64 / BR;
    static constexpr int F = KT / LPR;
    static constexpr int NQ = F / VEC;
    static constexpr int CHUNKS = KT / VEC;
    static constexpr bool SWAP = BR == 8 && NQ % 2 == 0 && LPR * VEC * (int)sizeof(T) == 128 &&
                                 (KT * (int)sizeof(T)) % 256 == 0;
    static constexpr int STRIDE = SWAP ? KT : KT + 32 / (int)sizeof(T);  // LDS row stride (elements)
    static constexpr int STAGE_ITERS = (BR * CHUNKS + 63) / 64;
    static_assert(F % VEC == 0 && NQ >= 1, "bad PBR tile");
};

// One wave per stripe and feature tile, software-pipelined PD blocks ahead:
// while block n is walked from LDS, the X rows of blocks n+1 .. n+PD and the
// values of their bit (r, c) -- one per lane -- are in flight into
// registers, and the metadata of block n+PD+1 behind them.  Every step issues
// the same loads (blocks past the stripe's end are clamped to its last), so
// no step waits on a load it issued itself, and a wave keeps PD blocks of X
// in flight (small feature tiles: several, so the many short X reads of a
// feature tile keep the memory system busy).  Lane (r, l) owns row r of the stripe and the VEC-chunks
// q*LPR + l of the tile; it walks its row's set bits with ctz, reading the
// bit's value and its X row slice from LDS.  Dense blocks are never formed.
template <typename T, typename I, int BR, int KT, int VEC, int PD, bool FULL, bool A32>
__device__ __forceinline__ void pbr_stripe_body(const PbrArgs<T, I>& a, int stripe, int kt, int b,
                                                T* tiles, T* vals) {
    typedef PbrGeom<T, BR, KT, VEC> G;
    constexpr int NBITS = BR * BR;
    const int lane = threadIdx.x;
    const int r = lane / G::LPR;
    const int l = lane % G::LPR;
    // acc[q] of this lane holds feature chunk q ^ par (chunk order of SWAP)
    const int par = G::SWAP ? (r & 1) : 0;
    auto fofs = [&](int q) { return ((q ^ par) * G::LPR + l) * VEC; };  // chunk's first feature in the tile
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

    // This row's remainder: its bounds are loaded first, and the column ids
    // of its first RU entries behind the first block's loads, so they land
    // during the block loop (the values are loaded beside the X rows, which
    // do not wait for them).  Rows longer than long_threshold are left to
    // rows_long_kernel.
    constexpr int RU = G::NQ * VEC <= 8 ? 4 : 2;  // remainder entries per round
    const long long rs = active ? (long long)a.rem_indptr[row] : 0;
    const long long re = active ? (long long)a.rem_indptr[row + 1] : 0;
    const bool rem_here = active && re - rs <= a.long_threshold;
    I rc[RU];  // -1: no entry
    auto rem_fetch = [&](long long j) {
#pragma unroll
        for (int u = 0; u < RU; ++u) rc[u] = rem_here && j + u < re ? a.rem_col_ind[j + u] : I(-1);
    };
    auto rem_prefetch = [&]() { rem_fetch(rs); };

    const int p0 = a.stripe_ptr[stripe], p1 = a.stripe_ptr[stripe + 1];
    if (p1 > p0) {
        const int plast = p1 - 1;
        // X rows of a block into registers (staging lane mapping: chunk ch of
        // column c; columns past the matrix load column col0 instead)
        auto load_x = [&](T (&xr)[G::STAGE_ITERS][VEC], long long col0) {
#pragma unroll
            for (int m = 0; m < G::STAGE_ITERS; ++m) {
                const int idx = m * 64 + lane;
                const int c = min(idx / G::CHUNKS, BR - 1);
                const int ch = idx % G::CHUNKS;
                const int f = FULL ? fbase + ch * VEC : min(fbase + ch * VEC, K - VEC);
                const long long xc = col0 + c < a.cols ? col0 + c : col0;
                load_vec<T, VEC>(x_at<T, A32>(Xb, xc, K, f), xr[m]);
            }
        };
        // the value of bit `lane` of a block (0 when the bit is clear)
        auto load_v = [&](uint64_t code, long long off) {
            const bool set = lane < NBITS && ((code >> lane) & 1ull);
            const int rank = __popcll(code & ((1ull << (lane & 63)) - 1ull));
            return set ? a.data[off + rank] : T(0);
        };
        // Block metadata, lane-held: lane i holds code, column and value
        // offset of block chunk + i (clamped to the stripe's last), one
        // coalesced load per 64 blocks; each step reads its block's with
        // readlane, so no step waits on a metadata load.
        int chunk = p0;
        uint64_t mcode;
        long long mcol, moff;
        auto meta_load = [&]() {
            const int q = min(chunk + lane, plast);
            mcode = (uint64_t)a.codes[q];
            mcol = (long long)a.coords[2 * (size_t)q + 1];
            moff = (long long)a.offsets[q];
        };
        auto rl64 = [](uint64_t v, int j) {
            const uint32_t lo = __builtin_amdgcn_readlane((int)(uint32_t)v, j);
            const uint32_t hi = __builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), j);
            return ((uint64_t)hi << 32) | lo;
        };
        meta_load();
        // The ring: slot s holds the X rows, the lane's bit value and the
        // code of the block PD steps ahead of the one it is walking next.
        T xr[PD][G::STAGE_ITERS][VEC];
        T vv[PD];
        uint64_t cd[PD];
#pragma unroll
        for (int s = 0; s < PD; ++s) {
            cd[s] = rl64(mcode, s);
            load_x(xr[s], (long long)rl64((uint64_t)mcol, s));
            vv[s] = load_v(cd[s], (long long)rl64((uint64_t)moff, s));
        }
        rem_prefetch();
        for (int base = p0; base < p1; base += PD) {
#pragma unroll
            for (int s = 0; s < PD; ++s) {
                const int blk = base + s;
                if (blk >= p1) break;  // uniform
                T* tile = tiles + ((blk - p0) & 1) * (BR * G::STRIDE);
                T* vb = vals + ((blk - p0) & 1) * 64;
                const uint64_t code = cd[s];
                // (1) block blk's X rows and values to LDS
#pragma unroll
                for (int m = 0; m < G::STAGE_ITERS; ++m) {
                    const int idx = m * 64 + lane;
                    const int c = idx / G::CHUNKS;
                    const int ch = idx % G::CHUNKS;
                    if (c < BR && (FULL || fbase + ch * VEC < K))
                        store_vec<T, VEC>(tile + c * G::STRIDE + ch * VEC, xr[s][m]);
                }
                vb[lane] = vv[s];
                wave_lds_fence();
                // (2) loads of block blk+PD (clamped to the stripe's last)
                // into the freed slot
                int jn = blk + PD - chunk;
                if (jn >= 64) {  // uniform; once per 64 blocks
                    chunk += 64;
                    jn -= 64;
                    meta_load();
                }
                cd[s] = rl64(mcode, jn);
                load_x(xr[s], (long long)rl64((uint64_t)mcol, jn));
                vv[s] = load_v(cd[s], (long long)rl64((uint64_t)moff, jn));
                // (3) walk block blk
                if (active) {
                    uint32_t rb = (uint32_t)((code >> (BR * r)) & rowbits);
                    // an entry's first feature chunk at one multiply-add from
                    // this lane's base in the tile, the others at fixed
                    // per-lane distances from it
                    const T* t0 = tile + fofs(0);
                    int dq[G::NQ];
#pragma unroll
                    for (int q = 0; q < G::NQ; ++q) dq[q] = fofs(q) - fofs(0);
                    while (rb) {
                        const int c = __builtin_ctz(rb);
                        rb &= rb - 1u;
                        const T v = vb[r * BR + c];
                        const T* x0 = t0 + c * G::STRIDE;
#pragma unroll
                        for (int q = 0; q < G::NQ; ++q) {
                            if (FULL || fbase + fofs(q) < K) {
                                T x[VEC];
                                load_vec<T, VEC>(x0 + dq[q], x);
#pragma unroll
                                for (int u = 0; u < VEC; ++u) acc[q][u] += v * x[u];
                            }
                        }
                    }
                }
                wave_lds_fence();
            }
        }
    } else {
        rem_prefetch();
    }

    // Remainder rounds: the X rows of RU entries in flight together, the
    // next round's column ids and values fetched behind them.
    if (rem_here) {
        for (long long j = rs; j < re; j += RU) {
            T xj[RU][G::NQ][VEC];
            // entries past the row's end load X row 0 (the row has an entry,
            // so X has rows) and carry the value 0
#pragma unroll
            for (int u = 0; u < RU; ++u) {
                const long long cu = rc[u] >= 0 ? (long long)rc[u] : 0;
#pragma unroll
                for (int q = 0; q < G::NQ; ++q) {
                    const int fq = fbase + fofs(q);
                    load_vec<T, VEC>(x_at<T, A32>(Xb, cu, K, FULL ? fq : min(fq, K - VEC)), xj[u][q]);
                }
            }
            T vj[RU];
#pragma unroll
            for (int u = 0; u < RU; ++u) vj[u] = rc[u] >= 0 ? a.rem_vals[j + u] : T(0);
            rem_fetch(j + RU);
#pragma unroll
            for (int u = 0; u < RU; ++u)
#pragma unroll
                for (int q = 0; q < G::NQ; ++q)
                    if (FULL || fbase + fofs(q) < K)
#pragma unroll
                        for (int e = 0; e < VEC; ++e) acc[q][e] += vj[u] * xj[u][q][e];
        }
    }
    if (!active) return;
    T* out = a.Y + ((size_t)b * a.rows + row) * K + fbase;
#pragma unroll
    for (int q = 0; q < G::NQ; ++q) {
        if (FULL || fbase + fofs(q) < K) store_vec<T, VEC>(out + fofs(q), acc[q]);
    }
}

template <typename T, typename I, int BR, int KT, int VEC, int PD, bool A32>
__global__ void __launch_bounds__(64) pbr_stripe_kernel(PbrArgs<T, I> a) {
    typedef PbrGeom<T, BR, KT, VEC> G;
    __shared__ __attribute__((aligned(16))) T tiles[2 * BR * G::STRIDE];
    __shared__ __attribute__((aligned(16))) T vals[2 * 64];
    const int stripe = xcd_remap(blockIdx.x, gridDim.x);
    if (stripe >= a.n_stripes) return;
    const int kt = a.kt0 + (int)blockIdx.y;
    const int b = blockIdx.z;
    if ((kt + 1) * KT <= a.K) {
        pbr_stripe_body<T, I, BR, KT, VEC, PD, true, A32>(a, stripe, kt, b, tiles, vals);
    } else {
        pbr_stripe_body<T, I, BR, KT, VEC, PD, false, A32>(a, stripe, kt, b, tiles, vals);
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

#ifndef SPMM_BOO_DEPTH
#define SPMM_BOO_DEPTH 1        // X tiles loaded this many tiles ahead
#endif
#ifndef SPMM_BOO_FAR
#define SPMM_BOO_FAR 2          // streaming tile data loaded this many tiles ahead
#endif
#ifndef SPMM_BOO_BLOB_DX
#define SPMM_BOO_BLOB_DX 1      // X tiles of the record kernel staged this many steps ahead
#endif

// Full feature tiles in one launch, a partial last tile (K % 2F != 0) in a
// second one compiled with the per-chunk feature guards.
template <typename T, int F, int VEC, bool A32>
int launch_boo_stream_a(const StreamArgs<T>& a, hipStream_t s) {
    constexpr int D = SPMM_BOO_DEPTH, DF = SPMM_BOO_FAR;
    constexpr int NST = BooGeom<T, F, VEC>::NST;
    // Workgroups of 4 waves share X tiles when the staging grouped slices by 4
    // and the tile splits 4 ways; otherwise each wave is its own workgroup
    // (every stream is complete on its own, so this is only slower).
    const bool wg4 = a.group == 4 && NST % 4 == 0;
    const int full = a.K / (2 * F);
    auto go = [&](auto kern, int wg, int ny, int kt) {
        const dim3 grid(round_up8(a.n_waves / wg), ny, a.batch);
        return launch("boo_stream_kernel", kern, grid, dim3(64 * wg), s, a, kt);
    };
    if constexpr (std::is_same<T, float>::value && F == 32 && VEC == 4 && A32) {
        if (wg4 && full > 0 && a.blobs && a.blob_first) {  // full 64-feature tiles, every load a DMA
            const dim3 grid(round_up8(a.n_waves / 4), full, a.batch);
            BlobArgs ba{a.rows, a.cols, a.K, a.batch, a.n_waves, a.blobs, a.blob_first, a.blob_xid, a.row_ids,
                        a.X, a.Y, a.P};
            const int rc = launch("boo_blob_kernel", boo_blob_kernel<SPMM_BOO_BLOB_DX>, grid, dim3(256), s, ba, 0);
            if (rc || a.K % (2 * F) == 0) return rc;
            return go(boo_stream_kernel<T, F, VEC, D, DF, 4, false, A32>, 4, 1, full);
        }
        if ((wg4 || a.group == 2) && full > 0) {  // full 64-feature tiles: X staged by LDS DMA
            const int wg = wg4 ? 4 : 2;
            const dim3 grid(round_up8(a.n_waves / wg), full, a.batch);
            const int rc = wg4 ? launch("boo_stream_dma_kernel", boo_stream_dma_kernel<DF, 4>, grid, dim3(256), s, a, 0)
                               : launch("boo_stream_dma_kernel", boo_stream_dma_kernel<DF, 2>, grid, dim3(128), s, a, 0);
            if (rc || a.K % (2 * F) == 0) return rc;
            return wg4 ? go(boo_stream_kernel<T, F, VEC, D, DF, 4, false, A32>, 4, 1, full)
                       : go(boo_stream_kernel<T, F, VEC, D, DF, 1, false, A32>, 1, 1, full);
        }
    }
    if (full > 0) {
        const int rc = wg4 ? go(boo_stream_kernel<T, F, VEC, D, DF, (NST % 4 == 0 ? 4 : 1), true, A32>, 4, full, 0)
                           : go(boo_stream_kernel<T, F, VEC, D, DF, 1, true, A32>, 1, full, 0);
        if (rc) return rc;
    }
    if (a.K % (2 * F)) {
        return wg4 ? go(boo_stream_kernel<T, F, VEC, D, DF, (NST % 4 == 0 ? 4 : 1), false, A32>, 4, 1, full)
                   : go(boo_stream_kernel<T, F, VEC, D, DF, 1, false, A32>, 1, 1, full);
    }
    return SPMM_OK;
}

// 32-bit X addressing when one batch's X slab is under 4 GiB.
template <typename T, int F, int VEC>
int launch_boo_stream(const StreamArgs<T>& a, hipStream_t s) {
    if ((uint64_t)a.cols * (uint64_t)a.K * sizeof(T) < (1ull << 32) && a.cols < (1 << 24) &&
        (uint64_t)a.K * sizeof(T) < (1ull << 24))
        return launch_boo_stream_a<T, F, VEC, true>(a, s);
    return launch_boo_stream_a<T, F, VEC, false>(a, s);
}

template <typename T>
int boo_dispatch(const StreamArgs<T>& a, hipStream_t s) {
    const int F = boo_pick_f<T>(a.K);
    const int VEC = pick_vec<T>(a.K, F, a.X, a.Y);
#define SPMM_BOO_CASE(FF, VV) \
    if (F == FF && VEC == VV) return launch_boo_stream<T, FF, VV>(a, s);
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
        return launch("rows_long_kernel", rows_long_kernel<T, I, V>, grid, dim3(256), s, long_rows, indptr,
                      col_ind, vals, X, Y, rows, cols, K);
    }
    const dim3 grid(n_long, (K + 15) / 16, batch);
    return launch("rows_long_kernel", rows_long_kernel<T, I, 1>, grid, dim3(256), s, long_rows, indptr, col_ind,
                  vals, X, Y, rows, cols, K);
}

// Workspace: the partial slots of split slices, then (256-byte aligned) the
// partial rows of the long gather rows' chunk tasks.
inline size_t boo_ws_slots_bytes(const spmm_boo_desc* A, size_t es, int64_t batch, int64_t K) {
    const size_t slots = A->n_slots > 0 ? (size_t)A->n_slots * (size_t)batch * (size_t)ST_ROWS * (size_t)K * es : 0;
    return (slots + 255) / 256 * 256;
}

template <typename T, int VEC, int LPR>
int launch_boo_rows_l(const spmm_boo_desc* A, const T* X, T* Y, int K, int batch, hipStream_t s) {
    constexpr int RPB = 256 / LPR;
    const int n_short = A->n_crow - A->n_crow_long;
    if (n_short <= 0) return SPMM_OK;
    const dim3 grid(round_up8((n_short + RPB - 1) / RPB), (K + LPR * VEC - 1) / (LPR * VEC), batch);
    return launch("boo_rows_kernel", boo_rows_kernel<T, VEC, LPR>, grid, dim3(256), s, A->crow_ptr, A->crow_id,
                  A->ccol, static_cast<const T*>(A->cval), n_short, X, Y, A->rows, A->cols, K);
}

template <typename T, int VEC>
int launch_boo_rows_v(const spmm_boo_desc* A, const T* X, T* Y, int K, int batch, hipStream_t s) {
    const int need = (K + VEC - 1) / VEC;  // lanes for the whole row
    if (need <= 1) return launch_boo_rows_l<T, VEC, 1>(A, X, Y, K, batch, s);
    if (need <= 2) return launch_boo_rows_l<T, VEC, 2>(A, X, Y, K, batch, s);
    if (need <= 4) return launch_boo_rows_l<T, VEC, 4>(A, X, Y, K, batch, s);
    if (need <= 8) return launch_boo_rows_l<T, VEC, 8>(A, X, Y, K, batch, s);
    if (need <= 16) return launch_boo_rows_l<T, VEC, 16>(A, X, Y, K, batch, s);
    if (need <= 32) return launch_boo_rows_l<T, VEC, 32>(A, X, Y, K, batch, s);
    return launch_boo_rows_l<T, VEC, 64>(A, X, Y, K, batch, s);
}

template <typename T, int VEC, int LPR>
int launch_gather_fix_l(const spmm_boo_desc* A, const T* P2, T* Y, int K, int batch, hipStream_t s) {
    constexpr int RPB = 256 / LPR;
    const int n_long = A->n_crow_long;
    const dim3 grid(round_up8((n_long + RPB - 1) / RPB), 1, batch);
    return launch("gather_fix_kernel", gather_fix_kernel<T, VEC, LPR>, grid, dim3(256), s, A->gtask_ptr,
                  A->crow_id, A->n_crow - n_long, n_long, P2, Y, A->rows, K, batch);
}

// The fixup of the chunk tasks: lanes for the whole row (at most 64).
template <typename T, int VEC>
int launch_gather_fix_v(const spmm_boo_desc* A, const T* P2, T* Y, int K, int batch, hipStream_t s) {
    const int need = (K + VEC - 1) / VEC;
    if (need <= 4) return launch_gather_fix_l<T, VEC, 4>(A, P2, Y, K, batch, s);
    if (need <= 8) return launch_gather_fix_l<T, VEC, 8>(A, P2, Y, K, batch, s);
    if (need <= 16) return launch_gather_fix_l<T, VEC, 16>(A, P2, Y, K, batch, s);
    if (need <= 32) return launch_gather_fix_l<T, VEC, 32>(A, P2, Y, K, batch, s);
    return launch_gather_fix_l<T, VEC, 64>(A, P2, Y, K, batch, s);
}

template <typename T>
int launch_boo_rows(const spmm_boo_desc* A, const T* X, T* Y, int K, int batch, T* P2, hipStream_t s) {
    constexpr int V = 16 / sizeof(T);
    const bool vec = K % V == 0 && aligned16(X) && aligned16(Y);
    int rc = vec ? launch_boo_rows_v<T, V>(A, X, Y, K, batch, s) : launch_boo_rows_v<T, 1>(A, X, Y, K, batch, s);
    if (rc || A->n_crow_long <= 0) return rc;
    if (A->n_gtask > 0) {
        const int v = vec ? V : 1;
        const dim3 grid(A->n_gtask, (K + 16 * v - 1) / (16 * v), batch);
        rc = vec ? launch("gather_chunk_kernel", gather_chunk_kernel<T, V>, grid, dim3(256), s, A->gtask,
                          A->gtask_order, A->ccol, static_cast<const T*>(A->cval), X, P2, A->cols, K, batch)
                 : launch("gather_chunk_kernel", gather_chunk_kernel<T, 1>, grid, dim3(256), s, A->gtask,
                          A->gtask_order, A->ccol, static_cast<const T*>(A->cval), X, P2, A->cols, K, batch);
        if (rc) return rc;
    }
    return vec && aligned16(P2) ? launch_gather_fix_v<T, V>(A, P2, Y, K, batch, s)
                                : launch_gather_fix_v<T, 1>(A, P2, Y, K, batch, s);
}

template <typename T>
int boo_matmul_t(const spmm_boo_desc* A, const void* Xv, void* Yv, int64_t batch, int64_t K,
                 void* ws, size_t ws_bytes, hipStream_t s) {
    const T* X = static_cast<const T*>(Xv);
    T* Y = static_cast<T*>(Yv);
    // Y rows come from the tile stream or the gather pass; a descriptor whose
    // counts do not add up to rows would leave rows of Y unwritten.
    if (A->n_stream_rows < 0 || A->n_crow < 0 || (long long)A->n_stream_rows + A->n_crow != A->rows)
        return fail(SPMM_EINVAL,
                    "BOO descriptor covers %d tile-stream rows + %d gather rows, not the matrix's %d rows; "
                    "copy n_stream_rows, n_crow and every gather-pass array from the staging",
                    A->n_stream_rows, A->n_crow, A->rows);
    if (A->n_stream_rows > 0 && A->n_tiles <= 0)
        return fail(SPMM_EINVAL, "BOO descriptor has %d tile-stream rows but no tiles", A->n_stream_rows);
    if (A->rows == 0 || K == 0 || batch == 0) return SPMM_OK;
    const bool stream = A->n_tiles > 0;
    if ((!stream && A->n_crow <= 0) || (stream && (A->n_waves <= 0 || !A->wave_tiles || !A->tiles)))
        return fail(SPMM_EINVAL, "BOO staging is empty; stage the matrix with spmm_boo_stage_create");
    if (A->n_crow > 0 && (!A->crow_ptr || !A->crow_id))  // ccol/cval may be null when the rows are empty
        return fail(SPMM_EINVAL, "BOO gather rows are null");
    if (A->n_crow_long < 0 || A->n_crow_long > A->n_crow || A->n_gtask < 0 ||
        (A->n_crow_long > 0 && !A->gtask_ptr) || (A->n_gtask > 0 && !A->gtask))
        return fail(SPMM_EINVAL, "bad BOO long gather rows");
    if (A->cols > 0 && !X) return fail(SPMM_EINVAL, "X is null");
    if (!Y) return fail(SPMM_EINVAL, "Y is null");
    const size_t need = spmm_boo_workspace_bytes(A, sizeof(T) == 4 ? SPMM_F32 : SPMM_F64, batch, K);
    if (need > ws_bytes || (need && !ws))
        return fail(SPMM_ENOMEM, "BOO workspace too small: need %zu bytes, got %zu", need, ws_bytes);

    if (A->cols == 0) {  // no entries: Y = 0
        const size_t n = (size_t)batch * (size_t)A->rows * (size_t)K;
        return launch("fill_zero_kernel", fill_zero_kernel<T>,
                      dim3((unsigned)std::min<size_t>((n + 255) / 256, 65535)), dim3(256), s, Y, n);
    }
    StreamArgs<T> a;
    a.rows = A->rows;
    a.cols = A->cols;
    a.K = (int)K;
    a.batch = (int)batch;
    a.n_waves = A->n_waves;
    a.n_tiles = A->n_tiles;
    a.group = A->group;
    if (a.group < 1 || a.n_waves % a.group) return fail(SPMM_EINVAL, "n_waves is not a multiple of group");
    a.tiles = A->tiles;
    a.tile_rs = A->tile_rs;
    a.ent_val = static_cast<const T*>(A->ent_val);
    a.ent_col = A->ent_col;
    a.tcols = A->tcols;
    a.row_ids = A->row_ids;
    a.wave_tiles = A->wave_tiles;
    a.X = X;
    a.Y = Y;
    a.P = static_cast<T*>(ws);
    const bool recs = A->n_blob16 > 0 && A->blobs && A->blob_first && A->blob_xid;
    a.blobs = recs ? static_cast<const uint32_t*>(A->blobs) : nullptr;
    a.blob_first = recs ? A->blob_first : nullptr;
    a.blob_xid = recs ? A->blob_xid : nullptr;
    int rc = stream ? boo_dispatch<T>(a, s) : SPMM_OK;
    if (rc) return rc;
    if (A->n_crow > 0) {
        rc = launch_boo_rows<T>(A, X, Y, (int)K, (int)batch,
                                ws ? reinterpret_cast<T*>(static_cast<char*>(ws) +
                                                          boo_ws_slots_bytes(A, sizeof(T), batch, K))
                                   : nullptr,
                                s);
        if (rc) return rc;
    }
    if (A->n_splits > 0) {
        const dim3 grid(A->n_splits, 1, (unsigned)batch);
        rc = launch("boo_fixup_kernel", boo_fixup_kernel<T>, grid, dim3(256), s, A->splits, A->row_ids,
                    (const T*)ws, Y, A->rows, (int)K, (int)batch);
        if (rc) return rc;
    }
    return launch_long_rows<T, int>(A->long_rows, A->n_long, A->rem_indptr, A->rem_col_ind,
                                    static_cast<const T*>(A->rem_vals), X, Y, A->rows, A->cols,
                                    (int)K, (int)batch, s);
}

// Blocks of X in flight per wave (1 measured best on configs 2 and 5, and
// no different on config 3: the walk, not X latency, sets the pace).
#ifndef SPMM_PBR_DEPTH_SMALL
#define SPMM_PBR_DEPTH_SMALL 1   // 256-byte feature tiles (64 float / 32 double)
#endif
#ifndef SPMM_PBR_DEPTH_BIG
#define SPMM_PBR_DEPTH_BIG 1     // 1 KiB feature tiles
#endif

// X of one batch above this many bytes: small feature tiles, one launch each
// (spmm_pbr_set_slab_bytes; 0, the default: never).
std::atomic<long long> g_pbr_slab_bytes{0};

// serial: one launch per feature tile, in order, so the X columns of one tile
// (cols x KT) stay in the MALL while every stripe reads them; otherwise one
// launch over all tiles (grid.y), whose stripes read every tile's X at once.
template <typename T, typename I, int BR, int KT, int VEC>
int launch_pbr(const PbrArgs<T, I>& a, int batch, bool serial, hipStream_t s) {
    const int nkt = (a.K + KT - 1) / KT;
    // 32-bit X offsets when one batch's X is under 4 GiB
    const bool a32 = (uint64_t)a.cols * (uint64_t)a.K * sizeof(T) < (1ull << 32);
    // blocks in flight per wave: X registers per block are STAGE_ITERS * VEC
    constexpr int PD = KT * (int)sizeof(T) <= 256 ? SPMM_PBR_DEPTH_SMALL : SPMM_PBR_DEPTH_BIG;
    auto kern = a32 ? pbr_stripe_kernel<T, I, BR, KT, VEC, PD, true> : pbr_stripe_kernel<T, I, BR, KT, VEC, PD, false>;
    if (!serial) return launch("pbr_stripe_kernel", kern, dim3(round_up8(a.n_stripes), nkt, batch), dim3(64), s, a);
    for (int kt = 0; kt < nkt; ++kt) {
        PbrArgs<T, I> ak = a;
        ak.kt0 = kt;
        const int rc = launch("pbr_stripe_kernel", kern, dim3(round_up8(a.n_stripes), 1, batch), dim3(64), s, ak);
        if (rc) return rc;
    }
    return SPMM_OK;
}

// KT (tile features) is 64 or 256 (float) / 32 or 128 (double); VEC is the
// widest load the lane's run of F features and the buffers allow.
template <typename T, typename I, int BR>
int pbr_dispatch_br(const PbrArgs<T, I>& a, int batch, hipStream_t s) {
    constexpr int small_kt = 256 / (int)sizeof(T);
    constexpr int big_kt = 1024 / (int)sizeof(T);
    // X too big for the MALL: small feature tiles, one launch each
    const long long slab = g_pbr_slab_bytes.load(std::memory_order_relaxed);
    const bool serial = slab > 0 && a.K > small_kt && (long long)a.cols * a.K * (long long)sizeof(T) > slab;
    const bool big = a.K >= big_kt && !serial;
    const int F = (big ? big_kt : small_kt) / (64 / BR);
    const int full = 16 / (int)sizeof(T);
    int vec = 1;
    if (F % full == 0 && a.K % full == 0 && aligned16(a.X) && aligned16(a.Y)) vec = full;
    if (big) {
        if (vec > 1) return launch_pbr<T, I, BR, big_kt, 16 / sizeof(T)>(a, batch, false, s);
        return launch_pbr<T, I, BR, big_kt, 1>(a, batch, false, s);
    }
    if constexpr ((small_kt / (64 / BR)) % (16 / sizeof(T)) == 0) {
        if (vec > 1) return launch_pbr<T, I, BR, small_kt, 16 / sizeof(T)>(a, batch, serial, s);
    }
    return launch_pbr<T, I, BR, small_kt, 1>(a, batch, serial, s);
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
    a.kt0 = 0;
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

// ---------------------------------------------------------------------------
// Scratch of the allocation-free BOO entry point: a file-scope device array
// (one copy per GPU, held until the process ends).  In host code `scratch`
// names a host-side stand-in, not device memory: its device address comes
// from hipGetSymbolAddress, once per device, with that device current.
// ---------------------------------------------------------------------------

constexpr size_t NOALLOC_SCRATCH_BYTES = (size_t)64 << 20;
constexpr int NOALLOC_MAX_DEVICES = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// Device address of this GPU's scratch (the current device's).
int scratch_for_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(SPMM_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) return fail(SPMM_EUNSUPPORTED, "device index %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr)
            return fail(SPMM_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = ptr;
    }
    *out = g_scratch_ptr[dev];
    return SPMM_OK;
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================

extern "C" {

const char* spmm_last_error(void) { return g_last_error.c_str(); }

const char* spmm_version(void) { return "spmm_amd 0.1 gfx950"; }

struct spmm_boo_stage {
    spmm_stage::Staged s;
    spmm_dtype dtype;
};

int spmm_boo_stage_create(const spmm_boo_host* H, int32_t max_item_nnz, int32_t long_threshold,
                          int32_t n_waves, int32_t group, float min_reuse, spmm_boo_stage** out) {
    if (!H || !out) return fail(SPMM_EINVAL, "null staging argument");
    *out = nullptr;
    if (H->rows < 0 || H->cols < 0 || H->n_row_groups < 0 || H->n_col_groups < 0 || H->num_blocks < 0)
        return fail(SPMM_EINVAL, "negative BOO sizes");
    if (!H->row_grp_ptr || !H->row_ids || !H->col_grp_ptr || (H->cols > 0 && !H->col_ids) ||
        !H->rem_indptr || (H->num_blocks > 0 && (!H->blk_row_grp || !H->blk_col_grp || !H->blk_nz_ptr ||
                                                 !H->blk_shift || !H->nz_idx || !H->nz_val)))
        return fail(SPMM_EINVAL, "null BOO host array");
    if (max_item_nnz < 1) return fail(SPMM_EINVAL, "max_item_nnz must be positive");
    if (n_waves < 1) return fail(SPMM_EINVAL, "n_waves must be positive");
    if (group != 1 && group != 2 && group != 4) return fail(SPMM_EINVAL, "group must be 1, 2 or 4");
    if (!(min_reuse >= 0.0f)) return fail(SPMM_EINVAL, "min_reuse must be >= 0");
    if (H->dtype != SPMM_F32 && H->dtype != SPMM_F64) return fail(SPMM_EINVAL, "unknown dtype %d", (int)H->dtype);
    spmm_boo_stage* st = new (std::nothrow) spmm_boo_stage();
    if (!st) return fail(SPMM_ENOMEM, "out of host memory");
    st->dtype = H->dtype;
    try {
        if (H->dtype == SPMM_F32) {
            spmm_stage::Builder<float>::In in{H->rows, H->cols, H->n_row_groups, H->n_col_groups, H->num_blocks,
                                              H->row_grp_ptr, H->row_ids, H->col_grp_ptr, H->col_ids,
                                              H->blk_row_grp, H->blk_col_grp, H->blk_nz_ptr, H->blk_shift,
                                              H->nz_idx, static_cast<const float*>(H->nz_val), H->rem_indptr,
                                              H->rem_col_ind, static_cast<const float*>(H->rem_vals)};
            spmm_stage::Builder<float>(in, max_item_nnz, long_threshold, n_waves, group, min_reuse).run(st->s);
        } else {
            spmm_stage::Builder<double>::In in{H->rows, H->cols, H->n_row_groups, H->n_col_groups, H->num_blocks,
                                               H->row_grp_ptr, H->row_ids, H->col_grp_ptr, H->col_ids,
                                               H->blk_row_grp, H->blk_col_grp, H->blk_nz_ptr, H->blk_shift,
                                               H->nz_idx, static_cast<const double*>(H->nz_val), H->rem_indptr,
                                               H->rem_col_ind, static_cast<const double*>(H->rem_vals)};
            spmm_stage::Builder<double>(in, max_item_nnz, long_threshold, n_waves, group, min_reuse).run(st->s);
        }
    } catch (const std::invalid_argument& e) {
        delete st;
        return fail(SPMM_EINVAL, "%s", e.what());
    } catch (const std::bad_alloc&) {
        delete st;
        return fail(SPMM_ENOMEM, "out of host memory");
    }
    if (st->s.ent_col.size() > (size_t)INT32_MAX || st->s.n_tiles() > (size_t)INT32_MAX / 64 ||
        st->s.tcols.size() > (size_t)INT32_MAX) {
        delete st;
        return fail(SPMM_EUNSUPPORTED, "BOO matrix too large for 32-bit tile offsets");
    }
    *out = st;
    return SPMM_OK;
}

int spmm_boo_stage_sizes(const spmm_boo_stage* st, spmm_boo_stage_info* info) {
    if (!st || !info) return fail(SPMM_EINVAL, "null staging argument");
    info->n_tiles = (int64_t)st->s.n_tiles();
    info->n_ent = (int64_t)st->s.ent_col.size();
    info->n_tcols = (int64_t)st->s.tcols.size();
    info->n_splits = (int64_t)(st->s.splits.size() / 4);
    info->n_long = (int64_t)st->s.long_rows.size();
    info->n_crow = (int64_t)st->s.crow_id.size();
    info->n_cnz = (int64_t)st->s.ccol.size();
    info->n_crow_long = st->s.n_crow_long;
    info->n_stream_rows = st->s.n_stream_rows;
    info->n_blob16 = (int64_t)(st->s.blobs.size() / 4);
    info->n_gtask = (int64_t)(st->s.gtask.size() / 2);
    info->n_gtask_order = (int64_t)st->s.gtask_order.size();
    info->n_slots = st->s.n_slots;
    info->n_waves = st->s.n_waves;
    info->group = st->s.group;
    return SPMM_OK;
}

int spmm_boo_stage_copy(const spmm_boo_stage* st, int32_t* tiles, uint8_t* tile_rs,
                        void* ent_val, uint8_t* ent_col, int32_t* tcols, int32_t* splits,
                        int32_t* long_rows, int32_t* wave_tiles, int32_t* crow_ptr, int32_t* crow_id,
                        int32_t* ccol, void* cval, int32_t* gtask, int32_t* gtask_ptr) {
    if (!st) return fail(SPMM_EINVAL, "null staging handle");
    const spmm_stage::Staged& s = st->s;
    auto put = [](void* dst, const void* src, size_t bytes) {
        if (bytes && dst) std::memcpy(dst, src, bytes);
        return bytes == 0 || dst != nullptr;
    };
    bool ok = put(tiles, s.tiles.data(), s.tiles.size() * 4) &&
              put(tile_rs, s.tile_rs.data(), s.tile_rs.size()) &&
              put(ent_val, s.ent_val.data(), s.ent_val.size()) &&
              put(ent_col, s.ent_col.data(), s.ent_col.size()) &&
              put(tcols, s.tcols.data(), s.tcols.size() * 4) &&
              put(splits, s.splits.data(), s.splits.size() * 4) &&
              put(long_rows, s.long_rows.data(), s.long_rows.size() * 4) &&
              put(wave_tiles, s.wave_tiles.data(), s.wave_tiles.size() * 4) &&
              put(crow_ptr, s.crow_ptr.data(), s.crow_ptr.size() * 4) &&
              put(crow_id, s.crow_id.data(), s.crow_id.size() * 4) &&
              put(ccol, s.ccol.data(), s.ccol.size() * 4) &&
              put(cval, s.cval.data(), s.cval.size()) &&
              put(gtask, s.gtask.data(), s.gtask.size() * 4) &&
              put(gtask_ptr, s.gtask_ptr.data(), s.gtask_ptr.size() * 4);
    return ok ? SPMM_OK : fail(SPMM_EINVAL, "null output array for a non-empty staging field");
}

int spmm_boo_stage_copy_blobs(const spmm_boo_stage* st, void* blobs, uint32_t* blob_first, uint32_t* blob_xid) {
    if (!st) return fail(SPMM_EINVAL, "null staging handle");
    const spmm_stage::Staged& s = st->s;
    if (s.blobs.empty()) return SPMM_OK;
    if (!blobs || !blob_first || !blob_xid) return fail(SPMM_EINVAL, "null output array for the record stream");
    std::memcpy(blobs, s.blobs.data(), s.blobs.size() * 4);
    std::memcpy(blob_first, s.blob_first.data(), s.blob_first.size() * 4);
    std::memcpy(blob_xid, s.blob_xid.data(), s.blob_xid.size() * 4);
    return SPMM_OK;
}

int spmm_boo_stage_copy_gtask_order(const spmm_boo_stage* st, int32_t* gtask_order) {
    if (!st) return fail(SPMM_EINVAL, "null staging handle");
    const spmm_stage::Staged& s = st->s;
    if (s.gtask_order.empty()) return SPMM_OK;
    if (!gtask_order) return fail(SPMM_EINVAL, "null output array for the chunk-task order");
    std::memcpy(gtask_order, s.gtask_order.data(), s.gtask_order.size() * 4);
    return SPMM_OK;
}

void spmm_boo_stage_destroy(spmm_boo_stage* st) { delete st; }

size_t spmm_boo_workspace_bytes(const spmm_boo_desc* A, spmm_dtype dtype, int64_t batch, int64_t K) {
    if (!A || batch <= 0 || K <= 0) return 0;
    const size_t es = dtype == SPMM_F64 ? 8 : 4;
    const size_t gather = A->n_gtask > 0 ? (size_t)A->n_gtask * (size_t)batch * (size_t)K * es : 0;
    return boo_ws_slots_bytes(A, es, batch, K) + gather;
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

int spmm_boo_matmul_noalloc(const spmm_boo_desc* A, spmm_dtype dtype, const void* X, void* Y,
                            int64_t batch, int64_t K, void* stream) {
    if (!A) return fail(SPMM_EINVAL, "null BOO descriptor");
    int rc = check_shape(batch, K);
    if (rc) return rc;
    if (dtype != SPMM_F32 && dtype != SPMM_F64) return fail(SPMM_EINVAL, "unknown dtype %d", (int)dtype);
    const size_t need = spmm_boo_workspace_bytes(A, dtype, batch, K);
    if (need > NOALLOC_SCRATCH_BYTES)
        return fail(SPMM_ENOMEM,
                    "spmm_boo_matmul_noalloc: this staging and shape need %zu bytes of workspace, more than its "
                    "%zu-byte scratch; call spmm_boo_matmul with a workspace instead",
                    need, NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if (need > 0) {
        rc = scratch_for_current_device(&ws);
        if (rc) return rc;
    }
    return spmm_boo_matmul(A, dtype, X, Y, batch, K, ws, need > 0 ? NOALLOC_SCRATCH_BYTES : 0, stream);
}

int spmm_pbr_set_slab_bytes(int64_t bytes) {
    if (bytes < 0) return fail(SPMM_EINVAL, "negative PBR slab size");
    g_pbr_slab_bytes.store(bytes, std::memory_order_relaxed);
    return SPMM_OK;
}

int64_t spmm_pbr_get_slab_bytes(void) { return g_pbr_slab_bytes.load(std::memory_order_relaxed); }

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

// ---------------------------------------------------------------------------
// Launch introspection: the multiply's own dispatch, recorded instead of
// launched, then each kernel's attributes and occupancy from the runtime.
// ---------------------------------------------------------------------------

namespace {

struct RecordGuard {
    explicit RecordGuard(std::vector<LaunchRec>* r) { t_record = r; }
    ~RecordGuard() { t_record = nullptr; }
};

int describe_launches(const std::vector<LaunchRec>& recs, spmm_launch_info* out, int32_t cap, int32_t* n_out) {
    if (n_out) *n_out = (int32_t)recs.size();
    for (size_t i = 0; i < recs.size() && (int64_t)i < cap; ++i) {
        const LaunchRec& r = recs[i];
        spmm_launch_info& o = out[i];
        std::memset(&o, 0, sizeof o);
        o.kernel = r.name;
        o.grid[0] = r.grid.x;
        o.grid[1] = r.grid.y;
        o.grid[2] = r.grid.z;
        o.block = r.block.x * r.block.y * r.block.z;
        hipFuncAttributes fa;
        hipError_t e = hipFuncGetAttributes(&fa, r.fn);
        if (e != hipSuccess) return fail(SPMM_ELAUNCH, "hipFuncGetAttributes(%s): %s", r.name, hipGetErrorString(e));
        o.registers = fa.numRegs;
        o.scratch_bytes = (int32_t)fa.localSizeBytes;
        o.lds_bytes = (int32_t)fa.sharedSizeBytes;
        o.max_threads = fa.maxThreadsPerBlock;
        int nb = 0;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, r.fn, (int)o.block, 0);
        if (e != hipSuccess)
            return fail(SPMM_ELAUNCH, "hipOccupancyMaxActiveBlocksPerMultiprocessor(%s): %s", r.name,
                        hipGetErrorString(e));
        o.wgs_per_cu = nb;
    }
    return SPMM_OK;
}

// Stand-in operand addresses for a recorded dispatch: nothing is launched, so
// they are never dereferenced; only their alignment steers the dispatch.
const void* stand_in(const void* p) { return p ? p : reinterpret_cast<const void*>(uintptr_t(1) << 12); }

}  // namespace

int spmm_boo_launch_info(const spmm_boo_desc* A, spmm_dtype dtype, const void* X, const void* Y, int64_t batch,
                         int64_t K, spmm_launch_info* out, int32_t cap, int32_t* n_out) {
    if (cap < 0 || (cap > 0 && !out)) return fail(SPMM_EINVAL, "null launch info array");
    std::vector<LaunchRec> recs;
    int rc;
    {
        RecordGuard g(&recs);
        void* ws = const_cast<void*>(stand_in(nullptr));
        rc = spmm_boo_matmul(A, dtype, stand_in(X), const_cast<void*>(stand_in(Y)), batch, K, ws, SIZE_MAX,
                             nullptr);
    }
    return rc ? rc : describe_launches(recs, out, cap, n_out);
}

int spmm_pbr_launch_info(const spmm_pbr_desc* A, spmm_dtype dtype, const void* X, const void* Y, int64_t batch,
                         int64_t K, spmm_launch_info* out, int32_t cap, int32_t* n_out) {
    if (cap < 0 || (cap > 0 && !out)) return fail(SPMM_EINVAL, "null launch info array");
    std::vector<LaunchRec> recs;
    int rc;
    {
        RecordGuard g(&recs);
        rc = spmm_pbr_matmul(A, dtype, stand_in(X), const_cast<void*>(stand_in(Y)), batch, K, nullptr);
    }
    return rc ? rc : describe_launches(recs, out, cap, n_out);
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
