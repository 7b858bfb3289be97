// Host-side staging of a BOO matrix into the tile stream the gfx950 kernel
// reads (no device work here).
//
// csr_to_boo (boo_matrix/boo_matrix.cpp:53-274) emits row groups, column
// groups, blocks with uint16 local indices sorted row-major inside each block,
// and a remainder CSR.  The kernel wants fixed-size units it can prefetch
// several steps ahead without any dependent lookup, so every row group is cut
// into 32-row slices and each slice's work into tiles:
//
//   * a tile is <= 32 rows x <= 32 columns with <= 96 entries, its entries
//     sorted by local row (the block's row-major order is kept), each entry a
//     value plus a one-byte local column, and a 33-entry row-start table;
//   * a block contributes one tile per 32-column chunk of its column group
//     (a chunk too full for 96 entries is cut between rows);
//   * the slice's short remainder rows (<= long_threshold entries) contribute
//     tiles over the sorted set of their distinct columns, 32 at a time;
//     longer rows are listed for the split-row pass;
//   * a slice with no entries still gets one empty tile, so its Y rows are
//     written (zeros);
//   * a tile whose entries crowd into a few rows (a remainder row, say) is
//     flagged to be computed one busy row at a time with lanes along K.
//
// Up to `group` slices that share column chunks form a group, run by one
// workgroup of `group` waves in lock step: step s stages one 32-column X tile
// in LDS for all members, and each member (wave) adds its own tile of that
// step.  Member streams therefore have equal length (padding tiles with no
// entries fill the gaps) and equal column ids per step.
//
// A slice heavier than max_item_nnz sits alone in its group and is cut at tile
// boundaries into several items: the first stores Y, the others write partial
// sums to workspace slots that a fixup pass adds in slot order.  Each XCD
// gets a contiguous share of groups of near-equal cost (an optimal min-max
// split into workgroup ranges), dealt round-robin to its workgroups.  Column
// ids of block tiles point into col_ids; those of remainder tiles are
// appended after it in the same array.
#pragma once

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>
#include <thread>
#include <type_traits>
#include <vector>

namespace spmm_stage {

constexpr int TILE_ROWS = 32;
constexpr int TILE_COLS = 32;
constexpr int TILE_ENT = 96;
static_assert(TILE_ENT < 256, "tile row starts are stored in bytes");
constexpr int TILE_RS = TILE_ROWS + 1;
constexpr int TILE_WORDS = 8;
constexpr uint32_t FLAG_LAST = 1u;    // last tile of its item
constexpr uint32_t FLAG_SERIAL = 2u;  // computed one busy row at a time
constexpr int SERIAL_MAX_BUSY = 4;    // busy rows a serial tile may have

// Cost model for dealing groups to workgroups, in units of one entry's work:
// a step (X tile staged, workgroup synchronised) and finishing an item.
constexpr long long COST_STEP = 256;
constexpr long long COST_ITEM = 512;
// A group's members all end their item at its last step, so in a uniform
// matrix every wave stores its 32 Y rows in the same step and the stores
// leave in one burst that the next step's loads queue behind.  In a group of
// at least EARLY_STORE_MIN_STEPS steps, its shared remainder tiles are walked
// first and each member stores at its own last tile with entries: in a
// stencil the members of the lower plane then finish a few steps before the
// others and the burst splits (27-point 64^3, K=64: -1 to -2.3 us).  Short
// groups keep one store step (5-point 256^2, K=128: 16.4 -> 18.0 us
// otherwise).
constexpr size_t EARLY_STORE_MIN_STEPS = 12;

// Gather-pass rows longer than the long-row threshold are summed in chunks of
// at most GATHER_CHUNK entries, one workgroup each, into partial rows that a
// fixup pass adds in chunk order.
constexpr int GATHER_CHUNK = 1024;
// When the gather rows' lengths are skewed (standard deviation above the
// mean, as in a power-law graph), rows longer than GATHER_SKEWED_LONG go to
// chunk tasks too: there the row pass's waves stall on a few mid-length rows
// that chunk tasks run wider (R-MAT 2^20, K=128: 2.52 -> 2.18 ms).  With even
// lengths the chunks' partial rows and fixup cost more than they save (48
// entries per row: 248 -> 423 us at K=32), so the threshold stays as given.
constexpr int GATHER_SKEWED_LONG = 32;
// Chunk tasks read X rows at random from every column, and on a power-law
// graph a few columns carry much of the entries, yet in one pass their X rows
// keep being evicted from L2 by the cold gathers in between (R-MAT 2^20: the
// 16,384 most used columns carry 55 % of the entries, yet an LRU model of
// the chunk pass hits L2 on only ~40 % of its reads).  When the GATHER_HOT_COLS most used columns of the
// long gather rows carry at least GATHER_HOT_SHARE of their entries (and
// GATHER_HOT_SKEW times their share of the columns), each long row's entries
// in those columns come first, in their own chunk tasks, and every such task
// is launched before the others: their X rows -- 256 bytes of each per
// workgroup's feature slab, 4 MiB for 16,384 of them, one XCD's L2 -- then
// stay resident while they run.  Each row's partial rows are still added in
// its task order, so its sum is deterministic.
constexpr int GATHER_HOT_COLS = 16384;
constexpr double GATHER_HOT_SHARE = 0.25;
constexpr double GATHER_HOT_SKEW = 4.0;
// The gather pass walks its short rows in staging order, and rows next to
// each other in that order run at about the same time on one XCD, so X rows
// they share are fetched once into that XCD's L2.  When a Cuthill-McKee order
// of the rows (breadth first over the rows their columns name) repeats more
// of the X rows within a window of GATHER_REUSE_WINDOW rows than the slice
// order does, by a factor of GATHER_REORDER_GAIN, the rows are walked in
// that order instead.  Each row keeps its own entries and their order, so
// its sum is the same; only which rows run side by side changes.  A randomly
// permuted 27-point stencil (128^3, K=32) repeats 9.3x more X rows in that
// order and its gather pass runs in 0.50 ms instead of 1.16 ms; an R-MAT
// graph (2^20, K=128) repeats 1.32x more but runs 5.6 % slower (its row
// order already keeps hub columns hot), hence a gain of 2 to switch.
constexpr int GATHER_REUSE_WINDOW = 8192;
constexpr double GATHER_REORDER_GAIN = 2.0;
// Both orders are compared on their first GATHER_REUSE_SAMPLE entries.
constexpr long long GATHER_REUSE_SAMPLE = 1ll << 23;

// Record stream (float, groups of 4): each wave's tiles again, one
// contiguous, 16-byte aligned record per step, so that a wave moves a whole
// step's entries into LDS with one DMA instruction, and beside it the ids of
// the X rows the wave stages at each step (8 per tile), so that the X tile
// can be staged without waiting for the step's record.  A record:
//   word 0   nnz | nr << 8 | nc << 14 | flags << 20 | nvec(record 4 steps later) << 24
//   word 1   slot (-1: the item stores Y)
//   word 2   offset, in 16-byte units, of this wave's record 4 steps later
//            (clamped to its last record)
//   word 3   ROWCONTIG: the slice's first Y row (row r is that + r);
//            otherwise its offset into row_ids
//   uint8 rs[32]      (absent when nnz = 0) first entry of each row; row r
//                     ends at rs[r + 1], row 31 at nnz
//   uint8 col[nnz]    local columns, then zero padding to 4 bytes
//   float val[nnz]    then zero padding to 16 bytes
// The X ids of tile t (the wave's tile index, as in tiles): xid[8 t + j] is
// the X row of column 2m + (j >> 2) + 8 (j & 3) of the step's X tile, m the
// wave's index in its workgroup, clamped to the tile's last column (X row 0
// for a tile without columns).
constexpr uint32_t BLOB_LAST = 1u, BLOB_SERIAL = 2u, BLOB_ROWCONTIG = 4u;
constexpr int BLOB_MAX_BYTES = 16 + 32 + TILE_ENT + 4 * TILE_ENT;  // 528
constexpr int BLOB_LOOKAHEAD = 4;



struct Staged {
    // [n_tiles][8]: ent_off, nnz|nc<<8|nr<<16|flags<<24, cid_off, row_off, slot, 0, 0, 0
    // (slot -1: the item stores Y; otherwise its partial slot)
    std::vector<int32_t> tiles;
    std::vector<uint8_t> tile_rs;    // [n_tiles][33]: row starts relative to ent_off (<= TILE_ENT)
    std::vector<uint8_t> ent_col;    // [n_ent] (zero padding after odd tiles and at the end)
    std::vector<char> ent_val;       // [n_ent] values (float or double bytes)
    std::vector<int32_t> tcols;      // [cols + extra]: col_ids, then remainder tile columns
    std::vector<int32_t> splits;     // [n_splits][4]: row_off, nr, slot_begin, slot_end
    std::vector<int32_t> long_rows;  // rows whose remainder exceeds long_threshold
    std::vector<int32_t> wave_tiles; // [n_waves+1]
    // rows of the gather pass: Y row ids, CSR of their entries (global columns)
    std::vector<int32_t> crow_ptr;   // [n_crow+1]
    std::vector<int32_t> crow_id;    // [n_crow]
    std::vector<int32_t> ccol;       // [n_cnz]
    std::vector<char> cval;          // [n_cnz] values (float or double bytes)
    // the last n_crow_long gather rows are long: chunk tasks (entry begin,
    // end) of long row i are gtask[gtask_ptr[i] .. gtask_ptr[i+1])
    int32_t n_crow_long = 0;
    std::vector<int32_t> gtask;      // [n_gtask][2]
    std::vector<int32_t> gtask_ptr;  // [n_crow_long+1]
    // launch order of the chunk tasks (hot-column tasks first), or empty:
    // task order
    std::vector<int32_t> gtask_order;
    int32_t n_slots = 0;
    int32_t n_waves = 0;
    int32_t group = 1;               // waves per workgroup sharing X tiles
    int32_t n_stream_rows = 0;       // rows the tile stream stores (the rest: crow_id)
    // record stream (float, group 4; empty otherwise): records in 16-byte
    // units (4 words each); per wave 8 words: offsets of its first 4 records
    // (clamped to its last), their 16-byte counts packed one per byte, its
    // step count, its first tile, 0; and the X ids, 8 per tile
    std::vector<uint32_t> blobs;
    std::vector<uint32_t> blob_first;
    std::vector<uint32_t> blob_xid;
    size_t n_tiles() const { return tiles.size() / TILE_WORDS; }
};

// f(begin, end) over [0, n) in contiguous ranges on up to 16 threads (the
// calling thread takes the first); small n runs inline.  f must not throw.
template <typename F>
inline void par_ranges(size_t n, F&& f) {
    const unsigned hw = std::thread::hardware_concurrency();
    const size_t nt = std::min<size_t>(std::min<size_t>(hw ? hw : 1, 16), (n + 4095) / 4096);
    if (nt <= 1) {
        f((size_t)0, n);
        return;
    }
    const size_t per = (n + nt - 1) / nt;
    std::vector<std::thread> th;
    for (size_t t = 1; t < nt; ++t) {
        const size_t b = t * per, e = std::min(n, b + per);
        if (b < e) th.emplace_back([&f, b, e]() { f(b, e); });
    }
    f((size_t)0, std::min(n, per));
    for (std::thread& x : th) x.join();
}

// One nonzero on its way into a tile.
struct Ent {
    int32_t src;      // index of the value in its source array
    uint8_t lr;       // local row in the slice
    uint8_t lc;       // local column in the tile
    uint8_t from_rem; // value comes from rem_vals rather than nz_val
    uint8_t pad;
};

template <typename T>
class Builder {
public:
    struct In {
        int32_t rows, cols, n_row_groups, n_col_groups, num_blocks;
        const int32_t *row_grp_ptr, *row_ids, *col_grp_ptr, *col_ids;
        const int32_t *blk_row_grp, *blk_col_grp, *blk_nz_ptr;
        const uint8_t* blk_shift;
        const uint16_t* nz_idx;
        const T* nz_val;
        const int32_t *rem_indptr, *rem_col_ind;
        const T* rem_vals;
    };

    // min_reuse: a slice with fewer than min_reuse nonzeros per X row its
    // tiles would stage (scattered columns: a permuted or power-law matrix)
    // gains nothing from staging X tiles, and its rows go to the row-wise
    // gather pass, as do empty slices; 0 keeps every slice in the tile stream.
    Builder(const In& in, int max_item_nnz, int long_threshold, int n_waves, int group, float min_reuse)
        : in_(in), max_item_nnz_(max_item_nnz), long_threshold_(long_threshold),
          want_waves_(n_waves), G_(group), min_reuse_(min_reuse) {}

    void run(Staged& S) {
        S = Staged();
        S.group = G_;
        S.tcols.assign(in_.col_ids, in_.col_ids + in_.cols);
        collect_slices(S);
        for (const Slice& sl : slices_) {  // long remainder rows of the tile stream's slices
            if (sl.csr) continue;
            S.n_stream_rows += sl.nr;
            for (size_t i = sl.g0; i < sl.g1; ++i) S.long_rows.push_back(longs_[i].row);
        }
        make_groups();
        for (size_t g = 0; g < groups_.size(); ++g) build_group_steps(S, g);
        split_heavy(S);
        deal_and_emit(S);
        emit_blobs(S);
        emit_csr(S);
    }

private:
    // ---- a 32-row slice of a row group: its block chunks and short remainder
    struct Chunk {
        int cid_off, nc;
        size_t e0, e1;  // entries in pool_, row-major
    };
    struct Slice {
        int row_off, nr;
        size_t c0, c1;  // chunks in chunks_
        size_t r0, r1;  // remainder entries in pool_ (lc = 0; column in rcol_)
        size_t g0, g1;  // its long remainder rows in longs_
        long long nnz;
        bool csr;       // rows go to the gather pass, not the tile stream; its short
                        // remainder is then read from the input CSR, not pool_
    };
    struct LongRow {
        int32_t lr, row;
    };
    // ---- one step of a group: one X tile, each member's entries in it
    struct Step {
        int cid_off, nc;
        size_t m0;      // member pieces in pieces_ [m0, m0 + G)
    };
    struct Piece {
        size_t e0, e1;  // entries in tent_ (lc = tile-local column)
    };
    struct Group {
        int members[4];
        int n_members;
        size_t s0, s1;  // steps in steps_
        long long cost;
        int slot;       // -1: stores Y; else the partial slot of an item of a split slice
        bool early = false;  // members store at their own last tile with entries
    };

    // Every index the staging later uses to address a host array is checked
    // here, so malformed input becomes invalid_argument (SPMM_EINVAL), never
    // an out-of-range access: row groups, column ids and the remainder CSR.
    void check_indices() const {
        if (in_.row_grp_ptr[0] != 0 || in_.row_grp_ptr[in_.n_row_groups] != in_.rows)
            throw std::invalid_argument("row_grp_ptr must run from 0 to rows");
        if (in_.col_grp_ptr[0] != 0 || in_.col_grp_ptr[in_.n_col_groups] != in_.cols)
            throw std::invalid_argument("col_grp_ptr must run from 0 to cols");
        for (int g = 0; g < in_.n_col_groups; ++g)
            if (in_.col_grp_ptr[g + 1] < in_.col_grp_ptr[g])
                throw std::invalid_argument("col_grp_ptr is not nondecreasing");
        for (int c = 0; c < in_.cols; ++c)
            if (in_.col_ids[c] < 0 || in_.col_ids[c] >= in_.cols) throw std::invalid_argument("col_ids out of range");
        if (in_.rem_indptr[0] != 0) throw std::invalid_argument("rem_indptr must start at 0");
        for (int r = 0; r < in_.rows; ++r)
            if (in_.rem_indptr[r + 1] < in_.rem_indptr[r])
                throw std::invalid_argument("rem_indptr is not nondecreasing");
        const int32_t n_rem = in_.rem_indptr[in_.rows];
        if (n_rem > 0 && !in_.rem_col_ind) throw std::invalid_argument("rem_col_ind is null");
        for (int32_t j = 0; j < n_rem; ++j)
            if (in_.rem_col_ind[j] < 0 || in_.rem_col_ind[j] >= in_.cols)
                throw std::invalid_argument("rem_col_ind out of range");
        if (in_.num_blocks > 0 && in_.blk_nz_ptr[0] != 0) throw std::invalid_argument("blk_nz_ptr must start at 0");
        for (int b = 0; b < in_.num_blocks; ++b)
            if (in_.blk_nz_ptr[b + 1] < in_.blk_nz_ptr[b])
                throw std::invalid_argument("blk_nz_ptr is not nondecreasing");
    }

    void collect_slices(Staged& S) {
        check_indices();
        {
            const size_t n_ent = (size_t)(in_.num_blocks > 0 ? in_.blk_nz_ptr[in_.num_blocks] : 0) +
                                 (size_t)in_.rem_indptr[in_.rows];
            pool_.reserve(n_ent);
            rcol_.reserve(n_ent);
        }
        // Send empty slices, and slices whose tiles would stage more X rows
        // than min_reuse per entry allows, to the gather pass.  A slice's
        // tiles stage every column of each block chunk it touches plus its
        // remainder's distinct columns (counted with stamp: the last slice
        // that counted the column).
        const bool use_stamp = min_reuse_ > 0.0f;
        std::vector<int32_t> stamp(use_stamp ? (size_t)in_.cols : 0, -1);
        int blk = 0;
        std::vector<Ent> ents;
        for (int rg = 0; rg < in_.n_row_groups; ++rg) {
            const int r0 = in_.row_grp_ptr[rg];
            const int nr_g = in_.row_grp_ptr[rg + 1] - r0;
            if (nr_g < 0) throw std::invalid_argument("row_grp_ptr is not nondecreasing");
            const int bb = blk;
            while (blk < in_.num_blocks && in_.blk_row_grp[blk] == rg) ++blk;
            if (blk < in_.num_blocks && in_.blk_row_grp[blk] < rg)
                throw std::invalid_argument("blocks are not sorted by row group");
            const int be = blk;
            for (int s0 = 0; s0 < nr_g; s0 += TILE_ROWS) {
                Slice sl;
                sl.nr = std::min(TILE_ROWS, nr_g - s0);
                sl.row_off = r0 + s0;
                sl.c0 = chunks_.size();
                sl.nnz = 0;
                sl.csr = false;
                for (int b = bb; b < be; ++b) {
                    const int cg = in_.blk_col_grp[b];
                    if (cg < 0 || cg >= in_.n_col_groups) throw std::invalid_argument("blk_col_grp out of range");
                    const int c0 = in_.col_grp_ptr[cg];
                    const int ncb = in_.col_grp_ptr[cg + 1] - c0;
                    const int sh = in_.blk_shift[b];
                    const uint32_t mask = (1u << sh) - 1u;
                    const int e0 = in_.blk_nz_ptr[b], e1 = in_.blk_nz_ptr[b + 1];
                    ents.clear();
                    int prev_row = -1;
                    for (int e = e0; e < e1; ++e) {
                        const int row = (int)((uint32_t)in_.nz_idx[e] >> sh);
                        const int col = (int)((uint32_t)in_.nz_idx[e] & mask);
                        if (row < prev_row) throw std::invalid_argument("block entries are not row-major");
                        prev_row = row;
                        if (row >= nr_g || col >= ncb) throw std::invalid_argument("block entry out of range");
                        if (row < s0 || row >= s0 + sl.nr) continue;
                        ents.push_back(Ent{e, (uint8_t)(row - s0), 0, 0, 0});
                        colx_.push_back(col);
                    }
                    if (ents.empty()) continue;
                    // one chunk per 32 columns of the column group
                    const size_t cx0 = colx_.size() - ents.size();
                    for (int k0 = 0; k0 < ncb; k0 += TILE_COLS) {
                        const size_t p0 = pool_.size();
                        for (size_t u = 0; u < ents.size(); ++u) {
                            const int col = colx_[cx0 + u];
                            if (col >= k0 && col < k0 + TILE_COLS) {
                                Ent x = ents[u];
                                x.lc = (uint8_t)(col - k0);
                                pool_.push_back(x);
                            }
                        }
                        if (pool_.size() > p0)
                            chunks_.push_back(Chunk{c0 + k0, std::min(TILE_COLS, ncb - k0), p0, pool_.size()});
                    }
                    colx_.resize(cx0);
                    sl.nnz += (long long)ents.size();
                }
                sl.c1 = chunks_.size();
                sl.r0 = pool_.size();
                sl.g0 = longs_.size();
                // the slice's short remainder: its entries and distinct
                // columns decide tile stream or gather pass (classify)
                long long staged = 0;
                for (size_t c = sl.c0; c < sl.c1; ++c) staged += chunks_[c].nc;
                const int32_t si = (int32_t)slices_.size();
                for (int lr = 0; lr < sl.nr; ++lr) {
                    const int row = in_.row_ids[sl.row_off + lr];
                    if (row < 0 || row >= in_.rows) throw std::invalid_argument("row_ids out of range");
                    const int rs = in_.rem_indptr[row], re = in_.rem_indptr[row + 1];
                    if (re == rs) continue;
                    if (re - rs > long_threshold_) {
                        longs_.push_back(LongRow{lr, row});
                        continue;
                    }
                    sl.nnz += re - rs;
                    if (use_stamp)
                        for (int j = rs; j < re; ++j) {
                            const int32_t col = in_.rem_col_ind[j];
                            if (stamp[col] != si) {
                                stamp[col] = si;
                                ++staged;
                            }
                        }
                }
                sl.g1 = longs_.size();
                sl.csr = use_stamp && (sl.nnz == 0 || (double)sl.nnz < (double)min_reuse_ * (double)staged);
                if (!sl.csr) {
                    rcol_.resize(pool_.size());  // block entries have no entry here
                    for (int lr = 0; lr < sl.nr; ++lr) {
                        const int row = in_.row_ids[sl.row_off + lr];
                        const int rs = in_.rem_indptr[row], re = in_.rem_indptr[row + 1];
                        if (re == rs || re - rs > long_threshold_) continue;
                        for (int j = rs; j < re; ++j) {
                            pool_.push_back(Ent{j, (uint8_t)lr, 0, 1, 0});
                            rcol_.push_back(in_.rem_col_ind[j]);
                        }
                    }
                }
                sl.r1 = pool_.size();
                slices_.push_back(sl);
            }
        }
        if (blk != in_.num_blocks) throw std::invalid_argument("block row groups out of range");
        rcol_.resize(pool_.size());
    }

    // f(lr, j) for each short remainder entry j of gather slice sl, row by
    // row, from the input CSR (the order pool_ would hold them in).
    template <typename F>
    void for_short_rem(const Slice& sl, F&& f) const {
        for (int lr = 0; lr < sl.nr; ++lr) {
            const int row = in_.row_ids[sl.row_off + lr];
            const int rs = in_.rem_indptr[row], re = in_.rem_indptr[row + 1];
            if (re - rs > long_threshold_) continue;
            for (int j = rs; j < re; ++j) f(lr, j);
        }
    }

    // Global column of a pool_ entry of slice chunk c (block) or remainder.
    int32_t ent_col_of(size_t e, const Chunk* c) const {
        return c ? in_.col_ids[c->cid_off + pool_[e].lc] : rcol_[e];
    }

    // Entries of each gather row (block entries plus remainder, long or not),
    // slice by slice; the long-row threshold of the gather pass follows from
    // their spread.
    int gather_long_threshold() const {
        double s1 = 0.0, s2 = 0.0;
        long long n = 0;
        std::vector<long long> cnt;
        for (const Slice& sl : slices_) {
            if (!sl.csr) continue;
            cnt.assign((size_t)sl.nr, 0);
            for (size_t c = sl.c0; c < sl.c1; ++c)
                for (size_t e = chunks_[c].e0; e < chunks_[c].e1; ++e) ++cnt[pool_[e].lr];
            for (int lr = 0; lr < sl.nr; ++lr) {  // short and long remainder rows alike
                const int row = in_.row_ids[sl.row_off + lr];
                cnt[lr] += in_.rem_indptr[row + 1] - in_.rem_indptr[row];
            }
            for (long long c : cnt) {
                s1 += (double)c;
                s2 += (double)c * (double)c;
            }
            n += sl.nr;
        }
        if (n == 0) return long_threshold_;
        const double mean = s1 / (double)n, var = s2 / (double)n - mean * mean;
        return var > mean * mean ? std::min(long_threshold_, GATHER_SKEWED_LONG) : long_threshold_;
    }

    // The gather pass's rows: every row of every slice sent there, whole (its
    // block entries in block order, then its remainder, long or not).  Rows of
    // at most the gather pass's long-row threshold come first, in slice order;
    // the longer ones follow, each cut into chunk tasks.
    void emit_csr(Staged& S) {
        const int thr = gather_long_threshold();
        // Pass 1, per gather slice: its rows' entry counts (block entries,
        // short remainder, long remainder) and its totals of short and long
        // rows and entries.  Pass 2 fills every slice's share of the output
        // at offsets from the prefix sums, each row's entries in the order
        // block entries, short remainder, long remainder.
        std::vector<size_t> gs;  // gather slices
        for (size_t i = 0; i < slices_.size(); ++i)
            if (slices_[i].csr) gs.push_back(i);
        const size_t ng = gs.size();
        std::vector<int32_t> rcnt(ng * TILE_ROWS, 0);
        std::vector<int64_t> n_sr(ng + 1, 0), n_se(ng + 1, 0), n_lr(ng + 1, 0), n_le(ng + 1, 0);
        par_ranges(ng, [&](size_t b0, size_t b1) {
            for (size_t k = b0; k < b1; ++k) {
                const Slice& sl = slices_[gs[k]];
                int32_t* cnt = &rcnt[k * TILE_ROWS];
                for (size_t c = sl.c0; c < sl.c1; ++c)
                    for (size_t e = chunks_[c].e0; e < chunks_[c].e1; ++e) ++cnt[pool_[e].lr];
                for (int lr = 0; lr < sl.nr; ++lr) {  // short and long remainder rows alike
                    const int row = in_.row_ids[sl.row_off + lr];
                    cnt[lr] += in_.rem_indptr[row + 1] - in_.rem_indptr[row];
                }
                for (int lr = 0; lr < sl.nr; ++lr) {
                    if (cnt[lr] > thr) {
                        ++n_lr[k + 1];
                        n_le[k + 1] += cnt[lr];
                    } else {
                        ++n_sr[k + 1];
                        n_se[k + 1] += cnt[lr];
                    }
                }
            }
        });
        for (size_t k = 0; k < ng; ++k) {
            n_sr[k + 1] += n_sr[k];
            n_se[k + 1] += n_se[k];
            n_lr[k + 1] += n_lr[k];
            n_le[k + 1] += n_le[k];
        }
        if (n_se[ng] + n_le[ng] > (int64_t)INT32_MAX) throw std::invalid_argument("too many gather-pass entries");
        S.crow_id.assign((size_t)n_sr[ng], 0);
        S.crow_ptr.assign((size_t)n_sr[ng] + 1, 0);
        S.ccol.assign((size_t)n_se[ng], 0);
        std::vector<T> short_val((size_t)n_se[ng]);
        std::vector<int32_t> long_id((size_t)n_lr[ng]), long_ptr((size_t)n_lr[ng] + 1, 0),
            long_col((size_t)n_le[ng]);
        std::vector<T> long_val((size_t)n_le[ng]);
        par_ranges(ng, [&](size_t b0, size_t b1) {
            std::vector<int32_t> at(TILE_ROWS);
            for (size_t k = b0; k < b1; ++k) {
                const Slice& sl = slices_[gs[k]];
                const int32_t* cnt = &rcnt[k * TILE_ROWS];
                // each row's first output position (short or long arrays)
                int64_t sr = n_sr[k], se = n_se[k], lrw = n_lr[k], le = n_le[k];
                for (int lr = 0; lr < sl.nr; ++lr) {
                    const int32_t row = in_.row_ids[sl.row_off + lr];
                    if (cnt[lr] > thr) {
                        at[lr] = (int32_t)le;
                        long_id[(size_t)lrw] = row;
                        le += cnt[lr];
                        long_ptr[(size_t)++lrw] = (int32_t)le;
                    } else {
                        at[lr] = (int32_t)se;
                        S.crow_id[(size_t)sr] = row;
                        se += cnt[lr];
                        S.crow_ptr[(size_t)++sr] = (int32_t)se;
                    }
                }
                auto put = [&](int lr, int32_t col, T x) {
                    const size_t q = (size_t)at[lr]++;
                    if (cnt[lr] > thr) {
                        long_col[q] = col;
                        long_val[q] = x;
                    } else {
                        S.ccol[q] = col;
                        short_val[q] = x;
                    }
                };
                for (size_t c = sl.c0; c < sl.c1; ++c)
                    for (size_t e = chunks_[c].e0; e < chunks_[c].e1; ++e)
                        put(pool_[e].lr, ent_col_of(e, &chunks_[c]), in_.nz_val[pool_[e].src]);
                for_short_rem(sl, [&](int lr, int j) { put(lr, in_.rem_col_ind[j], in_.rem_vals[j]); });
                for (size_t i = sl.g0; i < sl.g1; ++i) {
                    const int row = longs_[i].row;
                    for (int j = in_.rem_indptr[row]; j < in_.rem_indptr[row + 1]; ++j)
                        put(longs_[i].lr, in_.rem_col_ind[j], in_.rem_vals[j]);
                }
            }
        });
        S.cval.resize(short_val.size() * sizeof(T));
        if (!short_val.empty()) std::memcpy(S.cval.data(), short_val.data(), S.cval.size());
        std::vector<T>().swap(short_val);
        reorder_short_rows(S);
        S.n_crow_long = (int32_t)long_id.size();
        std::vector<int32_t> n_hot;  // per long row: entries in hot columns (empty: no split)
        hot_first(long_ptr, long_col, long_val, n_hot);
        S.gtask_ptr.assign(1, 0);
        S.gtask_order.clear();
        std::vector<int32_t> cold_tasks;
        const int32_t base = (int32_t)S.ccol.size();
        auto cut = [&](int32_t e0, int32_t e1, std::vector<int32_t>* order) {
            for (int32_t e = e0; e < e1; e += GATHER_CHUNK) {
                if (order) order->push_back((int32_t)(S.gtask.size() / 2));
                S.gtask.push_back(base + e);
                S.gtask.push_back(base + std::min(e1, e + GATHER_CHUNK));
            }
        };
        for (size_t i = 0; i < long_id.size(); ++i) {
            S.crow_id.push_back(long_id[i]);
            if (n_hot.empty()) {
                cut(long_ptr[i], long_ptr[i + 1], nullptr);
            } else {
                const int32_t ph = long_ptr[i] + n_hot[i];
                cut(long_ptr[i], ph, &S.gtask_order);
                cut(ph, long_ptr[i + 1], &cold_tasks);
            }
            S.gtask_ptr.push_back((int32_t)(S.gtask.size() / 2));
            S.crow_ptr.push_back(base + long_ptr[i + 1]);
        }
        S.gtask_order.insert(S.gtask_order.end(), cold_tasks.begin(), cold_tasks.end());
        S.ccol.insert(S.ccol.end(), long_col.begin(), long_col.end());
        const size_t v0 = S.cval.size();
        S.cval.resize(v0 + long_val.size() * sizeof(T));
        if (!long_val.empty()) std::memcpy(S.cval.data() + v0, long_val.data(), long_val.size() * sizeof(T));
    }

    // The hot-column split of the long gather rows (see GATHER_HOT_COLS): if
    // the matrix qualifies, each row's entries in the hot columns are moved
    // to its front (both parts keep their order) and n_hot gets each row's
    // count of them; otherwise n_hot is left empty.
    void hot_first(const std::vector<int32_t>& ptr, std::vector<int32_t>& col, std::vector<T>& val,
                   std::vector<int32_t>& n_hot) const {
        n_hot.clear();
        const size_t nrow = ptr.empty() ? 0 : ptr.size() - 1;
        const int32_t cols = in_.cols;
        if (nrow == 0 || col.empty() || cols <= GATHER_HOT_COLS) return;
        std::vector<int32_t> cnt((size_t)cols, 0);
        for (int32_t c : col) ++cnt[(size_t)c];
        // the GATHER_HOT_COLS most used columns (ties: lower column first)
        std::vector<int32_t> ids((size_t)cols);
        for (int32_t c = 0; c < cols; ++c) ids[(size_t)c] = c;
        auto more_used = [&](int32_t a, int32_t b) {
            const int32_t ca = cnt[(size_t)a], cb = cnt[(size_t)b];
            return ca != cb ? ca > cb : a < b;
        };
        std::nth_element(ids.begin(), ids.begin() + (GATHER_HOT_COLS - 1), ids.end(), more_used);
        std::vector<uint8_t> hot((size_t)cols, 0);
        long long n_in = 0;
        for (int k = 0; k < GATHER_HOT_COLS; ++k) {
            hot[(size_t)ids[(size_t)k]] = 1;
            n_in += cnt[(size_t)ids[(size_t)k]];
        }
        const double share = (double)n_in / (double)col.size();
        if (share < GATHER_HOT_SHARE || share < GATHER_HOT_SKEW * GATHER_HOT_COLS / (double)cols) return;
        n_hot.assign(nrow, 0);
        par_ranges(nrow, [&](size_t r0, size_t r1) {
            std::vector<int32_t> tc;
            std::vector<T> tv;
            for (size_t i = r0; i < r1; ++i) {
                const size_t p0 = (size_t)ptr[i], p1 = (size_t)ptr[i + 1];
                tc.clear();
                tv.clear();
                size_t q = p0;
                for (size_t p = p0; p < p1; ++p) {
                    if (hot[(size_t)col[p]]) {
                        col[q] = col[p];
                        val[q] = val[p];
                        ++q;
                    } else {
                        tc.push_back(col[p]);
                        tv.push_back(val[p]);
                    }
                }
                n_hot[i] = (int32_t)(q - p0);
                std::copy(tc.begin(), tc.end(), col.begin() + (std::ptrdiff_t)q);
                std::copy(tv.begin(), tv.end(), val.begin() + (std::ptrdiff_t)q);
            }
        });
    }

    // Entries among the first GATHER_REUSE_SAMPLE entries of the short gather
    // rows, taken in `order`, whose column was named by a row at most
    // GATHER_REUSE_WINDOW positions before (an X row another row nearby also
    // reads), per entry.  A prefix is enough to tell the two orders apart and
    // keeps the estimate's cost bounded on large matrices.
    double window_reuse(const Staged& S, const std::vector<int32_t>& order, std::vector<int32_t>& last) const {
        std::fill(last.begin(), last.end(), -1);
        long long hits = 0, seen = 0;
        for (int32_t p = 0; p < (int32_t)order.size() && seen < GATHER_REUSE_SAMPLE; ++p) {
            const int32_t i = order[p];
            for (int32_t e = S.crow_ptr[i]; e < S.crow_ptr[i + 1]; ++e) {
                const int32_t c = S.ccol[e];
                if (last[c] >= 0 && p - last[c] <= GATHER_REUSE_WINDOW) ++hits;
                last[c] = p;
            }
            seen += S.crow_ptr[i + 1] - S.crow_ptr[i];
        }
        return seen ? (double)hits / (double)seen : 0.0;
    }

    // Reorder the short gather rows (S.crow_id/crow_ptr/ccol/cval so far) by
    // Cuthill-McKee when that repeats X rows within the window more often.
    // Row i's neighbours are the short rows whose row id is one of its column
    // ids (the matrix read as a graph; any order is correct, this one is
    // local when the matrix is a graph with locality under some labelling).
    // Breadth first from the unvisited row of least length (ties: slice
    // order), each row's neighbours in the order of its entries.
    void reorder_short_rows(Staged& S) {
        const int32_t n = (int32_t)S.crow_id.size();
        if (n < 2 || in_.rows != in_.cols) return;
        std::vector<int32_t> pos_of_row((size_t)in_.rows, -1);
        for (int32_t i = 0; i < n; ++i) pos_of_row[S.crow_id[i]] = i;
        // start nodes: rows by ascending length, stable (a counting sort)
        int32_t max_deg = 0;
        for (int32_t i = 0; i < n; ++i) max_deg = std::max(max_deg, S.crow_ptr[i + 1] - S.crow_ptr[i]);
        std::vector<int32_t> first((size_t)max_deg + 2, 0), starts((size_t)n);
        for (int32_t i = 0; i < n; ++i) ++first[(size_t)(S.crow_ptr[i + 1] - S.crow_ptr[i]) + 1];
        for (int32_t d = 0; d <= max_deg; ++d) first[(size_t)d + 1] += first[(size_t)d];
        for (int32_t i = 0; i < n; ++i) starts[(size_t)first[(size_t)(S.crow_ptr[i + 1] - S.crow_ptr[i])]++] = i;
        // pos_of_row doubles as the visited mark: a row is set to -1 when it
        // joins the order (one random access per entry, not two)
        std::vector<int32_t> order;
        order.reserve(n);
        for (int32_t st : starts) {
            int32_t& ps = pos_of_row[S.crow_id[st]];
            if (ps < 0) continue;
            ps = -1;
            size_t head = order.size();
            order.push_back(st);
            while (head < order.size()) {
                const int32_t i = order[head++];
                for (int32_t e = S.crow_ptr[i]; e < S.crow_ptr[i + 1]; ++e) {
                    int32_t& pj = pos_of_row[S.ccol[e]];
                    if (pj >= 0) {
                        order.push_back(pj);
                        pj = -1;
                    }
                }
            }
        }
        std::vector<int32_t>().swap(pos_of_row);
        std::vector<int32_t> ident(n);
        for (int32_t i = 0; i < n; ++i) ident[i] = i;
        double h0 = 0.0, h1 = 0.0;
        {
            std::vector<int32_t> last0((size_t)in_.cols), last1((size_t)in_.cols);
            std::thread th([&]() { h1 = window_reuse(S, order, last1); });
            h0 = window_reuse(S, ident, last0);
            th.join();
        }
        if (h1 < GATHER_REORDER_GAIN * h0 || h1 == h0) return;
        std::vector<int32_t> rid((size_t)n), rptr((size_t)n + 1), col(S.ccol.size());
        std::vector<char> val(S.cval.size());
        rptr[0] = 0;
        for (int32_t p = 0; p < n; ++p) {
            const int32_t i = order[(size_t)p];
            rid[(size_t)p] = S.crow_id[(size_t)i];
            rptr[(size_t)p + 1] = rptr[(size_t)p] + (S.crow_ptr[(size_t)i + 1] - S.crow_ptr[(size_t)i]);
        }
        par_ranges((size_t)n, [&](size_t p0, size_t p1) {
            for (size_t p = p0; p < p1; ++p) {
                const int32_t i = order[p];
                const int32_t len = S.crow_ptr[(size_t)i + 1] - S.crow_ptr[(size_t)i];
                std::memcpy(col.data() + rptr[p], S.ccol.data() + S.crow_ptr[(size_t)i], (size_t)len * 4);
                std::memcpy(val.data() + (size_t)rptr[p] * sizeof(T),
                            S.cval.data() + (size_t)S.crow_ptr[(size_t)i] * sizeof(T), (size_t)len * sizeof(T));
            }
        });
        S.crow_id.swap(rid);
        S.crow_ptr.swap(rptr);
        S.ccol.swap(col);
        S.cval.swap(val);
    }

    // Slices that share column chunks go into one group (up to G): a group
    // loads each chunk's X tile once for all its members.  Greedy: take the
    // first free slice, then repeatedly the free slice with the most chunks in
    // common with the group so far (ties: lowest index).  A slice heavier than
    // max_item_nnz stays alone (it is cut into several items).
    void make_groups() {
        const int ns = (int)slices_.size();
        std::vector<std::pair<int, int>> kv;  // (chunk key, slice)
        kv.reserve(chunks_.size());
        for (int i = 0; i < ns; ++i)
            for (size_t c = slices_[i].c0; c < slices_[i].c1; ++c) kv.emplace_back(chunks_[c].cid_off, i);
        std::sort(kv.begin(), kv.end());
        auto heavy = [&](int i) { return slices_[i].nnz > max_item_nnz_; };
        std::vector<char> used(ns, 0);
        for (int i = 0; i < ns; ++i) used[i] = slices_[i].csr;
        // score: group keys a candidate shares; pair: its shared keys summed
        // over the members (ties on score go to the candidate closest to all
        // members, which keeps groups compact: a 2x2 block of stencil slices
        // touches fewer column groups than a line of four)
        std::vector<int> score(ns, 0), pair(ns, 0), touched;
        std::vector<int> keys;
        int fill = 0;
        for (int i = 0; i < ns; ++i) {
            if (used[i]) continue;
            Group g{};
            g.slot = -1;
            g.members[0] = i;
            g.n_members = 1;
            used[i] = 1;
            if (G_ > 1 && !heavy(i)) {
                keys.clear();
                touched.clear();
                auto add_keys = [&](int s) {
                    for (size_t c = slices_[s].c0; c < slices_[s].c1; ++c) {
                        const int k = chunks_[c].cid_off;
                        const bool fresh = std::find(keys.begin(), keys.end(), k) == keys.end();
                        if (fresh) keys.push_back(k);
                        // candidates: the next few slices (in order) that share the key
                        auto it = std::lower_bound(kv.begin(), kv.end(), std::make_pair(k, i));
                        for (int n = 0; it != kv.end() && it->first == k && n < 64; ++it, ++n) {
                            const int o = it->second;
                            if (used[o] || heavy(o)) continue;
                            if (score[o] == 0 && pair[o] == 0) touched.push_back(o);
                            score[o] += fresh;
                            ++pair[o];
                        }
                    }
                };
                add_keys(i);
                while (g.n_members < G_) {
                    int best = -1;
                    for (int o : touched)
                        if (!used[o] && score[o] > 0 &&
                            (best < 0 || score[o] > score[best] ||
                             (score[o] == score[best] && (pair[o] > pair[best] ||
                                                          (pair[o] == pair[best] && o < best)))))
                            best = o;
                    if (best < 0) {
                        // nothing shares a chunk: fill with the next free slice,
                        // so the number of groups stays near slices / G
                        while (fill < ns && (used[fill] || heavy(fill))) ++fill;
                        if (fill >= ns) break;
                        best = fill;
                    }
                    used[best] = 1;
                    g.members[g.n_members++] = best;
                    add_keys(best);
                }
                for (int o : touched) score[o] = pair[o] = 0;
            }
            groups_.push_back(g);
        }
    }

    // Cut a member's entries [e0, e1) of tent_ (row-major) between rows into
    // pieces of at most TILE_ENT entries; a row longer than that on its own
    // (duplicate entries) is cut inside, its parts in consecutive pieces of the
    // same item, so it keeps accumulating in the same registers.
    static void cut(const std::vector<Ent>& v, size_t e0, size_t e1, std::vector<Piece>& out) {
        size_t i = e0;
        do {
            const size_t start = i;
            while (i < e1) {
                size_t j = i;
                while (j < e1 && v[j].lr == v[i].lr) ++j;
                if (j - start > (size_t)TILE_ENT) {
                    if (i == start) i = start + TILE_ENT;
                    break;
                }
                i = j;
            }
            out.push_back(Piece{start, i});
        } while (i < e1);
    }

    // Append steps for one X tile shared by the members: member m's entries
    // are tent_[range[m]]; pieces too large are cut into extra steps.
    void add_steps(int cid_off, int nc, const std::vector<std::pair<size_t, size_t>>& range) {
        std::vector<std::vector<Piece>> pcs(G_);
        size_t n = 1;
        for (int m = 0; m < G_; ++m) {
            if (range[m].second > range[m].first) cut(tent_, range[m].first, range[m].second, pcs[m]);
            n = std::max(n, pcs[m].size());
        }
        for (size_t k = 0; k < n; ++k) {
            steps_.push_back(Step{cid_off, nc, pieces_.size()});
            for (int m = 0; m < G_; ++m)
                pieces_.push_back(k < pcs[m].size() ? pcs[m][k] : Piece{0, 0});
        }
    }

    void build_group_steps(Staged& S, size_t gi) {
        Group& g = groups_[gi];
        g.s0 = steps_.size();
        // block chunks, by key
        std::vector<std::pair<int, std::pair<int, size_t>>> keyed;  // (key, (member, chunk))
        for (int m = 0; m < g.n_members; ++m) {
            const Slice& sl = slices_[g.members[m]];
            for (size_t c = sl.c0; c < sl.c1; ++c) keyed.push_back({chunks_[c].cid_off, {m, c}});
        }
        std::sort(keyed.begin(), keyed.end());
        std::vector<std::pair<size_t, size_t>> range(G_);
        for (size_t i = 0; i < keyed.size();) {
            size_t j = i;
            for (auto& r : range) r = {0, 0};
            const Chunk& c0 = chunks_[keyed[i].second.second];
            while (j < keyed.size() && keyed[j].first == keyed[i].first) {
                const Chunk& c = chunks_[keyed[j].second.second];
                const size_t t0 = tent_.size();
                tent_.insert(tent_.end(), pool_.begin() + c.e0, pool_.begin() + c.e1);
                range[keyed[j].second.first] = {t0, tent_.size()};
                ++j;
            }
            add_steps(c0.cid_off, c0.nc, range);
            i = j;
        }
        const size_t b_end = steps_.size();
        // short remainder rows: tiles over the members' distinct columns
        std::vector<int32_t> ucols;
        for (int m = 0; m < g.n_members; ++m) {
            const Slice& sl = slices_[g.members[m]];
            for (size_t e = sl.r0; e < sl.r1; ++e) ucols.push_back(rcol_[e]);
        }
        if (!ucols.empty()) {
            std::sort(ucols.begin(), ucols.end());
            ucols.erase(std::unique(ucols.begin(), ucols.end()), ucols.end());
            for (size_t k0 = 0; k0 < ucols.size(); k0 += TILE_COLS) {
                const size_t k1 = std::min(ucols.size(), k0 + TILE_COLS);
                for (auto& r : range) r = {0, 0};
                for (int m = 0; m < g.n_members; ++m) {
                    const Slice& sl = slices_[g.members[m]];
                    const size_t t0 = tent_.size();
                    for (size_t e = sl.r0; e < sl.r1; ++e) {
                        const int col = rcol_[e];
                        if (col < ucols[k0] || col > ucols[k1 - 1]) continue;
                        Ent x = pool_[e];
                        x.lc = (uint8_t)(std::lower_bound(ucols.begin() + k0, ucols.begin() + k1, col) -
                                         (ucols.begin() + k0));
                        tent_.push_back(x);
                    }
                    range[m] = {t0, tent_.size()};
                }
                const int cid_off = (int)S.tcols.size();
                S.tcols.insert(S.tcols.end(), ucols.begin() + k0, ucols.begin() + k1);
                add_steps(cid_off, (int)(k1 - k0), range);
            }
        }
        if (steps_.size() == g.s0) {
            for (auto& r : range) r = {0, 0};
            add_steps(0, 0, range);
        }
        g.early = steps_.size() - g.s0 >= EARLY_STORE_MIN_STEPS;
        if (g.early && b_end > g.s0)  // the remainder tiles first
            std::rotate(steps_.begin() + (std::ptrdiff_t)g.s0, steps_.begin() + (std::ptrdiff_t)b_end, steps_.end());
        g.s1 = steps_.size();
        // A step costs about the same whatever its entries (the X tile is
        // loaded and the workgroup synchronises either way), and entries add
        // a little on top.
        long long nnz = 0;
        for (int m = 0; m < g.n_members; ++m) nnz += slices_[g.members[m]].nnz;
        g.cost = COST_ITEM + (long long)(g.s1 - g.s0) * COST_STEP + nnz / std::max(g.n_members, 1);
    }

    // Emit one member's tile of a step.
    void emit_tile(Staged& S, const Piece& pc, int cid_off, int nc, int row_off, int nr, uint32_t flags,
                   int slot) {
        const int nnz = (int)(pc.e1 - pc.e0);
        const int ent_off = (int)S.ent_col.size();
        uint8_t rs[TILE_RS];  // row starts fit a byte: TILE_ENT < 256
        int k = 0;
        for (int r = 0; r <= TILE_ROWS; ++r) {
            while (k < nnz && tent_[pc.e0 + k].lr < r) ++k;
            rs[r] = (uint8_t)k;
        }
        for (size_t u = pc.e0; u < pc.e1; ++u) {
            const Ent& x = tent_[u];
            S.ent_col.push_back(x.lc);
            const T v = x.from_rem ? in_.rem_vals[x.src] : in_.nz_val[x.src];
            const char* p = reinterpret_cast<const char*>(&v);
            S.ent_val.insert(S.ent_val.end(), p, p + sizeof(T));
        }
        // Rows in parallel cost one step per entry of the longest row; one
        // busy row at a time costs about a tenth of a step per entry plus a
        // step per busy row to hand its sums over.
        int busy = 0, longest = 0;
        for (int r = 0; r < TILE_ROWS; ++r) {
            const int len = rs[r + 1] - rs[r];
            busy += len > 0;
            longest = std::max(longest, len);
        }
        if (busy <= SERIAL_MAX_BUSY && 10 * longest > nnz + 10 * busy) flags |= FLAG_SERIAL;
        const int32_t w[TILE_WORDS] = {ent_off, (int32_t)(nnz | (nc << 8) | (nr << 16) | (flags << 24)),
                                       cid_off, row_off, slot, 0, 0, 0};
        S.tiles.insert(S.tiles.end(), w, w + TILE_WORDS);
        // entries of every tile start at an even index, so the kernel can load
        // them two at a time
        if (nnz & 1) {
            S.ent_col.push_back(0);
            S.ent_val.insert(S.ent_val.end(), sizeof(T), 0);
        }
        S.tile_rs.insert(S.tile_rs.end(), rs, rs + TILE_RS);
    }

    // A slice heavier than max_item_nnz (alone in its group) becomes several
    // items, each a group of its own so that different workgroups run them:
    // a run of its steps with at most max_item_nnz entries (or one step).
    // The first item stores Y, the others write partial slots that the fixup
    // pass adds in slot order.
    void split_heavy(Staged& S) {
        std::vector<Group> out;
        out.reserve(groups_.size());
        for (const Group& g : groups_) {
            const Slice& sl = slices_[g.members[0]];
            if (g.n_members != 1 || sl.nnz <= max_item_nnz_) {
                out.push_back(g);
                continue;
            }
            const int slot_begin = S.n_slots;
            size_t a = g.s0;
            long long nnz = 0;
            for (size_t st = g.s0; st < g.s1; ++st) {
                const Piece& pc = pieces_[steps_[st].m0];
                nnz += (long long)(pc.e1 - pc.e0);
                bool end = st + 1 == g.s1;
                if (!end) {
                    const Piece& nx = pieces_[steps_[st + 1].m0];
                    end = nnz + (long long)(nx.e1 - nx.e0) > max_item_nnz_;
                }
                if (!end) continue;
                Group it = g;
                it.s0 = a;
                it.s1 = st + 1;
                it.slot = a == g.s0 ? -1 : S.n_slots++;
                it.cost = COST_ITEM + (long long)(it.s1 - it.s0) * COST_STEP + nnz;
                out.push_back(it);
                a = st + 1;
                nnz = 0;
            }
            if (S.n_slots > slot_begin) {
                const int32_t sp4[4] = {sl.row_off, sl.nr, slot_begin, S.n_slots};
                S.splits.insert(S.splits.end(), sp4, sp4 + 4);
            }
        }
        groups_.swap(out);
    }

    // Deal groups to workgroups of G waves, then lay out each wave's stream:
    // for each of its workgroup's groups, its member's tile of every step.
    void deal_and_emit(Staged& S) {
        const int ng = (int)groups_.size();
        int nwg = std::max(1, std::min(std::max(want_waves_ / G_, 1), ng));
        if (ng == 0) {
            S.wave_tiles.assign(1, 0);
            S.n_waves = 0;
            finish(S);
            return;
        }
        // Contiguous ranges (neighbouring groups share X rows in L2) that
        // minimise the largest range cost: binary search on that bound, each
        // range filled greedily.
        long long lo = 0, hi = 0;
        for (const Group& g : groups_) {
            lo = std::max(lo, g.cost);
            hi += g.cost;
        }
        auto ranges_for = [&](long long bound, std::vector<int>* first) {
            int n = 0;
            long long acc = 0;
            for (int gi = 0; gi < ng; ++gi) {
                if (gi == 0 || acc + groups_[gi].cost > bound) {
                    ++n;
                    acc = 0;
                    if (first) first->push_back(gi);
                }
                acc += groups_[gi].cost;
            }
            return n;
        };
        while (lo < hi) {
            const long long mid = lo + (hi - lo) / 2;
            if (ranges_for(mid, nullptr) <= nwg) hi = mid;
            else lo = mid + 1;
        }
        std::vector<int> wg_first;
        ranges_for(lo, &wg_first);
        nwg = (int)wg_first.size();
        wg_first.push_back(ng);
        S.n_waves = nwg * G_;
        S.wave_tiles.assign(1, 0);
        // The launch gives XCD x the logical workgroups [x*per, (x+1)*per);
        // their ranges together are the XCD's contiguous share.  Inside it the
        // groups are dealt in order, each to the workgroup with the least cost
        // so far (the lowest index on ties: round-robin when the groups cost
        // the same), so the workgroups running at any one time hold
        // neighbouring groups, whose shared X rows then come from the XCD's L2
        // instead of being fetched again later, and uneven groups still leave
        // the workgroups' streams within about one group of each other.
        std::vector<std::vector<int>> wg_groups(nwg);
        std::vector<long long> load(nwg, 0);
        const int per = (nwg + 7) / 8;
        std::vector<int> order;
        for (int w0 = 0; w0 < nwg; w0 += per) {
            const int w1 = std::min(nwg, w0 + per);
            order.clear();
            for (int gi = wg_first[w0]; gi < wg_first[w1]; ++gi) order.push_back(gi);
            std::stable_sort(order.begin(), order.end(),
                             [&](int x, int y) { return groups_[x].cost > groups_[y].cost; });
            for (int gi : order) {
                int best = w0;
                for (int w = w0 + 1; w < w1; ++w)
                    if (load[w] < load[best]) best = w;
                wg_groups[best].push_back(gi);
                load[best] += groups_[gi].cost;
            }
        }
        for (int w = 0; w < nwg; ++w) {
            for (int m = 0; m < G_; ++m) {
                for (int gi : wg_groups[w]) {
                    const Group& g = groups_[gi];
                    const bool real = m < g.n_members;
                    const Slice* sl = real ? &slices_[g.members[m]] : nullptr;
                    const int row_off = real ? sl->row_off : 0, nr = real ? sl->nr : 0;
                    // the step at which this member stores (see EARLY_STORE_MIN_STEPS)
                    size_t store_at = g.s1 - 1;
                    if (g.early && real) {
                        for (size_t st = g.s1; st-- > g.s0;) {
                            const Piece& pc = pieces_[steps_[st].m0 + m];
                            if (pc.e1 > pc.e0) {
                                store_at = st;
                                break;
                            }
                        }
                    }
                    for (size_t st = g.s0; st < g.s1; ++st) {
                        const Step& sp = steps_[st];
                        const Piece& pc = pieces_[sp.m0 + m];
                        const uint32_t flags = st == store_at ? FLAG_LAST : 0u;
                        emit_tile(S, real ? pc : Piece{0, 0}, sp.cid_off, sp.nc, row_off, nr, flags, real ? g.slot : -1);
                    }
                }
                S.wave_tiles.push_back((int32_t)S.n_tiles());
            }
        }
        finish(S);
    }

    // The blob stream, derived from the tile arrays just emitted (see the
    // record layout above).  Only float matrices grouped by 4 get one; the
    // kernels that read it need both.
    void emit_blobs(Staged& S) {
        S.blobs.clear();
        S.blob_first.clear();
        S.blob_xid.clear();
        if (!std::is_same<T, float>::value || G_ != 4 || S.n_waves <= 0) return;
        S.blob_first.assign((size_t)S.n_waves * 8, 0u);
        S.blob_xid.assign(S.n_tiles() * 8, 0u);
        std::vector<uint32_t> offs, nvec;
        std::vector<uint8_t> rec;
        for (int w = 0; w < S.n_waves; ++w) {
            const int m = w % 4;
            const int t0 = S.wave_tiles[w], t1 = S.wave_tiles[w + 1];
            offs.clear();
            nvec.clear();
            for (int t = t0; t < t1; ++t) {
                const int32_t* tw = &S.tiles[(size_t)t * TILE_WORDS];
                const int ent_off = tw[0];
                const uint32_t w1 = (uint32_t)tw[1];
                const int nnz = (int)(w1 & 0xffu), nc = (int)((w1 >> 8) & 0xffu), nr = (int)((w1 >> 16) & 0xffu);
                const uint32_t tflags = w1 >> 24;
                const int cid_off = tw[2], row_off = tw[3], slot = tw[4];
                // the X rows this wave stages at this step
                for (int j = 0; j < 8; ++j) {
                    const int c = std::min(2 * m + (j >> 2) + 8 * (j & 3), nc - 1);
                    S.blob_xid[(size_t)t * 8 + j] = nc > 0 ? (uint32_t)S.tcols[(size_t)cid_off + c] : 0u;
                }
                uint32_t flags = 0;
                if (tflags & FLAG_LAST) flags |= BLOB_LAST;
                if (tflags & FLAG_SERIAL) flags |= BLOB_SERIAL;
                bool rcontig = nr > 0;
                for (int r = 1; r < nr && rcontig; ++r) rcontig = in_.row_ids[row_off + r] == in_.row_ids[row_off] + r;
                if (rcontig) flags |= BLOB_ROWCONTIG;
                rec.clear();
                auto put32 = [&](uint32_t v) {
                    for (int k = 0; k < 4; ++k) rec.push_back((uint8_t)(v >> (8 * k)));
                };
                put32((uint32_t)nnz | (uint32_t)nr << 8 | (uint32_t)std::min(nc, 63) << 14 | flags << 20);
                put32((uint32_t)slot);
                put32(0u);            // patched below
                put32(rcontig ? (uint32_t)in_.row_ids[row_off] : (uint32_t)row_off);
                if (nnz > 0)
                    for (int r = 0; r < TILE_ROWS; ++r) {
                        rec.push_back(S.tile_rs[(size_t)t * TILE_RS + r]);
                    }
                for (int e = 0; e < nnz; ++e) rec.push_back(S.ent_col[(size_t)ent_off + e]);
                while (rec.size() & 3) rec.push_back(0);
                const size_t vbytes = (size_t)nnz * sizeof(T);
                const char* vp = S.ent_val.data() + (size_t)ent_off * sizeof(T);
                rec.insert(rec.end(), vp, vp + vbytes);
                while (rec.size() & 15) rec.push_back(0);
                if ((int)rec.size() > BLOB_MAX_BYTES) throw std::invalid_argument("record too large");
                offs.push_back((uint32_t)(S.blobs.size() / 4));
                nvec.push_back((uint32_t)(rec.size() / 16));
                const size_t at = S.blobs.size();
                S.blobs.resize(at + rec.size() / 4);
                std::memcpy(&S.blobs[at], rec.data(), rec.size());
            }
            const int n = t1 - t0;
            for (int k = 0; k < n; ++k) {
                const int nx = std::min(k + BLOB_LOOKAHEAD, n - 1);
                uint32_t* hw = &S.blobs[(size_t)offs[k] * 4];
                hw[0] |= nvec[nx] << 24;
                hw[2] = offs[nx];
            }
            uint32_t* f = &S.blob_first[(size_t)w * 8];
            if (n > 0) {
                uint32_t packed = 0;
                for (int k = 0; k < BLOB_LOOKAHEAD; ++k) {
                    const int kk = std::min(k, n - 1);
                    f[k] = offs[kk];
                    packed |= nvec[kk] << (8 * k);
                }
                f[4] = packed;
            }
            f[5] = (uint32_t)n;
            f[6] = (uint32_t)t0;
        }
        // DMA offsets are 32-bit byte offsets: records and X ids under 4 GiB
        if (S.blobs.size() / 4 + 64 >= (size_t)1 << 28 || S.n_tiles() + 64 >= (size_t)1 << 27) {
            S.blobs.clear();
            S.blob_first.clear();
            S.blob_xid.clear();
        }
    }

    void finish(Staged& S) {
        // Two spare entries past the end: an empty tile's loads are clamped onto them.
        S.ent_col.insert(S.ent_col.end(), 2, 0);
        S.ent_val.insert(S.ent_val.end(), 2 * sizeof(T), 0);
    }

    In in_;
    int max_item_nnz_, long_threshold_, want_waves_, G_;
    float min_reuse_;
    std::vector<Ent> pool_, tent_;
    std::vector<int32_t> rcol_, colx_;
    std::vector<Chunk> chunks_;
    std::vector<LongRow> longs_;
    std::vector<Slice> slices_;
    std::vector<Group> groups_;
    std::vector<Step> steps_;
    std::vector<Piece> pieces_;
};

}  // namespace spmm_stage
