// Host-side format builders, decoders and CPU SpMM for BOO and PBR.
//
// These produce the reference's encodings bit for bit (the GPU consumes them
// unchanged), so each function states the reference routine whose output it
// must equal.  The algorithms are written for this library: BOO counts blocks
// per row group with a dense counter instead of a global hash map, and finds a
// nonzero's block by binary search over its row group's sorted column groups.
// PBR keeps libstdc++'s std::unordered_map for the per-stripe block set,
// because its iteration order IS the reference's block order.
#pragma once

#include <algorithm>
#include <bitset>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace spmm {

enum BooPolicy { BOO_KEEP = 0, BOO_MERGE = 1, BOO_REMAINDER = 2, BOO_TAIL_BATCH = 3 };
enum BooOrder { BOO_ROWMAJOR = 0, BOO_COLMAJOR = 1 };

template <typename I, typename S>
struct BooArrays {
    I rows = 0, cols = 0, total_nnz = 0;
    std::vector<I> row_grp_ptr, row_ids, col_grp_ptr, col_ids;
    std::vector<I> blk_row_grp, blk_col_grp, blk_nz_ptr;
    std::vector<uint8_t> blk_shift;
    std::vector<uint16_t> nz_idx;
    std::vector<S> nz_val;
    std::vector<I> rem_indptr, rem_col_ind;
    std::vector<S> rem_vals;
    std::vector<I> tail_row, tail_col;
    std::vector<S> tail_val;
    I max_nr = 0, max_nc = 0, max_nnz_blk = 0;
    int nz_order = BOO_ROWMAJOR;
};

// Bits for the column part of nz_idx: ceil(log2(n)), 0 for n <= 1
// (boo_matrix/boo_matrix.cpp:12-16).
inline uint8_t col_bits(uint32_t n) {
    uint8_t s = 0;
    while ((1u << s) < n) ++s;
    return s;
}

// Counting sort of labels into groups; ids ascend within a group and pos[i]
// is i's rank inside its group (boo_matrix/boo_matrix.cpp:23-48).
template <typename I>
void group_by_label(const int32_t* labels, I n, I n_groups, std::vector<I>& ptr,
                    std::vector<I>& ids, std::vector<I>& pos) {
    ptr.assign((size_t)n_groups + 1, 0);
    for (I i = 0; i < n; ++i) {
        const int32_t g = labels[i];
        if (g < 0 || (I)g >= n_groups)
            throw std::invalid_argument("csr_to_boo: cluster label out of range");
        ++ptr[(size_t)g + 1];
    }
    for (I g = 0; g < n_groups; ++g) ptr[(size_t)g + 1] += ptr[(size_t)g];
    ids.resize((size_t)n);
    pos.resize((size_t)n);
    std::vector<I> next(ptr.begin(), ptr.end() - 1);
    for (I i = 0; i < n; ++i) {
        const size_t g = (size_t)labels[i];
        const I slot = next[g]++;
        ids[(size_t)slot] = i;
        pos[(size_t)i] = slot - ptr[g];
    }
}

// csr_to_boo: output equal to boo_matrix/boo_matrix.cpp:53-274.
template <typename I, typename S>
BooArrays<I, S> build_boo(const I* indptr, const I* indices, const S* data, I rows, I cols,
                          const int32_t* row_labels, const int32_t* col_labels, int policy,
                          I threshold, int order) {
    if (policy == BOO_MERGE)
        throw std::invalid_argument(
            "csr_to_boo: 'merge' policy is a clustering-level column relabel, not a builder "
            "policy -- merge the column groups before building");
    if (policy != BOO_KEEP && policy != BOO_REMAINDER && policy != BOO_TAIL_BATCH)
        throw std::invalid_argument("csr_to_boo: unknown small_block_policy");
    if (order != BOO_ROWMAJOR && order != BOO_COLMAJOR)
        throw std::invalid_argument("csr_to_boo: unknown nz_order");

    BooArrays<I, S> A;
    A.rows = rows;
    A.cols = cols;
    A.total_nnz = rows > 0 ? indptr[rows] : 0;
    A.nz_order = order;

    I n_rg = 0, n_cg = 0;
    for (I r = 0; r < rows; ++r) n_rg = std::max<I>(n_rg, (I)row_labels[r] + 1);
    for (I c = 0; c < cols; ++c) n_cg = std::max<I>(n_cg, (I)col_labels[c] + 1);
    std::vector<I> row_pos, col_pos;
    group_by_label<I>(row_labels, rows, n_rg, A.row_grp_ptr, A.row_ids, row_pos);
    group_by_label<I>(col_labels, cols, n_cg, A.col_grp_ptr, A.col_ids, col_pos);

    // Pass 1: nonzeros per (row group, col group), row group by row group with
    // a dense counter, emitted in ascending (rg, cg) = the reference's key order.
    const bool spill = policy == BOO_REMAINDER || policy == BOO_TAIL_BATCH;
    std::vector<I> count((size_t)n_cg, 0);
    std::vector<I> touched;
    std::vector<I> rg_blk_begin((size_t)n_rg + 1, 0);
    A.blk_nz_ptr.push_back(0);
    I running = 0;
    for (I rg = 0; rg < n_rg; ++rg) {
        rg_blk_begin[(size_t)rg] = (I)A.blk_row_grp.size();
        touched.clear();
        for (I t = A.row_grp_ptr[(size_t)rg]; t < A.row_grp_ptr[(size_t)rg + 1]; ++t) {
            const I r = A.row_ids[(size_t)t];
            for (I j = indptr[r]; j < indptr[r + 1]; ++j) {
                const I cg = (I)col_labels[indices[j]];
                if (count[(size_t)cg]++ == 0) touched.push_back(cg);
            }
        }
        std::sort(touched.begin(), touched.end());
        const I n_r = A.row_grp_ptr[(size_t)rg + 1] - A.row_grp_ptr[(size_t)rg];
        for (const I cg : touched) {
            const I w = count[(size_t)cg];
            count[(size_t)cg] = 0;
            if (spill && w < threshold) continue;
            const I n_c = A.col_grp_ptr[(size_t)cg + 1] - A.col_grp_ptr[(size_t)cg];
            const uint8_t shift = col_bits((uint32_t)n_c);
            const uint64_t span = ((uint64_t)(n_r - 1) << shift) + (uint64_t)(n_c - 1);
            if (span > 0xFFFFull)
                throw std::invalid_argument(
                    "csr_to_boo: block local index space exceeds uint16 -- reduce max_nr/max_nc "
                    "in the clustering");
            A.blk_row_grp.push_back(rg);
            A.blk_col_grp.push_back(cg);
            A.blk_shift.push_back(shift);
            running += w;
            A.blk_nz_ptr.push_back(running);
            A.max_nr = std::max(A.max_nr, n_r);
            A.max_nc = std::max(A.max_nc, n_c);
            A.max_nnz_blk = std::max(A.max_nnz_blk, w);
        }
    }
    rg_blk_begin[(size_t)n_rg] = (I)A.blk_row_grp.size();

    // Pass 2: place nonzeros in global row order, CSR order within a row.
    const size_t nb = A.blk_row_grp.size();
    A.nz_idx.resize((size_t)running);
    A.nz_val.resize((size_t)running);
    std::vector<I> cursor(A.blk_nz_ptr.begin(), A.blk_nz_ptr.end() - 1);
    std::vector<std::vector<std::pair<I, S>>> bins;
    if (policy != BOO_TAIL_BATCH) bins.resize((size_t)rows);
    for (I r = 0; r < rows; ++r) {
        const I rg = (I)row_labels[r];
        const auto first = A.blk_col_grp.begin() + rg_blk_begin[(size_t)rg];
        const auto last = A.blk_col_grp.begin() + rg_blk_begin[(size_t)rg + 1];
        const uint32_t lrow = (uint32_t)row_pos[(size_t)r];
        for (I j = indptr[r]; j < indptr[r + 1]; ++j) {
            const I c = indices[j];
            const I cg = (I)col_labels[c];
            const auto hit = std::lower_bound(first, last, cg);
            if (hit == last || *hit != cg) {
                if (policy == BOO_TAIL_BATCH) {
                    A.tail_row.push_back(r);
                    A.tail_col.push_back(c);
                    A.tail_val.push_back(data[j]);
                } else {
                    bins[(size_t)r].emplace_back(c, data[j]);
                }
                continue;
            }
            const size_t b = (size_t)(hit - A.blk_col_grp.begin());
            const I slot = cursor[b]++;
            A.nz_idx[(size_t)slot] =
                (uint16_t)((lrow << A.blk_shift[b]) | (uint32_t)col_pos[(size_t)c]);
            A.nz_val[(size_t)slot] = data[j];
        }
    }

    // Order inside each block: by nz_idx (rowmajor) or (local col, local row)
    // (colmajor); equal keys keep placement order.
    std::vector<std::pair<uint32_t, uint32_t>> key;
    std::vector<uint16_t> idx_tmp;
    std::vector<S> val_tmp;
    for (size_t b = 0; b < nb; ++b) {
        const size_t lo = (size_t)A.blk_nz_ptr[b], hi = (size_t)A.blk_nz_ptr[b + 1];
        if (hi - lo < 2) continue;
        const uint32_t sh = A.blk_shift[b];
        const uint32_t cm = (1u << sh) - 1u;
        key.clear();
        for (size_t k = lo; k < hi; ++k) {
            const uint32_t v = A.nz_idx[k];
            key.emplace_back(order == BOO_ROWMAJOR ? v : (((v & cm) << 16) | (v >> sh)),
                             (uint32_t)(k - lo));
        }
        std::sort(key.begin(), key.end());
        idx_tmp.assign(A.nz_idx.begin() + lo, A.nz_idx.begin() + hi);
        val_tmp.assign(A.nz_val.begin() + lo, A.nz_val.begin() + hi);
        for (size_t t = 0; t < key.size(); ++t) {
            A.nz_idx[lo + t] = idx_tmp[key[t].second];
            A.nz_val[lo + t] = val_tmp[key[t].second];
        }
    }

    // Remainder bins -> CSR, each row sorted by (col, value).
    A.rem_indptr.assign((size_t)rows + 1, 0);
    for (I r = 0; r < rows; ++r) {
        if (!bins.empty()) {
            auto& bin = bins[(size_t)r];
            std::sort(bin.begin(), bin.end());
            for (const auto& e : bin) {
                A.rem_col_ind.push_back(e.first);
                A.rem_vals.push_back(e.second);
            }
        }
        A.rem_indptr[(size_t)r + 1] = (I)A.rem_col_ind.size();
    }
    return A;
}

// boo_to_csr: output equal to boo_matrix/boo_matrix.cpp:277-333.
template <typename I, typename S>
void boo_decode(I rows, const I* row_grp_ptr, const I* row_ids, const I* col_grp_ptr,
                const I* col_ids, I nb, const I* blk_row_grp, const I* blk_col_grp,
                const I* blk_nz_ptr, const uint8_t* blk_shift, const uint16_t* nz_idx,
                const S* nz_val, const I* rem_indptr, const I* rem_col_ind, const S* rem_vals,
                I tail_n, const I* tail_row, const I* tail_col, const S* tail_val, I* out_indptr,
                I* out_indices, S* out_data) {
    std::vector<std::vector<std::pair<I, S>>> bins((size_t)rows);
    for (I b = 0; b < nb; ++b) {
        const I rbase = row_grp_ptr[blk_row_grp[b]];
        const I cbase = col_grp_ptr[blk_col_grp[b]];
        const uint32_t sh = blk_shift[b];
        const uint32_t cm = (1u << sh) - 1u;
        for (I k = blk_nz_ptr[b]; k < blk_nz_ptr[b + 1]; ++k) {
            const uint32_t v = nz_idx[k];
            bins[(size_t)row_ids[rbase + (I)(v >> sh)]].emplace_back(col_ids[cbase + (I)(v & cm)],
                                                                     nz_val[k]);
        }
    }
    for (I r = 0; r < rows; ++r)
        for (I j = rem_indptr[r]; j < rem_indptr[r + 1]; ++j)
            bins[(size_t)r].emplace_back(rem_col_ind[j], rem_vals[j]);
    for (I k = 0; k < tail_n; ++k) bins[(size_t)tail_row[k]].emplace_back(tail_col[k], tail_val[k]);
    I n = 0;
    out_indptr[0] = 0;
    for (I r = 0; r < rows; ++r) {
        auto& bin = bins[(size_t)r];
        std::sort(bin.begin(), bin.end());
        for (const auto& e : bin) {
            out_indices[n] = e.first;
            out_data[n] = e.second;
            ++n;
        }
        out_indptr[r + 1] = n;
    }
}

// boo_batched_matmul_cpu: same loop order, and so the same rounding, as
// boo_matrix/boo_matrix.cpp:336-396 (blocks, then remainder rows, then tail;
// y += v*x with separate multiply and add).  y must be zeroed.
template <typename I, typename S>
void boo_matmul_host(I rows, I cols, const I* row_grp_ptr, const I* row_ids,
                     const I* col_grp_ptr, const I* col_ids, I nb, const I* blk_row_grp,
                     const I* blk_col_grp, const I* blk_nz_ptr, const uint8_t* blk_shift,
                     const uint16_t* nz_idx, const S* nz_val, const I* rem_indptr,
                     const I* rem_col_ind, const S* rem_vals, I tail_n, const I* tail_row,
                     const I* tail_col, const S* tail_val, const S* x, S* y, int64_t batch,
                     int64_t K) {
    for (int64_t bt = 0; bt < batch; ++bt) {
        const S* xb = x + bt * (int64_t)cols * K;
        S* yb = y + bt * (int64_t)rows * K;
        for (I b = 0; b < nb; ++b) {
            const I rbase = row_grp_ptr[blk_row_grp[b]];
            const I cbase = col_grp_ptr[blk_col_grp[b]];
            const uint32_t sh = blk_shift[b];
            const uint32_t cm = (1u << sh) - 1u;
            for (I k = blk_nz_ptr[b]; k < blk_nz_ptr[b + 1]; ++k) {
                const uint32_t v = nz_idx[k];
                const S a = nz_val[k];
                const S* xr = xb + (int64_t)col_ids[cbase + (I)(v & cm)] * K;
                S* yr = yb + (int64_t)row_ids[rbase + (I)(v >> sh)] * K;
                for (int64_t f = 0; f < K; ++f) yr[f] += a * xr[f];
            }
        }
        for (I r = 0; r < rows; ++r) {
            S* yr = yb + (int64_t)r * K;
            for (I j = rem_indptr[r]; j < rem_indptr[r + 1]; ++j) {
                const S a = rem_vals[j];
                const S* xr = xb + (int64_t)rem_col_ind[j] * K;
                for (int64_t f = 0; f < K; ++f) yr[f] += a * xr[f];
            }
        }
        for (I k = 0; k < tail_n; ++k) {
            const S a = tail_val[k];
            const S* xr = xb + (int64_t)tail_col[k] * K;
            S* yr = yb + (int64_t)tail_row[k] * K;
            for (int64_t f = 0; f < K; ++f) yr[f] += a * xr[f];
        }
    }
}

// ---------------------------------------------------------------------------
// PBR
// ---------------------------------------------------------------------------

template <typename I, typename S>
struct PbrArrays {
    I rows = 0, cols = 0, block_rows = 0, block_cols = 0, total_nnz = 0;
    std::vector<uint64_t> codes;
    std::vector<I> coords;   // interleaved (row, col)
    std::vector<I> offsets;
    std::vector<S> data;
    std::vector<I> rem_indptr, rem_col_ind;
    std::vector<S> rem_vals;
};

// csr_to_pbr: output equal to pbr_matrix/pbr_matrix.cpp:333-448.  The block
// order inside a stripe is the iteration order of a std::unordered_map keyed
// by the block index narrowed to I, created with sqrt(#block columns) buckets,
// filled in CSR order and cleared (keeping its buckets) after each stripe --
// the same container operations in the same sequence as the reference, which
// is what fixes that order.  A block's values are its entries in CSR order;
// a spilled block pairs its k-th set bit (row-major) with its k-th value.
template <typename I, typename S>
PbrArrays<I, S> build_pbr(const I* indptr, const I* indices, const S* data, I rows, I cols,
                          I block_rows, I block_cols, uint8_t min_nnz) {
    if (block_rows <= 0 || block_cols <= 0 || (uint64_t)block_rows * (uint64_t)block_cols > 64)
        throw std::invalid_argument("csr_to_pbr: block_rows*block_cols must be in [1, 64]");
    PbrArrays<I, S> P;
    P.rows = rows;
    P.cols = cols;
    P.block_rows = block_rows;
    P.block_cols = block_cols;
    P.total_nnz = rows > 0 ? indptr[rows] : 0;
    const uint64_t ncb = ((uint64_t)cols + (uint64_t)block_cols - 1) / (uint64_t)block_cols;
    P.offsets.push_back(0);
    P.data.reserve((size_t)P.total_nnz);

    // key -> (code, block column); only the key sequence shapes the order.
    std::unordered_map<I, std::pair<uint64_t, uint64_t>> stripe((size_t)std::sqrt((double)ncb));
    // Values of each block column of the current stripe, in CSR order.
    std::vector<std::vector<S>> vals((size_t)ncb);
    std::vector<std::vector<std::pair<I, S>>> bins((size_t)rows);
    std::vector<uint64_t> live;  // block columns touched in this stripe
    I offset = 0;
    for (uint64_t row = 0; row < (uint64_t)rows; ++row) {
        const I brow = (I)(row / (uint64_t)block_rows);
        const uint64_t roff = row % (uint64_t)block_rows;
        for (uint64_t j = (uint64_t)indptr[row]; j < (uint64_t)indptr[row + 1]; ++j) {
            const uint64_t col = (uint64_t)indices[j];
            const uint64_t bcol = col / (uint64_t)block_cols;
            const I key = (I)((uint64_t)brow * ncb + bcol);
            auto ins = stripe.emplace(key, std::pair<uint64_t, uint64_t>(0ull, bcol));
            if (ins.second) live.push_back(bcol);
            ins.first->second.first |= 1ull << (roff * (uint64_t)block_cols + col % (uint64_t)block_cols);
            vals[(size_t)bcol].push_back(data[j]);
        }
        if ((row + 1) / (uint64_t)block_rows > (uint64_t)brow || row + 1 == (uint64_t)rows) {
            const I row0 = (I)(brow * block_rows);
            for (const auto& kv : stripe) {
                const uint64_t code = kv.second.first;
                const uint64_t bc = kv.second.second;
                auto& v = vals[(size_t)bc];
                const int n = __builtin_popcountll(code);
                const I col0 = (I)(bc * (uint64_t)block_cols);
                if (n >= (int)min_nnz) {
                    P.codes.push_back(code);
                    P.coords.push_back(row0);
                    P.coords.push_back(col0);
                    P.data.insert(P.data.end(), v.begin(), v.end());
                    offset += (I)n;
                    P.offsets.push_back(offset);
                } else {
                    size_t k = 0;
                    for (I ro = 0; ro < block_rows; ++ro)
                        for (I co = 0; co < block_cols; ++co)
                            if ((code >> (uint64_t)(ro * block_cols + co)) & 1ull)
                                bins[(size_t)(row0 + ro)].emplace_back(col0 + co, v[k++]);
                }
            }
            for (const uint64_t bc : live) vals[(size_t)bc].clear();
            live.clear();
            stripe.clear();
        }
    }
    P.rem_indptr.assign((size_t)rows + 1, 0);
    for (I r = 0; r < rows; ++r) {
        auto& bin = bins[(size_t)r];
        std::sort(bin.begin(), bin.end());
        for (const auto& e : bin) {
            P.rem_col_ind.push_back(e.first);
            P.rem_vals.push_back(e.second);
        }
        P.rem_indptr[(size_t)r + 1] = (I)P.rem_col_ind.size();
    }
    return P;
}

// pbr_to_csr: output equal to pbr_matrix/pbr_matrix.cpp:279-331 (values are
// consumed in bit order across all blocks; a set bit in a padding row past the
// last matrix row is an error).  Returns the number of entries written.
template <typename I, typename S>
I pbr_decode(I rows, I cols, I block_rows, I block_cols, size_t nb, const uint64_t* codes,
             const I* coords, const S* data, const I* rem_indptr, const I* rem_col_ind,
             const S* rem_vals, I* out_indptr, I* out_indices, S* out_data) {
    std::vector<std::vector<std::pair<I, S>>> bins((size_t)rows);
    size_t di = 0;
    for (size_t b = 0; b < nb; ++b) {
        const uint64_t code = codes[b];
        const I r0 = coords[2 * b], c0 = coords[2 * b + 1];
        for (I r = 0; r < block_rows; ++r) {
            if (r0 + r >= rows) {
                for (I c = 0; c < block_cols; ++c)
                    if ((code >> (uint64_t)(r * block_cols + c)) & 1ull)
                        throw std::runtime_error(
                            "Block has a nonzero past the last matrix row. Check block size and "
                            "matrix dimensions for compatibility.");
                continue;
            }
            for (I c = 0; c < block_cols; ++c) {
                if (c0 + c >= cols) continue;
                if ((code >> (uint64_t)(r * block_cols + c)) & 1ull)
                    bins[(size_t)(r0 + r)].emplace_back(c0 + c, data[di++]);
            }
        }
    }
    for (I r = 0; r < rows; ++r)
        for (I j = rem_indptr[r]; j < rem_indptr[r + 1]; ++j)
            bins[(size_t)r].emplace_back(rem_col_ind[j], rem_vals[j]);
    I n = 0;
    out_indptr[0] = 0;
    for (I r = 0; r < rows; ++r) {
        auto& bin = bins[(size_t)r];
        std::sort(bin.begin(), bin.end());
        for (const auto& e : bin) {
            out_indices[n] = e.first;
            out_data[n] = e.second;
            ++n;
        }
        out_indptr[r + 1] = n;
    }
    return n;
}

// pbr_batched_matmul_cpu: same loop order as pbr_matrix/pbr_matrix.cpp:17-68
// (blocks in order, bits row-major, values consumed sequentially; then the
// remainder rows).  y must be zeroed.
template <typename I, typename S>
void pbr_matmul_host(I rows, I cols, I block_rows, I block_cols, size_t nb, const uint64_t* codes,
                     const I* coords, const S* data, const I* rem_indptr, const I* rem_col_ind,
                     const S* rem_vals, const S* x, S* y, int64_t batch, int64_t K) {
    for (int64_t bt = 0; bt < batch; ++bt) {
        const S* xb = x + bt * (int64_t)cols * K;
        S* yb = y + bt * (int64_t)rows * K;
        size_t di = 0;
        for (size_t b = 0; b < nb; ++b) {
            const uint64_t code = codes[b];
            const I r0 = coords[2 * b], c0 = coords[2 * b + 1];
            for (I r = 0; r < block_rows; ++r) {
                const I gr = r0 + r;
                if (gr >= rows) continue;
                for (I c = 0; c < block_cols; ++c) {
                    const I gc = c0 + c;
                    if (gc >= cols) continue;
                    if ((code >> (uint64_t)(r * block_cols + c)) & 1ull) {
                        const S a = data[di++];
                        S* yr = yb + (int64_t)gr * K;
                        const S* xr = xb + (int64_t)gc * K;
                        for (int64_t f = 0; f < K; ++f) yr[f] += a * xr[f];
                    }
                }
            }
        }
        for (I r = 0; r < rows; ++r) {
            S* yr = yb + (int64_t)r * K;
            for (I j = rem_indptr[r]; j < rem_indptr[r + 1]; ++j) {
                const S a = rem_vals[j];
                const S* xr = xb + (int64_t)rem_col_ind[j] * K;
                for (int64_t f = 0; f < K; ++f) yr[f] += a * xr[f];
            }
        }
    }
}

}  // namespace spmm
