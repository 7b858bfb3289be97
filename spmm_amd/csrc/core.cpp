// spmm_amd._core -- the pybind11 host layer.
//
// Mirrors the module surface of the reference's torch_fast_spdmm_core
// (bindings/bindings.cpp:157-232): csr_to_boo / boo_to_csr / the CPU BOO op,
// csr_to_pbr / pbr_to_csr / the CPU PBR op, and the GPU entry points.  It
// holds no tensors: Python hands over numpy arrays for host work and raw
// device pointers + a hipStream_t for GPU work, and the GPU calls go through
// the C ABI of libspmm_amd.so (include/spmm_amd.h).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "formats.hpp"
#include "spmm_amd.h"

namespace py = pybind11;

namespace {

// Hand a vector to numpy without copying: the array owns it via a capsule.
template <typename T>
py::array_t<T> give(std::vector<T>&& v) {
    auto* heap = new std::vector<T>(std::move(v));
    py::capsule owner(heap, [](void* p) { delete static_cast<std::vector<T>*>(p); });
    return py::array_t<T>({(py::ssize_t)heap->size()}, {(py::ssize_t)sizeof(T)}, heap->data(), owner);
}

template <typename T>
const T* ptr_of(const py::array& a, const char* name) {
    if (!py::isinstance<py::array_t<T>>(a) || !(a.flags() & py::array::c_style))
        throw std::invalid_argument(std::string(name) + ": expected a contiguous array of the right dtype");
    return static_cast<const T*>(a.data());
}

template <typename T>
T* mut_ptr_of(py::array& a, const char* name) {
    if (!py::isinstance<py::array_t<T>>(a) || !(a.flags() & py::array::c_style) || !a.writeable())
        throw std::invalid_argument(std::string(name) + ": expected a writable contiguous array");
    return static_cast<T*>(a.mutable_data());
}

bool is_i64(const py::array& a) { return a.dtype().is(py::dtype::of<int64_t>()); }
bool is_f64(const py::array& a) { return a.dtype().is(py::dtype::of<double>()); }

void raise_status(int rc) {
    if (rc == SPMM_OK) return;
    const std::string msg = spmm_last_error();
    if (rc == SPMM_EINVAL || rc == SPMM_EUNSUPPORTED) throw std::invalid_argument(msg);
    throw std::runtime_error(msg);
}

// ---------------------------------------------------------------- BOO host
template <typename I, typename S>
py::dict boo_build_t(const py::array& indptr, const py::array& indices, const py::array& data,
                     int64_t rows, int64_t cols, const py::array& rl, const py::array& cl,
                     int policy, int64_t threshold, int order) {
    const I* ip = ptr_of<I>(indptr, "indptr");
    const I* ix = ptr_of<I>(indices, "indices");
    const S* dv = ptr_of<S>(data, "data");
    const int32_t* rlp = ptr_of<int32_t>(rl, "row_labels");
    const int32_t* clp = ptr_of<int32_t>(cl, "col_labels");
    if ((int64_t)rl.size() != rows || (int64_t)cl.size() != cols)
        throw std::invalid_argument("csr_to_boo: label array length must match matrix dims");
    if ((int64_t)indptr.size() != rows + 1)
        throw std::invalid_argument("csr_to_boo: indptr must have rows+1 entries");
    spmm::BooArrays<I, S> A;
    {
        py::gil_scoped_release nogil;
        A = spmm::build_boo<I, S>(ip, ix, dv, (I)rows, (I)cols, rlp, clp, policy, (I)threshold, order);
    }
    py::dict d;
    d["rows"] = (int64_t)A.rows;
    d["cols"] = (int64_t)A.cols;
    d["total_nnz"] = (int64_t)A.total_nnz;
    d["max_nr"] = (int64_t)A.max_nr;
    d["max_nc"] = (int64_t)A.max_nc;
    d["max_nnz_blk"] = (int64_t)A.max_nnz_blk;
    d["nz_order"] = A.nz_order;
    d["row_grp_ptr"] = give(std::move(A.row_grp_ptr));
    d["row_ids"] = give(std::move(A.row_ids));
    d["col_grp_ptr"] = give(std::move(A.col_grp_ptr));
    d["col_ids"] = give(std::move(A.col_ids));
    d["blk_row_grp"] = give(std::move(A.blk_row_grp));
    d["blk_col_grp"] = give(std::move(A.blk_col_grp));
    d["blk_nz_ptr"] = give(std::move(A.blk_nz_ptr));
    d["blk_shift"] = give(std::move(A.blk_shift));
    d["nz_idx"] = give(std::move(A.nz_idx));
    d["nz_val"] = give(std::move(A.nz_val));
    d["rem_indptr"] = give(std::move(A.rem_indptr));
    d["rem_col_ind"] = give(std::move(A.rem_col_ind));
    d["rem_vals"] = give(std::move(A.rem_vals));
    d["tail_row"] = give(std::move(A.tail_row));
    d["tail_col"] = give(std::move(A.tail_col));
    d["tail_val"] = give(std::move(A.tail_val));
    return d;
}

py::dict boo_build(const py::array& indptr, const py::array& indices, const py::array& data,
                   int64_t rows, int64_t cols, const py::array& rl, const py::array& cl, int policy,
                   int64_t threshold, int order) {
    const bool i64 = is_i64(indptr), f64 = is_f64(data);
    if (i64 && f64) return boo_build_t<int64_t, double>(indptr, indices, data, rows, cols, rl, cl, policy, threshold, order);
    if (i64) return boo_build_t<int64_t, float>(indptr, indices, data, rows, cols, rl, cl, policy, threshold, order);
    if (f64) return boo_build_t<int32_t, double>(indptr, indices, data, rows, cols, rl, cl, policy, threshold, order);
    return boo_build_t<int32_t, float>(indptr, indices, data, rows, cols, rl, cl, policy, threshold, order);
}

// The BOO arrays travel as a dict (the Python object's __dict__ subset).
template <typename I, typename S>
struct BooView {
    I rows, cols, nb, tail_n;
    const I *row_grp_ptr, *row_ids, *col_grp_ptr, *col_ids, *blk_row_grp, *blk_col_grp, *blk_nz_ptr;
    const uint8_t* blk_shift;
    const uint16_t* nz_idx;
    const S* nz_val;
    const I *rem_indptr, *rem_col_ind;
    const S* rem_vals;
    const I *tail_row, *tail_col;
    const S* tail_val;
};

template <typename I, typename S>
BooView<I, S> boo_view(const py::dict& d) {
    BooView<I, S> v;
    v.rows = (I)d["rows"].cast<int64_t>();
    v.cols = (I)d["cols"].cast<int64_t>();
    auto arr = [&](const char* k) { return d[k].cast<py::array>(); };
    v.row_grp_ptr = ptr_of<I>(arr("row_grp_ptr"), "row_grp_ptr");
    v.row_ids = ptr_of<I>(arr("row_ids"), "row_ids");
    v.col_grp_ptr = ptr_of<I>(arr("col_grp_ptr"), "col_grp_ptr");
    v.col_ids = ptr_of<I>(arr("col_ids"), "col_ids");
    v.blk_row_grp = ptr_of<I>(arr("blk_row_grp"), "blk_row_grp");
    v.nb = (I)arr("blk_row_grp").size();
    v.blk_col_grp = ptr_of<I>(arr("blk_col_grp"), "blk_col_grp");
    v.blk_nz_ptr = ptr_of<I>(arr("blk_nz_ptr"), "blk_nz_ptr");
    v.blk_shift = ptr_of<uint8_t>(arr("blk_shift"), "blk_shift");
    v.nz_idx = ptr_of<uint16_t>(arr("nz_idx"), "nz_idx");
    v.nz_val = ptr_of<S>(arr("nz_val"), "nz_val");
    v.rem_indptr = ptr_of<I>(arr("rem_indptr"), "rem_indptr");
    v.rem_col_ind = ptr_of<I>(arr("rem_col_ind"), "rem_col_ind");
    v.rem_vals = ptr_of<S>(arr("rem_vals"), "rem_vals");
    v.tail_row = ptr_of<I>(arr("tail_row"), "tail_row");
    v.tail_col = ptr_of<I>(arr("tail_col"), "tail_col");
    v.tail_val = ptr_of<S>(arr("tail_val"), "tail_val");
    v.tail_n = (I)arr("tail_val").size();
    return v;
}

template <typename I, typename S>
void boo_to_csr_t(const py::dict& d, py::array& out_indptr, py::array& out_indices, py::array& out_data) {
    auto v = boo_view<I, S>(d);
    I* op = mut_ptr_of<I>(out_indptr, "indptr");
    I* oi = mut_ptr_of<I>(out_indices, "indices");
    S* od = mut_ptr_of<S>(out_data, "data");
    py::gil_scoped_release nogil;
    spmm::boo_decode<I, S>(v.rows, v.row_grp_ptr, v.row_ids, v.col_grp_ptr, v.col_ids, v.nb,
                           v.blk_row_grp, v.blk_col_grp, v.blk_nz_ptr, v.blk_shift, v.nz_idx,
                           v.nz_val, v.rem_indptr, v.rem_col_ind, v.rem_vals, v.tail_n, v.tail_row,
                           v.tail_col, v.tail_val, op, oi, od);
}

template <typename I, typename S>
void boo_matmul_cpu_t(const py::dict& d, const py::array& x, py::array& y, int64_t batch, int64_t K) {
    auto v = boo_view<I, S>(d);
    const S* xp = ptr_of<S>(x, "x");
    S* yp = mut_ptr_of<S>(y, "y");
    if ((int64_t)x.size() != batch * (int64_t)v.cols * K || (int64_t)y.size() != batch * (int64_t)v.rows * K)
        throw std::invalid_argument("boo_matmul_cpu: x/y sizes do not match the matrix");
    py::gil_scoped_release nogil;
    spmm::boo_matmul_host<I, S>(v.rows, v.cols, v.row_grp_ptr, v.row_ids, v.col_grp_ptr, v.col_ids,
                                v.nb, v.blk_row_grp, v.blk_col_grp, v.blk_nz_ptr, v.blk_shift,
                                v.nz_idx, v.nz_val, v.rem_indptr, v.rem_col_ind, v.rem_vals,
                                v.tail_n, v.tail_row, v.tail_col, v.tail_val, xp, yp, batch, K);
}

#define SPMM_DISPATCH_IS(i64, f64, FN, ...)                      \
    do {                                                         \
        if (i64 && f64) return FN<int64_t, double>(__VA_ARGS__); \
        if (i64) return FN<int64_t, float>(__VA_ARGS__);         \
        if (f64) return FN<int32_t, double>(__VA_ARGS__);        \
        return FN<int32_t, float>(__VA_ARGS__);                  \
    } while (0)

// ---------------------------------------------------------------- PBR host
template <typename I, typename S>
py::dict pbr_build_t(const py::array& indptr, const py::array& indices, const py::array& data,
                     int64_t rows, int64_t cols, int64_t br, int64_t bc, int min_nnz) {
    const I* ip = ptr_of<I>(indptr, "indptr");
    const I* ix = ptr_of<I>(indices, "indices");
    const S* dv = ptr_of<S>(data, "data");
    if ((int64_t)indptr.size() != rows + 1)
        throw std::invalid_argument("csr_to_pbr: indptr must have rows+1 entries");
    spmm::PbrArrays<I, S> P;
    {
        py::gil_scoped_release nogil;
        P = spmm::build_pbr<I, S>(ip, ix, dv, (I)rows, (I)cols, (I)br, (I)bc, (uint8_t)min_nnz);
    }
    py::dict d;
    d["rows"] = (int64_t)P.rows;
    d["cols"] = (int64_t)P.cols;
    d["block_rows"] = (int64_t)P.block_rows;
    d["block_cols"] = (int64_t)P.block_cols;
    d["total_nnz"] = (int64_t)P.total_nnz;
    d["block_codes"] = give(std::move(P.codes));
    d["block_coords"] = give(std::move(P.coords));
    d["block_offsets"] = give(std::move(P.offsets));
    d["block_data"] = give(std::move(P.data));
    d["remainder_indptr"] = give(std::move(P.rem_indptr));
    d["remainder_col_ind"] = give(std::move(P.rem_col_ind));
    d["remainder_data"] = give(std::move(P.rem_vals));
    return d;
}

py::dict pbr_build(const py::array& indptr, const py::array& indices, const py::array& data,
                   int64_t rows, int64_t cols, int64_t br, int64_t bc, int min_nnz) {
    if (min_nnz < 0 || min_nnz > 255)
        throw std::invalid_argument("csr_to_pbr: min_nnz_per_block must fit in uint8 (0..255)");
    SPMM_DISPATCH_IS(is_i64(indptr), is_f64(data), pbr_build_t, indptr, indices, data, rows, cols, br, bc, min_nnz);
}

template <typename I, typename S>
int64_t pbr_to_csr_t(const py::dict& d, py::array& out_indptr, py::array& out_indices, py::array& out_data) {
    auto arr = [&](const char* k) { return d[k].cast<py::array>(); };
    const I rows = (I)d["rows"].cast<int64_t>(), cols = (I)d["cols"].cast<int64_t>();
    const I br = (I)d["block_rows"].cast<int64_t>(), bc = (I)d["block_cols"].cast<int64_t>();
    const py::array codes = arr("block_codes");
    const uint64_t* cp = ptr_of<uint64_t>(codes, "block_codes");
    const I* co = ptr_of<I>(arr("block_coords"), "block_coords");
    const S* dp = ptr_of<S>(arr("block_data"), "block_data");
    const I* ri = ptr_of<I>(arr("remainder_indptr"), "remainder_indptr");
    const I* rc = ptr_of<I>(arr("remainder_col_ind"), "remainder_col_ind");
    const S* rv = ptr_of<S>(arr("remainder_data"), "remainder_data");
    I* op = mut_ptr_of<I>(out_indptr, "indptr");
    I* oi = mut_ptr_of<I>(out_indices, "indices");
    S* od = mut_ptr_of<S>(out_data, "data");
    py::gil_scoped_release nogil;
    return (int64_t)spmm::pbr_decode<I, S>(rows, cols, br, bc, (size_t)codes.size(), cp, co, dp, ri, rc,
                                           rv, op, oi, od);
}

template <typename I, typename S>
void pbr_matmul_cpu_t(const py::dict& d, const py::array& x, py::array& y, int64_t batch, int64_t K) {
    auto arr = [&](const char* k) { return d[k].cast<py::array>(); };
    const I rows = (I)d["rows"].cast<int64_t>(), cols = (I)d["cols"].cast<int64_t>();
    const I br = (I)d["block_rows"].cast<int64_t>(), bc = (I)d["block_cols"].cast<int64_t>();
    const py::array codes = arr("block_codes");
    const uint64_t* cp = ptr_of<uint64_t>(codes, "block_codes");
    const I* co = ptr_of<I>(arr("block_coords"), "block_coords");
    const S* dp = ptr_of<S>(arr("block_data"), "block_data");
    const I* ri = ptr_of<I>(arr("remainder_indptr"), "remainder_indptr");
    const I* rc = ptr_of<I>(arr("remainder_col_ind"), "remainder_col_ind");
    const S* rv = ptr_of<S>(arr("remainder_data"), "remainder_data");
    const S* xp = ptr_of<S>(x, "x");
    S* yp = mut_ptr_of<S>(y, "y");
    if ((int64_t)x.size() != batch * (int64_t)cols * K || (int64_t)y.size() != batch * (int64_t)rows * K)
        throw std::invalid_argument("pbr_matmul_cpu: x/y sizes do not match the matrix");
    py::gil_scoped_release nogil;
    spmm::pbr_matmul_host<I, S>(rows, cols, br, bc, (size_t)codes.size(), cp, co, dp, ri, rc, rv, xp,
                                yp, batch, K);
}

// ---------------------------------------------------------------- GPU glue
uintptr_t P(const py::dict& d, const char* k) { return d[k].cast<uintptr_t>(); }

spmm_boo_desc boo_desc(const py::dict& d) {
    spmm_boo_desc A{};
    A.rows = d["rows"].cast<int32_t>();
    A.cols = d["cols"].cast<int32_t>();
    A.n_stream_rows = d["n_stream_rows"].cast<int32_t>();
    A.row_ids = reinterpret_cast<const int32_t*>(P(d, "row_ids"));
    A.n_tiles = d["n_tiles"].cast<int32_t>();
    A.tiles = reinterpret_cast<const int32_t*>(P(d, "tiles"));
    A.tile_rs = reinterpret_cast<const uint8_t*>(P(d, "tile_rs"));
    A.ent_val = reinterpret_cast<const void*>(P(d, "ent_val"));
    A.ent_col = reinterpret_cast<const uint8_t*>(P(d, "ent_col"));
    A.tcols = reinterpret_cast<const int32_t*>(P(d, "tcols"));
    A.n_waves = d["n_waves"].cast<int32_t>();
    A.group = d["group"].cast<int32_t>();
    A.wave_tiles = reinterpret_cast<const int32_t*>(P(d, "wave_tiles"));
    A.n_slots = d["n_slots"].cast<int32_t>();
    A.n_splits = d["n_splits"].cast<int32_t>();
    A.splits = reinterpret_cast<const int32_t*>(P(d, "splits"));
    A.n_long = d["n_long"].cast<int32_t>();
    A.long_rows = reinterpret_cast<const int32_t*>(P(d, "long_rows"));
    A.n_crow = d["n_crow"].cast<int32_t>();
    A.crow_ptr = reinterpret_cast<const int32_t*>(P(d, "crow_ptr"));
    A.crow_id = reinterpret_cast<const int32_t*>(P(d, "crow_id"));
    A.ccol = reinterpret_cast<const int32_t*>(P(d, "ccol"));
    A.cval = reinterpret_cast<const void*>(P(d, "cval"));
    A.n_crow_long = d["n_crow_long"].cast<int32_t>();
    A.n_gtask = d["n_gtask"].cast<int32_t>();
    A.gtask = reinterpret_cast<const int32_t*>(P(d, "gtask"));
    A.gtask_ptr = reinterpret_cast<const int32_t*>(P(d, "gtask_ptr"));
    A.rem_indptr = reinterpret_cast<const int32_t*>(P(d, "rem_indptr"));
    A.rem_col_ind = reinterpret_cast<const int32_t*>(P(d, "rem_col_ind"));
    A.rem_vals = reinterpret_cast<const void*>(P(d, "rem_vals"));
    if (d.contains("n_blob16")) {
        A.n_blob16 = d["n_blob16"].cast<int64_t>();
        A.blobs = reinterpret_cast<const void*>(P(d, "blobs"));
        A.blob_first = reinterpret_cast<const uint32_t*>(P(d, "blob_first"));
        A.blob_xid = reinterpret_cast<const uint32_t*>(P(d, "blob_xid"));
    }
    if (d.contains("gtask_order")) A.gtask_order = reinterpret_cast<const int32_t*>(P(d, "gtask_order"));
    return A;
}

// Host staging of a BOO matrix into the kernel's tile stream (spmm_boo_stage_*).
// h: the BOO arrays as int32 / uint8 / uint16 numpy arrays plus the sizes.
py::dict boo_stage(const py::dict& h, int32_t max_item_nnz, int32_t long_threshold, int32_t n_waves,
                   int32_t group, float min_reuse) {
    auto arr = [&](const char* k) { return h[k].cast<py::array>(); };
    const py::array nz_val = arr("nz_val"), rem_vals = arr("rem_vals");
    const bool f64 = is_f64(nz_val);
    if (f64 != is_f64(rem_vals)) throw std::invalid_argument("nz_val and rem_vals dtypes differ");
    spmm_boo_host H{};
    H.rows = h["rows"].cast<int32_t>();
    H.cols = h["cols"].cast<int32_t>();
    H.n_row_groups = h["n_row_groups"].cast<int32_t>();
    H.n_col_groups = h["n_col_groups"].cast<int32_t>();
    H.num_blocks = h["num_blocks"].cast<int32_t>();
    H.dtype = f64 ? SPMM_F64 : SPMM_F32;
    H.row_grp_ptr = ptr_of<int32_t>(arr("row_grp_ptr"), "row_grp_ptr");
    H.row_ids = ptr_of<int32_t>(arr("row_ids"), "row_ids");
    H.col_grp_ptr = ptr_of<int32_t>(arr("col_grp_ptr"), "col_grp_ptr");
    H.col_ids = ptr_of<int32_t>(arr("col_ids"), "col_ids");
    H.blk_row_grp = ptr_of<int32_t>(arr("blk_row_grp"), "blk_row_grp");
    H.blk_col_grp = ptr_of<int32_t>(arr("blk_col_grp"), "blk_col_grp");
    H.blk_nz_ptr = ptr_of<int32_t>(arr("blk_nz_ptr"), "blk_nz_ptr");
    H.blk_shift = ptr_of<uint8_t>(arr("blk_shift"), "blk_shift");
    H.nz_idx = ptr_of<uint16_t>(arr("nz_idx"), "nz_idx");
    H.nz_val = nz_val.data();
    H.rem_indptr = ptr_of<int32_t>(arr("rem_indptr"), "rem_indptr");
    H.rem_col_ind = ptr_of<int32_t>(arr("rem_col_ind"), "rem_col_ind");
    H.rem_vals = rem_vals.data();
    if (!(nz_val.flags() & py::array::c_style) || !(rem_vals.flags() & py::array::c_style))
        throw std::invalid_argument("values must be contiguous");
    spmm_boo_stage* st = nullptr;
    raise_status(spmm_boo_stage_create(&H, max_item_nnz, long_threshold, n_waves, group, min_reuse, &st));
    spmm_boo_stage_info inf{};
    spmm_boo_stage_sizes(st, &inf);
    std::vector<int32_t> tiles((size_t)inf.n_tiles * 8), tcols((size_t)inf.n_tcols),
        splits((size_t)inf.n_splits * 4), longr((size_t)inf.n_long), wt((size_t)inf.n_waves + 1),
        crp((size_t)inf.n_crow + 1), cri((size_t)inf.n_crow), ccol((size_t)inf.n_cnz),
        gt((size_t)inf.n_gtask * 2), gtp((size_t)inf.n_crow_long + 1);
    std::vector<uint8_t> rs((size_t)inf.n_tiles * 33);
    std::vector<uint8_t> ecol((size_t)inf.n_ent);
    py::array ev = f64 ? py::array(py::array_t<double>((py::ssize_t)inf.n_ent))
                       : py::array(py::array_t<float>((py::ssize_t)inf.n_ent));
    py::array cv = f64 ? py::array(py::array_t<double>((py::ssize_t)inf.n_cnz))
                       : py::array(py::array_t<float>((py::ssize_t)inf.n_cnz));
    const int rc = spmm_boo_stage_copy(st, tiles.data(), rs.data(), inf.n_ent ? ev.mutable_data() : nullptr,
                                       ecol.data(), tcols.data(), splits.data(), longr.data(), wt.data(),
                                       crp.data(), cri.data(), ccol.data(),
                                       inf.n_cnz ? cv.mutable_data() : nullptr, gt.data(), gtp.data());
    std::vector<uint32_t> blobs((size_t)inf.n_blob16 * 4), bfirst(inf.n_blob16 > 0 ? (size_t)inf.n_waves * 8 : 0),
        bxid(inf.n_blob16 > 0 ? (size_t)inf.n_tiles * 8 : 0);
    const int rc2 = rc ? rc : spmm_boo_stage_copy_blobs(st, blobs.data(), bfirst.data(), bxid.data());
    std::vector<int32_t> gord((size_t)inf.n_gtask_order);
    const int rc3 = rc2 ? rc2 : spmm_boo_stage_copy_gtask_order(st, gord.data());
    spmm_boo_stage_destroy(st);
    raise_status(rc);
    raise_status(rc2);
    raise_status(rc3);
    py::dict d;
    d["gtask_order"] = give(std::move(gord));
    d["n_gtask_order"] = inf.n_gtask_order;
    d["blobs"] = give(std::move(blobs));
    d["blob_first"] = give(std::move(bfirst));
    d["blob_xid"] = give(std::move(bxid));
    d["n_blob16"] = inf.n_blob16;
    d["tiles"] = give(std::move(tiles));
    d["tile_rs"] = give(std::move(rs));
    d["ent_val"] = ev;
    d["ent_col"] = give(std::move(ecol));
    d["tcols"] = give(std::move(tcols));
    d["splits"] = give(std::move(splits));
    d["long_rows"] = give(std::move(longr));
    d["wave_tiles"] = give(std::move(wt));
    d["crow_ptr"] = give(std::move(crp));
    d["crow_id"] = give(std::move(cri));
    d["ccol"] = give(std::move(ccol));
    d["cval"] = cv;
    d["n_crow"] = inf.n_crow;
    d["gtask"] = give(std::move(gt));
    d["gtask_ptr"] = give(std::move(gtp));
    d["n_crow_long"] = inf.n_crow_long;
    d["n_stream_rows"] = inf.n_stream_rows;
    d["n_gtask"] = inf.n_gtask;
    d["n_tiles"] = inf.n_tiles;
    d["n_slots"] = inf.n_slots;
    d["n_splits"] = inf.n_splits;
    d["n_long"] = inf.n_long;
    d["n_waves"] = inf.n_waves;
    d["group"] = inf.group;
    return d;
}

size_t boo_workspace_bytes(const py::dict& d, int dtype, int64_t batch, int64_t K) {
    spmm_boo_desc A = boo_desc(d);
    return spmm_boo_workspace_bytes(&A, (spmm_dtype)dtype, batch, K);
}

void boo_matmul_gpu(const py::dict& d, int dtype, uintptr_t x, uintptr_t y, int64_t batch, int64_t K,
                    uintptr_t ws, size_t ws_bytes, uintptr_t stream) {
    spmm_boo_desc A = boo_desc(d);
    raise_status(spmm_boo_matmul(&A, (spmm_dtype)dtype, reinterpret_cast<const void*>(x),
                                 reinterpret_cast<void*>(y), batch, K, reinterpret_cast<void*>(ws),
                                 ws_bytes, reinterpret_cast<void*>(stream)));
}

spmm_pbr_desc pbr_desc(const py::dict& d) {
    spmm_pbr_desc A{};
    A.rows = d["rows"].cast<int64_t>();
    A.cols = d["cols"].cast<int64_t>();
    A.block_rows = d["block_rows"].cast<int32_t>();
    A.block_cols = d["block_cols"].cast<int32_t>();
    A.num_blocks = d["num_blocks"].cast<int64_t>();
    A.itype = (spmm_itype)d["itype"].cast<int>();
    A.codes = reinterpret_cast<const int64_t*>(P(d, "codes"));
    A.coords = reinterpret_cast<const void*>(P(d, "coords"));
    A.offsets = reinterpret_cast<const void*>(P(d, "offsets"));
    A.data = reinterpret_cast<const void*>(P(d, "data"));
    A.rem_indptr = reinterpret_cast<const void*>(P(d, "rem_indptr"));
    A.rem_col_ind = reinterpret_cast<const void*>(P(d, "rem_col_ind"));
    A.rem_vals = reinterpret_cast<const void*>(P(d, "rem_vals"));
    A.stripe_ptr = reinterpret_cast<const int32_t*>(P(d, "stripe_ptr"));
    A.n_long = d["n_long"].cast<int32_t>();
    A.long_rows = reinterpret_cast<const int32_t*>(P(d, "long_rows"));
    A.long_threshold = d["long_threshold"].cast<int32_t>();
    return A;
}

void pbr_matmul_gpu(const py::dict& d, int dtype, uintptr_t x, uintptr_t y, int64_t batch, int64_t K,
                    uintptr_t stream) {
    spmm_pbr_desc A = pbr_desc(d);
    raise_status(spmm_pbr_matmul(&A, (spmm_dtype)dtype, reinterpret_cast<const void*>(x),
                                 reinterpret_cast<void*>(y), batch, K, reinterpret_cast<void*>(stream)));
}

// ---- launch introspection: the kernels a multiply launches, with their
// runtime attributes, as a list of dicts (one per launch, in order) ----

py::list launch_list(const std::vector<spmm_launch_info>& v, int32_t n) {
    py::list out;
    for (int32_t i = 0; i < n; ++i) {
        const spmm_launch_info& o = v[i];
        py::dict d;
        d["kernel"] = std::string(o.kernel);
        d["grid"] = py::make_tuple(o.grid[0], o.grid[1], o.grid[2]);
        d["threads"] = o.block;
        d["registers_per_thread"] = o.registers;
        d["local_bytes_per_thread"] = o.scratch_bytes;
        d["static_shared_bytes"] = o.lds_bytes;
        d["max_threads_per_block"] = o.max_threads;
        d["max_active_blocks_per_cu"] = o.wgs_per_cu;
        out.append(d);
    }
    return out;
}

template <typename Desc, typename Fn>
py::list launch_info(const Desc& A, int dtype, uintptr_t x, uintptr_t y, int64_t batch, int64_t K, Fn fn) {
    int32_t n = 0;
    raise_status(fn(&A, (spmm_dtype)dtype, reinterpret_cast<const void*>(x), reinterpret_cast<const void*>(y),
                    batch, K, nullptr, 0, &n));
    std::vector<spmm_launch_info> v(n);
    raise_status(fn(&A, (spmm_dtype)dtype, reinterpret_cast<const void*>(x), reinterpret_cast<const void*>(y),
                    batch, K, v.data(), n, &n));
    return launch_list(v, std::min<int32_t>(n, (int32_t)v.size()));
}

py::list boo_launch_info(const py::dict& d, int dtype, uintptr_t x, uintptr_t y, int64_t batch, int64_t K) {
    return launch_info(boo_desc(d), dtype, x, y, batch, K, spmm_boo_launch_info);
}

py::list pbr_launch_info(const py::dict& d, int dtype, uintptr_t x, uintptr_t y, int64_t batch, int64_t K) {
    return launch_info(pbr_desc(d), dtype, x, y, batch, K, spmm_pbr_launch_info);
}

// ---- measurement adjuncts: timers, C++-timed calls, the vendor SpMM plan ----
// Handles cross into Python as integers; the Python classes own them.

uintptr_t new_timer() {
    spmm_timer* t = nullptr;
    raise_status(spmm_timer_create(&t));
    return reinterpret_cast<uintptr_t>(t);
}

float boo_matmul_gpu_timed(const py::dict& d, int dtype, uintptr_t x, uintptr_t y, int64_t batch,
                           int64_t K, uintptr_t ws, size_t ws_bytes, uintptr_t stream, uintptr_t timer) {
    spmm_boo_desc A = boo_desc(d);
    float ms = 0.f;
    raise_status(spmm_boo_matmul_timed(&A, (spmm_dtype)dtype, reinterpret_cast<const void*>(x),
                                       reinterpret_cast<void*>(y), batch, K, reinterpret_cast<void*>(ws),
                                       ws_bytes, reinterpret_cast<void*>(stream),
                                       reinterpret_cast<spmm_timer*>(timer), &ms));
    return ms;
}

float pbr_matmul_gpu_timed(const py::dict& d, int dtype, uintptr_t x, uintptr_t y, int64_t batch, int64_t K,
                           uintptr_t stream, uintptr_t timer) {
    spmm_pbr_desc A = pbr_desc(d);
    float ms = 0.f;
    raise_status(spmm_pbr_matmul_timed(&A, (spmm_dtype)dtype, reinterpret_cast<const void*>(x),
                                       reinterpret_cast<void*>(y), batch, K, reinterpret_cast<void*>(stream),
                                       reinterpret_cast<spmm_timer*>(timer), &ms));
    return ms;
}

uintptr_t vendor_create(int64_t rows, int64_t cols, int64_t nnz, uintptr_t crow, uintptr_t col, uintptr_t val,
                        uintptr_t x, int64_t K, uintptr_t y, int alg, uintptr_t stream) {
    spmm_vendor_spmm* p = nullptr;
    raise_status(spmm_vendor_spmm_create(rows, cols, nnz, reinterpret_cast<const int32_t*>(crow),
                                         reinterpret_cast<const int32_t*>(col),
                                         reinterpret_cast<const float*>(val), reinterpret_cast<const float*>(x),
                                         K, reinterpret_cast<float*>(y), alg, reinterpret_cast<void*>(stream), &p));
    return reinterpret_cast<uintptr_t>(p);
}

py::dict vendor_info(uintptr_t plan) {
    spmm_vendor_info inf{};
    raise_status(spmm_vendor_spmm_info(reinterpret_cast<const spmm_vendor_spmm*>(plan), &inf));
    py::dict d;
    d["version"] = inf.version;
    d["header_version"] = inf.header_version;
    d["workspace_bytes"] = inf.workspace_bytes;
    d["supported"] = inf.supported != 0;
    d["preprocess_status"] = inf.preprocess_status;
    return d;
}

float vendor_run_timed(uintptr_t plan, uintptr_t stream, uintptr_t timer) {
    float ms = 0.f;
    raise_status(spmm_vendor_spmm_run_timed(reinterpret_cast<spmm_vendor_spmm*>(plan),
                                            reinterpret_cast<void*>(stream),
                                            reinterpret_cast<spmm_timer*>(timer), &ms));
    return ms;
}

void csr_naive_gpu(uintptr_t indptr, uintptr_t col, uintptr_t vals, int itype, int dtype, int64_t rows,
                   int64_t cols, uintptr_t x, uintptr_t y, int64_t K, uintptr_t stream) {
    raise_status(spmm_csr_naive(reinterpret_cast<const void*>(indptr), reinterpret_cast<const void*>(col),
                                reinterpret_cast<const void*>(vals), (spmm_itype)itype, (spmm_dtype)dtype,
                                rows, cols, reinterpret_cast<const void*>(x), reinterpret_cast<void*>(y), K,
                                reinterpret_cast<void*>(stream)));
}

}  // namespace

PYBIND11_MODULE(_core, m) {
    m.doc() = "spmm_amd native host layer (format builders, CPU ops, C-ABI GPU glue)";
    m.def("csr_to_boo", &boo_build);
    m.def("boo_to_csr", [](const py::dict& d, py::array& ip, py::array& ix, py::array& dv) {
        SPMM_DISPATCH_IS(is_i64(ip), is_f64(dv), boo_to_csr_t, d, ip, ix, dv);
    });
    m.def("boo_matmul_cpu", [](const py::dict& d, const py::array& x, py::array& y, int64_t batch, int64_t K) {
        SPMM_DISPATCH_IS(is_i64(d["row_ids"].cast<py::array>()), is_f64(x), boo_matmul_cpu_t, d, x, y, batch, K);
    });
    m.def("csr_to_pbr", &pbr_build);
    m.def("pbr_to_csr", [](const py::dict& d, py::array& ip, py::array& ix, py::array& dv) -> int64_t {
        SPMM_DISPATCH_IS(is_i64(ip), is_f64(dv), pbr_to_csr_t, d, ip, ix, dv);
    });
    m.def("pbr_matmul_cpu", [](const py::dict& d, const py::array& x, py::array& y, int64_t batch, int64_t K) {
        SPMM_DISPATCH_IS(is_i64(d["block_offsets"].cast<py::array>()), is_f64(x), pbr_matmul_cpu_t, d, x, y,
                         batch, K);
    });
    m.def("boo_stage", &boo_stage, py::arg("h"), py::arg("max_item_nnz"), py::arg("long_threshold"),
          py::arg("n_waves"), py::arg("group") = 1, py::arg("min_reuse") = 0.0f);
    m.def("boo_workspace_bytes", &boo_workspace_bytes);
    m.def("boo_matmul_gpu", &boo_matmul_gpu);
    m.def("pbr_matmul_gpu", &pbr_matmul_gpu);
    m.def("csr_naive_gpu", &csr_naive_gpu);
    m.def("boo_launch_info", &boo_launch_info);
    m.def("pbr_set_slab_bytes", [](int64_t b) { raise_status(spmm_pbr_set_slab_bytes(b)); });
    m.def("pbr_get_slab_bytes", []() { return spmm_pbr_get_slab_bytes(); });
    m.def("pbr_launch_info", &pbr_launch_info);
    m.def("timer_create", &new_timer);
    m.def("timer_destroy", [](uintptr_t t) { spmm_timer_destroy(reinterpret_cast<spmm_timer*>(t)); });
    m.def("boo_matmul_gpu_timed", &boo_matmul_gpu_timed);
    m.def("pbr_matmul_gpu_timed", &pbr_matmul_gpu_timed);
    m.def("vendor_create", &vendor_create);
    m.def("vendor_info", &vendor_info);
    m.def("vendor_preprocess", [](uintptr_t plan, uintptr_t ws, size_t bytes) {
        raise_status(spmm_vendor_spmm_preprocess(reinterpret_cast<spmm_vendor_spmm*>(plan),
                                                 reinterpret_cast<void*>(ws), bytes));
    });
    m.def("vendor_run", [](uintptr_t plan, uintptr_t stream) {
        raise_status(spmm_vendor_spmm_run(reinterpret_cast<spmm_vendor_spmm*>(plan),
                                          reinterpret_cast<void*>(stream)));
    });
    m.def("vendor_run_timed", &vendor_run_timed);
    m.def("vendor_destroy", [](uintptr_t plan) {
        spmm_vendor_spmm_destroy(reinterpret_cast<spmm_vendor_spmm*>(plan));
    });
    m.def("version", []() { return std::string(spmm_version()); });
}
