// Measurement adjuncts of the C ABI (include/spmm_amd.h):
//
//  * spmm_timer and the *_timed entry points: an event pair recorded on the
//    caller's stream around exactly one product call, with nothing else
//    between the two records -- the scope of the reference's C++-timed
//    harnesses (bindings/bindings_boo_timed.cu:254-270,
//    bindings/bindings_pbr_timed.cu:160-180, bindings/bindings_cusparse.cu:
//    122-134).
//  * spmm_vendor_spmm: a persistent rocSPARSE generic-SpMM plan over a CSR
//    matrix, the vendor baseline (the reference's DirectSpMM over cuSPARSE,
//    bindings/bindings_cusparse.cu:21-160).  librocsparse is opened with
//    dlopen on the first plan, so the library has no link-time dependency on
//    it and the product path never loads it.
//
// Host code only: no kernels are defined here.

#include <hip/hip_runtime.h>
#include <rocsparse/rocsparse.h>

#include <dlfcn.h>

#include <cstdio>
#include <mutex>
#include <string>

#include "spmm_amd.h"
#include "internal.hpp"

namespace {

int fail(int code, const std::string& msg) { return spmm_internal::set_error(code, msg.c_str()); }

int hip_fail(const char* what, hipError_t e) {
    return fail(SPMM_ELAUNCH, std::string(what) + ": " + hipGetErrorString(e));
}

// The rocSPARSE entry points the plan uses, typed from the header.
struct Rocsparse {
    decltype(&rocsparse_create_handle) create_handle = nullptr;
    decltype(&rocsparse_destroy_handle) destroy_handle = nullptr;
    decltype(&rocsparse_set_stream) set_stream = nullptr;
    decltype(&rocsparse_set_pointer_mode) set_pointer_mode = nullptr;
    decltype(&rocsparse_get_version) get_version = nullptr;
    decltype(&rocsparse_get_status_name) status_name = nullptr;
    decltype(&rocsparse_create_csr_descr) create_csr = nullptr;
    decltype(&rocsparse_destroy_spmat_descr) destroy_spmat = nullptr;
    decltype(&rocsparse_create_dnmat_descr) create_dnmat = nullptr;
    decltype(&rocsparse_destroy_dnmat_descr) destroy_dnmat = nullptr;
    decltype(&rocsparse_spmm) spmm = nullptr;
    std::string error;  // empty when every symbol resolved
};

const Rocsparse& rocsparse() {
    static Rocsparse r;
    static std::once_flag once;
    std::call_once(once, [] {
        void* h = dlopen("librocsparse.so.1", RTLD_NOW | RTLD_LOCAL);
        if (!h) h = dlopen("librocsparse.so", RTLD_NOW | RTLD_LOCAL);
        if (!h) {
            const char* e = dlerror();
            r.error = std::string("cannot load librocsparse: ") + (e ? e : "unknown error");
            return;
        }
        auto sym = [&](auto& fn, const char* name) {
            fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name));
            if (!fn && r.error.empty()) r.error = std::string("librocsparse lacks ") + name;
        };
        sym(r.create_handle, "rocsparse_create_handle");
        sym(r.destroy_handle, "rocsparse_destroy_handle");
        sym(r.set_stream, "rocsparse_set_stream");
        sym(r.set_pointer_mode, "rocsparse_set_pointer_mode");
        sym(r.get_version, "rocsparse_get_version");
        sym(r.status_name, "rocsparse_get_status_name");
        sym(r.create_csr, "rocsparse_create_csr_descr");
        sym(r.destroy_spmat, "rocsparse_destroy_spmat_descr");
        sym(r.create_dnmat, "rocsparse_create_dnmat_descr");
        sym(r.destroy_dnmat, "rocsparse_destroy_dnmat_descr");
        sym(r.spmm, "rocsparse_spmm");
    });
    return r;
}

int sparse_fail(const Rocsparse& api, const char* what, rocsparse_status s) {
    const char* name = api.status_name ? api.status_name(s) : "?";
    return fail(s == rocsparse_status_not_implemented ? SPMM_EUNSUPPORTED : SPMM_ELAUNCH,
                std::string("rocSPARSE ") + what + ": " + name);
}

rocsparse_spmm_alg vendor_alg(int32_t code) {
    switch (code) {
        case SPMM_VENDOR_ALG_CSR: return rocsparse_spmm_alg_csr;
        case SPMM_VENDOR_ALG_CSR_ROW_SPLIT: return rocsparse_spmm_alg_csr_row_split;
        case SPMM_VENDOR_ALG_CSR_NNZ_SPLIT: return rocsparse_spmm_alg_csr_nnz_split;
        case SPMM_VENDOR_ALG_CSR_MERGE_PATH: return rocsparse_spmm_alg_csr_merge_path;
        default: return rocsparse_spmm_alg_default;
    }
}

// Records start, runs body, records end, waits for it: ms is the GPU time
// between the two records.  The end is recorded even when body fails, so
// the stream never holds a dangling start.
template <class F>
int timed(spmm_timer* t, hipStream_t s, float* ms, F&& body);

}  // namespace

extern "C" {

struct spmm_timer {
    hipEvent_t start = nullptr, end = nullptr;
};

struct spmm_vendor_spmm {
    rocsparse_handle handle = nullptr;
    rocsparse_spmat_descr A = nullptr;
    rocsparse_dnmat_descr B = nullptr, C = nullptr;
    rocsparse_spmm_alg alg = rocsparse_spmm_alg_default;
    hipStream_t stream = nullptr;
    size_t bytes = 0;
    void* workspace = nullptr;
    int32_t supported = 1;
    int32_t preprocessed = 0;
    int32_t preprocess_status = -1;  // rocsparse_status of the preprocess stage, -1 before it
    float alpha = 1.f, beta = 0.f;
};

int spmm_timer_create(spmm_timer** out) {
    if (!out) return fail(SPMM_EINVAL, "null timer output");
    *out = nullptr;
    auto* t = new (std::nothrow) spmm_timer();
    if (!t) return fail(SPMM_ENOMEM, "cannot allocate a timer");
    hipError_t e = hipEventCreate(&t->start);
    if (e == hipSuccess) e = hipEventCreate(&t->end);
    // first records outside any measurement
    if (e == hipSuccess) e = hipEventRecord(t->start, nullptr);
    if (e == hipSuccess) e = hipEventRecord(t->end, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(t->end);
    if (e != hipSuccess) {
        spmm_timer_destroy(t);
        return hip_fail("timer events", e);
    }
    *out = t;
    return SPMM_OK;
}

void spmm_timer_destroy(spmm_timer* t) {
    if (!t) return;
    if (t->start) (void)hipEventDestroy(t->start);
    if (t->end) (void)hipEventDestroy(t->end);
    delete t;
}

int spmm_boo_matmul_timed(const spmm_boo_desc* A, spmm_dtype dtype, const void* X, void* Y,
                          int64_t batch, int64_t K, void* workspace, size_t workspace_bytes,
                          void* stream, spmm_timer* timer, float* ms) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    return timed(timer, s, ms, [&] {
        return spmm_boo_matmul(A, dtype, X, Y, batch, K, workspace, workspace_bytes, stream);
    });
}

int spmm_pbr_matmul_timed(const spmm_pbr_desc* A, spmm_dtype dtype, const void* X, void* Y,
                          int64_t batch, int64_t K, void* stream, spmm_timer* timer, float* ms) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    return timed(timer, s, ms, [&] { return spmm_pbr_matmul(A, dtype, X, Y, batch, K, stream); });
}

int spmm_vendor_spmm_create(int64_t rows, int64_t cols, int64_t nnz, const int32_t* crow,
                            const int32_t* col, const float* val, const float* X, int64_t K,
                            float* Y, int32_t alg, void* stream, spmm_vendor_spmm** out) {
    if (!out) return fail(SPMM_EINVAL, "null plan output");
    *out = nullptr;
    if (rows < 0 || cols < 0 || nnz < 0 || K < 0) return fail(SPMM_EINVAL, "negative CSR SpMM sizes");
    if (!crow || (nnz > 0 && (!col || !val)) || (cols > 0 && K > 0 && !X) || (rows > 0 && K > 0 && !Y))
        return fail(SPMM_EINVAL, "null CSR SpMM array");
    if (alg < SPMM_VENDOR_ALG_DEFAULT || alg > SPMM_VENDOR_ALG_CSR_MERGE_PATH)
        return fail(SPMM_EINVAL, "unknown vendor SpMM algorithm " + std::to_string(alg));
    const Rocsparse& api = rocsparse();
    if (!api.error.empty()) return fail(SPMM_EUNSUPPORTED, api.error);

    auto* p = new (std::nothrow) spmm_vendor_spmm();
    if (!p) return fail(SPMM_ENOMEM, "cannot allocate a vendor plan");
    p->alg = vendor_alg(alg);
    p->stream = static_cast<hipStream_t>(stream);
    auto bail = [&](int rc) {
        spmm_vendor_spmm_destroy(p);
        return rc;
    };
    rocsparse_status st = api.create_handle(&p->handle);
    if (st != rocsparse_status_success) return bail(sparse_fail(api, "create_handle", st));
    st = api.set_stream(p->handle, p->stream);
    if (st == rocsparse_status_success) st = api.set_pointer_mode(p->handle, rocsparse_pointer_mode_host);
    if (st != rocsparse_status_success) return bail(sparse_fail(api, "handle setup", st));
    st = api.create_csr(&p->A, rows, cols, nnz, const_cast<int32_t*>(crow), const_cast<int32_t*>(col),
                        const_cast<float*>(val), rocsparse_indextype_i32, rocsparse_indextype_i32,
                        rocsparse_index_base_zero, rocsparse_datatype_f32_r);
    if (st == rocsparse_status_success)
        st = api.create_dnmat(&p->B, cols, K, K, const_cast<float*>(X), rocsparse_datatype_f32_r,
                              rocsparse_order_row);
    if (st == rocsparse_status_success)
        st = api.create_dnmat(&p->C, rows, K, K, Y, rocsparse_datatype_f32_r, rocsparse_order_row);
    if (st != rocsparse_status_success) return bail(sparse_fail(api, "descriptors", st));
    st = api.spmm(p->handle, rocsparse_operation_none, rocsparse_operation_none, &p->alpha, p->A, p->B,
                  &p->beta, p->C, rocsparse_datatype_f32_r, p->alg, rocsparse_spmm_stage_buffer_size,
                  &p->bytes, nullptr);
    if (st == rocsparse_status_not_implemented) {
        p->supported = 0;  // reported by info(); run() refuses
    } else if (st != rocsparse_status_success) {
        return bail(sparse_fail(api, "buffer size", st));
    }
    *out = p;
    return SPMM_OK;
}

int spmm_vendor_spmm_info(const spmm_vendor_spmm* p, spmm_vendor_info* info) {
    if (!p || !info) return fail(SPMM_EINVAL, "null vendor plan or info");
    const Rocsparse& api = rocsparse();
    int version = 0;
    rocsparse_status st = api.get_version(p->handle, &version);
    if (st != rocsparse_status_success) return sparse_fail(api, "get_version", st);
    info->version = version;
    info->header_version = ROCSPARSE_VERSION_MAJOR * 100000 + ROCSPARSE_VERSION_MINOR * 100 +
                           ROCSPARSE_VERSION_PATCH;
    info->workspace_bytes = p->bytes;
    info->supported = p->supported;
    info->preprocess_status = p->preprocess_status;
    return SPMM_OK;
}

int spmm_vendor_spmm_preprocess(spmm_vendor_spmm* p, void* workspace, size_t workspace_bytes) {
    if (!p) return fail(SPMM_EINVAL, "null vendor plan");
    if (!p->supported) return fail(SPMM_EUNSUPPORTED, "rocSPARSE does not implement this SpMM");
    if (workspace_bytes < p->bytes || (p->bytes > 0 && !workspace))
        return fail(SPMM_ENOMEM, "vendor SpMM workspace needs " + std::to_string(p->bytes) + " bytes");
    const Rocsparse& api = rocsparse();
    size_t bytes = p->bytes;
    rocsparse_status st = api.spmm(p->handle, rocsparse_operation_none, rocsparse_operation_none, &p->alpha,
                                   p->A, p->B, &p->beta, p->C, rocsparse_datatype_f32_r, p->alg,
                                   rocsparse_spmm_stage_preprocess, &bytes, workspace);
    p->preprocess_status = (int32_t)st;
    if (st != rocsparse_status_success) return sparse_fail(api, "preprocess", st);
    p->workspace = workspace;
    p->preprocessed = 1;
    const hipError_t e = hipStreamSynchronize(p->stream);
    if (e != hipSuccess) return hip_fail("vendor SpMM preprocess", e);
    return SPMM_OK;
}

int spmm_vendor_spmm_run(spmm_vendor_spmm* p, void* stream) {
    if (!p) return fail(SPMM_EINVAL, "null vendor plan");
    if (static_cast<hipStream_t>(stream) != p->stream)
        return fail(SPMM_EINVAL, "the vendor SpMM plan must run on its construction stream");
    if (!p->supported) return fail(SPMM_EUNSUPPORTED, "rocSPARSE does not implement this SpMM");
    if (!p->preprocessed) return fail(SPMM_EINVAL, "vendor SpMM plan run before preprocess");
    const Rocsparse& api = rocsparse();
    size_t bytes = p->bytes;
    const rocsparse_status st = api.spmm(p->handle, rocsparse_operation_none, rocsparse_operation_none,
                                         &p->alpha, p->A, p->B, &p->beta, p->C, rocsparse_datatype_f32_r,
                                         p->alg, rocsparse_spmm_stage_compute, &bytes, p->workspace);
    if (st != rocsparse_status_success) return sparse_fail(api, "compute", st);
    return SPMM_OK;
}

int spmm_vendor_spmm_run_timed(spmm_vendor_spmm* p, void* stream, spmm_timer* timer, float* ms) {
    return timed(timer, static_cast<hipStream_t>(stream), ms, [&] { return spmm_vendor_spmm_run(p, stream); });
}

void spmm_vendor_spmm_destroy(spmm_vendor_spmm* p) {
    if (!p) return;
    const Rocsparse& api = rocsparse();
    if (p->handle) (void)hipStreamSynchronize(p->stream);
    if (p->C) api.destroy_dnmat(p->C);
    if (p->B) api.destroy_dnmat(p->B);
    if (p->A) api.destroy_spmat(p->A);
    if (p->handle) api.destroy_handle(p->handle);
    delete p;
}

}  // extern "C"

namespace {

template <class F>
int timed(spmm_timer* t, hipStream_t s, float* ms, F&& body) {
    if (!t || !ms) return fail(SPMM_EINVAL, "null timer or result");
    *ms = 0.f;
    hipError_t e = hipEventRecord(t->start, s);
    if (e != hipSuccess) return hip_fail("timer start", e);
    const int rc = body();
    e = hipEventRecord(t->end, s);
    if (e == hipSuccess) e = hipEventSynchronize(t->end);
    if (rc != SPMM_OK) return rc;
    if (e != hipSuccess) return hip_fail("timer end", e);
    e = hipEventElapsedTime(ms, t->start, t->end);
    if (e != hipSuccess) return hip_fail("timer elapsed", e);
    return SPMM_OK;
}

}  // namespace
