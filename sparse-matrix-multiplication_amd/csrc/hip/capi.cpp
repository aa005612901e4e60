// C ABI (include/spmm_capi.h) over the C++ API and the launch layer.

#include "spmm_capi.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <new>
#include <stdexcept>
#include <string>
#include <vector>

#include "engine.h"
#include "spmm/bsr.h"
#include "spmm/csr.h"
#include "spmm/metrics.h"
#include "spmm/partition.h"
#include "spmm/patterns.h"
#include "spmm/spmm_hybrid.h"

namespace {

thread_local std::string g_last_error;

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int ok() { return SPMM_OK; }

spmm::CSR to_cpp(const spmm_csr_t& c) {
    spmm::CSR m;
    m.num_rows = c.num_rows;
    m.num_cols = c.num_cols;
    m.nnz      = c.nnz;
    m.row_ptr  = c.row_ptr;
    m.col_idx  = c.col_idx;
    m.values   = c.values;
    return m;
}

spmm_csr_t to_c(const spmm::CSR& m) {
    spmm_csr_t c;
    c.num_rows = m.num_rows;
    c.num_cols = m.num_cols;
    c.nnz      = m.nnz;
    c.row_ptr  = m.row_ptr;
    c.col_idx  = m.col_idx;
    c.values   = m.values;
    return c;
}

spmm::BSR to_cpp(const spmm_bsr_t& c) {
    spmm::BSR b;
    b.num_rows   = c.num_rows;
    b.num_cols   = c.num_cols;
    b.block_rows = c.block_rows;
    b.block_cols = c.block_cols;
    b.num_blocks = c.num_blocks;
    b.nnz        = c.nnz;
    b.row_ptr    = c.row_ptr;
    b.col_idx    = c.col_idx;
    b.values     = reinterpret_cast<half*>(c.values);
    return b;
}

spmm::BSR_host host_bsr_from_c(const spmm_bsr_t& c) {
    spmm::BSR_host h;
    h.num_rows   = c.num_rows;
    h.num_cols   = c.num_cols;
    h.block_rows = c.block_rows;
    h.block_cols = c.block_cols;
    h.num_blocks = c.num_blocks;
    h.nnz        = c.nnz;
    h.row_ptr.assign(c.row_ptr, c.row_ptr + c.block_rows + 1);
    h.col_idx.assign(c.col_idx, c.col_idx + c.num_blocks);
    const size_t nv = static_cast<size_t>(c.num_blocks) * 256;
    h.values.resize(nv);
    std::memcpy(h.values.data(), c.values, nv * sizeof(uint16_t));
    return h;
}

template <typename T>
T* malloc_copy(const T* src, size_t n) {
    T* p = static_cast<T*>(std::malloc(sizeof(T) * (n > 0 ? n : 1)));
    if (p == nullptr) throw std::bad_alloc();
    if (n > 0) std::memcpy(p, src, sizeof(T) * n);
    return p;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

int from_engine(const spmm::engine::Error& e) {
    if (e.status == spmm::engine::kOk) return SPMM_OK;
    switch (e.status) {
        case spmm::engine::kInvalid: return set_error(SPMM_INVALID, e.message);
        case spmm::engine::kUnsupported: return set_error(SPMM_UNSUPPORTED, e.message);
        default: return set_error(SPMM_HIP_ERROR, e.message);
    }
}

int from_hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return SPMM_OK;
    return set_error(SPMM_HIP_ERROR, std::string(what) + ": " + hipGetErrorString(e));
}

// Runs f, mapping C++ exceptions to error codes.
template <typename F>
int guarded(F f) {
    try {
        return f();
    } catch (const std::bad_alloc&) {
        return set_error(SPMM_NO_MEMORY, "host allocation failed");
    } catch (const std::runtime_error& e) {
        const std::string msg = e.what();
        const bool io = msg.find("cannot open") != std::string::npos ||
                        msg.find("short read") != std::string::npos;
        return set_error(io ? SPMM_IO_ERROR : SPMM_INVALID, msg);
    } catch (const std::exception& e) {
        return set_error(SPMM_INVALID, e.what());
    }
}

spmm::engine::CsrRole role_of(int id) { return static_cast<spmm::engine::CsrRole>(id); }

int launch_id(int kernel_id, const void* d_A_any, const void* d_B, float* d_C, int N,
              void* stream) {
    if (d_A_any == nullptr) return set_error(SPMM_INVALID, "null matrix descriptor");
    if (kernel_id >= 0 && kernel_id <= 6) {
        const spmm::CSR A = to_cpp(*static_cast<const spmm_csr_t*>(d_A_any));
        return from_engine(spmm::engine::launch_csr(role_of(kernel_id), A,
                                                    static_cast<const float*>(d_B), d_C, N,
                                                    as_stream(stream)));
    }
    if (kernel_id == 7) {
        const spmm::BSR A = to_cpp(*static_cast<const spmm_bsr_t*>(d_A_any));
        return from_engine(spmm::engine::launch_bsr(A, static_cast<const half*>(d_B), d_C, N,
                                                    as_stream(stream)));
    }
    return set_error(SPMM_INVALID, "unknown kernel id " + std::to_string(kernel_id));
}

spmm::engine::EngineOpts opts_from_c(const spmm_engine_opts_t* o) {
    spmm::engine::EngineOpts e;
    if (o != nullptr) {
        e.vec            = o->vec;
        e.waves          = o->waves;
        e.unroll         = o->unroll;
        e.rows_per_block = o->rows_per_block;
        e.groups         = o->groups;
        e.slices         = o->slices;
        e.global_loads   = o->global_loads;
        e.row_groups     = o->row_groups;
        e.entry_lanes    = o->entry_lanes;
        e.max_row_hint   = o->max_row_hint;
    }
    return e;
}

}  // namespace

extern "C" {

const char* spmm_c_last_error(void) { return g_last_error.c_str(); }
const char* spmm_c_version(void) { return "spmm_amd 0.1 gfx950"; }

// ---- host CSR -------------------------------------------------------------

int spmm_c_csr_alloc_host(int rows, int cols, int nnz, spmm_csr_t* out) {
    if (out == nullptr || rows < 0 || cols < 0 || nnz < 0) {
        return set_error(SPMM_INVALID, "spmm_c_csr_alloc_host: bad argument");
    }
    *out = to_c(spmm::csr_alloc_host(rows, cols, nnz));
    return ok();
}

void spmm_c_csr_free_host(spmm_csr_t* m) {
    if (m == nullptr) return;
    spmm::CSR c = to_cpp(*m);
    spmm::csr_free_host(c);
    *m = to_c(c);
}

int spmm_c_csr_from_coo_host(int rows, int cols, int n, const int* r, const int* c,
                             const float* v, spmm_csr_t* out) {
    if (out == nullptr || n < 0 || rows < 0 || cols < 0 ||
        (n > 0 && (r == nullptr || c == nullptr || v == nullptr))) {
        return set_error(SPMM_INVALID, "spmm_c_csr_from_coo_host: bad argument");
    }
    return guarded([&] {
        std::vector<int> rv(r, r + n), cv(c, c + n);
        std::vector<float> vv(v, v + n);
        *out = to_c(spmm::csr_from_coo_host(rows, cols, rv, cv, vv));
        return ok();
    });
}

int spmm_c_generate_uniform_random_csr(int rows, int cols, float density, int seed,
                                       spmm_csr_t* out) {
    if (out == nullptr || rows < 0 || cols < 0) {
        return set_error(SPMM_INVALID, "spmm_c_generate_uniform_random_csr: bad argument");
    }
    return guarded([&] {
        *out = to_c(spmm::generate_uniform_random_csr(rows, cols, density, seed));
        return ok();
    });
}

int spmm_c_csr_row_slice_host(const spmm_csr_t* m, int b, int e, spmm_csr_t* out) {
    if (m == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        *out = to_c(spmm::csr_row_slice_host(to_cpp(*m), b, e));
        return ok();
    });
}

int spmm_c_csr_read_binary_host(const char* path, spmm_csr_t* out) {
    if (path == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        *out = to_c(spmm::csr_read_binary_host(path));
        return ok();
    });
}

int spmm_c_csr_write_binary_host(const spmm_csr_t* m, const char* path) {
    if (path == nullptr || m == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        spmm::csr_write_binary_host(to_cpp(*m), path);
        return ok();
    });
}

int spmm_c_csr_to_device(const spmm_csr_t* h, spmm_csr_t* d) {
    if (h == nullptr || d == nullptr || h->num_rows < 0 || h->nnz < 0) {
        return set_error(SPMM_INVALID, "spmm_c_csr_to_device: bad argument");
    }
    spmm_csr_t out{h->num_rows, h->num_cols, h->nnz, nullptr, nullptr, nullptr};
    const size_t rp = sizeof(int) * (static_cast<size_t>(h->num_rows) + 1);
    const size_t nz = static_cast<size_t>(h->nnz > 0 ? h->nnz : 1);
    int rc = from_hip(hipMalloc(&out.row_ptr, rp), "hipMalloc");
    if (rc == SPMM_OK) rc = from_hip(hipMalloc(&out.col_idx, sizeof(int) * nz), "hipMalloc");
    if (rc == SPMM_OK) rc = from_hip(hipMalloc(&out.values, sizeof(float) * nz), "hipMalloc");
    if (rc == SPMM_OK) {
        rc = from_hip(hipMemcpy(out.row_ptr, h->row_ptr, rp, hipMemcpyHostToDevice), "hipMemcpy");
    }
    if (rc == SPMM_OK && h->nnz > 0) {
        rc = from_hip(hipMemcpy(out.col_idx, h->col_idx, sizeof(int) * h->nnz,
                                hipMemcpyHostToDevice), "hipMemcpy");
        if (rc == SPMM_OK) {
            rc = from_hip(hipMemcpy(out.values, h->values, sizeof(float) * h->nnz,
                                    hipMemcpyHostToDevice), "hipMemcpy");
        }
    }
    if (rc != SPMM_OK) {
        (void)hipFree(out.row_ptr);
        (void)hipFree(out.col_idx);
        (void)hipFree(out.values);
        return rc;
    }
    *d = out;
    return ok();
}

int spmm_c_csr_free_device(spmm_csr_t* d) {
    if (d == nullptr) return ok();
    int rc = SPMM_OK;
    if (d->row_ptr) rc |= from_hip(hipFree(d->row_ptr), "hipFree");
    if (d->col_idx) rc |= from_hip(hipFree(d->col_idx), "hipFree");
    if (d->values) rc |= from_hip(hipFree(d->values), "hipFree");
    *d = spmm_csr_t{0, 0, 0, nullptr, nullptr, nullptr};
    return rc == SPMM_OK ? ok() : SPMM_HIP_ERROR;
}

// ---- BSR ------------------------------------------------------------------

int spmm_c_bsr_from_csr_host(const spmm_csr_t* h, spmm_bsr_t* out) {
    if (h == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        const spmm::BSR_host b = spmm::bsr_from_csr_host(to_cpp(*h));
        spmm_bsr_t r;
        r.num_rows   = b.num_rows;
        r.num_cols   = b.num_cols;
        r.block_rows = b.block_rows;
        r.block_cols = b.block_cols;
        r.num_blocks = b.num_blocks;
        r.nnz        = b.nnz;
        r.row_ptr    = malloc_copy(b.row_ptr.data(), b.row_ptr.size());
        r.col_idx    = malloc_copy(b.col_idx.data(), b.col_idx.size());
        r.values     = malloc_copy(reinterpret_cast<const uint16_t*>(b.values.data()),
                                   b.values.size());
        *out = r;
        return ok();
    });
}

void spmm_c_bsr_free_host(spmm_bsr_t* h) {
    if (h == nullptr) return;
    std::free(h->row_ptr);
    std::free(h->col_idx);
    std::free(h->values);
    *h = spmm_bsr_t{0, 0, 0, 0, 0, 0, nullptr, nullptr, nullptr};
}

int spmm_c_bsr_to_device(const spmm_bsr_t* h, spmm_bsr_t* d) {
    if (h == nullptr || d == nullptr || h->block_rows < 0 || h->num_blocks < 0) {
        return set_error(SPMM_INVALID, "spmm_c_bsr_to_device: bad argument");
    }
    spmm_bsr_t out = *h;
    out.row_ptr = nullptr;
    out.col_idx = nullptr;
    out.values  = nullptr;
    const size_t rp = sizeof(int) * (static_cast<size_t>(h->block_rows) + 1);
    const size_t nb = static_cast<size_t>(h->num_blocks > 0 ? h->num_blocks : 1);
    int rc = from_hip(hipMalloc(&out.row_ptr, rp), "hipMalloc");
    if (rc == SPMM_OK) rc = from_hip(hipMalloc(&out.col_idx, sizeof(int) * nb), "hipMalloc");
    if (rc == SPMM_OK) rc = from_hip(hipMalloc(&out.values, sizeof(uint16_t) * 256 * nb), "hipMalloc");
    if (rc == SPMM_OK) {
        rc = from_hip(hipMemcpy(out.row_ptr, h->row_ptr, rp, hipMemcpyHostToDevice), "hipMemcpy");
    }
    if (rc == SPMM_OK && h->num_blocks > 0) {
        rc = from_hip(hipMemcpy(out.col_idx, h->col_idx, sizeof(int) * h->num_blocks,
                                hipMemcpyHostToDevice), "hipMemcpy");
        if (rc == SPMM_OK) {
            rc = from_hip(hipMemcpy(out.values, h->values,
                                    sizeof(uint16_t) * 256 * static_cast<size_t>(h->num_blocks),
                                    hipMemcpyHostToDevice), "hipMemcpy");
        }
    }
    if (rc != SPMM_OK) {
        (void)hipFree(out.row_ptr);
        (void)hipFree(out.col_idx);
        (void)hipFree(out.values);
        return rc;
    }
    *d = out;
    return ok();
}

int spmm_c_bsr_free_device(spmm_bsr_t* d) {
    if (d == nullptr) return ok();
    int rc = SPMM_OK;
    if (d->row_ptr) rc |= from_hip(hipFree(d->row_ptr), "hipFree");
    if (d->col_idx) rc |= from_hip(hipFree(d->col_idx), "hipFree");
    if (d->values) rc |= from_hip(hipFree(d->values), "hipFree");
    d->row_ptr = nullptr;
    d->col_idx = nullptr;
    d->values  = nullptr;
    return rc == SPMM_OK ? ok() : SPMM_HIP_ERROR;
}

int spmm_c_bsr_compute_stats(const spmm_bsr_t* h, spmm_bsr_stats_t* out) {
    if (h == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    spmm::BSR_host b;  // statistics only read the scalar fields
    b.num_rows   = h->num_rows;
    b.num_cols   = h->num_cols;
    b.block_rows = h->block_rows;
    b.block_cols = h->block_cols;
    b.num_blocks = h->num_blocks;
    b.nnz        = h->nnz;
    const spmm::BSR_stats s = spmm::bsr_compute_stats(b);
    out->num_blocks      = s.num_blocks;
    out->stored_elements = s.stored_elements;
    out->original_nnz    = s.original_nnz;
    out->fill_in_ratio   = s.fill_in_ratio;
    out->block_density   = s.block_density;
    return ok();
}

namespace {

void stats_to_c(const spmm::BSR_stats& s, spmm_bsr_stats_t* out) {
    out->num_blocks      = s.num_blocks;
    out->stored_elements = s.stored_elements;
    out->original_nnz    = s.original_nnz;
    out->fill_in_ratio   = s.fill_in_ratio;
    out->block_density   = s.block_density;
}

}  // namespace

int spmm_c_bsr_stats_from_csr_host(const spmm_csr_t* h, spmm_bsr_stats_t* out) {
    if (h == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        stats_to_c(spmm::bsr_stats_from_csr_host(to_cpp(*h)), out);
        return ok();
    });
}

int spmm_c_bsr_from_csr_device(const spmm_csr_t* d_A, spmm_bsr_t* d_out, void* stream) {
    if (d_A == nullptr || d_out == nullptr) return set_error(SPMM_INVALID, "null argument");
    spmm::BSR b;
    const int rc = from_engine(spmm::engine::build_bsr_device(to_cpp(*d_A), &b, as_stream(stream)));
    if (rc != SPMM_OK) return rc;
    spmm_bsr_t r;
    r.num_rows   = b.num_rows;
    r.num_cols   = b.num_cols;
    r.block_rows = b.block_rows;
    r.block_cols = b.block_cols;
    r.num_blocks = b.num_blocks;
    r.nnz        = b.nnz;
    r.row_ptr    = b.row_ptr;
    r.col_idx    = b.col_idx;
    r.values     = reinterpret_cast<uint16_t*>(b.values);
    *d_out = r;
    return ok();
}

int spmm_c_bsr_stats_from_csr_device(const spmm_csr_t* d_A, spmm_bsr_stats_t* out, void* stream) {
    if (d_A == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    spmm::BSR_stats s{};
    const int rc = from_engine(spmm::engine::bsr_stats_device(to_cpp(*d_A), &s, as_stream(stream)));
    if (rc != SPMM_OK) return rc;
    stats_to_c(s, out);
    return ok();
}

int spmm_c_bsr_to_host(const spmm_bsr_t* d, spmm_bsr_t* h_out) {
    if (d == nullptr || h_out == nullptr || d->block_rows < 0 || d->num_blocks < 0) {
        return set_error(SPMM_INVALID, "spmm_c_bsr_to_host: bad argument");
    }
    spmm_bsr_t r = *d;
    const size_t rp = static_cast<size_t>(d->block_rows) + 1;
    const size_t nb = static_cast<size_t>(d->num_blocks);
    r.row_ptr = static_cast<int*>(std::malloc(sizeof(int) * rp));
    r.col_idx = static_cast<int*>(std::malloc(sizeof(int) * std::max<size_t>(nb, 1)));
    r.values  = static_cast<uint16_t*>(std::malloc(sizeof(uint16_t) * std::max<size_t>(nb * 256, 1)));
    if (r.row_ptr == nullptr || r.col_idx == nullptr || r.values == nullptr) {
        spmm_c_bsr_free_host(&r);
        return set_error(SPMM_NO_MEMORY, "spmm_c_bsr_to_host: out of host memory");
    }
    int rc = from_hip(hipMemcpy(r.row_ptr, d->row_ptr, sizeof(int) * rp, hipMemcpyDeviceToHost),
                      "hipMemcpy");
    if (rc == SPMM_OK && nb > 0) {
        rc = from_hip(hipMemcpy(r.col_idx, d->col_idx, sizeof(int) * nb, hipMemcpyDeviceToHost),
                      "hipMemcpy");
        if (rc == SPMM_OK) {
            rc = from_hip(hipMemcpy(r.values, d->values, sizeof(uint16_t) * nb * 256,
                                    hipMemcpyDeviceToHost), "hipMemcpy");
        }
    }
    if (rc != SPMM_OK) {
        spmm_c_bsr_free_host(&r);
        return rc;
    }
    *h_out = r;
    return ok();
}

// ---- synthetic inputs ----------------------------------------------------------

int spmm_c_generate_dense_row_major(int rows, int cols, int seed, float* out) {
    if (out == nullptr && static_cast<long>(rows) * cols > 0) {
        return set_error(SPMM_INVALID, "null output");
    }
    return guarded([&] {
        const std::vector<float> v = spmm::generate_dense_row_major(rows, cols, seed);
        if (!v.empty()) std::memcpy(out, v.data(), sizeof(float) * v.size());
        return ok();
    });
}

int spmm_c_generate_banded_csr(int rows, int cols, int hb, int seed, spmm_csr_t* out) {
    if (out == nullptr) return set_error(SPMM_INVALID, "null output");
    return guarded([&] {
        *out = to_c(spmm::generate_banded_csr(rows, cols, hb, seed));
        return ok();
    });
}

int spmm_c_generate_block_diagonal_csr(int rows, int cols, int block, int seed, float scale,
                                       spmm_csr_t* out) {
    if (out == nullptr) return set_error(SPMM_INVALID, "null output");
    return guarded([&] {
        *out = to_c(spmm::generate_block_diagonal_csr(rows, cols, block, seed, scale));
        return ok();
    });
}

int spmm_c_generate_block_diagonal_uniform_csr(int rows, int cols, int block, int seed,
                                               spmm_csr_t* out) {
    if (out == nullptr) return set_error(SPMM_INVALID, "null output");
    return guarded([&] {
        *out = to_c(spmm::generate_block_diagonal_uniform_csr(rows, cols, block, seed));
        return ok();
    });
}

int spmm_c_generate_power_law_csr(int rows, int cols, double mean_deg, double alpha, int cap,
                                  int seed, spmm_csr_t* out) {
    if (out == nullptr) return set_error(SPMM_INVALID, "null output");
    return guarded([&] {
        *out = to_c(spmm::generate_power_law_csr(rows, cols, mean_deg, alpha, cap, seed));
        return ok();
    });
}

int spmm_c_round_to_fp16(float* v, long n) {
    if (n < 0 || (n > 0 && v == nullptr)) return set_error(SPMM_INVALID, "bad argument");
    spmm::dense_round_to_fp16(v, n);
    return ok();
}

// ---- partition and metrics ------------------------------------------------

int spmm_c_nnz_balanced_bounds(const spmm_csr_t* h, int parts, int* out) {
    if (h == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        const std::vector<int> b = spmm::nnz_balanced_bounds(to_cpp(*h), parts);
        std::memcpy(out, b.data(), sizeof(int) * b.size());
        return ok();
    });
}

int spmm_c_nnz_split_rows(const spmm_csr_t* h, int parts, int* out) {
    if (h == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    return guarded([&] {
        const std::vector<int> r = spmm::nnz_split_rows(to_cpp(*h), parts);
        std::memcpy(out, r.data(), sizeof(int) * r.size());
        return ok();
    });
}

int spmm_c_compare(const float* ours, const float* ref, long n, float* max_abs, float* max_rel,
                   float* rel_l2) {
    if (n < 0 || (n > 0 && (ours == nullptr || ref == nullptr))) {
        return set_error(SPMM_INVALID, "bad argument");
    }
    return guarded([&] {
        const std::vector<float> a(ours, ours + n), b(ref, ref + n);
        const spmm::ErrorStats s = spmm::compare(a, b);
        if (max_abs) *max_abs = s.max_abs;
        if (max_rel) *max_rel = s.max_rel;
        if (rel_l2) *rel_l2 = s.rel_l2;
        return ok();
    });
}

int spmm_c_host_reference_f64(const spmm_csr_t* h_A, const float* h_B, int N, int threads,
                              float* h_C) {
    if (h_A == nullptr || h_C == nullptr || N < 0) return set_error(SPMM_INVALID, "bad argument");
    return guarded([&] {
        const std::vector<float> c = spmm::spmm_host_reference_f64(to_cpp(*h_A), h_B, N, threads);
        if (!c.empty()) std::memcpy(h_C, c.data(), sizeof(float) * c.size());
        return ok();
    });
}

int spmm_c_host_reference_bsr_f32(const spmm_bsr_t* h_A, const float* h_B, int N, int threads,
                                  float* h_C) {
    if (h_A == nullptr || h_C == nullptr || N < 0) return set_error(SPMM_INVALID, "bad argument");
    return guarded([&] {
        const std::vector<float> c =
            spmm::spmm_host_reference_bsr_f32(host_bsr_from_c(*h_A), h_B, N, threads);
        if (!c.empty()) std::memcpy(h_C, c.data(), sizeof(float) * c.size());
        return ok();
    });
}

// ---- kernel entry points -----------------------------------------------------

#define SPMM_C_CSR_ENTRY(fn, id)                                                          \
    int fn(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N, void* stream) {    \
        return launch_id(id, d_A, d_B, d_C, N, stream);                                    \
    }

SPMM_C_CSR_ENTRY(spmm_c_baseline, 0)
SPMM_C_CSR_ENTRY(spmm_c_memopt, 1)
SPMM_C_CSR_ENTRY(spmm_c_memopt_v2, 2)
SPMM_C_CSR_ENTRY(spmm_c_tiled, 3)
SPMM_C_CSR_ENTRY(spmm_c_tiled_v2, 4)
SPMM_C_CSR_ENTRY(spmm_c_tiled_v3, 5)
SPMM_C_CSR_ENTRY(spmm_c_tiled_v4, 6)

#undef SPMM_C_CSR_ENTRY

int spmm_c_tiled_v3_partitioned(const spmm_csr_t* d_A, const int* d_bounds, int parts,
                                const float* d_B, float* d_C, int N, void* stream) {
    if (d_A == nullptr || d_bounds == nullptr) return set_error(SPMM_INVALID, "null argument");
    return from_engine(spmm::engine::launch_csr(spmm::engine::CsrRole::TiledV3, to_cpp(*d_A),
                                                d_B, d_C, N, as_stream(stream), d_bounds, parts));
}

int spmm_c_default_partition_parts(int num_rows, int nnz) {
    return spmm::engine::default_partition_parts(num_rows, nnz);
}

int spmm_c_tiled_v3_split(const spmm_csr_t* d_A, const int* d_split_rows, int parts,
                          const float* d_B, float* d_C, int N, float* d_carry, void* stream) {
    if (d_A == nullptr || d_split_rows == nullptr) return set_error(SPMM_INVALID, "null argument");
    spmm::engine::SplitPlan plan;
    plan.rows  = d_split_rows;
    plan.parts = parts;
    plan.carry = d_carry;
    return from_engine(spmm::engine::launch_csr_split(to_cpp(*d_A), d_B, d_C, N,
                                                      as_stream(stream), plan));
}

int spmm_c_tiled_v3_split_noalloc(const spmm_csr_t* d_A, const int* d_split_rows, int parts,
                                  const float* d_B, float* d_C, int N, void* stream) {
    if (d_A == nullptr || d_split_rows == nullptr) return set_error(SPMM_INVALID, "null argument");
    return from_engine(spmm::engine::launch_csr_split_noalloc(to_cpp(*d_A), d_split_rows, parts,
                                                              d_B, d_C, N, as_stream(stream)));
}

int spmm_c_split_partition_parts(int nnz) { return spmm::engine::split_partition_parts(nnz); }

int spmm_c_csr_auto_form(const spmm_csr_t* h, int N, int* form_out, spmm_engine_opts_t* opts_out,
                         int* parts_out) {
    if (h == nullptr || form_out == nullptr || opts_out == nullptr || parts_out == nullptr) {
        return set_error(SPMM_INVALID, "null argument");
    }
    if (N < 0 || h->num_rows < 0 || h->nnz < 0 || (h->num_rows > 0 && h->row_ptr == nullptr) ||
        (h->nnz > 0 && h->col_idx == nullptr)) {
        return set_error(SPMM_INVALID, "bad CSR or N");
    }
    const spmm::engine::CsrChoice ch = spmm::engine::choose_csr_form(to_cpp(*h), N);
    *form_out  = ch.form == spmm::engine::CsrForm::RowGroups ? 1
                 : ch.form == spmm::engine::CsrForm::Split   ? 2
                 : ch.form == spmm::engine::CsrForm::KHalf   ? 3
                                                             : 0;
    *opts_out  = spmm_engine_opts_t{};
    opts_out->row_groups   = ch.opts.row_groups;
    opts_out->max_row_hint = ch.opts.max_row_hint;
    *parts_out = ch.parts;
    return ok();
}

struct spmm_khalf_plan {
    spmm::engine::KHalfPlan p;
};

int spmm_c_khalf_plan_create(const spmm_csr_t* h_A, int N, spmm_khalf_plan_t** plan_out) {
    if (h_A == nullptr || plan_out == nullptr) return set_error(SPMM_INVALID, "null argument");
    *plan_out = nullptr;
    spmm_khalf_plan_t* plan = new (std::nothrow) spmm_khalf_plan_t;
    if (plan == nullptr) return set_error(SPMM_INVALID, "out of host memory");
    const int rc = from_engine(spmm::engine::khalf_plan_build(to_cpp(*h_A), N, &plan->p));
    if (rc != SPMM_OK) {
        delete plan;
        return rc;
    }
    *plan_out = plan;
    return ok();
}

int spmm_c_khalf_launch(const spmm_khalf_plan_t* plan, const float* d_B, float* d_C,
                        void* stream) {
    if (plan == nullptr) return set_error(SPMM_INVALID, "null plan");
    return from_engine(spmm::engine::launch_csr_khalf(plan->p, d_B, d_C, as_stream(stream)));
}

void spmm_c_khalf_plan_destroy(spmm_khalf_plan_t* plan) {
    if (plan == nullptr) return;
    spmm::engine::khalf_plan_free(&plan->p);
    delete plan;
}

int spmm_c_khalf_runs(const int* row_ptr, int M, long long nnz, const int* split_rows, int parts,
                      int* first_out, int* last_out) {
    if (M < 0 || nnz < 0 || parts < 1) return set_error(SPMM_INVALID, "bad size");
    if ((M > 0 && (row_ptr == nullptr || first_out == nullptr || last_out == nullptr)) ||
        split_rows == nullptr) {
        return set_error(SPMM_INVALID, "null argument");
    }
    spmm::engine::khalf_runs(row_ptr, M, nnz, split_rows, parts, first_out, last_out);
    return ok();
}

struct spmm_bsr_tile_plan {
    spmm::engine::BsrTilePlan p;
};

int spmm_c_bsr_tile_plan_create(const spmm_bsr_t* d_A, int rows_per_panel, void* stream,
                                spmm_bsr_tile_plan_t** plan_out) {
    if (d_A == nullptr || plan_out == nullptr) return set_error(SPMM_INVALID, "null argument");
    *plan_out = nullptr;
    spmm_bsr_tile_plan_t* plan = new (std::nothrow) spmm_bsr_tile_plan_t;
    if (plan == nullptr) return set_error(SPMM_NO_MEMORY, "host allocation failed");
    const int rc = guarded([&] {
        return from_engine(spmm::engine::bsr_tile_plan_build(to_cpp(*d_A), rows_per_panel,
                                                             &plan->p, as_stream(stream)));
    });
    if (rc != SPMM_OK) {
        spmm::engine::bsr_tile_plan_free(&plan->p);
        delete plan;
        return rc;
    }
    *plan_out = plan;
    return ok();
}

int spmm_c_bsr_tile_launch(const spmm_bsr_tile_plan_t* plan, const spmm_bsr_t* d_A,
                           const uint16_t* d_B_fp16, float* d_C, int N, int shape,
                           void* stream) {
    if (plan == nullptr || d_A == nullptr) return set_error(SPMM_INVALID, "null argument");
    return from_engine(spmm::engine::launch_bsr_tile(plan->p, to_cpp(*d_A),
                                                     reinterpret_cast<const half*>(d_B_fp16),
                                                     d_C, N, as_stream(stream), shape));
}

void spmm_c_bsr_tile_plan_destroy(spmm_bsr_tile_plan_t* plan) {
    if (plan == nullptr) return;
    spmm::engine::bsr_tile_plan_free(&plan->p);
    delete plan;
}

int spmm_c_bsr_tile_plan_info(const spmm_bsr_tile_plan_t* plan, int* panels_out,
                              int* rows_per_panel_out, int* max_union_out) {
    if (plan == nullptr) return set_error(SPMM_INVALID, "null plan");
    if (panels_out) *panels_out = plan->p.panels;
    if (rows_per_panel_out) *rows_per_panel_out = plan->p.R;
    if (max_union_out) *max_union_out = plan->p.max_union;
    return ok();
}

int spmm_c_bsr_tile_records(const int* row_ptr, const int* col_idx, int block_rows,
                            int block_cols, int rows_per_panel, int* records_out,
                            int* max_union_out) {
    if (row_ptr == nullptr || records_out == nullptr || max_union_out == nullptr ||
        (block_rows > 0 && row_ptr[block_rows] > 0 && col_idx == nullptr)) {
        return set_error(SPMM_INVALID, "null argument");
    }
    return guarded([&] {
        std::vector<int> desc;
        int mu = 0;
        const int rc = from_engine(spmm::engine::bsr_tile_plan_from_host(
            row_ptr, col_idx, block_rows, block_cols, rows_per_panel, &desc, &mu));
        if (rc != SPMM_OK) return rc;
        std::copy(desc.begin(), desc.end(), records_out);
        *max_union_out = mu;
        return ok();
    });
}

int spmm_c_bsr_tile_shape_count(void) { return spmm::engine::tile_shape_count(); }

int spmm_c_bsr_tile_shape(int id, int* fields_out) {
    if (fields_out == nullptr) return set_error(SPMM_INVALID, "null argument");
    if (id < 0 || id >= spmm::engine::tile_shape_count()) {
        return set_error(SPMM_INVALID, "unknown tile shape");
    }
    const spmm::engine::TileShape& t = spmm::engine::kTileShapes[id];
    const int f[6] = {t.R, t.NT, t.WC, t.CS, t.NB, t.KIND};
    std::copy(f, f + 6, fields_out);
    return ok();
}

int spmm_c_bsr_tile_default_shape(const spmm_bsr_tile_plan_t* plan, int N) {
    if (plan == nullptr) return set_error(SPMM_INVALID, "null plan");
    return spmm::engine::default_tile_shape(plan->p.R, plan->p.max_union, plan->p.num_rows, N);
}

int spmm_c_launch_repeat_bsr_tile(const spmm_bsr_tile_plan_t* plan, const spmm_bsr_t* d_A,
                                  const uint16_t* d_B_fp16, float* d_C, int N, int shape,
                                  int reps, void* stream) {
    if (plan == nullptr || d_A == nullptr) return set_error(SPMM_INVALID, "null argument");
    const spmm::BSR A = to_cpp(*d_A);
    for (int i = 0; i < reps; ++i) {
        const int rc = from_engine(spmm::engine::launch_bsr_tile(
            plan->p, A, reinterpret_cast<const half*>(d_B_fp16), d_C, N, as_stream(stream),
            shape));
        if (rc != SPMM_OK) return rc;
    }
    return ok();
}

int spmm_c_tiled_v3_opts(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                         const spmm_engine_opts_t* opts, void* stream) {
    if (d_A == nullptr) return set_error(SPMM_INVALID, "null argument");
    const spmm::engine::EngineOpts o = opts_from_c(opts);
    return from_engine(spmm::engine::launch_csr(spmm::engine::CsrRole::TiledV3, to_cpp(*d_A),
                                                d_B, d_C, N, as_stream(stream), nullptr, 0, &o));
}

int spmm_c_shader_clock_trace(uint64_t* d_out, int samples, int interval_ticks, void* stream) {
    return from_engine(spmm::engine::launch_shader_clock_trace(
        reinterpret_cast<unsigned long long*>(d_out), samples, interval_ticks, as_stream(stream)));
}

int spmm_c_float_to_half(const float* d_src, uint16_t* d_dst, long n, void* stream) {
    return from_engine(spmm::engine::launch_float_to_half(d_src, reinterpret_cast<half*>(d_dst),
                                                          n, as_stream(stream)));
}

int spmm_c_wmma(const spmm_bsr_t* d_bsr, const uint16_t* d_B16, float* d_C, int N,
                void* stream) {
    return launch_id(7, d_bsr, d_B16, d_C, N, stream);
}

int spmm_c_wmma_opts(const spmm_bsr_t* d_bsr, const uint16_t* d_B16, float* d_C, int N,
                     const spmm_bsr_opts_t* opts, void* stream) {
    if (d_bsr == nullptr) return set_error(SPMM_INVALID, "null matrix descriptor");
    spmm::engine::BsrOpts o;
    if (opts != nullptr) {
        if (opts->reserved0 != 0 || opts->reserved1 != 0) {
            return set_error(SPMM_INVALID,
                             "spmm_bsr_opts_t reserved fields must be 0 (the multi-row and "
                             "split-K wave variants were removed)");
        }
        o.row_group = opts->row_group;
        o.tiles     = opts->tiles;
        o.per_wave  = opts->per_wave;
        o.depth     = opts->depth;
        o.xcd_order = opts->xcd_order;
        o.addressing = opts->addressing;
    }
    return from_engine(spmm::engine::launch_bsr(to_cpp(*d_bsr),
                                                reinterpret_cast<const half*>(d_B16), d_C, N,
                                                as_stream(stream), &o));
}

int spmm_c_launch_repeat_wmma_opts(const spmm_bsr_t* d_bsr, const uint16_t* d_B16, float* d_C,
                                   int N, const spmm_bsr_opts_t* opts, int reps, void* stream) {
    for (int i = 0; i < reps; ++i) {
        const int rc = spmm_c_wmma_opts(d_bsr, d_B16, d_C, N, opts, stream);
        if (rc != SPMM_OK) return rc;
    }
    return ok();
}

// ---- hybrid ------------------------------------------------------------------

namespace {
// A host CSR whose arrays the host-in entry points may read: non-negative
// sizes, row_ptr present, and (with entries) col_idx, plus values when the
// numbers are used.  The C++ API trusts its caller as the reference does.
bool host_csr_ok(const spmm_csr_t& h, bool values) {
    return h.num_rows >= 0 && h.num_cols >= 0 && h.nnz >= 0 && h.row_ptr != nullptr &&
           (h.nnz == 0 || (h.col_idx != nullptr && (!values || h.values != nullptr)));
}
}  // namespace

float spmm_c_hybrid_default_threshold(void) { return spmm::kHybridDefaultThreshold; }
float spmm_c_hybrid_default_threshold_for(int N) { return spmm::hybrid_default_threshold(N); }

int spmm_c_hybrid_choose(const spmm_csr_t* h_A, int N, float thr, spmm_hybrid_plan_t* out) {
    if (h_A == nullptr || out == nullptr) return set_error(SPMM_INVALID, "null argument");
    if (!host_csr_ok(*h_A, false)) return set_error(SPMM_INVALID, "bad host CSR");
    return guarded([&] {
        const spmm::HybridPlan p = spmm::hybrid_choose(to_cpp(*h_A), N, thr);
        out->backend       = p.backend == spmm::Backend::TENSOR_WMMA ? SPMM_BACKEND_WMMA
                                                                      : SPMM_BACKEND_CSR;
        out->fill_in_ratio = p.fill_in_ratio;
        out->block_density = p.block_density;
        out->threshold     = p.threshold;
        out->n_aligned     = p.n_aligned ? 1 : 0;
        out->reason        = p.reason;
        return ok();
    });
}

const char* spmm_c_backend_name(int backend) {
    return spmm::backend_name(backend == SPMM_BACKEND_WMMA ? spmm::Backend::TENSOR_WMMA
                                                           : spmm::Backend::CSR_TILED);
}

int spmm_c_hybrid_run(const spmm_hybrid_plan_t* plan, const spmm_csr_t* h_A, const float* h_B,
                      float* h_C, int N, int warmup, int iters, float* ms_out) {
    if (plan == nullptr || h_A == nullptr || h_C == nullptr || N < 0 || warmup < 0 ||
        iters < 0) {
        return set_error(SPMM_INVALID, "bad argument");
    }
    if (!host_csr_ok(*h_A, true)) return set_error(SPMM_INVALID, "bad host CSR");
    if (h_B == nullptr && static_cast<long>(h_A->num_cols) * N > 0) {
        return set_error(SPMM_INVALID, "null B");
    }
    return guarded([&] {
        spmm::HybridPlan p;
        p.backend       = plan->backend == SPMM_BACKEND_WMMA ? spmm::Backend::TENSOR_WMMA
                                                             : spmm::Backend::CSR_TILED;
        p.fill_in_ratio = plan->fill_in_ratio;
        p.block_density = plan->block_density;
        p.threshold     = plan->threshold;
        p.n_aligned     = plan->n_aligned != 0;
        p.reason        = plan->reason ? plan->reason : "";
        float ms = 0.f;
        const int rc = from_engine(
            spmm::engine::run_hybrid(p, to_cpp(*h_A), h_B, h_C, N, warmup, iters, &ms));
        if (rc == SPMM_OK && ms_out) *ms_out = ms;
        return rc;
    });
}

int spmm_c_gpu_count(void) {
    int n = 0;
    return hipGetDeviceCount(&n) == hipSuccess ? n : 0;
}

int spmm_c_unified(const spmm_csr_t* h_A, const float* h_B, float* h_C, int N, int warmup,
                   int iters, float* ms_out, int* prefetched_out) {
    if (h_A == nullptr || h_C == nullptr || N < 0 || warmup < 0 || iters < 0) {
        return set_error(SPMM_INVALID, "bad argument");
    }
    if (!host_csr_ok(*h_A, true)) return set_error(SPMM_INVALID, "bad host CSR");
    if (h_B == nullptr && static_cast<long>(h_A->num_cols) * N > 0) {
        return set_error(SPMM_INVALID, "null B");
    }
    return guarded([&] {
        float ms = 0.f;
        int residency = spmm::engine::kUnifiedPrefetched;
        const int rc = from_engine(spmm::engine::run_unified(to_cpp(*h_A), h_B, h_C, N, warmup,
                                                             iters, &ms, &residency));
        if (rc == SPMM_OK) {
            if (ms_out) *ms_out = ms;
            if (prefetched_out) *prefetched_out = residency;
        }
        return rc;
    });
}

// ---- measurement helpers -------------------------------------------------------

int spmm_c_launch_repeat(int kernel_id, const void* d_A_any, const void* d_B, float* d_C, int N,
                         int reps, void* stream) {
    for (int i = 0; i < reps; ++i) {
        const int rc = launch_id(kernel_id, d_A_any, d_B, d_C, N, stream);
        if (rc != SPMM_OK) return rc;
    }
    return ok();
}

int spmm_c_launch_repeat_opts(const spmm_csr_t* d_A, const float* d_B, float* d_C, int N,
                              const spmm_engine_opts_t* opts, int reps, void* stream) {
    if (d_A == nullptr) return set_error(SPMM_INVALID, "null argument");
    const spmm::engine::EngineOpts o = opts_from_c(opts);
    const spmm::CSR A = to_cpp(*d_A);
    for (int i = 0; i < reps; ++i) {
        const int rc = from_engine(spmm::engine::launch_csr(
            spmm::engine::CsrRole::TiledV3, A, d_B, d_C, N, as_stream(stream), nullptr, 0, &o));
        if (rc != SPMM_OK) return rc;
    }
    return ok();
}

int spmm_c_launch_repeat_khalf(const spmm_khalf_plan_t* plan, const float* d_B, float* d_C,
                               int reps, void* stream) {
    if (plan == nullptr) return set_error(SPMM_INVALID, "null plan");
    for (int i = 0; i < reps; ++i) {
        const int rc = from_engine(
            spmm::engine::launch_csr_khalf(plan->p, d_B, d_C, as_stream(stream)));
        if (rc != SPMM_OK) return rc;
    }
    return ok();
}

int spmm_c_launch_repeat_split(const spmm_csr_t* d_A, const int* d_split_rows, int parts,
                               const float* d_B, float* d_C, int N, float* d_carry, int reps,
                               void* stream) {
    if (d_A == nullptr || d_split_rows == nullptr) return set_error(SPMM_INVALID, "null argument");
    spmm::engine::SplitPlan plan;
    plan.rows  = d_split_rows;
    plan.parts = parts;
    plan.carry = d_carry;
    const spmm::CSR A = to_cpp(*d_A);
    for (int i = 0; i < reps; ++i) {
        const int rc = from_engine(
            spmm::engine::launch_csr_split(A, d_B, d_C, N, as_stream(stream), plan));
        if (rc != SPMM_OK) return rc;
    }
    return ok();
}

int spmm_c_time_repeat(int kernel_id, const void* d_A_any, const void* d_B, float* d_C, int N,
                       int reps, void* stream, float* ms_out) {
    if (ms_out == nullptr || reps < 1) return set_error(SPMM_INVALID, "bad argument");
    hipEvent_t e0, e1;
    int rc = from_hip(hipEventCreate(&e0), "hipEventCreate");
    if (rc != SPMM_OK) return rc;
    rc = from_hip(hipEventCreate(&e1), "hipEventCreate");
    if (rc != SPMM_OK) {
        (void)hipEventDestroy(e0);
        return rc;
    }
    rc = from_hip(hipEventRecord(e0, as_stream(stream)), "hipEventRecord");
    if (rc == SPMM_OK) rc = spmm_c_launch_repeat(kernel_id, d_A_any, d_B, d_C, N, reps, stream);
    if (rc == SPMM_OK) rc = from_hip(hipEventRecord(e1, as_stream(stream)), "hipEventRecord");
    if (rc == SPMM_OK) rc = from_hip(hipEventSynchronize(e1), "hipEventSynchronize");
    if (rc == SPMM_OK) rc = from_hip(hipEventElapsedTime(ms_out, e0, e1), "hipEventElapsedTime");
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return rc;
}

int spmm_c_device_synchronize(void) { return from_hip(hipDeviceSynchronize(), "hipDeviceSynchronize"); }

}  // extern "C"
