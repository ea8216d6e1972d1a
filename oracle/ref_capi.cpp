// ref_capi.cpp -- C entry points over the reference's own sequential kernels.
//
// TEST INFRASTRUCTURE ONLY (see tg_oracle.c).  Compiled together with the
// reference's cpp/src/ref.cpp, where it lies under /root/reference, into
// oracle/_ref/libtilegen_ref.so by oracle/Makefile.  This glue is this
// repository's own code; it only moves pointers into the reference's
// tilegen::Csr<double> / std::vector types (cpp/include/tilegen/ref.hpp:11-43)
// and back.  A handle keeps the matrix and operands resident so repeated calls
// time the reference kernel, not the copies.
#include <chrono>
#include <cstdint>
#include <cstring>
#include <vector>

#include "tilegen/ref.hpp"

namespace {

struct Handle {
  tilegen::Csr<double> A;
  std::vector<double> x, B, U, V, out;
  int64_t K = 0;
};

}  // namespace

extern "C" {

void* ref_create(int64_t rows, int64_t cols, int64_t nnz, const int64_t* indptr,
                 const int64_t* indices, const double* data) {
  Handle* h = new Handle;
  h->A.rows = rows;
  h->A.cols = cols;
  h->A.indptr.assign(indptr, indptr + rows + 1);
  h->A.indices.assign(indices, indices + nnz);
  h->A.data.assign(data, data + nnz);
  return h;
}

void ref_destroy(void* handle) { delete static_cast<Handle*>(handle); }

// Set dense operands: x (cols), B (cols x K), U (rows x K), V (cols x K).
// Any pointer may be null.
void ref_set_operands(void* handle, int64_t K, const double* x, const double* B,
                      const double* U, const double* V) {
  Handle* h = static_cast<Handle*>(handle);
  h->K = K;
  const size_t n = static_cast<size_t>(h->A.cols), m = static_cast<size_t>(h->A.rows);
  if (x) h->x.assign(x, x + n);
  if (B) h->B.assign(B, B + n * K);
  if (U) h->U.assign(U, U + m * K);
  if (V) h->V.assign(V, V + n * K);
}

// Run kernel `which` (0 spmv, 1 spmm, 2 sddmm) `iters` times; copy the last
// result into out (may be null); return seconds per call (steady clock).
double ref_run(void* handle, int which, int iters, double* out) {
  Handle* h = static_cast<Handle*>(handle);
  auto t0 = std::chrono::steady_clock::now();
  for (int it = 0; it < iters; ++it) {
    if (which == 0)
      tilegen::csr_spmv(h->A, h->x, h->out);
    else if (which == 1)
      tilegen::csr_spmm(h->A, h->B, h->K, h->out);
    else
      tilegen::sddmm(h->A, h->U, h->V, h->K, h->out);
  }
  auto t1 = std::chrono::steady_clock::now();
  if (out && !h->out.empty()) std::memcpy(out, h->out.data(), h->out.size() * sizeof(double));
  return std::chrono::duration<double>(t1 - t0).count() / (iters > 0 ? iters : 1);
}

// dense_spmv (ref.cpp:18-28): y = A x, A row-major m x n
void ref_dense_spmv(int64_t m, int64_t n, const double* A, const double* x, double* y) {
  std::vector<double> a(A, A + m * n), xv(x, x + n), yv;
  tilegen::dense_spmv(a, m, n, xv, yv);
  std::memcpy(y, yv.data(), yv.size() * sizeof(double));
}

// fused_spmv_axpy (ref.cpp:61-73)
void ref_fused_spmv_axpy(void* handle, const double* w, double alpha, double beta,
                         double* z) {
  Handle* h = static_cast<Handle*>(handle);
  std::vector<double> wv(w, w + h->A.rows), zv;
  tilegen::fused_spmv_axpy(h->A, h->x, wv, alpha, beta, zv);
  std::memcpy(z, zv.data(), zv.size() * sizeof(double));
}

}  // extern "C"
