/*
 * tg_oracle.c -- CPU restatement of the reference's sequential CSR kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (tilegen_amd/) may call,
 * link or load this file; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg use it, and only as the checker.
 *
 * Each function follows the plain sequential definition of the reference
 * (cpp/src/ref.cpp, templates declared in cpp/include/tilegen/ref.hpp):
 * one accumulator per output, summed in increasing nonzero order, products
 * formed as data * operand.  Built with -ffp-contract=off so every product is
 * rounded before it is added, exactly like the reference compiled without FMA
 * contraction; that makes this file and the reference bit-identical on the
 * same inputs (checked in tests/test_oracle.py against oracle/_ref).
 *
 * Pinning (tests/test_oracle.py): the known-answer tests of
 * cpp/tests/test_ref.cpp:25-116, brute-force dense products on tiny inputs,
 * float64 SciPy, and bit-for-bit agreement with oracle/_ref.
 */
#include <stdint.h>
#include <string.h>

/* y[i] = sum_{p in row i} data[p] * x[indices[p]]   (ref.cpp:6-16 csr_spmv) */
void oracle_csr_spmv(int64_t M, const int64_t* indptr, const int64_t* indices,
                     const double* data, const double* x, double* y) {
  for (int64_t i = 0; i < M; ++i) {
    double acc = 0.0;
    for (int64_t p = indptr[i]; p < indptr[i + 1]; ++p) acc += data[p] * x[indices[p]];
    y[i] = acc;
  }
}

/* y = A x with A dense row-major m x n   (ref.cpp:18-28 dense_spmv) */
void oracle_dense_spmv(int64_t m, int64_t n, const double* A, const double* x, double* y) {
  for (int64_t i = 0; i < m; ++i) {
    double acc = 0.0;
    for (int64_t j = 0; j < n; ++j) acc += A[i * n + j] * x[j];
    y[i] = acc;
  }
}

/* C = A B: C zeroed, then for each nonzero C[i,:] += data[p] * B[j,:]
 * (ref.cpp:31-43 csr_spmm) */
void oracle_csr_spmm(int64_t M, int64_t K, const int64_t* indptr, const int64_t* indices,
                     const double* data, const double* B, double* C) {
  memset(C, 0, (size_t)M * (size_t)K * sizeof(double));
  for (int64_t i = 0; i < M; ++i) {
    for (int64_t p = indptr[i]; p < indptr[i + 1]; ++p) {
      const int64_t j = indices[p];
      const double a = data[p];
      for (int64_t k = 0; k < K; ++k) C[i * K + k] += a * B[j * K + k];
    }
  }
}

/* out[p] = data[p] * sum_k U[i,k] V[j,k]   (ref.cpp:46-59 sddmm) */
void oracle_sddmm(int64_t M, int64_t K, const int64_t* indptr, const int64_t* indices,
                  const double* data, const double* U, const double* V, double* out) {
  for (int64_t i = 0; i < M; ++i) {
    for (int64_t p = indptr[i]; p < indptr[i + 1]; ++p) {
      const int64_t j = indices[p];
      double acc = 0.0;
      for (int64_t k = 0; k < K; ++k) acc += U[i * K + k] * V[j * K + k];
      out[p] = data[p] * acc;
    }
  }
}

/* z[i] = alpha * (A x)[i] + beta * w[i]   (ref.cpp:62-73 fused_spmv_axpy) */
void oracle_fused_spmv_axpy(int64_t M, const int64_t* indptr, const int64_t* indices,
                            const double* data, const double* x, const double* w,
                            double alpha, double beta, double* z) {
  for (int64_t i = 0; i < M; ++i) {
    double acc = 0.0;
    for (int64_t p = indptr[i]; p < indptr[i + 1]; ++p) acc += data[p] * x[indices[p]];
    z[i] = alpha * acc + beta * w[i];
  }
}

/* z[i] = alpha * x[i] + beta * w[i]   (reference verify.py:369-370 axpy) */
void oracle_axpy(int64_t M, const double* x, const double* w, double alpha, double beta,
                 double* z) {
  for (int64_t i = 0; i < M; ++i) z[i] = alpha * x[i] + beta * w[i];
}
