// libtg_vendor: rocSPARSE CSR SpMV, SpMM and SDDMM timed on the same device
// buffers as the generated kernels, for the vendor comparison the reference
// runs against cuSPARSE (reference scripts/compare_cusparse.py:80-96).  Not on
// the product path: nothing in tilegen_amd's launch/verify code calls it.
//
// One entry point per operation, plain C types: each builds one rocSPARSE
// descriptor set per argument set (rotation over input copies, as in
// tg_time_launches), runs the preprocess stage once per set outside the timed
// region, then times `iters` compute calls with hipEvents recorded around each
// call on the handle's stream.
#include <hip/hip_runtime_api.h>
#include <rocsparse/rocsparse.h>

#include <cstdint>
#include <cstdio>
#include <vector>

namespace {
thread_local char g_msg[512] = "";
int fail(int code, const char* what) {
  std::snprintf(g_msg, sizeof(g_msg), "%s failed (%d)", what, code);
  return code ? code : -1;
}

// A rocSPARSE handle on its own non-blocking stream; both are released by the
// destructor, whatever happened in between.
struct Session {
  rocsparse_handle h = nullptr;
  hipStream_t stream = nullptr;
  int rc = 0;
  Session() {
    rocsparse_status st = rocsparse_create_handle(&h);
    if (st != rocsparse_status_success) {
      h = nullptr;
      rc = fail(st, "rocsparse_create_handle");
      return;
    }
    hipError_t e = hipStreamCreateWithFlags(&stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
      stream = nullptr;
      rc = fail(e, "hipStreamCreateWithFlags");
      return;
    }
    st = rocsparse_set_stream(h, stream);
    if (st != rocsparse_status_success) rc = fail(st, "rocsparse_set_stream");
  }
  ~Session() {
    if (h) rocsparse_destroy_handle(h);
    if (stream) (void)hipStreamDestroy(stream);
  }
};

// Shared timing loop: `call(s)` runs one compute call on argument set s
// (launch i uses set i % n_sets); events are recorded around each timed call.
template <typename F>
int time_calls(hipStream_t stream, int n_sets, int warmup, int iters, float* ms_each,
               float* wall_ms, F call) {
  std::vector<hipEvent_t> ev(2 * static_cast<size_t>(iters), nullptr);
  int rc = 0;
  for (auto& e : ev) {
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      e = nullptr;
      rc = fail(err, "hipEventCreate");
      break;
    }
  }
  for (int i = 0; rc == 0 && i < warmup + iters; ++i) {
    const int s = i % n_sets, t = i - warmup;
    if (t >= 0 && hipEventRecord(ev[2 * t], stream) != hipSuccess) rc = fail(-1, "hipEventRecord");
    if (rc == 0) rc = call(s);
    if (rc == 0 && t >= 0 && hipEventRecord(ev[2 * t + 1], stream) != hipSuccess)
      rc = fail(-1, "hipEventRecord");
  }
  // drain whatever was enqueued, also after a failure, before the events go
  hipError_t sync = hipStreamSynchronize(stream);
  if (rc == 0 && sync != hipSuccess) rc = fail(sync, "hipStreamSynchronize");
  for (int t = 0; rc == 0 && t < iters; ++t) {
    hipError_t err = hipEventElapsedTime(&ms_each[t], ev[2 * t], ev[2 * t + 1]);
    if (err != hipSuccess) rc = fail(err, "hipEventElapsedTime");
  }
  if (rc == 0 && wall_ms) {
    hipError_t err = hipEventElapsedTime(wall_ms, ev[0], ev[2 * iters - 1]);
    if (err != hipSuccess) rc = fail(err, "hipEventElapsedTime(wall)");
  }
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}
}  // namespace

extern "C" {

const char* tgv_vendor_last_error(void) { return g_msg; }

// sets: n_sets x 5 device pointers (indptr, indices, data, x, y).
// alg: rocsparse_spmv_alg value (2 adaptive, 3 rowsplit, 7 lrb, 8 nnzsplit).
int tgv_vendor_spmv_time(int alg, int64_t M, int64_t N, int64_t nnz, const uint64_t* sets,
                         int n_sets, int warmup, int iters, float* ms_each, float* wall_ms) {
  if (!sets || n_sets <= 0 || iters <= 0 || warmup < 0 || !ms_each) return fail(-1, "arguments");
  Session ses;
  if (ses.rc) return ses.rc;
  const double alpha = 1.0, beta = 0.0;
  const auto a_alg = (rocsparse_spmv_alg)alg;
  std::vector<rocsparse_spmat_descr> A(n_sets, nullptr);
  std::vector<rocsparse_dnvec_descr> X(n_sets, nullptr), Y(n_sets, nullptr);
  std::vector<void*> buf(n_sets, nullptr);
  std::vector<size_t> bytes(n_sets, 0);
  int rc = 0;
  for (int s = 0; s < n_sets && rc == 0; ++s) {
    const uint64_t* p = sets + 5 * s;
    rocsparse_status st = rocsparse_create_csr_descr(
        &A[s], M, N, nnz, (void*)p[0], (void*)p[1], (void*)p[2], rocsparse_indextype_i64,
        rocsparse_indextype_i64, rocsparse_index_base_zero, rocsparse_datatype_f64_r);
    if (st == rocsparse_status_success)
      st = rocsparse_create_dnvec_descr(&X[s], N, (void*)p[3], rocsparse_datatype_f64_r);
    if (st == rocsparse_status_success)
      st = rocsparse_create_dnvec_descr(&Y[s], M, (void*)p[4], rocsparse_datatype_f64_r);
    if (st == rocsparse_status_success)
      st = rocsparse_spmv(ses.h, rocsparse_operation_none, &alpha, A[s], X[s], &beta, Y[s],
                          rocsparse_datatype_f64_r, a_alg, rocsparse_spmv_stage_buffer_size,
                          &bytes[s], nullptr);
    if (st == rocsparse_status_success && bytes[s]) {
      if (hipMalloc(&buf[s], bytes[s]) != hipSuccess) st = rocsparse_status_memory_error;
    }
    if (st == rocsparse_status_success)
      st = rocsparse_spmv(ses.h, rocsparse_operation_none, &alpha, A[s], X[s], &beta, Y[s],
                          rocsparse_datatype_f64_r, a_alg, rocsparse_spmv_stage_preprocess,
                          &bytes[s], buf[s]);
    if (st != rocsparse_status_success) rc = fail(st, "rocsparse spmv setup");
  }
  if (rc == 0)
    rc = time_calls(ses.stream, n_sets, warmup, iters, ms_each, wall_ms, [&](int s) {
      rocsparse_status r = rocsparse_spmv(ses.h, rocsparse_operation_none, &alpha, A[s], X[s],
                                          &beta, Y[s], rocsparse_datatype_f64_r, a_alg,
                                          rocsparse_spmv_stage_compute, &bytes[s], buf[s]);
      return r == rocsparse_status_success ? 0 : fail(r, "rocsparse_spmv compute");
    });
  (void)hipStreamSynchronize(ses.stream);  // setup work, if timing never ran
  for (int s = 0; s < n_sets; ++s) {
    if (buf[s]) (void)hipFree(buf[s]);
    if (A[s]) rocsparse_destroy_spmat_descr(A[s]);
    if (X[s]) rocsparse_destroy_dnvec_descr(X[s]);
    if (Y[s]) rocsparse_destroy_dnvec_descr(Y[s]);
  }
  return rc;
}

// C = A * B.  sets: n_sets x 5 device pointers (indptr, indices, data, B, C);
// B is N x K and C is M x K, both row-major.  alg: rocsparse_spmm_alg value.
int tgv_vendor_spmm_time(int alg, int64_t M, int64_t N, int64_t K, int64_t nnz,
                         const uint64_t* sets, int n_sets, int warmup, int iters,
                         float* ms_each, float* wall_ms) {
  if (!sets || n_sets <= 0 || iters <= 0 || warmup < 0 || !ms_each) return fail(-1, "arguments");
  Session ses;
  if (ses.rc) return ses.rc;
  const double alpha = 1.0, beta = 0.0;
  const auto a_alg = (rocsparse_spmm_alg)alg;
  std::vector<rocsparse_spmat_descr> A(n_sets, nullptr);
  std::vector<rocsparse_dnmat_descr> B(n_sets, nullptr), C(n_sets, nullptr);
  std::vector<void*> buf(n_sets, nullptr);
  std::vector<size_t> bytes(n_sets, 0);
  int rc = 0;
  for (int s = 0; s < n_sets && rc == 0; ++s) {
    const uint64_t* p = sets + 5 * s;
    rocsparse_status st = rocsparse_create_csr_descr(
        &A[s], M, N, nnz, (void*)p[0], (void*)p[1], (void*)p[2], rocsparse_indextype_i64,
        rocsparse_indextype_i64, rocsparse_index_base_zero, rocsparse_datatype_f64_r);
    if (st == rocsparse_status_success)
      st = rocsparse_create_dnmat_descr(&B[s], N, K, K, (void*)p[3], rocsparse_datatype_f64_r,
                                        rocsparse_order_row);
    if (st == rocsparse_status_success)
      st = rocsparse_create_dnmat_descr(&C[s], M, K, K, (void*)p[4], rocsparse_datatype_f64_r,
                                        rocsparse_order_row);
    if (st == rocsparse_status_success)
      st = rocsparse_spmm(ses.h, rocsparse_operation_none, rocsparse_operation_none, &alpha,
                          A[s], B[s], &beta, C[s], rocsparse_datatype_f64_r, a_alg,
                          rocsparse_spmm_stage_buffer_size, &bytes[s], nullptr);
    if (st == rocsparse_status_success && bytes[s]) {
      if (hipMalloc(&buf[s], bytes[s]) != hipSuccess) st = rocsparse_status_memory_error;
    }
    if (st == rocsparse_status_success)
      st = rocsparse_spmm(ses.h, rocsparse_operation_none, rocsparse_operation_none, &alpha,
                          A[s], B[s], &beta, C[s], rocsparse_datatype_f64_r, a_alg,
                          rocsparse_spmm_stage_preprocess, &bytes[s], buf[s]);
    if (st != rocsparse_status_success) rc = fail(st, "rocsparse spmm setup");
  }
  if (rc == 0)
    rc = time_calls(ses.stream, n_sets, warmup, iters, ms_each, wall_ms, [&](int s) {
      rocsparse_status r = rocsparse_spmm(ses.h, rocsparse_operation_none,
                                          rocsparse_operation_none, &alpha, A[s], B[s], &beta,
                                          C[s], rocsparse_datatype_f64_r, a_alg,
                                          rocsparse_spmm_stage_compute, &bytes[s], buf[s]);
      return r == rocsparse_status_success ? 0 : fail(r, "rocsparse_spmm compute");
    });
  (void)hipStreamSynchronize(ses.stream);
  for (int s = 0; s < n_sets; ++s) {
    if (buf[s]) (void)hipFree(buf[s]);
    if (A[s]) rocsparse_destroy_spmat_descr(A[s]);
    if (B[s]) rocsparse_destroy_dnmat_descr(B[s]);
    if (C[s]) rocsparse_destroy_dnmat_descr(C[s]);
  }
  return rc;
}

// out[p] = (U * V^T)[i, indices[p]] on A's pattern.  rocSPARSE's SDDMM does
// not multiply by A's values (C := alpha (U V^T) o spy(C) + beta C), so the
// vendor call does one multiply per nonzero less than this build's kernel.
// sets: n_sets x 5 device pointers (indptr, indices, U, V, out); U is M x K,
// V is N x K, both row-major (V is read as the column-major K x N matrix V^T).
int tgv_vendor_sddmm_time(int alg, int64_t M, int64_t N, int64_t K, int64_t nnz,
                          const uint64_t* sets, int n_sets, int warmup, int iters,
                          float* ms_each, float* wall_ms) {
  if (!sets || n_sets <= 0 || iters <= 0 || warmup < 0 || !ms_each) return fail(-1, "arguments");
  Session ses;
  if (ses.rc) return ses.rc;
  const double alpha = 1.0, beta = 0.0;
  const auto a_alg = (rocsparse_sddmm_alg)alg;
  std::vector<rocsparse_spmat_descr> C(n_sets, nullptr);
  std::vector<rocsparse_dnmat_descr> Ud(n_sets, nullptr), Vt(n_sets, nullptr);
  std::vector<void*> buf(n_sets, nullptr);
  int rc = 0;
  for (int s = 0; s < n_sets && rc == 0; ++s) {
    const uint64_t* p = sets + 5 * s;
    rocsparse_status st = rocsparse_create_csr_descr(
        &C[s], M, N, nnz, (void*)p[0], (void*)p[1], (void*)p[4], rocsparse_indextype_i64,
        rocsparse_indextype_i64, rocsparse_index_base_zero, rocsparse_datatype_f64_r);
    if (st == rocsparse_status_success)
      st = rocsparse_create_dnmat_descr(&Ud[s], M, K, K, (void*)p[2], rocsparse_datatype_f64_r,
                                        rocsparse_order_row);
    if (st == rocsparse_status_success)
      st = rocsparse_create_dnmat_descr(&Vt[s], K, N, K, (void*)p[3], rocsparse_datatype_f64_r,
                                        rocsparse_order_column);
    size_t bytes = 0;
    if (st == rocsparse_status_success)
      st = rocsparse_sddmm_buffer_size(ses.h, rocsparse_operation_none, rocsparse_operation_none,
                                       &alpha, Ud[s], Vt[s], &beta, C[s],
                                       rocsparse_datatype_f64_r, a_alg, &bytes);
    if (st == rocsparse_status_success && bytes) {
      if (hipMalloc(&buf[s], bytes) != hipSuccess) st = rocsparse_status_memory_error;
    }
    if (st == rocsparse_status_success)
      st = rocsparse_sddmm_preprocess(ses.h, rocsparse_operation_none, rocsparse_operation_none,
                                      &alpha, Ud[s], Vt[s], &beta, C[s],
                                      rocsparse_datatype_f64_r, a_alg, buf[s]);
    if (st != rocsparse_status_success) rc = fail(st, "rocsparse sddmm setup");
  }
  if (rc == 0)
    rc = time_calls(ses.stream, n_sets, warmup, iters, ms_each, wall_ms, [&](int s) {
      rocsparse_status r = rocsparse_sddmm(ses.h, rocsparse_operation_none,
                                           rocsparse_operation_none, &alpha, Ud[s], Vt[s], &beta,
                                           C[s], rocsparse_datatype_f64_r, a_alg, buf[s]);
      return r == rocsparse_status_success ? 0 : fail(r, "rocsparse_sddmm");
    });
  (void)hipStreamSynchronize(ses.stream);
  for (int s = 0; s < n_sets; ++s) {
    if (buf[s]) (void)hipFree(buf[s]);
    if (C[s]) rocsparse_destroy_spmat_descr(C[s]);
    if (Ud[s]) rocsparse_destroy_dnmat_descr(Ud[s]);
    if (Vt[s]) rocsparse_destroy_dnmat_descr(Vt[s]);
  }
  return rc;
}

}  // extern "C"
