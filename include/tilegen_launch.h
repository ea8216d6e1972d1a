/*
 * tilegen_launch.h -- the per-kernel launch ABI every generated HIP variant
 * library exports (one shared object per (kernel, schedule), produced by
 * tilegen_amd.verify.compile_generated).
 *
 * The launch_* entry points are the reference's plugin interface for the CSR
 * hot path (spmv, spmm, sddmm) and for the two standard kernels around it
 * (fused_spmv_axpy, axpy), with identical argument order and types: each reference
 * variant is one `extern "C" void launch_<name>(...)` (reference
 * tilegen/codegen.py:226-280 `_abi`, :814-818; ctypes argtypes at
 * tilegen/verify.py:166-173 `_SIGNATURES`; dlsym binding at
 * cpp/src/harness.cpp:130-141).
 *
 * Contract (same as the reference's device path, verify.py:155-163):
 *   - every pointer is a device pointer the caller allocated;
 *   - indptr has M+1 entries; row i's nonzeros are the positions
 *     [indptr[i], indptr[i+1]) of indices/data, so the rows' nonzeros are
 *     [indptr[0], indptr[M]).  indptr[0] may be nonzero: a block of rows of a
 *     larger matrix, passed as a pointer into that matrix's indptr together
 *     with its whole indices/data, as the reference's kernels allow (they walk
 *     rows by indptr alone and never read nnz; tilegen/codegen.py:274,
 *     :593-714);
 *   - indices/data hold at least max(nnz, indptr[M]) entries.  nnz sizes the
 *     launch and changes nothing else: every nnz gives the product, bit for bit
 *     the same whenever nnz >= indptr[M] - indptr[0] (an undercount may sum
 *     some rows in another order).  No position outside [indptr[0], indptr[M])
 *     is used; the merge-path, hybrid and stream SpMV variants and the row
 *     tiles with sorted gathers may load positions below nnz outside it (they
 *     start on nnz's numbers and check them against indptr);
 *   - indptr/indices are never written;
 *   - the call is synchronous (returns after the kernel finished);
 *   - it returns void: a failure is recorded and reported by tg_last_status()
 *     / tg_last_error() of libtgrt (the reference surfaces device errors at
 *     its next synchronizing call);
 *   - spmm: every element of C is written (C = A*B). The reference adds into
 *     C (C += A*B) and all its callers pass C zeroed; both give A*B there.
 *
 * The tgv_* functions let a harness time or stream the same kernel without
 * the synchronizing wrapper.  Launches of one merge-path, hybrid or stream
 * variant share that variant's module scratch: launch_* and tgv_launch_async
 * order each of them after the previous one on any stream, except under HIP
 * graph capture, where the caller must not let a replay overlap an eager launch
 * of the same variant (tgrt.h, tg_graph_begin).
 */
#ifndef TILEGEN_LAUNCH_H
#define TILEGEN_LAUNCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* y[i] = sum_p data[p] * x[indices[p]], p in [indptr[i], indptr[i+1]) */
void launch_spmv(const int64_t* indptr, const int64_t* indices, const double* data,
                 const double* x, double* y, int64_t M, int64_t N, int64_t nnz);

/* C[i,:] = sum_p data[p] * B[indices[p], :]; B is N x K, C is M x K, row-major */
void launch_spmm(const int64_t* indptr, const int64_t* indices, const double* data,
                 const double* B, double* C, int64_t M, int64_t N, int64_t K,
                 int64_t nnz);

/* C[p] = data[p] * sum_k U[i,k] * V[indices[p],k]; U is M x K, V is N x K */
void launch_sddmm(const int64_t* indptr, const int64_t* indices, const double* data,
                  const double* U, const double* V, double* C, int64_t M, int64_t N,
                  int64_t K, int64_t nnz);

/* z[i] = alpha * sum_p data[p] * x[indices[p]] + beta * w[i]  (reference
 * dsl.py fused_spmv_axpy after loop_fusion; argtypes verify.py:170-171) */
void launch_fused_spmv_axpy(const int64_t* indptr, const int64_t* indices, const double* data,
                            const double* x, const double* w, double* z, double alpha,
                            double beta, int64_t M, int64_t N, int64_t nnz);

/* z[i] = alpha * x[i] + beta * w[i]  (reference dsl.py axpy; argtypes verify.py:172) */
void launch_axpy(const double* x, const double* w, double* z, double alpha, double beta,
                 int64_t M);

/* Harness side of a variant library (no counterpart in the reference). */
void* tgv_function(void);                  /* the variant's kernel, current device */
const char* tgv_kernel_name(void);         /* "spmv", "spmm", ... */
/* grid and block of a launch; *lds_bytes is the dynamic LDS to pass, always 0:
 * every generated kernel declares its LDS statically */
int tgv_geometry(int64_t M, int64_t N, int64_t K, int64_t nnz, int64_t* grid,
                 int32_t* block, int32_t* lds_bytes);

/* tgv_launch_async: the same launch, enqueued on `stream` (0 = the null stream)
 * without waiting for it; returns 0 or the libtgrt status.  Each variant library
 * exports one tgv_launch_async whose arguments after the stream are its
 * launch_<name> arguments, so it is bound through the typedef of its kernel
 * (dlsym(lib, "tgv_launch_async") cast to that type).  Launches of one merge-path,
 * hybrid or stream variant are ordered after that variant's previous launch on any
 * stream (they combine row pieces through the module's scratch); a launch
 * captured into a HIP graph skips that ordering, so a graph replay must not overlap
 * an eager launch of the same variant. */
typedef int (*tgv_launch_async_spmv_fn)(void* stream, const int64_t* indptr,
                                        const int64_t* indices, const double* data,
                                        const double* x, double* y, int64_t M, int64_t N,
                                        int64_t nnz);
typedef int (*tgv_launch_async_spmm_fn)(void* stream, const int64_t* indptr,
                                        const int64_t* indices, const double* data,
                                        const double* B, double* C, int64_t M, int64_t N,
                                        int64_t K, int64_t nnz);
typedef int (*tgv_launch_async_sddmm_fn)(void* stream, const int64_t* indptr,
                                         const int64_t* indices, const double* data,
                                         const double* U, const double* V, double* C,
                                         int64_t M, int64_t N, int64_t K, int64_t nnz);
typedef int (*tgv_launch_async_fused_spmv_axpy_fn)(void* stream, const int64_t* indptr,
                                                   const int64_t* indices,
                                                   const double* data, const double* x,
                                                   const double* w, double* z, double alpha,
                                                   double beta, int64_t M, int64_t N,
                                                   int64_t nnz);
typedef int (*tgv_launch_async_axpy_fn)(void* stream, const double* x, const double* w,
                                        double* z, double alpha, double beta, int64_t M);

#ifdef __cplusplus
}
#endif

#endif /* TILEGEN_LAUNCH_H */
