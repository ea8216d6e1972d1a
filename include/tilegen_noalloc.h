/*
 * tilegen_noalloc.h -- libtgna.so (tilegen_amd/csrc/spmv_noalloc.hip): an SpMV
 * entry point that allocates nothing.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc.  Same arguments and result as launch_spmv
 * (tilegen_launch.h) at the hybrid-tile schedule T128/TPR4/U2/B512 (row tiles
 * plus long-row workgroups over equal nonzero ranges), plus a stream:
 *
 *   - y[i] = sum_p data[p] * x[indices[p]] over row i; every pointer is a
 *     device pointer the caller allocated; indptr/indices are never written;
 *   - asynchronous: the kernels are enqueued on `stream` (NULL = the null
 *     stream) and the call returns; the caller synchronizes;
 *   - allocates nothing: the long-row partial sums go to a 1 MiB static device
 *     array of the library (131072 slots, one copy per GPU, held until the
 *     process ends).  The first call on a device resolves that device's copy
 *     (hipGetSymbolAddress); make it outside graph capture.  Each call clears
 *     the slots it uses with a small kernel before the SpMV kernel;
 *   - limit: nnz <= 65536 ranges x the schedule's range length (2 x block x
 *     unroll nonzeros: 134,217,728 at the shipped schedule); larger calls are
 *     refused with -2, as are rows beyond one launch's 2^32 work-items;
 *   - calls that overlap on one device (two streams, concurrent graph
 *     replays) share the slots and race: order them;
 *   - returns 0 on success, -1 for a bad argument, -2 for a size beyond the
 *     limit, or a hipError_t; the message is in libtgrt's tg_last_error().
 */
#ifndef TILEGEN_NOALLOC_H
#define TILEGEN_NOALLOC_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

int launch_spmv_noalloc(const int64_t* indptr, const int64_t* indices, const double* data,
                        const double* x, double* y, int64_t M, int64_t N, int64_t nnz,
                        void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TILEGEN_NOALLOC_H */
