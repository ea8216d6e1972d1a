/*
 * tgrt.h -- TileGen HIP runtime, the C ABI under every generated kernel
 * (libtgrt.so, built from tilegen_amd/csrc/tgrt.cpp for gfx950 hosts).
 *
 * The reference drives its kernels from Python through libcudart via ctypes
 * and an nvcc subprocess (reference tilegen/verify.py:52-163 `_cuda_runtime`,
 * `_CudaBuffers`, `_invoke`; compile at verify.py:264-312). These functions are
 * what replaces that layer: runtime compilation with hipRTC, module loading,
 * kernel launch, device memory and GPU-side timing.
 *
 * Conventions: every function returns 0 on success, otherwise a nonzero code
 * (a hipError_t, a hiprtcResult + 1000, or -1 for an argument error) and
 * records a message readable with tg_last_error() on the calling thread.
 * Pointers named d_* are device pointers. Nothing here allocates behind the
 * caller's back except tg_malloc, the module/function cache of
 * tg_code_function, and the host buffers tg_rtc_compile returns (release those
 * with tg_host_free).
 */
#ifndef TILEGEN_TGRT_H
#define TILEGEN_TGRT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void* tg_module;
typedef void* tg_function;

/* ---- errors (replaces verify.py:93-100 `_cuda_check`) ---- */
const char* tg_last_error(void);
int tg_last_status(void);
void tg_clear_error(void);
/* Records `code` and `message` for tg_last_status/tg_last_error on the calling
 * thread and returns `code`: how libraries layered on libtgrt report. */
int tg_fail(int code, const char* message);

/* ---- devices (replaces env.py:55-83 `_gpu_info` for the HIP backend) ---- */
int tg_device_count(int* count);
int tg_set_device(int device);
int tg_get_device(int* device);
/* name/arch are NUL-terminated into caller buffers of the given lengths */
int tg_device_props(int device, char* name, int name_len, char* arch, int arch_len,
                    int* cu_count, int64_t* global_mem_bytes, int* clock_khz,
                    int* l2_bytes);
int tg_runtime_version(int* hip_version, int* hiprtc_major, int* hiprtc_minor);

/* ---- runtime compilation (replaces the nvcc subprocess, verify.py:279-296) ---- */
/* Compiles `source` with hipRTC. On success *code and *code_size hold the code
 * object; *log (may be NULL on return) holds the compiler log. Both are
 * malloc'd: free with tg_host_free. On a compile error the return is nonzero
 * and *log still carries the diagnostics. */
int tg_rtc_compile(const char* source, const char* name, const char* const* options,
                   int n_options, void** code, size_t* code_size, char** log);
void tg_host_free(void* p);

/* ---- modules and functions ---- */
int tg_module_load(const void* code, size_t code_size, tg_module* module);
int tg_module_unload(tg_module module);
int tg_module_function(tg_module module, const char* name, tg_function* fn);
/* Function `name` of an embedded code object on the current device. Loaded
 * once per (code pointer, device) and kept until tg_code_release. */
int tg_code_function(const void* code, size_t code_size, const char* name,
                     tg_function* fn);
/* Forgets the cached modules of an embedded code object on every device, so
 * that another object later placed at the same address is loaded afresh.
 * Generated launcher libraries call it as they are unloaded.  The modules are
 * not unloaded (this may run during process exit), so this makes no HIP call. */
int tg_code_release(const void* code, size_t code_size);
/* Registers, static LDS bytes, scratch bytes per lane, max lanes per workgroup. */
int tg_function_attrs(tg_function fn, int* num_regs, int* lds_bytes, int* scratch_bytes,
                      int* max_threads);

/* ---- launch (replaces the <<<>>> + cudaDeviceSynchronize of codegen.py:797-798) ---- */
/* One-dimensional launch of `grid` workgroups of `block` lanes. `args` holds
 * one 8-byte slot per kernel parameter (pointer, int64 or double bits).
 * stream NULL = the null stream; sync != 0 waits for completion. */
int tg_launch(tg_function fn, int64_t grid, int32_t block, int32_t lds_bytes,
              const uint64_t* args, int n_args, void* stream, int sync);

/* tg_launch, ordered after the previous launch made with the same order_key on
 * the current device: when that launch went to another stream, `stream` first
 * waits for its end (an event recorded after every such launch).  Generated
 * launchers of kernels that combine row pieces through module scratch pass
 * their embedded code object as the key, so calls that overlap on two streams
 * run one after the other instead of racing on the scratch.  A launch into a
 * stream under graph capture is passed to tg_launch unordered.  No counterpart
 * in the reference, whose launchers are synchronous on the null stream. */
int tg_launch_ordered(const void* order_key, tg_function fn, int64_t grid, int32_t block,
                      int32_t lds_bytes, const uint64_t* args, int n_args, void* stream,
                      int sync);

/* GPU-side timing. Launches `warmup` + `iters` times on `stream`, launch i
 * using argument set (i % n_sets) of `arg_sets` (n_sets x n_args slots), so a
 * caller can rotate among input copies that do not fit in cache together.
 * kernel_ms[i] (iters entries) is the duration of timed launch i as recorded
 * by start/stop events attached to the kernel dispatch itself
 * (hipExtModuleLaunchKernel); *wall_ms is the event time from the first timed
 * launch's start to the last one's end, gaps between kernels included. */
int tg_time_launches(tg_function fn, int64_t grid, int32_t block, int32_t lds_bytes,
                     const uint64_t* arg_sets, int n_args, int n_sets, int warmup,
                     int iters, void* stream, float* kernel_ms, float* wall_ms);

/* Enqueue `iters` launches back to back (launch i uses argument set
 * i % n_sets) without waiting; the caller synchronizes.  The timed region of
 * bench.py. */
int tg_run_launches(tg_function fn, int64_t grid, int32_t block, int32_t lds_bytes,
                    const uint64_t* arg_sets, int n_args, int n_sets, int iters,
                    void* stream);

/* ---- device memory (replaces verify.py:103-142 `_CudaBuffers`) ---- */
int tg_malloc(void** d_ptr, size_t bytes);
int tg_free(void* d_ptr);
int tg_memcpy_htod(void* d_dst, const void* src, size_t bytes);
int tg_memcpy_dtoh(void* dst, const void* d_src, size_t bytes);
int tg_memcpy_dtod(void* d_dst, const void* d_src, size_t bytes);
int tg_memset(void* d_ptr, int value, size_t bytes);
int tg_synchronize(void);

/* ---- streams (default priority only) ---- */
int tg_stream_create(void** stream);
int tg_stream_destroy(void* stream);
int tg_stream_synchronize(void* stream);

/* ---- HIP graphs ----
 * tg_graph_begin starts capturing `stream` (not the null stream; thread-local
 * mode); launches enqueued on it are recorded, not run.  tg_graph_end ends the
 * capture and instantiates the graph into *exec; tg_graph_launch replays it on
 * `stream` (sync != 0 waits); tg_graph_destroy frees it.  The generated
 * launchers' tgv_launch_async and launch_spmv_noalloc may be captured.  A
 * captured launch of a module with scratch is not ordered against that
 * module's eager launches: the caller orders replays and eager calls.  No
 * counterpart in the reference, which has no graph layer. */
int tg_graph_begin(void* stream);
int tg_graph_end(void* stream, void** exec);
int tg_graph_launch(void* exec, void* stream, int sync);
int tg_graph_destroy(void* exec);

#ifdef __cplusplus
}
#endif

#endif /* TILEGEN_TGRT_H */
