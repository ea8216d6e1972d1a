// libtgrt: the TileGen HIP runtime behind every generated kernel.
//
// Runtime compilation (hipRTC), code-object loading, 1-D kernel launch from
// packed 8-byte argument slots, GPU-side timing and device memory, exported as
// the plain C ABI declared in include/tgrt.h.  The reference reaches CUDA
// through ctypes on libcudart plus an nvcc subprocess (reference
// tilegen/verify.py:52-163, :264-312); this library is the HIP-native
// replacement for that whole layer.  Host code only: no device code lives here.
#include "tgrt.h"

#include <hip/hip_runtime_api.h>
#include <hip/hiprtc.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

// From hip/hip_ext.h, whose templated launch helpers need the HIP compiler;
// this file is plain host C++.
extern "C" hipError_t hipExtModuleLaunchKernel(hipFunction_t f, uint32_t globalWorkSizeX,
                                               uint32_t globalWorkSizeY, uint32_t globalWorkSizeZ,
                                               uint32_t localWorkSizeX, uint32_t localWorkSizeY,
                                               uint32_t localWorkSizeZ, size_t sharedMemBytes,
                                               hipStream_t hStream, void** kernelParams,
                                               void** extra, hipEvent_t startEvent,
                                               hipEvent_t stopEvent, uint32_t flags);

namespace {

thread_local int g_status = 0;
thread_local char g_message[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_message, sizeof(g_message), fmt, ap);
  va_end(ap);
  g_status = code;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(static_cast<int>(e), "%s: %s (hipError %d)", what, hipGetErrorString(e),
              static_cast<int>(e));
}

#define TG_HIP(call, what)                        \
  do {                                            \
    hipError_t e_ = (call);                       \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

constexpr int kRtcBase = 1000;

// Module cache of tg_code_function: key = (code pointer, size, device).
struct CodeKey {
  const void* code;
  size_t size;
  int device;
  bool operator<(const CodeKey& o) const {
    return std::tie(code, size, device) < std::tie(o.code, o.size, o.device);
  }
};
struct CodeCache {
  std::mutex mu;
  std::map<CodeKey, hipModule_t> modules;
  std::map<std::tuple<hipModule_t, std::string>, hipFunction_t> functions;
};

// Never destroyed: launcher libraries call tg_code_release from their own ELF
// destructors, which at process exit can run after this library's static
// objects would have been torn down.
CodeCache& code_cache() {
  static CodeCache* c = new CodeCache;
  return *c;
}

// Launch order of tg_launch_ordered: key = (caller's order key, device).  The
// event marks the end of the key's latest launch, which went to `last`.
struct OrderState {
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
  bool pending = false;
};
struct OrderTable {
  std::mutex mu;
  std::map<std::pair<const void*, int>, OrderState> keys;
};
// Never destroyed, like the code cache (tg_code_release drops entries at exit).
OrderTable& order_table() {
  static OrderTable* t = new OrderTable;
  return *t;
}

bool valid_geometry(int64_t grid, int32_t block) {
  if (grid <= 0 || block <= 0 || block > 1024) return false;
  // the dispatch packet's grid size is a 32-bit count of work-items
  return grid * static_cast<int64_t>(block) <= 0xFFFFFFFFLL;
}

}  // namespace

extern "C" {

const char* tg_last_error(void) { return g_message; }
int tg_last_status(void) { return g_status; }
void tg_clear_error(void) {
  g_status = 0;
  g_message[0] = '\0';
}

int tg_fail(int code, const char* message) { return fail(code, "%s", message ? message : ""); }

int tg_device_count(int* count) {
  if (!count) return fail(-1, "tg_device_count: null output");
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return 0;
  }
  TG_HIP(e, "hipGetDeviceCount");
  return 0;
}

int tg_set_device(int device) {
  TG_HIP(hipSetDevice(device), "hipSetDevice");
  return 0;
}

int tg_get_device(int* device) {
  if (!device) return fail(-1, "tg_get_device: null output");
  TG_HIP(hipGetDevice(device), "hipGetDevice");
  return 0;
}

int tg_device_props(int device, char* name, int name_len, char* arch, int arch_len,
                    int* cu_count, int64_t* global_mem_bytes, int* clock_khz,
                    int* l2_bytes) {
  hipDeviceProp_t p;
  TG_HIP(hipGetDeviceProperties(&p, device), "hipGetDeviceProperties");
  if (name && name_len > 0) std::snprintf(name, name_len, "%s", p.name);
  if (arch && arch_len > 0) std::snprintf(arch, arch_len, "%s", p.gcnArchName);
  if (cu_count) *cu_count = p.multiProcessorCount;
  if (global_mem_bytes) *global_mem_bytes = static_cast<int64_t>(p.totalGlobalMem);
  if (clock_khz) *clock_khz = p.clockRate;
  if (l2_bytes) *l2_bytes = p.l2CacheSize;
  return 0;
}

int tg_runtime_version(int* hip_version, int* hiprtc_major, int* hiprtc_minor) {
  if (hip_version) {
    *hip_version = 0;
    TG_HIP(hipRuntimeGetVersion(hip_version), "hipRuntimeGetVersion");
  }
  int maj = 0, min = 0;
  hiprtcResult r = hiprtcVersion(&maj, &min);
  if (r != HIPRTC_SUCCESS)
    return fail(kRtcBase + r, "hiprtcVersion: %s", hiprtcGetErrorString(r));
  if (hiprtc_major) *hiprtc_major = maj;
  if (hiprtc_minor) *hiprtc_minor = min;
  return 0;
}

int tg_rtc_compile(const char* source, const char* name, const char* const* options,
                   int n_options, void** code, size_t* code_size, char** log) {
  if (!source || !code || !code_size) return fail(-1, "tg_rtc_compile: null argument");
  *code = nullptr;
  *code_size = 0;
  if (log) *log = nullptr;
  hiprtcProgram prog;
  hiprtcResult r = hiprtcCreateProgram(&prog, source, name ? name : "tilegen.hip", 0,
                                       nullptr, nullptr);
  if (r != HIPRTC_SUCCESS)
    return fail(kRtcBase + r, "hiprtcCreateProgram: %s", hiprtcGetErrorString(r));
  r = hiprtcCompileProgram(prog, n_options, const_cast<const char**>(options));
  size_t log_size = 0;
  if (hiprtcGetProgramLogSize(prog, &log_size) == HIPRTC_SUCCESS && log_size > 1 && log) {
    char* text = static_cast<char*>(std::malloc(log_size + 1));
    if (text && hiprtcGetProgramLog(prog, text) == HIPRTC_SUCCESS) {
      text[log_size] = '\0';
      *log = text;
    } else {
      std::free(text);
    }
  }
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    return fail(kRtcBase + r, "hiprtcCompileProgram(%s): %s", name ? name : "?",
                hiprtcGetErrorString(r));
  }
  size_t n = 0;
  r = hiprtcGetCodeSize(prog, &n);
  if (r != HIPRTC_SUCCESS || n == 0) {
    hiprtcDestroyProgram(&prog);
    return fail(kRtcBase + r, "hiprtcGetCodeSize: %s", hiprtcGetErrorString(r));
  }
  void* buf = std::malloc(n);
  if (!buf) {
    hiprtcDestroyProgram(&prog);
    return fail(-1, "tg_rtc_compile: out of host memory (%zu bytes)", n);
  }
  r = hiprtcGetCode(prog, static_cast<char*>(buf));
  hiprtcDestroyProgram(&prog);
  if (r != HIPRTC_SUCCESS) {
    std::free(buf);
    return fail(kRtcBase + r, "hiprtcGetCode: %s", hiprtcGetErrorString(r));
  }
  *code = buf;
  *code_size = n;
  return 0;
}

void tg_host_free(void* p) { std::free(p); }

int tg_module_load(const void* code, size_t code_size, tg_module* module) {
  if (!code || !code_size || !module) return fail(-1, "tg_module_load: null argument");
  hipModule_t m;
  TG_HIP(hipModuleLoadData(&m, code), "hipModuleLoadData");
  *module = m;
  return 0;
}

int tg_module_unload(tg_module module) {
  TG_HIP(hipModuleUnload(static_cast<hipModule_t>(module)), "hipModuleUnload");
  return 0;
}

int tg_module_function(tg_module module, const char* name, tg_function* fn) {
  if (!module || !name || !fn) return fail(-1, "tg_module_function: null argument");
  hipFunction_t f;
  hipError_t e = hipModuleGetFunction(&f, static_cast<hipModule_t>(module), name);
  if (e != hipSuccess)
    return fail(static_cast<int>(e), "hipModuleGetFunction(%s): %s", name, hipGetErrorString(e));
  *fn = f;
  return 0;
}

int tg_code_function(const void* code, size_t code_size, const char* name,
                     tg_function* fn) {
  if (!code || !code_size || !name || !fn) return fail(-1, "tg_code_function: null argument");
  int device = 0;
  TG_HIP(hipGetDevice(&device), "hipGetDevice");
  CodeCache& c = code_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  CodeKey key{code, code_size, device};
  auto it = c.modules.find(key);
  hipModule_t m;
  if (it == c.modules.end()) {
    TG_HIP(hipModuleLoadData(&m, code), "hipModuleLoadData");
    c.modules.emplace(key, m);
  } else {
    m = it->second;
  }
  auto fkey = std::make_tuple(m, std::string(name));
  auto fit = c.functions.find(fkey);
  if (fit != c.functions.end()) {
    *fn = fit->second;
    return 0;
  }
  hipFunction_t f;
  hipError_t e = hipModuleGetFunction(&f, m, name);
  if (e != hipSuccess)
    return fail(static_cast<int>(e), "hipModuleGetFunction(%s): %s", name, hipGetErrorString(e));
  c.functions.emplace(fkey, f);
  *fn = f;
  return 0;
}

int tg_code_release(const void* code, size_t code_size) {
  {
    // launch order kept under this code object's address (its event is left
    // alive: this may run during process exit, so no HIP call is made)
    OrderTable& t = order_table();
    std::lock_guard<std::mutex> lock(t.mu);
    for (auto it = t.keys.begin(); it != t.keys.end();)
      it = it->first.first == code ? t.keys.erase(it) : std::next(it);
  }
  CodeCache& c = code_cache();
  std::lock_guard<std::mutex> lock(c.mu);
  for (auto it = c.modules.begin(); it != c.modules.end();) {
    if (it->first.code == code && it->first.size == code_size) {
      const hipModule_t m = it->second;
      for (auto f = c.functions.begin(); f != c.functions.end();)
        f = std::get<0>(f->first) == m ? c.functions.erase(f) : std::next(f);
      it = c.modules.erase(it);
    } else {
      ++it;
    }
  }
  return 0;
}

int tg_function_attrs(tg_function fn, int* num_regs, int* lds_bytes, int* scratch_bytes,
                      int* max_threads) {
  if (!fn) return fail(-1, "tg_function_attrs: null function");
  hipFunction_t f = static_cast<hipFunction_t>(fn);
  if (num_regs) TG_HIP(hipFuncGetAttribute(num_regs, HIP_FUNC_ATTRIBUTE_NUM_REGS, f), "NUM_REGS");
  if (lds_bytes)
    TG_HIP(hipFuncGetAttribute(lds_bytes, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f), "SHARED");
  if (scratch_bytes)
    TG_HIP(hipFuncGetAttribute(scratch_bytes, HIP_FUNC_ATTRIBUTE_LOCAL_SIZE_BYTES, f), "LOCAL");
  if (max_threads)
    TG_HIP(hipFuncGetAttribute(max_threads, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f),
           "MAX_THREADS");
  return 0;
}

int tg_launch(tg_function fn, int64_t grid, int32_t block, int32_t lds_bytes,
              const uint64_t* args, int n_args, void* stream, int sync) {
  if (!fn) return fail(-1, "tg_launch: null function");
  if (n_args < 0 || n_args > 64 || (n_args && !args)) return fail(-1, "tg_launch: bad args");
  if (grid == 0) return 0;
  if (!valid_geometry(grid, block))
    return fail(-1, "tg_launch: invalid geometry grid=%lld block=%d", (long long)grid, block);
  void* params[64];
  for (int i = 0; i < n_args; ++i) params[i] = const_cast<uint64_t*>(args + i);
  hipStream_t s = static_cast<hipStream_t>(stream);
  TG_HIP(hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), static_cast<unsigned>(grid), 1, 1,
                               static_cast<unsigned>(block), 1, 1,
                               static_cast<unsigned>(lds_bytes), s, params, nullptr),
         "hipModuleLaunchKernel");
  if (sync) TG_HIP(s ? hipStreamSynchronize(s) : hipDeviceSynchronize(), "synchronize");
  return 0;
}

int tg_launch_ordered(const void* order_key, tg_function fn, int64_t grid, int32_t block,
                      int32_t lds_bytes, const uint64_t* args, int n_args, void* stream,
                      int sync) {
  if (!order_key) return fail(-1, "tg_launch_ordered: null order key");
  if (!fn) return fail(-1, "tg_launch_ordered: null function");
  if (grid == 0) return 0;
  if (!valid_geometry(grid, block))
    return fail(-1, "tg_launch_ordered: invalid geometry grid=%lld block=%d", (long long)grid,
                block);
  int device = 0;
  TG_HIP(hipGetDevice(&device), "hipGetDevice");
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  // the null stream is never captured
  if (s) TG_HIP(hipStreamIsCapturing(s, &cap), "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone) {
    // a captured launch runs when its graph is replayed, so ordering it
    // against eager launches here would be meaningless; the graph orders its
    // own nodes
    return tg_launch(fn, grid, block, lds_bytes, args, n_args, stream, 0);
  }
  OrderTable& t = order_table();
  // held across wait, launch and record, so two host threads cannot both
  // launch after the same recorded end
  std::lock_guard<std::mutex> lock(t.mu);
  OrderState& st = t.keys[std::make_pair(order_key, device)];
  if (!st.done) TG_HIP(hipEventCreateWithFlags(&st.done, hipEventDisableTiming), "hipEventCreate");
  if (st.pending && st.last != s)
    TG_HIP(hipStreamWaitEvent(s, st.done, 0), "hipStreamWaitEvent");
  const int rc = tg_launch(fn, grid, block, lds_bytes, args, n_args, stream, 0);
  if (rc != 0) return rc;
  TG_HIP(hipEventRecord(st.done, s), "hipEventRecord");
  st.last = s;
  st.pending = true;
  if (sync) TG_HIP(s ? hipStreamSynchronize(s) : hipDeviceSynchronize(), "synchronize");
  return 0;
}

int tg_time_launches(tg_function fn, int64_t grid, int32_t block, int32_t lds_bytes,
                     const uint64_t* arg_sets, int n_args, int n_sets, int warmup,
                     int iters, void* stream, float* kernel_ms, float* wall_ms) {
  if (!fn || !arg_sets || n_sets <= 0 || iters <= 0 || warmup < 0 || n_args < 0 ||
      n_args > 64 || !kernel_ms)
    return fail(-1, "tg_time_launches: bad argument");
  if (!valid_geometry(grid, block))
    return fail(-1, "tg_time_launches: invalid geometry grid=%lld block=%d",
                (long long)grid, block);
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipFunction_t f = static_cast<hipFunction_t>(fn);
  const uint32_t gx = static_cast<uint32_t>(grid * block);
  std::vector<hipEvent_t> ev(2 * static_cast<size_t>(iters), nullptr);
  int rc = 0;
  for (auto& e : ev) {
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) {
      rc = hip_fail(err, "hipEventCreate");
      break;
    }
  }
  void* params[64];
  for (int i = 0; rc == 0 && i < warmup + iters; ++i) {
    const uint64_t* a = arg_sets + static_cast<size_t>(i % n_sets) * n_args;
    for (int k = 0; k < n_args; ++k) params[k] = const_cast<uint64_t*>(a + k);
    const int t = i - warmup;
    hipEvent_t start = t >= 0 ? ev[2 * t] : nullptr;
    hipEvent_t stop = t >= 0 ? ev[2 * t + 1] : nullptr;
    hipError_t err = hipExtModuleLaunchKernel(f, gx, 1, 1, static_cast<uint32_t>(block), 1, 1,
                                              static_cast<size_t>(lds_bytes), s, params,
                                              nullptr, start, stop, 0);
    if (err != hipSuccess) rc = hip_fail(err, "hipExtModuleLaunchKernel");
  }
  if (rc == 0) {
    hipError_t err = s ? hipStreamSynchronize(s) : hipDeviceSynchronize();
    if (err != hipSuccess) rc = hip_fail(err, "synchronize after timed launches");
  }
  for (int t = 0; rc == 0 && t < iters; ++t) {
    hipError_t err = hipEventElapsedTime(&kernel_ms[t], ev[2 * t], ev[2 * t + 1]);
    if (err != hipSuccess) rc = hip_fail(err, "hipEventElapsedTime");
  }
  if (rc == 0 && wall_ms) {
    hipError_t err = hipEventElapsedTime(wall_ms, ev[0], ev[2 * (iters - 1) + 1]);
    if (err != hipSuccess) rc = hip_fail(err, "hipEventElapsedTime(wall)");
  }
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int tg_run_launches(tg_function fn, int64_t grid, int32_t block, int32_t lds_bytes,
                    const uint64_t* arg_sets, int n_args, int n_sets, int iters, void* stream) {
  if (!fn || !arg_sets || n_sets <= 0 || iters < 0 || n_args < 0 || n_args > 64)
    return fail(-1, "tg_run_launches: bad argument");
  if (!valid_geometry(grid, block))
    return fail(-1, "tg_run_launches: invalid geometry grid=%lld block=%d", (long long)grid,
                block);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* params[64];
  for (int i = 0; i < iters; ++i) {
    const uint64_t* a = arg_sets + static_cast<size_t>(i % n_sets) * n_args;
    for (int k = 0; k < n_args; ++k) params[k] = const_cast<uint64_t*>(a + k);
    TG_HIP(hipModuleLaunchKernel(static_cast<hipFunction_t>(fn), static_cast<unsigned>(grid), 1,
                                 1, static_cast<unsigned>(block), 1, 1,
                                 static_cast<unsigned>(lds_bytes), s, params, nullptr),
           "hipModuleLaunchKernel");
  }
  return 0;
}

int tg_malloc(void** d_ptr, size_t bytes) {
  if (!d_ptr) return fail(-1, "tg_malloc: null output");
  *d_ptr = nullptr;
  TG_HIP(hipMalloc(d_ptr, bytes ? bytes : 1), "hipMalloc");
  return 0;
}

int tg_free(void* d_ptr) {
  if (d_ptr) TG_HIP(hipFree(d_ptr), "hipFree");
  return 0;
}

int tg_memcpy_htod(void* d_dst, const void* src, size_t bytes) {
  if (bytes) TG_HIP(hipMemcpy(d_dst, src, bytes, hipMemcpyHostToDevice), "hipMemcpy H2D");
  return 0;
}

int tg_memcpy_dtoh(void* dst, const void* d_src, size_t bytes) {
  if (bytes) TG_HIP(hipMemcpy(dst, d_src, bytes, hipMemcpyDeviceToHost), "hipMemcpy D2H");
  return 0;
}

int tg_memcpy_dtod(void* d_dst, const void* d_src, size_t bytes) {
  if (bytes) TG_HIP(hipMemcpy(d_dst, d_src, bytes, hipMemcpyDeviceToDevice), "hipMemcpy D2D");
  return 0;
}

int tg_memset(void* d_ptr, int value, size_t bytes) {
  if (bytes) TG_HIP(hipMemset(d_ptr, value, bytes), "hipMemset");
  return 0;
}

int tg_synchronize(void) {
  TG_HIP(hipDeviceSynchronize(), "hipDeviceSynchronize");
  return 0;
}

int tg_stream_create(void** stream) {
  if (!stream) return fail(-1, "tg_stream_create: null output");
  hipStream_t s;
  TG_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreate");
  *stream = s;
  return 0;
}

int tg_stream_destroy(void* stream) {
  if (stream) TG_HIP(hipStreamDestroy(static_cast<hipStream_t>(stream)), "hipStreamDestroy");
  return 0;
}

int tg_stream_synchronize(void* stream) {
  TG_HIP(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "hipStreamSynchronize");
  return 0;
}

int tg_graph_begin(void* stream) {
  // the null stream cannot be captured; thread-local mode leaves other threads free
  if (!stream) return fail(-1, "tg_graph_begin: the null stream cannot be captured");
  TG_HIP(hipStreamBeginCapture(static_cast<hipStream_t>(stream),
                               hipStreamCaptureModeThreadLocal),
         "hipStreamBeginCapture");
  return 0;
}

int tg_graph_end(void* stream, void** exec) {
  if (!stream) return fail(-1, "tg_graph_end: null stream");
  hipGraph_t graph = nullptr;
  // the capture is ended even when the caller gave no output, so the stream is usable again
  TG_HIP(hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph), "hipStreamEndCapture");
  // the captured graph is released whatever happens next (its executable, when one is
  // made, does not need it); a failure to release it changes nothing for the caller
  if (!exec) {
    if (graph) (void)hipGraphDestroy(graph);
    return fail(-1, "tg_graph_end: null output");
  }
  hipGraphExec_t e = nullptr;
  const hipError_t err = hipGraphInstantiate(&e, graph, nullptr, nullptr, 0);
  (void)hipGraphDestroy(graph);
  if (err != hipSuccess) return hip_fail(err, "hipGraphInstantiate");
  *exec = e;
  return 0;
}

int tg_graph_launch(void* exec, void* stream, int sync) {
  if (!exec) return fail(-1, "tg_graph_launch: null graph");
  hipStream_t s = static_cast<hipStream_t>(stream);
  TG_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), s), "hipGraphLaunch");
  if (sync) TG_HIP(s ? hipStreamSynchronize(s) : hipDeviceSynchronize(), "synchronize");
  return 0;
}

int tg_graph_destroy(void* exec) {
  if (exec) TG_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)), "hipGraphExecDestroy");
  return 0;
}

}  // extern "C"
