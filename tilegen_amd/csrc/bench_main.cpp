// tilegen_bench: host harness for one generated variant (the HIP-native
// counterpart of the reference's cpp/src/harness.cpp:117-268).
//
//   tilegen_bench --kernel spmv --matrix A.bin --lib variant.so
//                 [--backend hip|cpu] [--K 32] [--iters 20] [--warmup 5]
//                 [--rotate 1] [--config JSON]
//
// Loads a TGM1 matrix (magic 0x54474D31, rows/cols/nnz int64, indptr, indices,
// data; reference tilegen/matrices.py:38-46), dlopens the variant library,
// binds launch_<kernel>, runs it on deterministic inputs, checks the result
// against a sequential CPU product computed here, and prints one JSON line
// with the reference's keys (kernel, config, backend, matrix, rows, cols, nnz,
// ms_mean, ms_min, gflops, bandwidth_gbs, max_abs_err, max_rel_err).
//
// Differences from the reference harness: with --backend hip every operand
// lives in device memory (the reference passes host pointers even to its CUDA
// variants), ms_* are GPU times of the kernel dispatch (start/stop events on
// the dispatch, tg_time_launches) with the synchronous launch_<kernel> wall time
// reported beside them, and --rotate N keeps N device copies of the inputs so
// timed launches read cold memory.  Exit codes: 2 usage or input error, 3
// library/symbol error, 4 runtime error, as in the reference for 2 and 3.
#include <dlfcn.h>

#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <fstream>
#include <string>
#include <vector>

#include "tgrt.h"

namespace {

struct Csr {
  int64_t rows = 0, cols = 0, nnz = 0;
  std::vector<int64_t> indptr, indices;
  std::vector<double> data;
};

bool load_tgm1(const std::string& path, Csr* m, std::string* err) {
  std::ifstream fh(path, std::ios::binary);
  if (!fh) {
    *err = "cannot open matrix " + path;
    return false;
  }
  uint32_t magic = 0;
  fh.read(reinterpret_cast<char*>(&magic), 4);
  fh.read(reinterpret_cast<char*>(&m->rows), 8);
  fh.read(reinterpret_cast<char*>(&m->cols), 8);
  fh.read(reinterpret_cast<char*>(&m->nnz), 8);
  if (!fh || magic != 0x54474D31u || m->rows < 0 || m->cols < 0 || m->nnz < 0) {
    *err = "not a TGM1 matrix: " + path;
    return false;
  }
  m->indptr.resize(static_cast<size_t>(m->rows) + 1);
  m->indices.resize(static_cast<size_t>(m->nnz));
  m->data.resize(static_cast<size_t>(m->nnz));
  fh.read(reinterpret_cast<char*>(m->indptr.data()), 8 * (m->rows + 1));
  fh.read(reinterpret_cast<char*>(m->indices.data()), 8 * m->nnz);
  fh.read(reinterpret_cast<char*>(m->data.data()), 8 * m->nnz);
  if (!fh) {
    *err = "truncated TGM1 payload: " + path;
    return false;
  }
  if (m->indptr[0] != 0 || m->indptr[m->rows] != m->nnz) {
    *err = "inconsistent indptr in " + path;
    return false;
  }
  for (int64_t p = 0; p < m->nnz; ++p)
    if (m->indices[p] < 0 || m->indices[p] >= m->cols) {
      *err = "column index out of range in " + path;
      return false;
    }
  return true;
}

struct Args {
  std::string kernel, matrix, lib, config = "{}", backend = "hip";
  int iters = 20, warmup = 5, rotate = 1;
  int64_t K = 32;
};

bool parse(int argc, char** argv, Args* a) {
  for (int i = 1; i < argc; ++i) {
    std::string k = argv[i];
    if (i + 1 >= argc) {
      std::fprintf(stderr, "error: missing value for %s\n", k.c_str());
      return false;
    }
    std::string v = argv[++i];
    if (k == "--kernel") a->kernel = v;
    else if (k == "--matrix") a->matrix = v;
    else if (k == "--lib") a->lib = v;
    else if (k == "--config") a->config = v;
    else if (k == "--backend") a->backend = v;
    else if (k == "--iters") a->iters = std::atoi(v.c_str());
    else if (k == "--warmup") a->warmup = std::atoi(v.c_str());
    else if (k == "--rotate") a->rotate = std::atoi(v.c_str());
    else if (k == "--K") a->K = std::atoll(v.c_str());
    else {
      std::fprintf(stderr, "error: unknown flag %s\n", k.c_str());
      return false;
    }
  }
  return !a->kernel.empty() && !a->matrix.empty() && !a->lib.empty() && a->iters > 0 &&
         a->warmup >= 0 && a->rotate >= 1 && a->K >= 1 &&
         (a->backend == "hip" || a->backend == "cpu");
}

std::string escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o.push_back('\\');
    o.push_back(c);
  }
  return o;
}

// deterministic operand values in [-0.5, 0.5), distinct per array
void fill(std::vector<double>* v, uint64_t salt) {
  for (size_t i = 0; i < v->size(); ++i) {
    uint64_t h = (i + 1) * 0x9E3779B97F4A7C15ull ^ (salt * 0xC2B2AE3D27D4EB4Full);
    h ^= h >> 29;
    (*v)[i] = static_cast<double>(h % 1000003) / 1000003.0 - 0.5;
  }
}

double now_ms() {
  using namespace std::chrono;
  return duration<double, std::milli>(steady_clock::now().time_since_epoch()).count();
}

}  // namespace

int main(int argc, char** argv) {
  Args a;
  if (!parse(argc, argv, &a)) {
    std::fprintf(stderr,
                 "usage: tilegen_bench --kernel K --matrix M.bin --lib L.so [--backend hip|cpu] "
                 "[--K 32] [--iters N] [--warmup N] [--rotate N] [--config JSON]\n");
    return 2;
  }
  Csr m;
  std::string err;
  if (!load_tgm1(a.matrix, &m, &err)) {
    std::fprintf(stderr, "error: %s\n", err.c_str());
    return 2;
  }
  const int64_t M = m.rows, N = m.cols, nnz = m.nnz, K = a.K;
  const std::string& kn = a.kernel;
  if (kn != "spmv" && kn != "spmm" && kn != "sddmm") {
    std::fprintf(stderr, "error: unknown kernel %s (spmv|spmm|sddmm)\n", kn.c_str());
    return 2;
  }
  void* h = dlopen(a.lib.c_str(), RTLD_NOW);
  if (!h) {
    std::fprintf(stderr, "error: dlopen failed: %s\n", dlerror());
    return 3;
  }
  void* fn = dlsym(h, ("launch_" + kn).c_str());
  if (!fn) {
    std::fprintf(stderr, "error: symbol launch_%s not found: %s\n", kn.c_str(), dlerror());
    return 3;
  }

  // operands and the sequential CPU product they are checked against
  std::vector<double> x, B, U, V, ref, out;
  double flops = 0.0, bytes_ref = 0.0;
  if (kn == "spmv") {
    x.resize(N);
    fill(&x, 1);
    ref.assign(M, 0.0);
    for (int64_t i = 0; i < M; ++i) {
      double acc = 0.0;
      for (int64_t p = m.indptr[i]; p < m.indptr[i + 1]; ++p) acc += m.data[p] * x[m.indices[p]];
      ref[i] = acc;
    }
    flops = 2.0 * nnz;
    bytes_ref = 24.0 * nnz + 8.0 * (M + 1) + 8.0 * M;
  } else if (kn == "spmm") {
    B.resize(static_cast<size_t>(N) * K);
    fill(&B, 2);
    ref.assign(static_cast<size_t>(M) * K, 0.0);
    for (int64_t i = 0; i < M; ++i)
      for (int64_t p = m.indptr[i]; p < m.indptr[i + 1]; ++p)
        for (int64_t k = 0; k < K; ++k) ref[i * K + k] += m.data[p] * B[m.indices[p] * K + k];
    flops = 2.0 * nnz * K;
    bytes_ref = 16.0 * nnz + 8.0 * (M + 1) + 8.0 * nnz * K + 8.0 * M * K;
  } else {
    U.resize(static_cast<size_t>(M) * K);
    V.resize(static_cast<size_t>(N) * K);
    fill(&U, 3);
    fill(&V, 4);
    ref.assign(nnz, 0.0);
    for (int64_t i = 0; i < M; ++i)
      for (int64_t p = m.indptr[i]; p < m.indptr[i + 1]; ++p) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) acc += U[i * K + k] * V[m.indices[p] * K + k];
        ref[p] = m.data[p] * acc;
      }
    flops = 2.0 * nnz * K;
    bytes_ref = 16.0 * nnz + 8.0 * (M + 1) + 16.0 * nnz * K + 8.0 * nnz;
  }
  out.assign(ref.size(), 0.0);
  const std::vector<double>& dense0 = kn == "spmv" ? x : (kn == "spmm" ? B : U);

  using Fv = void (*)(const int64_t*, const int64_t*, const double*, const double*, double*,
                      int64_t, int64_t, int64_t);
  using Fm = void (*)(const int64_t*, const int64_t*, const double*, const double*, double*,
                      int64_t, int64_t, int64_t, int64_t);
  using Fs = void (*)(const int64_t*, const int64_t*, const double*, const double*,
                      const double*, double*, int64_t, int64_t, int64_t, int64_t);

  struct Set {
    const int64_t *ip, *ind;
    const double *dat, *d0, *d1;
    double* o;
  };
  std::vector<Set> sets;
  std::vector<void*> owned;
  const bool hip = a.backend == "hip";
  auto dev = [&](const void* src, size_t bytes) -> void* {
    void* p = nullptr;
    if (tg_malloc(&p, bytes) != 0 || tg_memcpy_htod(p, src, bytes) != 0) return nullptr;
    owned.push_back(p);
    return p;
  };
  for (int c = 0; c < (hip ? a.rotate : 1); ++c) {
    Set s{};
    if (hip) {
      s.ip = static_cast<const int64_t*>(dev(m.indptr.data(), 8 * (M + 1)));
      s.ind = static_cast<const int64_t*>(dev(m.indices.data(), 8 * nnz));
      s.dat = static_cast<const double*>(dev(m.data.data(), 8 * nnz));
      s.d0 = static_cast<const double*>(dev(dense0.data(), 8 * dense0.size()));
      s.d1 = kn == "sddmm" ? static_cast<const double*>(dev(V.data(), 8 * V.size())) : nullptr;
      s.o = static_cast<double*>(dev(out.data(), 8 * out.size()));
      if (!s.ip || !s.ind || !s.dat || !s.d0 || !s.o || (kn == "sddmm" && !s.d1)) {
        std::fprintf(stderr, "error: device allocation failed: %s\n", tg_last_error());
        return 4;
      }
    } else {
      s = Set{m.indptr.data(), m.indices.data(), m.data.data(), dense0.data(),
              kn == "sddmm" ? V.data() : nullptr, out.data()};
    }
    sets.push_back(s);
  }

  auto call = [&](const Set& s) {
    // the OpenMP variants accumulate into C (reference semantics): start from zero
    if (!hip && kn == "spmm") std::fill(out.begin(), out.end(), 0.0);
    if (kn == "spmv")
      reinterpret_cast<Fv>(fn)(s.ip, s.ind, s.dat, s.d0, s.o, M, N, nnz);
    else if (kn == "spmm")
      reinterpret_cast<Fm>(fn)(s.ip, s.ind, s.dat, s.d0, s.o, M, N, K, nnz);
    else
      reinterpret_cast<Fs>(fn)(s.ip, s.ind, s.dat, s.d0, s.d1, s.o, M, N, K, nnz);
  };

  // synchronous calls through the ABI: checked result + wall time
  tg_clear_error();
  for (int i = 0; i < a.warmup; ++i) call(sets[i % sets.size()]);
  std::vector<double> wall;
  for (int i = 0; i < a.iters; ++i) {
    const double t0 = now_ms();
    call(sets[i % sets.size()]);
    wall.push_back(now_ms() - t0);
  }
  if (hip && tg_last_status() != 0) {
    std::fprintf(stderr, "error: launch_%s failed: %s\n", kn.c_str(), tg_last_error());
    return 4;
  }
  std::vector<double> got(out.size());
  if (hip) {
    if (tg_memcpy_dtoh(got.data(), sets[0].o, 8 * got.size()) != 0) {
      std::fprintf(stderr, "error: %s\n", tg_last_error());
      return 4;
    }
  } else {
    got = out;
  }

  // GPU time of the dispatch itself
  std::vector<float> kms;
  double enqueue_async_us = -1.0, enqueue_raw_us = -1.0;
  if (hip) {
    using Fn = void* (*)(void);
    using Fg = int (*)(int64_t, int64_t, int64_t, int64_t, int64_t*, int32_t*, int32_t*);
    Fn getfn = reinterpret_cast<Fn>(dlsym(h, "tgv_function"));
    Fg geom = reinterpret_cast<Fg>(dlsym(h, "tgv_geometry"));
    if (getfn && geom) {
      int64_t grid = 0;
      int32_t block = 0, lds = 0;
      geom(M, N, K, nnz, &grid, &block, &lds);
      void* kfn = getfn();
      if (kfn && grid > 0) {
        std::vector<uint64_t> slots;
        for (const Set& s : sets) {
          std::vector<uint64_t> one = {reinterpret_cast<uint64_t>(s.ip),
                                       reinterpret_cast<uint64_t>(s.ind),
                                       reinterpret_cast<uint64_t>(s.dat),
                                       reinterpret_cast<uint64_t>(s.d0)};
          if (kn == "sddmm") one.push_back(reinterpret_cast<uint64_t>(s.d1));
          one.push_back(reinterpret_cast<uint64_t>(s.o));
          one.push_back(static_cast<uint64_t>(M));
          one.push_back(static_cast<uint64_t>(N));
          if (kn != "spmv") one.push_back(static_cast<uint64_t>(K));
          one.push_back(static_cast<uint64_t>(nnz));
          slots.insert(slots.end(), one.begin(), one.end());
        }
        const int nargs = static_cast<int>(slots.size() / sets.size());
        kms.assign(a.iters, 0.0f);
        float ev_wall = 0.0f;
        if (tg_time_launches(kfn, grid, block, lds, slots.data(), nargs,
                             static_cast<int>(sets.size()), a.warmup, a.iters, nullptr,
                             kms.data(), &ev_wall) != 0) {
          std::fprintf(stderr, "error: %s\n", tg_last_error());
          return 4;
        }
        // host cost of enqueueing one launch: a.iters back-to-back launches through
        // the variant's tgv_launch_async (the product path: ordered launches for
        // variants with module scratch) and through tg_run_launches (the raw
        // dispatch), host clock around the enqueue loop only
        if (kn == "spmv") {
          using Fa = int (*)(void*, const int64_t*, const int64_t*, const double*, const double*,
                             double*, int64_t, int64_t, int64_t);
          Fa async = reinterpret_cast<Fa>(dlsym(h, "tgv_launch_async"));
          if (async) {
            tg_synchronize();
            double t0 = now_ms();
            for (int i = 0; i < a.iters; ++i) {
              const Set& s = sets[i % sets.size()];
              if (async(nullptr, s.ip, s.ind, s.dat, s.d0, s.o, M, N, nnz) != 0) {
                std::fprintf(stderr, "error: tgv_launch_async: %s\n", tg_last_error());
                return 4;
              }
            }
            enqueue_async_us = (now_ms() - t0) * 1e3 / a.iters;
            tg_synchronize();
            t0 = now_ms();
            if (tg_run_launches(kfn, grid, block, lds, slots.data(), nargs,
                                static_cast<int>(sets.size()), a.iters, nullptr) != 0) {
              std::fprintf(stderr, "error: %s\n", tg_last_error());
              return 4;
            }
            enqueue_raw_us = (now_ms() - t0) * 1e3 / a.iters;
            tg_synchronize();
          }
        }
      }
    }
  }

  double max_abs = 0.0, max_rel = 0.0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double d = std::fabs(got[i] - ref[i]);
    max_abs = std::fmax(max_abs, d);
    max_rel = std::fmax(max_rel, d / std::fmax(std::fabs(ref[i]), 1e-300));
  }
  std::vector<double> t;
  if (!kms.empty())
    for (float v : kms) t.push_back(v);
  else
    t = wall;
  double sum = 0.0, mn = t.empty() ? 0.0 : t[0];
  for (double v : t) {
    sum += v;
    mn = std::fmin(mn, v);
  }
  double wsum = 0.0;
  for (double v : wall) wsum += v;
  const double mean = t.empty() ? 0.0 : sum / t.size();
  std::printf(
      "{\"kernel\":\"%s\",\"config\":%s,\"backend\":\"%s\",\"matrix\":\"%s\",\"rows\":%lld,"
      "\"cols\":%lld,\"nnz\":%lld,\"K\":%lld,\"ms_mean\":%.6g,\"ms_min\":%.6g,"
      "\"gflops\":%.6g,\"bandwidth_gbs\":%.6g,\"max_abs_err\":%.6g,\"max_rel_err\":%.6g,"
      "\"timer\":\"%s\",\"launch_wall_ms_mean\":%.6g,\"rotate\":%d,"
      "\"enqueue_us_async\":%.4g,\"enqueue_us_raw\":%.4g}\n",
      escape(kn).c_str(), a.config.c_str(), escape(a.backend).c_str(), escape(a.matrix).c_str(),
      (long long)M, (long long)N, (long long)nnz, (long long)(kn == "spmv" ? 0 : K), mean, mn,
      mn > 0 ? flops / (mn * 1e6) : 0.0, mn > 0 ? bytes_ref / (mn * 1e6) : 0.0, max_abs, max_rel,
      kms.empty() ? "host clock around launch" : "dispatch events (tg_time_launches)",
      wall.empty() ? 0.0 : wsum / wall.size(), hip ? a.rotate : 1, enqueue_async_us,
      enqueue_raw_us);
  for (void* p : owned) tg_free(p);
  // no dlclose: an OpenMP variant's worker threads still run code from it; the
  // library goes away with the process
  return 0;
}
