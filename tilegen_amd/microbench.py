"""Hardware microbenchmarks behind the roofline analysis of the CSR kernels.

Four probes, each a small kernel compiled with hipRTC and timed with
dispatch-attached events (``tg_time_launches``); none is on the product path.

gather
    Random 8-byte loads from an 800 KB array (the size of c1's ``x``, which
    stays resident in each XCD's L2), 8 per lane, indices streamed from HBM.
    Run with 64, 32, 16 and 8 active lanes per wave: if the rate in gathers/s
    stays flat as lanes drop, the limit is per gathered line, not per load
    instruction.  A second kernel routes the gathers of the first S lanes of
    each wave through uniform (scalar-cache) loads instead, to see whether
    that path adds capacity.
stream
    A plain 128-bit read-and-sum over cold (rotated) copies of 8, 27, 128 and
    512 MB: the practical HBM read rate at the BASELINE sizes, including one
    launch's ramp-up and first-byte latency.
rowgather
    SpMM's B-row access without the A stream: 1.6 M random 512-byte rows
    gathered from a 51.2 MB table (larger than an XCD's L2, smaller than the
    Infinity Cache) and from a 3.2 MB one, with one 512-byte row written per
    16 gathered, cold (table copies rotated) and warm.
flat
    A SpMV case's accesses without its rows (every SpMV case by default): the
    matrix's own ``indices`` and ``data`` streamed with one 128-bit load of
    each per lane, ``x`` gathered at those indices, 8 lanes summing 16
    products and one double stored per 16, with no row pointers, LDS or
    barriers.  Cold (every array rotated) and warm, with the gathers and
    without them (the stream alone): the floor for the bytes and gathers the
    case makes, against which the row logic is measured.

``python -m tilegen_amd.microbench --out results`` writes ``microbench.json``
and ``microbench.md``.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
from typing import Dict, List

import numpy as np

from . import runtime as rt
from .verify import hiprtc_options

__all__ = ["gather_probe", "stream_probe", "rowgather_probe", "flat_probe", "main"]

_GATHER_SRC = r'''
typedef long long i64;
// 8 gathers per lane from x; lanes at or past `active` in each wave skip theirs
extern "C" __global__ __launch_bounds__(256)
void mb_gather(const i64* __restrict__ idx, const double* __restrict__ x, double* __restrict__ out,
               int active) {
  const i64 t = (i64)blockIdx.x * 256 + threadIdx.x;
  double acc = 0.0;
  if ((int)(threadIdx.x & 63) < active) {
    i64 c[8];
    #pragma unroll
    for (int u = 0; u < 8; ++u) c[u] = idx[t * 8 + u];
    #pragma unroll
    for (int u = 0; u < 8; ++u) acc += x[c[u]];
  }
  out[t] = acc;
}
// the first S lanes' gathers go through wave-uniform loads, one lane at a time
extern "C" __global__ __launch_bounds__(256)
void mb_gather_uniform(const i64* __restrict__ idx, const double* __restrict__ x,
                       double* __restrict__ out, int S) {
  const i64 t = (i64)blockIdx.x * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63;
  i64 c[8];
  #pragma unroll
  for (int u = 0; u < 8; ++u) c[u] = idx[t * 8 + u];
  double acc = 0.0;
  if (lane >= S) {
    #pragma unroll
    for (int u = 0; u < 8; ++u) acc += x[c[u]];
  }
  for (int l = 0; l < S; ++l) {
    #pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int lo = __builtin_amdgcn_readlane((int)c[u], l);
      const int hi = __builtin_amdgcn_readlane((int)(c[u] >> 32), l);
      const double v = x[((i64)hi << 32) | (unsigned)lo];
      acc += lane == l ? v : 0.0;
    }
  }
  out[t] = acc;
}
'''

_ROWGATHER_SRC = r'''
typedef long long i64;
typedef double f64x2 __attribute__((ext_vector_type(2)));
// each 32-lane group gathers `per` random 512-byte rows of T (64 doubles, one
// 128-bit load per lane, 4 rows in flight), sums them and writes its 512-byte
// result row: SpMM's B-row gathers and C stores without the A stream
extern "C" __global__ __launch_bounds__(256)
void mb_rowgather(const i64* __restrict__ idx, const f64x2* __restrict__ T, f64x2* __restrict__ out,
                  i64 n_groups, int per) {
  const i64 g = ((i64)blockIdx.x * 256 + threadIdx.x) / 32;
  const int l = threadIdx.x % 32;
  if (g >= n_groups) return;
  f64x2 acc = {0.0, 0.0};
  for (int r = 0; r < per; r += 4) {
    i64 j[4];
    #pragma unroll
    for (int u = 0; u < 4; ++u) j[u] = idx[g * per + r + u];
    f64x2 v[4];
    #pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = T[j[u] * 32 + l];
    #pragma unroll
    for (int u = 0; u < 4; ++u) acc += v[u];
  }
  __builtin_nontemporal_store(acc, out + g * 32 + l);
}
'''

_FLAT_SRC = r'''
typedef long long i64;
typedef long long i64x2 __attribute__((ext_vector_type(2)));
typedef double f64x2 __attribute__((ext_vector_type(2)));
// thread t takes nonzeros 2t and 2t+1 (one 128-bit load of indices and one of
// values); the 8 threads of group g = t / 8 cover nonzeros 16g .. 16g+15 and
// store their sum as out[g].  With gather == 0 the index itself stands in for
// x[index], so the index loads stay live and x is never read.
extern "C" __global__ __launch_bounds__(256)
void mb_flat(const i64x2* __restrict__ idx, const f64x2* __restrict__ val,
             const double* __restrict__ x, double* __restrict__ out, i64 n_groups, int gather) {
  const i64 t = (i64)blockIdx.x * blockDim.x + threadIdx.x;
  const i64 g = t / 8;
  double s = 0.0;
  if (g < n_groups) {
    const i64x2 c = __builtin_nontemporal_load(idx + t);
    const f64x2 v = __builtin_nontemporal_load(val + t);
    s = gather ? v.x * x[c.x] + v.y * x[c.y] : v.x * (double)c.x + v.y * (double)c.y;
  }
  s += __shfl_xor(s, 1);
  s += __shfl_xor(s, 2);
  s += __shfl_xor(s, 4);
  if (g < n_groups && (threadIdx.x & 7) == 0) __builtin_nontemporal_store(s, out + g);
}
'''

_STREAM_SRC = r'''
typedef double f64x2 __attribute__((ext_vector_type(2)));
// each workgroup sums its contiguous share of the array with 128-bit loads;
// the sum is stored only if it equals a sentinel, so the loads cannot be elided
extern "C" __global__ __launch_bounds__(256)
void mb_stream(const f64x2* __restrict__ a, double* __restrict__ out, long long n2,
               long long per_block) {
  const long long lo = (long long)blockIdx.x * per_block;
  long long hi = lo + per_block;
  if (hi > n2) hi = n2;
  double s = 0.0;
  for (long long i = lo + threadIdx.x; i < hi; i += 1024) {
    f64x2 v[4];
    #pragma unroll
    for (int u = 0; u < 4; ++u) {
      const long long k = i + u * 256;
      v[u] = k < hi ? __builtin_nontemporal_load(a + k) : (f64x2){0.0, 0.0};
    }
    #pragma unroll
    for (int u = 0; u < 4; ++u) s += v[u].x + v[u].y;
  }
  if (s == 12345.678) out[blockIdx.x] = s;
}
'''


def _load(src: str, names: List[str]) -> Dict[str, int]:
    code, _ = rt.rtc_compile(src, "microbench.hip", hiprtc_options())
    blob = ctypes.create_string_buffer(code, len(code))
    mod = ctypes.c_void_p()
    rt.check(rt.lib().tg_module_load(blob, len(code), ctypes.byref(mod)), "module load")
    _load.keep.append(blob)
    out = {}
    for n in names:
        f = ctypes.c_void_p()
        rt.check(rt.lib().tg_module_function(mod, n.encode(), ctypes.byref(f)), n)
        out[n] = f.value
    return out


_load.keep = []


def gather_probe(n: int = 100_000, workgroups: int = 4000, iters: int = 30) -> List[dict]:
    fns = _load(_GATHER_SRC, ["mb_gather", "mb_gather_uniform"])
    threads = 256 * workgroups
    rng = np.random.default_rng(0)
    idx = rng.integers(0, n, threads * 8, dtype=np.int64)
    if idx.min() < 0 or idx.max() >= n:  # every gather stays inside x
        raise AssertionError("index out of range")
    bi, bx = rt.DeviceBuffer(idx), rt.DeviceBuffer(rng.uniform(-1, 1, n))
    bo = rt.DeviceBuffer(np.zeros(threads))
    waves = threads // 64
    rows = []
    try:
        for name, arg in [("mb_gather", 64), ("mb_gather", 32), ("mb_gather", 16),
                          ("mb_gather", 8), ("mb_gather_uniform", 0), ("mb_gather_uniform", 4),
                          ("mb_gather_uniform", 8), ("mb_gather_uniform", 16)]:
            kms, _ = rt.time_launches(fns[name], workgroups, 256, 0, [[bi, bx, bo, arg]], 5,
                                      iters)
            sec = float(np.median(kms)) * 1e-3
            gathers = waves * 8 * (arg if name == "mb_gather" else 64)
            rows.append({"kernel": name, "lanes_or_uniform": arg, "us": sec * 1e6,
                         "gathers_per_s": gathers / sec, "gather_instr_per_s": waves * 8 / sec})
    finally:
        for b in (bi, bx, bo):
            b.free()
    return rows


def stream_probe(sizes_mb=(8, 27, 128, 512), rotate_mb: int = 1280, iters: int = 100
                 ) -> List[dict]:
    fn = _load(_STREAM_SRC, ["mb_stream"])["mb_stream"]
    out = rt.DeviceBuffer(np.zeros(1 << 16))
    rows = []
    try:
        for mb in sizes_mb:
            n = (mb << 20) // 8
            copies = max(2, rotate_mb // mb)
            bufs = [rt.DeviceBuffer(np.random.default_rng(c).standard_normal(n))
                    for c in range(copies)]
            try:
                best = None
                for blocks in (2048, 4096, 8192, 16384):
                    per = -(-(n // 2) // blocks)
                    kms, _ = rt.time_launches(fn, blocks, 256, 0,
                                              [[b, out, n // 2, per] for b in bufs], 10, iters)
                    sec = float(np.median(kms)) * 1e-3
                    if best is None or sec < best[0]:
                        best = (sec, blocks)
                rows.append({"mb": mb, "bytes": n * 8, "us": best[0] * 1e6,
                             "gb_per_s": n * 8 / best[0] / 1e9, "workgroups": best[1],
                             "copies": copies})
            finally:
                for b in bufs:
                    b.free()
    finally:
        out.free()
    return rows


def rowgather_probe(table_rows=(100_000, 6_250), n_groups: int = 100_000, per: int = 16,
                    rotate_mb: int = 640, iters: int = 50) -> List[dict]:
    """Random 512-byte row gathers (c4's B-row access: 100000 groups x 16
    rows from a 100000 x 64 fp64 table), cold (table copies rotated past the
    256 MB Infinity Cache) and warm (one copy)."""
    if per % 4:
        raise ValueError("per must be a multiple of 4")
    fn = _load(_ROWGATHER_SRC, ["mb_rowgather"])["mb_rowgather"]
    rng = np.random.default_rng(1)
    out = rt.DeviceBuffer(nbytes=n_groups * 512)
    grid = -(-n_groups * 32 // 256)
    rows = []
    try:
        for n in table_rows:
            idx = rng.integers(0, n, n_groups * per, dtype=np.int64)
            if idx.min() < 0 or idx.max() >= n:  # every gather stays inside the table
                raise AssertionError("index out of range")
            bi = rt.DeviceBuffer(idx)
            table = rng.uniform(-1, 1, (n, 64))
            try:
                for cold in (True, False):
                    copies = max(2, -(-(rotate_mb << 20) // table.nbytes)) if cold else 1
                    bufs = [rt.DeviceBuffer(table) for _ in range(copies)]
                    try:
                        kms, _ = rt.time_launches(fn, grid, 256, 0,
                                                  [[bi, b, out, n_groups, per] for b in bufs],
                                                  10, iters)
                    finally:
                        for b in bufs:
                            b.free()
                    sec = float(np.median(kms)) * 1e-3
                    g = n_groups * per
                    rows.append({"table_mb": table.nbytes / 1e6, "cold": cold, "copies": copies,
                                 "rows_gathered": g, "us": sec * 1e6,
                                 "g_rows_per_s": g / sec / 1e9,
                                 "gathered_gb_per_s": g * 512 / sec / 1e9,
                                 "written_gb_per_s": n_groups * 512 / sec / 1e9})
            finally:
                bi.free()
    finally:
        out.free()
    return rows


def flat_probe(rotate_mb: int = 1280, iters: int = 100, blocks=(128, 256),
               case: str = "c1") -> List[dict]:
    """A SpMV case's indices/data/x accesses with no row structure (see the
    module docstring), on that BASELINE matrix itself.  The nonzeros are taken
    in groups of 16; a tail of fewer than 16 is left out."""
    from .matrices import baseline_operands, make_baseline
    fn = _load(_FLAT_SRC, ["mb_flat"])["mb_flat"]
    A = make_baseline(case)
    M, N = A.shape
    nnz = int(A.nnz) // 16 * 16
    if nnz == 0:
        raise ValueError("the flat probe needs at least 16 nonzeros")
    indices = np.ascontiguousarray(A.indices[:nnz], dtype=np.int64)
    if indices.min() < 0 or indices.max() >= N:  # every gather stays inside x
        raise AssertionError("index out of range")
    data = np.ascontiguousarray(A.data[:nnz], dtype=np.float64)
    x = baseline_operands("spmv", M, N, 1)["x"]
    n_groups = nnz // 16
    per_copy = indices.nbytes + data.nbytes + x.nbytes
    want = {1: np.add.reduceat(data * x[indices], np.arange(0, nnz, 16)),
            0: np.add.reduceat(data * indices.astype(np.float64), np.arange(0, nnz, 16))}
    out = rt.DeviceBuffer(nbytes=n_groups * 8)
    rows = []
    try:
        for cold in (True, False):
            copies = max(2, -(-(rotate_mb << 20) // per_copy)) if cold else 1
            sets = [(rt.DeviceBuffer(indices), rt.DeviceBuffer(data), rt.DeviceBuffer(x))
                    for _ in range(copies)]
            try:
                for gather in (1, 0):
                    for block in blocks:
                        grid = -(-n_groups * 8 // block)
                        kms, _ = rt.time_launches(
                            fn, grid, block, 0,
                            [[bi, bv, bx, out, n_groups, gather] for bi, bv, bx in sets],
                            10, iters)
                        got = out.to_host(np.empty(n_groups))
                        err = float(np.abs(got - want[gather]).max()
                                    / max(np.abs(want[gather]).max(), 1e-300))
                        if not err <= 1e-12:
                            raise AssertionError("mb_flat result off by %.3e" % err)
                        sec = float(np.median(kms)) * 1e-3
                        streamed = indices.nbytes + data.nbytes + n_groups * 8
                        rows.append({"case": case, "cold": cold, "copies": copies,
                                     "gather": bool(gather),
                                     "block": block, "nnz": nnz, "us": sec * 1e6,
                                     "streamed_bytes": streamed,
                                     "streamed_gb_per_s": streamed / sec / 1e9,
                                     "g_gathers_per_s": (nnz / sec / 1e9) if gather else 0.0})
            finally:
                for st in sets:
                    for b in st:
                        b.free()
    finally:
        out.free()
    return rows


def render(gather: List[dict], stream: List[dict], device: str,
           rowgather: List[dict] = (), flat: List[dict] = ()) -> str:
    md = ["# Microbenchmarks (%s)" % device, "",
          "Written by `python -m tilegen_amd.microbench`; kernel times are medians of "
          "dispatch-attached events."]
    if gather:
        md += ["", "## Random 8-byte gathers from an 800 KB (L2-resident) array", "",
               "| kernel | active lanes / lanes routed through uniform loads | µs | "
               "G gathers/s | G gather instructions/s |", "|---|---:|---:|---:|---:|"]
        for r in gather:
            md.append("| %s | %d | %.2f | %.1f | %.2f |" % (
                r["kernel"], r["lanes_or_uniform"], r["us"], r["gathers_per_s"] / 1e9,
                r["gather_instr_per_s"] / 1e9))
    if stream:
        md += ["", "## Streaming 128-bit reads over cold copies", "",
               "| MB | µs | GB/s | workgroups |", "|---:|---:|---:|---:|"]
        for r in stream:
            md.append("| %d | %.2f | %.0f | %d |" % (r["mb"], r["us"], r["gb_per_s"],
                                                     r["workgroups"]))
    if rowgather:
        md += ["", "## Random 512-byte row gathers (SpMM's B rows: 100000 x 16 gathers, "
               "one 512-byte row written per 16)", "",
               "| table MB | inputs | µs | G rows/s | GB/s gathered | GB/s written |",
               "|---:|---|---:|---:|---:|---:|"]
        for r in rowgather:
            md.append("| %.1f | %s | %.2f | %.2f | %.0f | %.0f |" % (
                r["table_mb"], "cold (%d copies)" % r["copies"] if r["cold"] else "warm",
                r["us"], r["g_rows_per_s"], r["gathered_gb_per_s"], r["written_gb_per_s"]))
    if flat:
        md += ["", "## SpMV accesses without rows (the case's own indices and values, 16 "
               "nonzeros per 8-lane group, no row pointers, LDS or barriers)", "",
               "| case | inputs | x gathers | block | µs | GB/s streamed (indices, values, out) | "
               "G gathers/s |", "|---|---|---|---:|---:|---:|---:|"]
        for r in flat:
            md.append("| %s | %s | %s | %d | %.2f | %.0f | %s |" % (
                r.get("case", "c1"), "cold (%d copies)" % r["copies"] if r["cold"] else "warm",
                "yes" if r["gather"] else "no", r["block"], r["us"], r["streamed_gb_per_s"],
                "%.1f" % r["g_gathers_per_s"] if r["gather"] else "-"))
    return "\n".join(md) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="Gather and streaming-read microbenchmarks.")
    ap.add_argument("--out", default="results")
    ap.add_argument("--only", choices=["flat"], default=None,
                    help="run one probe and print its table (results/ is left as it is)")
    ap.add_argument("--flat-cases", default="c1,c2,c3a,c3b",
                    help="SpMV cases the flat probe runs on (comma-separated)")
    a = ap.parse_args(argv)
    if rt.device_count() < 1:
        print("microbench: no HIP device visible", file=sys.stderr)
        return 2
    dev = rt.device_info(0)
    cases = [c for c in a.flat_cases.split(",") if c]
    if a.only == "flat":
        print(render([], [], dev["arch"], flat=[r for c in cases for r in flat_probe(case=c)]),
              flush=True)
        return 0
    g = gather_probe()
    print("[microbench] gather done", flush=True)
    s = stream_probe()
    print("[microbench] stream done", flush=True)
    rg = rowgather_probe()
    print("[microbench] rowgather done", flush=True)
    fl = [r for c in cases for r in flat_probe(case=c)]
    os.makedirs(a.out, exist_ok=True)
    with open(os.path.join(a.out, "microbench.json"), "w") as fh:
        json.dump({"device": dev, "gather": g, "stream": s, "rowgather": rg, "flat": fl}, fh,
                  indent=1)
    with open(os.path.join(a.out, "microbench.md"), "w") as fh:
        fh.write(render(g, s, "%s %s" % (dev["name"], dev["arch"]), rg, fl))
    print(render(g, s, dev["arch"], rg, fl))
    return 0


if __name__ == "__main__":
    sys.exit(main())
