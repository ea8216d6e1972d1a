"""Hardware probes behind the measured ceilings of the CSR SpMV path on MI355X.

These kernels are not part of the product path: they time one access pattern
in isolation so that a kernel's time can be set against the floor of the loads
it has to make.  Each probe reads a BASELINE matrix's own ``indices`` and
``data``, rotates over enough input copies that every launch reads HBM, times
every launch with dispatch-attached events (the same ``tg_time_launches`` as
``bench.py``) and checks its own output against numpy.

``flat`` makes a SpMV's loads with no rows at all: workgroup w takes the
nonzeros [w CH, (w+1) CH), CH = BLK x U; lane t loads its U (index, value)
pairs as 128-bit loads at positions 2 (k BLK + t) + h (k < U/2, h in {0, 1}),
gathers ``x`` at each index, and SEG lanes sum their products into one output.
The gather instruction for (k, h) therefore covers, for the 64 lanes of one
wave, the items s = (2k + h) BLK + t of the range in the order the host laid
them out.

Orders (how the host lays out each range of CH nonzeros before upload):

* ``matrix``: the matrix's own order;
* ``b<S>``: sorted by ``col >> S`` (stable), then placed so that gather
  instruction j of wave w takes the sorted items j BLK + 64 w ... + 63, that is
  64 consecutive items of the sorted range.  This is the order a kernel would
  reach by counting-sorting each range in LDS; the probe pays none of that
  sort, so it bounds what such a kernel could gain;
* ``line``: the same with S = 4 (one 128-byte line of ``x`` per key);
* ``lsort``: the matrix order, sorted by the workgroup itself in LDS
  (``lsort_source``): what the host-sorted orders bound, with the sort paid.

Gather modes: ``x`` (``x[col]``), ``none`` (the index itself used as the
operand, so the index loads stay live but nothing is gathered) and ``one``
(``x[col & 7]``: every address in one line, so the gather's address work is
kept and its line traffic removed).

    python -m tilegen_amd.probes flat --case c1 --order matrix,b9,line \\
        --shape 1024x4,1024x8 [--gather x,none,one] [--json out.json]
    python -m tilegen_amd.probes --build          # compile every probe (no GPU)

``placement`` launches workgroups of a kernel's footprint (block, static LDS) at
several grid sizes and reports how many CUs took them and how many took two or
more (``run_placement``):

    python -m tilegen_amd.probes placement --grids 194,239,256 --block 1024 --lds 45264

``stream`` reads a buffer once with 128-bit loads, cold over rotated copies at each
size and re-reading one resident buffer (``run_stream``); ``rowgather`` makes SpMM's
512-byte row gathers from a 64-wide fp64 table, 16 per output row, with no values or
FMAs (``run_rowgather``):

    python -m tilegen_amd.probes stream --mib 8,27,128,512 --resident-mib 96
    python -m tilegen_amd.probes rowgather --table-rows 100000,6250

``gather`` makes random 8-byte loads from an L2-resident array of 100000 doubles at
addresses hashed in registers, with 64, 32 or 16 lanes of each wave active
(``run_gather``):

    python -m tilegen_amd.probes gather --active 64,32,16
"""

from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import sys
import time
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np

__all__ = ["flat_source", "flat_layout", "flat_expected", "gather_lines", "main"]

_GATHER = {"x": "x[c]", "none": "(double)c", "one": "x[c & 7]"}


def flat_source(name: str, blk: int, u: int, seg: int, gather: str) -> str:
    """HIP source of one ``flat`` probe kernel (``extern "C"`` ``name``)."""
    from .codegen import _HIP_PRELUDE
    if u % 2 or u < 2 or blk % 64 or seg not in (1, 2, 4, 8, 16, 32, 64):
        raise ValueError("flat probe needs an even U, a block of whole waves and SEG | 64")
    ch = blk * u
    lines = [_HIP_PRELUDE,
             '#define TG_GATHER(c) (%s)' % _GATHER[gather],
             'extern "C" __global__ __launch_bounds__(%d)' % blk,
             "void %s(const tg_i64* __restrict__ indices, const double* __restrict__ data," % name,
             "        const double* __restrict__ x, double* __restrict__ out, const tg_i64 nnz) {",
             "  const tg_i64 p0 = (tg_i64)blockIdx.x * %d;" % ch,
             "  const int cnt = (int)(nnz - p0 < %d ? nnz - p0 : %d);" % (ch, ch),
             "  const int t = threadIdx.x;",
             "  tg_i64 ci[%d]; double cv[%d];" % (u, u)]
    for k in range(u // 2):
        q = "2 * (%d + t)" % (k * blk)
        lines += ["  {",
                  "    const int q = %s;" % q,
                  "    if (q + 1 < cnt) {",
                  "      const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + p0 + q));",
                  "      const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + p0 + q));",
                  "      ci[%d] = a.x; ci[%d] = a.y; cv[%d] = b.x; cv[%d] = b.y;" % (2 * k, 2 * k + 1,
                                                                              2 * k, 2 * k + 1),
                  "    } else {",
                  "      ci[%d] = q < cnt ? indices[p0 + q] : 0;" % (2 * k),
                  "      cv[%d] = q < cnt ? data[p0 + q] : 0.0;" % (2 * k),
                  "      ci[%d] = 0; cv[%d] = 0.0;" % (2 * k + 1, 2 * k + 1),
                  "    }",
                  "  }"]
    lines.append("  double xv[%d];" % u)
    for j in range(u):
        lines.append("  { const tg_i64 c = ci[%d]; xv[%d] = TG_GATHER(c); }" % (j, j))
    lines.append("  double acc = 0.0;")
    for j in range(u):
        lines.append("  acc += cv[%d] * xv[%d];" % (j, j))
    lines += ["  acc = tg_segsum<%d>(acc);" % seg,
              "  if (t %% %d == 0) out[((tg_i64)blockIdx.x * %d + t) / %d] = acc;" % (seg, blk, seg),
              "}"]
    return "\n".join(lines) + "\n"


def lsort_source(name: str, blk: int, u: int, seg: int, nb: int) -> str:
    """HIP source of the ``lsort`` probe: the flat probe's loads and sums, with
    the gathers made in an order the workgroup sorts itself, in LDS.

    Each of the BLK x U nonzeros of a range gets a slot s = u BLK + t.  Keys are
    ``col >> shift`` (a kernel argument, so that NB buckets cover the columns):
    an LDS histogram (atomic adds that return each item's rank in its bucket),
    an exclusive scan over the NB buckets, then every item writes (col << 13 |
    slot) to its sorted place.  Lane t then gathers sorted entries k BLK + t,
    so the 64 lanes of a gather instruction take 64 consecutive sorted items,
    and stores x[col] at x_lds[slot]; each lane finally reads its own slots
    back and sums exactly as the flat probe does (same products, same order,
    same bits)."""
    from .codegen import _HIP_PRELUDE
    ch = blk * u
    if ch > 8192 or nb != blk or blk % 64 or u % 2:
        raise ValueError("lsort probe: BLK x U <= 8192, NB == BLK, even U")
    waves = blk // 64
    L = [_HIP_PRELUDE,
         'extern "C" __global__ __launch_bounds__(%d)' % blk,
         "void %s(const tg_i64* __restrict__ indices, const double* __restrict__ data," % name,
         "        const double* __restrict__ x, double* __restrict__ out, const tg_i64 nnz,",
         "        const int shift) {",
         "  __shared__ unsigned s_hist[%d];" % nb,
         "  __shared__ unsigned long long s_ent[%d];" % ch,
         "  __shared__ double s_x[%d];" % ch,
         "  __shared__ unsigned s_wsum[%d];" % waves,
         "  const tg_i64 p0 = (tg_i64)blockIdx.x * %d;" % ch,
         "  const int cnt = (int)(nnz - p0 < %d ? nnz - p0 : %d);" % (ch, ch),
         "  const int t = threadIdx.x, l = t & 63, wv = t >> 6;",
         "  s_hist[t] = 0u;",
         "  tg_i64 ci[%d]; double cv[%d];" % (u, u)]
    for k in range(u // 2):
        L += ["  {",
              "    const int q = 2 * (%d + t);" % (k * blk),
              "    if (q + 1 < cnt) {",
              "      const tg_i64x2 a = __builtin_nontemporal_load((const tg_i64x2*)(indices + p0 + q));",
              "      const tg_f64x2 b = __builtin_nontemporal_load((const tg_f64x2*)(data + p0 + q));",
              "      ci[%d] = a.x; ci[%d] = a.y; cv[%d] = b.x; cv[%d] = b.y;" % (2 * k, 2 * k + 1,
                                                                          2 * k, 2 * k + 1),
              "    } else {",
              "      ci[%d] = q < cnt ? indices[p0 + q] : 0;" % (2 * k),
              "      cv[%d] = q < cnt ? data[p0 + q] : 0.0;" % (2 * k),
              "      ci[%d] = 0; cv[%d] = 0.0;" % (2 * k + 1, 2 * k + 1),
              "    }",
              "  }"]
    L += ["  __syncthreads();",
          "  // each item's rank in its bucket",
          "  unsigned rk[%d]; int key[%d];" % (u, u)]
    for j in range(u):
        q = "2 * (%d + t) + %d" % ((j // 2) * blk, j % 2)
        L.append("  { const int q = %s; key[%d] = (int)(ci[%d] >> shift); "
                 "rk[%d] = q < cnt ? atomicAdd(&s_hist[key[%d]], 1u) : 0u; }" % (q, j, j, j, j))
    L += ["  __syncthreads();",
          "  // exclusive scan of the buckets: wave scans, then the waves' totals",
          "  {",
          "    const unsigned h = s_hist[t];",
          "    unsigned v = h;",
          "    #pragma unroll",
          "    for (int d = 1; d < 64; d <<= 1) { const unsigned o = __shfl_up(v, d); if (l >= d) v += o; }",
          "    if (l == 63) s_wsum[wv] = v;",
          "    __syncthreads();",
          "    unsigned base = 0;",
          "    for (int w = 0; w < wv; ++w) base += s_wsum[w];",
          "    s_hist[t] = base + v - h;",
          "  }",
          "  __syncthreads();"]
    for j in range(u):
        q = "2 * (%d + t) + %d" % ((j // 2) * blk, j % 2)
        L.append("  { const int q = %s; if (q < cnt) s_ent[s_hist[key[%d]] + rk[%d]] = "
                 "((unsigned long long)ci[%d] << 13) | (unsigned)(%d + t); }"
                 % (q, j, j, j, j * blk))
    L += ["  __syncthreads();",
          "  // gathers in sorted order: 64 consecutive sorted items per instruction"]
    for k in range(u):
        L.append("  { const int s = %d + t; if (s < cnt) { const unsigned long long e = s_ent[s]; "
                 "s_x[e & 8191u] = x[e >> 13]; } }" % (k * blk))
    L += ["  __syncthreads();",
          "  double acc = 0.0;"]
    for j in range(u):
        q = "2 * (%d + t) + %d" % ((j // 2) * blk, j % 2)
        L.append("  { const int q = %s; acc += cv[%d] * (q < cnt ? s_x[%d + t] : 0.0); }"
                 % (q, j, j * blk))
    L += ["  acc = tg_segsum<%d>(acc);" % seg,
          "  if (t %% %d == 0) out[((tg_i64)blockIdx.x * %d + t) / %d] = acc;" % (seg, blk, seg),
          "}"]
    return "\n".join(L) + "\n"


def _slot_of_sorted(blk: int, u: int) -> np.ndarray:
    """pos[s]: the position in a range of CH = blk*u nonzeros that the flat
    kernel's gather instruction j = s // blk, lane t = s % blk reads."""
    s = np.arange(blk * u)
    j, t = s // blk, s % blk
    return 2 * ((j // 2) * blk + t) + (j % 2)


def flat_layout(indices: np.ndarray, data: np.ndarray, blk: int, u: int, order: str
                ) -> Tuple[np.ndarray, np.ndarray]:
    """``indices``/``data`` laid out in ``order`` per range of blk*u nonzeros
    (the last, partial range keeps the matrix order)."""
    if order == "matrix":
        return indices.copy(), data.copy()
    shift = 4 if order == "line" else int(order[1:])
    ch = blk * u
    full = (len(indices) // ch) * ch
    ind, val = indices.copy(), data.copy()
    if full:
        ki = indices[:full].reshape(-1, ch)
        kv = data[:full].reshape(-1, ch)
        srt = np.argsort(ki >> shift, axis=1, kind="stable")
        si = np.take_along_axis(ki, srt, axis=1)
        sv = np.take_along_axis(kv, srt, axis=1)
        pos = _slot_of_sorted(blk, u)
        oi = np.empty_like(ki)
        ov = np.empty_like(kv)
        oi[:, pos] = si
        ov[:, pos] = sv
        ind[:full] = oi.ravel()
        val[:full] = ov.ravel()
    return ind, val


def flat_expected(ind: np.ndarray, val: np.ndarray, x: np.ndarray, blk: int, u: int, seg: int,
                  gather: str) -> np.ndarray:
    """What the flat kernel writes for the laid-out arrays."""
    ch = blk * u
    nnz = len(ind)
    grid = -(-nnz // ch)
    pi = np.zeros(grid * ch, dtype=np.int64)
    pv = np.zeros(grid * ch)
    pi[:nnz] = ind
    pv[:nnz] = val
    if gather == "x":
        g = x[pi]
    elif gather == "one":
        g = x[pi & 7]
    else:
        g = pi.astype(np.float64)
    prod = (pv * g).reshape(grid, u // 2, blk, 2)   # [range][pair k][lane t][half h]
    lane = prod.sum(axis=(1, 3))                      # [range][lane]
    return lane.reshape(grid, blk // seg, seg).sum(axis=2).ravel()


def gather_lines(ind: np.ndarray, blk: int, u: int) -> float:
    """Distinct 128-byte lines of ``x`` per gathered address, counted per
    64-lane gather instruction of the flat kernel (the L1->L2 requests that
    gather would make if no line were found in L1)."""
    ch = blk * u
    full = (len(ind) // ch) * ch
    if not full:
        return float("nan")
    r = ind[:full].reshape(-1, u // 2, blk // 64, 64, 2) >> 4   # [range][k][wave][lane][h]
    r = np.moveaxis(r, 4, 2).reshape(-1, 64)                     # one row per instruction
    r = np.sort(r, axis=1)
    distinct = 1 + (np.diff(r, axis=1) != 0).sum(axis=1)
    return float(distinct.sum() / r.size)


def _cache_dir() -> str:
    from .verify import cache_dir
    return cache_dir()


def _code_object(name: str, src: str) -> bytes:
    """hipRTC code object of ``src``, cached in the kernel cache by hash."""
    from . import runtime as rt
    from .verify import hiprtc_options
    opts = hiprtc_options()
    key = hashlib.sha1("\0".join([src] + opts).encode()).hexdigest()[:20]
    path = os.path.join(_cache_dir(), "%s_%s.co" % (name, key))
    if os.path.exists(path):
        with open(path, "rb") as fh:
            return fh.read()
    code, _log = rt.rtc_compile(src, name + ".hip", opts)
    tmp = path + ".tmp%d" % os.getpid()
    with open(tmp, "wb") as fh:
        fh.write(code)
    os.replace(tmp, path)
    return code


def _function(name: str, src: str) -> int:
    from . import runtime as rt
    code = _code_object(name, src)
    blob = ctypes.create_string_buffer(code, len(code))
    mod, fn = ctypes.c_void_p(), ctypes.c_void_p()
    rt.check(rt.lib().tg_module_load(blob, len(code), ctypes.byref(mod)), "tg_module_load")
    rt.check(rt.lib().tg_module_function(mod, name.encode(), ctypes.byref(fn)),
             "tg_module_function")
    return int(fn.value)


STREAM_BLOCK, STREAM_UNROLL = 256, 8


def stream_source(name: str) -> str:
    """``stream``: a plain read of n2 16-byte pairs.  Workgroup w reads the
    contiguous pairs [w BLK U, (w+1) BLK U), lane t the pairs k BLK + t, every load
    issued before any is used (the buffer is padded to whole workgroups, so no load
    is conditional); one double per wave is written so that the loads stay live."""
    blk, u = STREAM_BLOCK, STREAM_UNROLL
    L = ["typedef double tg_f64x2 __attribute__((ext_vector_type(2)));",
         'extern "C" __global__ __launch_bounds__(%d)' % blk,
         "void %s(const double* __restrict__ a, double* __restrict__ out) {" % name,
         "  const long long t = (long long)blockIdx.x * %d + threadIdx.x;" % blk,
         "  const tg_f64x2* p = (const tg_f64x2*)a + (long long)blockIdx.x * %d + threadIdx.x;"
         % (blk * u),
         "  tg_f64x2 v[%d];" % u]
    L += ["  v[%d] = __builtin_nontemporal_load(p + %d);" % (k, k * blk) for k in range(u)]
    L += ["  double s = 0.0;"]
    L += ["  s += v[%d].x + v[%d].y;" % (k, k) for k in range(u)]
    L += ["  for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d);",
          "  if ((threadIdx.x & 63) == 0) out[t >> 6] = s;",
          "}", ""]
    return "\n".join(L)


def run_stream(sizes_mib: Sequence[float], resident_mib: Sequence[float], warmup: int,
               iters: int) -> List[dict]:
    """Read rate of the ``stream`` probe: over rotated copies (cold, so every launch
    reads HBM) at each size, and re-reading one buffer (resident in the Infinity
    Cache when it fits its 256 MB)."""
    from . import runtime as rt
    from .profiling import bench_copies
    name = "probe_stream_b%du%d" % (STREAM_BLOCK, STREAM_UNROLL)
    fn = _function(name, stream_source(name))
    per_launch = STREAM_BLOCK * STREAM_UNROLL      # pairs per workgroup
    out = []
    for mode, sizes in (("cold", sizes_mib), ("resident", resident_mib)):
        for mib in sizes:
            grid = max(1, int(round(mib * (1 << 20) / (16 * per_launch))))
            n2 = grid * per_launch
            copies = bench_copies(16 * n2) if mode == "cold" else 1
            rng = np.random.default_rng(7)
            host = rng.uniform(-1, 1, 2 * n2)
            bufs = [rt.DeviceBuffer(host) for _ in range(copies)]
            outs = [rt.DeviceBuffer(nbytes=grid * STREAM_BLOCK // 64 * 8) for _ in range(copies)]
            sets = [[b, o] for b, o in zip(bufs, outs)]
            rt.launch(fn, grid, STREAM_BLOCK, 0, sets[0])
            got = float(outs[0].to_host(np.empty(grid * STREAM_BLOCK // 64)).sum())
            want = float(host.sum())
            assert abs(got - want) <= 1e-9 * max(1.0, float(np.abs(host).sum())), (got, want)
            kms, _ = rt.time_launches(fn, grid, STREAM_BLOCK, 0, sets, warmup, iters)
            us = float(np.mean(kms)) * 1e3
            out.append({"probe": "stream", "mode": mode, "mib": round(16 * n2 / (1 << 20), 2),
                        "copies": copies, "us_avg": round(us, 3),
                        "us_median": round(float(np.median(kms)) * 1e3, 3),
                        "tb_s": round(16 * n2 / (us * 1e-6) / 1e12, 3)})
            for b in bufs + outs:
                b.free()
    return out


GATHER_BLOCK, GATHER_PER_LANE = 256, 64


def gather_source(name: str, active: int) -> str:
    """``gather``: random 8-byte loads from an array of n doubles (L2-resident at
    0.8 MB).  The first ``active`` lanes of each wave make GATHER_PER_LANE loads at
    indices hashed in registers (no index stream), 8 in flight; one double per wave
    is written so that the loads stay live."""
    return "\n".join([
        'extern "C" __global__ __launch_bounds__(%d)' % GATHER_BLOCK,
        "void %s(const double* __restrict__ x, double* __restrict__ out, const unsigned n) {"
        % name,
        "  const unsigned t = blockIdx.x * %du + threadIdx.x;" % GATHER_BLOCK,
        "  double s = 0.0;",
        "  if ((threadIdx.x & 63) < %d) {" % active,
        "    unsigned h = t * 0x9E3779B9u + 0x7F4A7C15u;",
        "    #pragma unroll 1",
        "    for (int k = 0; k < %d; k += 8) {" % GATHER_PER_LANE,
        "      double v[8];",
        "      #pragma unroll",
        "      for (int j = 0; j < 8; ++j) {",
        "        h ^= h << 13; h ^= h >> 17; h ^= h << 5;   // xorshift32",
        "        v[j] = x[h % n];",
        "      }",
        "      #pragma unroll",
        "      for (int j = 0; j < 8; ++j) s += v[j];",
        "    }",
        "  }",
        "  for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d);",
        "  if ((threadIdx.x & 63) == 0) out[t >> 6] = s;",
        "}", ""])


def gather_expected(grid: int, active: int, x: np.ndarray) -> np.ndarray:
    """What the gather probe writes: per wave, the sum of its active lanes' loads."""
    n = np.uint32(len(x))
    lanes = np.arange(grid * GATHER_BLOCK, dtype=np.uint64)
    act = (lanes & 63) < active
    h = ((lanes * 0x9E3779B9 + 0x7F4A7C15) & 0xFFFFFFFF).astype(np.uint32)
    s = np.zeros(lanes.size)
    for _ in range(GATHER_PER_LANE):
        h ^= h << np.uint32(13)
        h ^= h >> np.uint32(17)
        h ^= h << np.uint32(5)
        s += np.where(act, x[h % n], 0.0)
    return s.reshape(-1, 64).sum(axis=1)


def run_gather(actives: Sequence[int], n: int, waves: int, warmup: int, iters: int
               ) -> List[dict]:
    """Random-gather rate (G gathered addresses per second) from an n-double array."""
    from . import runtime as rt
    x = np.random.default_rng(5).uniform(-1, 1, n)
    bx = rt.DeviceBuffer(x)
    grid = max(1, waves * 64 // GATHER_BLOCK)
    bout = rt.DeviceBuffer(nbytes=grid * GATHER_BLOCK // 64 * 8)
    out = []
    for a in actives:
        name = "probe_gather_a%d" % a
        fn = _function(name, gather_source(name, a))
        args = [bx, bout, np.uint32(n)]
        rt.launch(fn, grid, GATHER_BLOCK, 0, args)
        got = bout.to_host(np.empty(grid * GATHER_BLOCK // 64))
        assert np.allclose(got, gather_expected(grid, a, x), rtol=1e-10, atol=1e-10)
        kms, _ = rt.time_launches(fn, grid, GATHER_BLOCK, 0, [args], warmup, iters)
        us = float(np.mean(kms)) * 1e3
        g = grid * GATHER_BLOCK // 64 * a * GATHER_PER_LANE
        out.append({"probe": "gather", "active_lanes": a, "array_kb": n * 8 // 1024,
                    "gathers": g, "us_avg": round(us, 3),
                    "g_gathers_per_s": round(g / (us * 1e-6) / 1e9, 1)})
    bx.free()
    bout.free()
    return out


ROWGATHER_ROW_NNZ = 16


def rowgather_source(name: str) -> str:
    """``rowgather``: SpMM's row gathers without values or FMAs.  A 32-lane group
    takes one output row of ROWGATHER_ROW_NNZ column indices; lane j loads 16 bytes
    of each gathered 512-byte row of the 64-wide table, four rows in flight, adds
    them and writes its 16 bytes of the output row."""
    L = ["typedef double tg_f64x2 __attribute__((ext_vector_type(2)));",
         'extern "C" __global__ __launch_bounds__(256)',
         "void %s(const long long* __restrict__ cols, const double* __restrict__ B," % name,
         "        double* __restrict__ C, const long long M) {",
         "  const long long row = (long long)blockIdx.x * 8 + (threadIdx.x >> 5);",
         "  const int j = threadIdx.x & 31;",
         "  if (row >= M) return;",
         "  const long long* c = cols + row * %d;" % ROWGATHER_ROW_NNZ,
         "  tg_f64x2 acc = {0.0, 0.0};",
         "  #pragma unroll",
         "  for (int q = 0; q < %d; q += 4) {" % ROWGATHER_ROW_NNZ,
         "    long long cc[4];",
         "    #pragma unroll",
         "    for (int k = 0; k < 4; ++k) cc[k] = c[q + k];",
         "    tg_f64x2 v[4];",
         "    #pragma unroll",
         "    for (int k = 0; k < 4; ++k) v[k] = *((const tg_f64x2*)(B + cc[k] * 64) + j);",
         "    #pragma unroll",
         "    for (int k = 0; k < 4; ++k) acc += v[k];",
         "  }",
         "  __builtin_nontemporal_store(acc, (tg_f64x2*)(C + row * 64) + j);",
         "}", ""]
    return "\n".join(L)


def run_rowgather(table_rows: Sequence[int], M: int, warmup: int, iters: int,
                  seed: int = 11) -> List[dict]:
    """Gathered rate of the ``rowgather`` probe: M x 16 random rows of a
    table_rows x 64 fp64 table, cold (rotated copies of table, indices and output)."""
    from . import runtime as rt
    from .profiling import bench_copies
    name = "probe_rowgather"
    fn = _function(name, rowgather_source(name))
    out = []
    for n in table_rows:
        rng = np.random.default_rng(seed)
        cols = rng.integers(0, n, M * ROWGATHER_ROW_NNZ).astype(np.int64)
        table = rng.uniform(-1, 1, (n, 64))
        nbytes = 8 * cols.size + 8 * table.size + 8 * M * 64
        copies = bench_copies(nbytes)
        sets = [[rt.DeviceBuffer(cols), rt.DeviceBuffer(table), rt.DeviceBuffer(nbytes=M * 64 * 8), M]
                for _ in range(copies)]
        grid = -(-M // 8)
        rt.launch(fn, grid, 256, 0, sets[0])
        got = sets[0][2].to_host(np.empty((M, 64)))
        want = table[cols].reshape(M, ROWGATHER_ROW_NNZ, 64).sum(axis=1)
        assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
        kms, _ = rt.time_launches(fn, grid, 256, 0, sets, warmup, iters)
        us = float(np.mean(kms)) * 1e3
        out.append({"probe": "rowgather", "table_mb": round(8 * table.size / 1e6, 1),
                    "gathers": int(cols.size), "copies": copies, "us_avg": round(us, 3),
                    "us_median": round(float(np.median(kms)) * 1e3, 3),
                    "gathered_tb_s": round(cols.size * 512 / (us * 1e-6) / 1e12, 3)})
        for st in sets:
            for b in st[:3]:
                b.free()
    return out


def placement_source(name: str, blk: int, lds_bytes: int, spin_ticks: int) -> str:
    """``placement``: where the dispatcher puts the workgroups of a grid.  Each
    workgroup of ``blk`` lanes and ``lds_bytes`` of static LDS (the footprint of the
    kernel whose placement is in question) records its XCC and hardware id
    (``HW_REG_XCC_ID``, ``HW_REG_HW_ID``: SIMD, CU, shader array and engine) and its
    start time, then stays resident for ``spin_ticks`` of the 100 MHz real-time
    clock (at most 2^22 polls), so that the whole grid is resident at once."""
    return "\n".join([
        "typedef unsigned long long u64;",
        'extern "C" __global__ __launch_bounds__(%d)' % blk,
        "void %s(u64* __restrict__ rec, const int pad_index) {" % name,
        "  __shared__ unsigned char s_pad[%d];" % lds_bytes,
        "  unsigned hw, xcc;",
        '  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));',
        '  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));',
        "  const u64 t0 = __builtin_amdgcn_s_memrealtime();",
        "  // keep the LDS allocation: one byte written, read back after the barrier",
        "  if (threadIdx.x == 0) s_pad[pad_index] = 1;",
        "  __syncthreads();",
        "  #pragma unroll 1",
        "  for (int i = 0; i < (1 << 22); ++i)",
        "    if (__builtin_amdgcn_s_memrealtime() - t0 >= %dull) break;" % spin_ticks,
        "  if (threadIdx.x == 0) {",
        "    rec[3 * blockIdx.x] = ((u64)(xcc & 0xffffu) << 32) | hw;",
        "    rec[3 * blockIdx.x + 1] = t0;",
        "    rec[3 * blockIdx.x + 2] = s_pad[pad_index];",
        "  }",
        "}",
        ""])


def placement_cu(rec_word: int) -> Tuple[int, int]:
    """(XCC, CU key) of a placement record: the HW_ID bits above the wave's SIMD and
    slot (CU, shader array, shader engine, bits 8-15)."""
    return int(rec_word >> 32) & 0xF, (int(rec_word) >> 8) & 0xFF


def run_placement(grids: Sequence[int], blk: int, lds_bytes: int,
                  spin_ticks: int = 2000) -> List[dict]:
    """Launch the placement probe at each grid size; per grid, how many CUs took
    workgroups and how many took more than one."""
    from . import runtime as rt
    name = "probe_placement_b%d_l%d" % (blk, lds_bytes)
    fn = _function(name, placement_source(name, blk, lds_bytes, spin_ticks))
    out = []
    for g in grids:
        buf = rt.DeviceBuffer(np.zeros(3 * g, dtype=np.uint64))
        pad = np.int32(lds_bytes - 1)
        rt.launch(fn, g, blk, 0, [buf, pad])
        rt.synchronize()
        rec = buf.to_host().view(np.uint64).reshape(g, 3)
        buf.free()
        cus = {}
        for b in range(g):
            cus.setdefault(placement_cu(int(rec[b, 0])), []).append(b)
        per = np.bincount([len(v) for v in cus.values()])
        xcc_of = [placement_cu(int(rec[b, 0]))[0] for b in range(g)]
        out.append({"grid": g, "block": blk, "lds_bytes": lds_bytes, "cus": len(cus),
                    "max_per_cu": int(max(len(v) for v in cus.values())),
                    "cus_with_2_or_more": int(sum(per[2:])) if len(per) > 2 else 0,
                    "xcc_is_block_mod_8": all(xcc_of[b] == b % 8 for b in range(g)),
                    "all_loaded_pad": bool(np.all(rec[:, 2] == 1)),
                    "start_spread_us": float((rec[:, 1].max() - rec[:, 1].min()) / 100.0)})
    return out


def _shapes(text: str) -> List[Tuple[int, int]]:
    out = []
    for part in text.split(","):
        b, u = part.lower().split("x")
        out.append((int(b), int(u)))
    return out


def _variants(orders: Sequence[str], shapes: Sequence[Tuple[int, int]],
              gathers: Sequence[str], seg: int) -> List[Tuple[str, str, int, int, str]]:
    """(kernel name, order, blk, u, gather); every order has a kernel of its
    own name, so a rocprofv3 run tells them apart.  Order ``lsort`` is the
    matrix layout sorted by the workgroup itself (``lsort_source``)."""
    out = []
    for blk, u in shapes:
        for g in gathers:
            for o in (orders if g == "x" else ("matrix",)):
                if o == "lsort" and (blk * u > 8192 or u % 2):
                    continue
                out.append(("probe_flat_%s_%s_b%du%d" % (g, o, blk, u), o, blk, u, g))
    return out


def _source(name: str, order: str, blk: int, u: int, seg: int, g: str) -> str:
    if order == "lsort":
        return lsort_source(name, blk, u, seg, blk)
    return flat_source(name, blk, u, seg, g)


def lsort_shift(N: int, nb: int) -> int:
    """The smallest shift that maps columns 0..N-1 onto fewer than nb buckets."""
    s = 0
    while ((max(N, 1) - 1) >> s) >= nb:
        s += 1
    return s


def build(orders=("matrix", "b9", "line", "lsort"), shapes=((1024, 4), (1024, 8), (512, 8)),
          gathers=("x", "none", "one"), seg: int = 4, others: bool = True) -> int:
    """Compile the flat probe's variants and (``others``) the placement, stream,
    rowgather and gather probes into the kernel cache; returns how many."""
    n = 0
    for name, o, blk, u, g in _variants(orders, shapes, gathers, seg):
        _code_object(name, _source(name, o, blk, u, seg, g))
        n += 1
    if others:
        for blk, lds in ((1024, 45264), (512, 28816)):
            nm = "probe_placement_b%d_l%d" % (blk, lds)
            _code_object(nm, placement_source(nm, blk, lds, 2000))
        nm = "probe_stream_b%du%d" % (STREAM_BLOCK, STREAM_UNROLL)
        _code_object(nm, stream_source(nm))
        _code_object("probe_rowgather", rowgather_source("probe_rowgather"))
        for act in (64, 32, 16):
            _code_object("probe_gather_a%d" % act, gather_source("probe_gather_a%d" % act, act))
        n += 7
    return n


def run_flat(case_id: str, orders: Sequence[str], shapes: Sequence[Tuple[int, int]],
             gathers: Sequence[str], seg: int, warmup: int, iters: int, repeats: int,
             control: bool) -> List[Dict[str, object]]:
    from . import runtime as rt
    from .matrices import baseline_case, baseline_operands, compulsory_bytes, make_baseline
    from .profiling import bench_copies
    A = make_baseline(case_id)
    case = baseline_case(case_id)
    if case.kernel != "spmv":
        raise SystemExit("the flat probe takes an SpMV case")
    M, N = A.shape
    nnz = int(A.nnz)
    x = baseline_operands("spmv", M, N, 1)["x"]
    ind0 = A.indices.astype(np.int64)
    val0 = A.data.astype(np.float64)
    nbytes = compulsory_bytes("spmv", M, N, nnz)
    copies = bench_copies(nbytes)
    print("[probe] %s M=%d N=%d nnz=%d, %d copies" % (case_id, M, N, nnz, copies), flush=True)
    variants = _variants(orders, shapes, gathers, seg)
    layouts: Dict[Tuple[str, int, int], Tuple[list, np.ndarray, np.ndarray, float]] = {}
    xs = [rt.DeviceBuffer(x) for _ in range(copies)]
    records = []
    timed: Dict[str, List[np.ndarray]] = {}
    meta: Dict[str, Dict[str, object]] = {}
    tuned = None
    if control:
        from .schedules import TUNED
        from .variant import Variant
        v = Variant("spmv", TUNED[case_id])
        bufs = []
        for c in range(copies):
            b = {"indptr": rt.DeviceBuffer(A.indptr.astype(np.int64)),
                 "indices": rt.DeviceBuffer(ind0), "data": rt.DeviceBuffer(val0),
                 "x": xs[c], "y": rt.DeviceBuffer(nbytes=M * 8)}
            bufs.append(b)
        sets = [v.abi_values(A, b, {}, M, N, case.K, nnz) for b in bufs]
        g, bl, lds = v.geometry(M, N, case.K, nnz)
        tuned = (v.function(), g, bl, lds, sets, bufs, TUNED[case_id].short())
    for _rep in range(repeats):
        if tuned is not None:
            fn, g, bl, lds, sets, _b, sched = tuned
            kms, _ = rt.time_launches(fn, g, bl, lds, sets, warmup, iters)
            timed.setdefault("tuned", []).append(kms)
            meta["tuned"] = {"kernel": "spmv tuned " + sched, "order": "matrix"}
            print("[probe] tuned %s: avg %.2f us median %.2f us" % (
                sched, kms.mean() * 1e3, np.median(kms) * 1e3), flush=True)
        for name, order, blk, u, g in variants:
            key = (order, blk, u)
            if key not in layouts:
                ind, val = flat_layout(ind0, val0, blk, u,
                                       "matrix" if order == "lsort" else order)
                dev = [(rt.DeviceBuffer(ind), rt.DeviceBuffer(val)) for _ in range(copies)]
                layouts[key] = (dev, ind, val, gather_lines(ind, blk, u))
            dev, ind, val, lpg = layouts[key]
            fn = _function(name, _source(name, order, blk, u, seg, g))
            ch = blk * u
            grid = -(-nnz // ch)
            out = rt.DeviceBuffer(nbytes=grid * (blk // seg) * 8)
            extra = [lsort_shift(N, blk)] if order == "lsort" else []
            sets = [[dev[c][0], dev[c][1], xs[c], out, nnz] + extra for c in range(copies)]
            kms, _ = rt.time_launches(fn, grid, blk, 0, sets, warmup, iters)
            got = out.to_host(np.empty(grid * (blk // seg)))
            exp = flat_expected(ind, val, x, blk, u, seg, g)
            err = float(np.abs(got - exp).max() / max(np.abs(exp).max(), 1e-300))
            out.free()
            if not err <= 1e-12:
                raise SystemExit("probe %s output check failed: rel err %.3e" % (name, err))
            timed.setdefault(name, []).append(kms)
            meta[name] = {"order": order, "block": blk, "unroll": u, "range": ch, "grid": grid,
                          "gather": g, "lines_per_gather": round(lpg, 4), "err": err}
            print("[probe] %-34s avg %.2f us median %.2f us (lines/gather %.3f, err %.1e)" % (
                name, kms.mean() * 1e3, np.median(kms) * 1e3, lpg, err), flush=True)
    for name, runs in timed.items():
        rec = dict(meta[name])
        rec.update({"name": name, "case": case_id,
                    "us_avg": [round(float(k.mean()) * 1e3, 3) for k in runs],
                    "us_median": [round(float(np.median(k)) * 1e3, 3) for k in runs],
                    "launches": iters, "copies": copies})
        records.append(rec)
    return records


def main(argv: Optional[Sequence[str]] = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("probe", nargs="?",
                    choices=["flat", "placement", "stream", "rowgather", "gather"], default="flat")
    ap.add_argument("--active", default="64,32,16", help="gather: active lanes per wave")
    ap.add_argument("--waves", type=int, default=65536, help="gather: waves launched")
    ap.add_argument("--mib", default="8,27,128,512", help="stream: cold read sizes (MiB)")
    ap.add_argument("--resident-mib", default="96", help="stream: re-read sizes (MiB)")
    ap.add_argument("--table-rows", default="100000,6250", help="rowgather: table rows")
    ap.add_argument("--rows", type=int, default=100000, help="rowgather: output rows")
    ap.add_argument("--grids", default="194,207,222,239,250,256,259",
                    help="placement: grid sizes")
    ap.add_argument("--block", type=int, default=1024, help="placement: workgroup size")
    ap.add_argument("--lds", type=int, default=45264, help="placement: static LDS bytes")
    ap.add_argument("--build", action="store_true", help="compile the probes and exit")
    ap.add_argument("--case", default="c1")
    ap.add_argument("--order", default="matrix,b9,line",
                    help="matrix, line, b<shift> (host-sorted) or lsort (sorted in LDS)")
    ap.add_argument("--shape", default="1024x4,1024x8,512x8",
                    help="BLOCKxU per probe (U nonzeros per lane, even)")
    ap.add_argument("--gather", default="x,none,one")
    ap.add_argument("--seg", type=int, default=4, help="lanes summed into one output")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iters", type=int, default=200)
    ap.add_argument("--repeats", type=int, default=3, help="interleaved repeats")
    ap.add_argument("--no-control", action="store_true",
                    help="skip the tuned product kernel timed beside the probes")
    ap.add_argument("--json", default=None, help="also write the records here")
    args = ap.parse_args(argv)
    orders = [o for o in args.order.split(",") if o]
    for o in orders:
        if o not in ("matrix", "line", "lsort") and not (o[0] == "b" and o[1:].isdigit()):
            raise SystemExit("bad order %r (matrix, line or b<shift>)" % o)
    shapes = _shapes(args.shape)
    gathers = [g for g in args.gather.split(",") if g]
    if args.build:
        t0 = time.time()
        n = build(orders, shapes, gathers, args.seg)
        print("built %d probe code objects in %.1fs" % (n, time.time() - t0))
        return 0
    if args.probe == "placement":
        grids = [int(g) for g in args.grids.split(",") if g]
        recs = run_placement(grids, args.block, args.lds)
    elif args.probe == "stream":
        recs = run_stream([float(m) for m in args.mib.split(",") if m],
                          [float(m) for m in args.resident_mib.split(",") if m],
                          args.warmup, args.iters)
    elif args.probe == "gather":
        recs = run_gather([int(a) for a in args.active.split(",") if a], 100000, args.waves,
                          args.warmup, args.iters)
    elif args.probe == "rowgather":
        recs = run_rowgather([int(n) for n in args.table_rows.split(",") if n], args.rows,
                             args.warmup, args.iters)
    else:
        recs = run_flat(args.case, orders, shapes, gathers, args.seg, args.warmup, args.iters,
                        args.repeats, not args.no_control)
    for r in recs:
        print(json.dumps(r, separators=(",", ":")), flush=True)
    if args.json:
        with open(args.json, "w") as fh:
            json.dump(recs, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
