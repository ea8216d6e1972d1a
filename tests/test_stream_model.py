"""(CPU) The work split of the stream SpMV (``Config.balance == "stream"``) as a
model: which rows each range of nonzeros writes, which row pieces it commits
and which rows it sums whole, replayed from the same rules the emitted kernel
follows (``codegen._hip_stream_reduce``).

The rows' nonzeros are the positions [pbase, pend) = [indptr[0], indptr[M]):
indptr[0] may be nonzero (a block of rows of a larger matrix).  Range e stages
the positions [pa, pa + CH), pa = (pbase & ~1) + e CH, clipped to [p0, ps)
inside [pbase, pend), and owns the rows from the row holding p0 (row 0 for
e = 0) up to the row holding the next range's first position.  The grid comes
from the launch's nnz (floor(nnz / CH) + 1 workgroups), so only the first
NL = min(NR, grid) ranges exist: the last of them owns every row up to M and
sums, with its own loads, what lies past its staged positions (nothing when
nnz covers the rows' nonzeros).  For every matrix below the model checks:

* every row is finished exactly once: written whole by the one range that owns
  it, or combined from pieces, or (past the scratch) summed whole by its first
  range;
* a combined row has exactly one piece in each range it spans (its last range
  clamped to NL - 1), the pieces are disjoint and cover its nonzeros in range
  order, and their slots lie inside the scratch;
* a row written whole is covered by the owning range's own positions;
* the staged positions of the ranges are disjoint, lie inside [pbase, pend),
  and only the last range reads past them.

The matrices put the rules at their edges: empty rows before, between and after
the nonzeros, rows ending exactly at a range boundary, one row holding every
nonzero, no nonzeros at all, a count of nonzeros that is a multiple of the range,
a scratch so small that long rows take the whole-row path, the same rows as a
block of a larger matrix (indptr[0] odd and even), and launches whose nnz is
exact, too large, zero or too small.
"""

from __future__ import annotations

import bisect
from collections import Counter, defaultdict

import numpy as np
import pytest

from tilegen_amd import codegen as cg
from tilegen_amd.codegen import Config, generate
from tilegen_amd.dsl import standard_kernels
from tilegen_amd.schedules import TUNED


def _row_holding(indptr, p):
    """The row r with indptr[r] <= p < indptr[r + 1] (what tg_st_row returns)."""
    return bisect.bisect_right(indptr, p) - 1


def stream_split(indptr, CH, cap=cg.MERGE_CAP, nnz=None):
    """Replay the kernel's decisions for a launch with ``nnz`` (default: the
    rows' own count).  Returns (writes, pieces, whole, grid, staged):
    writes[r] = list of (range, lo, hi) covered by a whole-row write, pieces[r] =
    list of (range, lo, hi, slot) committed, whole[r] = ranges that sum r with
    their own loads, staged = (range, lo, hi, tail) per existing range."""
    indptr = [int(v) for v in indptr]
    M = len(indptr) - 1
    if M == 0:
        return defaultdict(list), defaultdict(list), Counter(), 0, []
    pbase, pend = indptr[0], indptr[M]
    if nnz is None:
        nnz = pend - pbase
    G = max(0, nnz) // CH + 1
    pal = pbase & ~1
    NR = -(-(pend - pal) // CH) if pend > pbase else 1
    NL = min(NR, G)
    writes, pieces, whole, staged = defaultdict(list), defaultdict(list), Counter(), []
    for e in range(NL):
        last = e == NL - 1
        pa = pal + e * CH
        p0, ps = max(pa, pbase), min(pa + CH, pend)
        p1 = pend if last else ps
        staged.append((e, p0, ps, last and p1 > ps))
        if e == 0:
            ra, ra_s, ra_e = 0, pbase, pbase
        else:
            ra = _row_holding(indptr, p0)
            ra_s, ra_e = indptr[ra], indptr[ra + 1]
        if p1 < pend:
            rb = _row_holding(indptr, p1)
            rb_s, rb_e = indptr[rb], indptr[rb + 1]
        else:
            rb, rb_s, rb_e = M, pend, pend
        ra_cut = e > 0 and ra < rb and ra_s < p0
        if ra_cut:
            ef = (ra_s - pal) // CH
            assert min((ra_e - 1 - pal) // CH, NL - 1) == e
            if e < cap:
                pieces[ra].append((e, p0, ra_e, 2 * e + (1 if e == ef else 0)))
        if rb < M and rb_s < p1:
            ef, el = (rb_s - pal) // CH, min((rb_e - 1 - pal) // CH, NL - 1)
            if el < cap:
                assert rb_e > ps and not last
                pieces[rb].append((e, max(rb_s, p0), p1, 2 * e + (1 if e == ef else 0)))
            elif ef == e:
                whole[rb] += 1
        for r in range(ra, rb):
            if r == ra and ra_cut:
                continue
            st, en = max(indptr[r], p0), indptr[r + 1]
            assert p0 <= st <= en <= p1 or (st == en), (e, r, st, en, p0, p1)
            writes[r].append((e, st, en))
    return writes, pieces, whole, G, staged


def check_split(indptr, CH, cap=cg.MERGE_CAP, nnz=None):
    writes, pieces, whole, G, staged = stream_split(indptr, CH, cap, nnz)
    indptr = [int(v) for v in indptr]
    M = len(indptr) - 1
    if M == 0:
        return G
    pbase, pend = indptr[0], indptr[M]
    pal = pbase & ~1
    NL = len(staged)
    for a, b in zip(staged, staged[1:]):
        assert a[2] == b[1] and not a[3], (a, b)   # disjoint, in order, no tail but the last
    assert staged[0][1] == pbase and staged[-1][2] <= pend
    assert all(pbase <= lo <= hi <= pend for _e, lo, hi, _t in staged)
    for r in range(M):
        s, t = indptr[r], indptr[r + 1]
        ways = (len(writes[r]) > 0) + (len(pieces[r]) > 0) + (whole[r] > 0)
        assert ways == 1, "row %d finished %d ways" % (r, ways)
        if writes[r]:
            assert len(writes[r]) == 1, "row %d written %d times" % (r, len(writes[r]))
            _e, lo, hi = writes[r][0]
            assert (lo, hi) == (s, t) or s == t, (r, lo, hi, s, t)
        elif whole[r]:
            assert whole[r] == 1
            assert min((t - 1 - pal) // CH, NL - 1) >= cap
        else:
            wf, wl = (s - pal) // CH, min((t - 1 - pal) // CH, NL - 1)
            assert wl > wf and wl < cap
            es = [p[0] for p in pieces[r]]
            assert sorted(es) == list(range(wf, wl + 1)), (r, es, wf, wl)
            spans = sorted((lo, hi) for _e, lo, hi, _s in pieces[r])
            assert spans[0][0] == s and spans[-1][1] == t
            for (a0, a1), (b0, b1) in zip(spans, spans[1:]):
                assert a1 == b0
            assert all(0 <= slot < 2 * cap for *_x, slot in pieces[r])
            assert len({slot for *_x, slot in pieces[r]}) == len(pieces[r])
    return G


def _views(ip, CH):
    """The same rows as a block of a larger matrix: indptr shifted by offsets of
    both parities, with launches whose nnz is exact, too large, zero and too
    small."""
    ip = np.asarray(ip, dtype=np.int64)
    own = int(ip[-1] - ip[0]) if len(ip) > 1 else 0
    for off in (0, 1, 2, 7, CH + 3):
        for nnz in (own, own + 5 * CH + 1, 0, own // 3):
            yield ip + off, nnz


def _indptr(lengths):
    return np.concatenate([[0], np.cumsum(np.asarray(lengths, dtype=np.int64))])


@pytest.mark.parametrize("CH", [1, 2, 7, 64, 512])
def test_edge_layouts(CH):
    cases = {
        "no_rows": [0],
        "no_nonzeros": [0] * 11,
        "one_row_all": _indptr([5 * CH + 3]),
        "one_row_exact": _indptr([4 * CH]),
        "empty_around": _indptr([0, 0, 3, 0, 0, CH, 0, 1, 0, 0]),
        "rows_end_on_boundaries": _indptr([CH, CH, 2 * CH, CH]),
        "row_ends_one_past": _indptr([CH + 1, CH - 1, CH]),
        "leading_and_trailing_empty": _indptr([0] * 5 + [2 * CH + 1] + [0] * 7),
        "singletons": _indptr([1] * (3 * CH + 2)),
    }
    for name, ip in cases.items():
        ip = np.asarray(ip, dtype=np.int64)
        G = check_split(ip, CH)
        M, nnz = len(ip) - 1, int(ip[-1])
        assert G == (0 if M == 0 else nnz // CH + 1), name
        for view, n in _views(ip, CH):
            check_split(view, CH, nnz=n)


@pytest.mark.parametrize("seed", range(12))
def test_random_skew(seed):
    rng = np.random.default_rng(seed)
    M = int(rng.integers(1, 400))
    lengths = np.minimum(rng.zipf(1.6, size=M) - 1, 3000)
    lengths[rng.random(M) < 0.2] = 0
    CH = int(rng.choice([3, 16, 64, 256, 512]))
    check_split(_indptr(lengths), CH)
    for view, n in _views(_indptr(lengths), CH):
        check_split(view, CH, nnz=n)
        check_split(view, CH, cap=3, nnz=n)


def test_scratch_edge_sends_long_rows_whole():
    """With room for only 4 ranges of slots, rows reaching past range 3 are
    summed whole by their first range and rows inside it are combined."""
    CH = 8
    ip = _indptr([3, 20, 2, 30, 0, 41, 5])
    writes, pieces, whole, _G, _st = stream_split(ip, CH, cap=4)
    assert pieces[1] and not whole[1]          # nonzeros 3..22: ranges 0..2
    assert whole[3] == 1 and not pieces[3]     # nonzeros 25..54: ranges 3..6
    assert whole[5] == 1                       # nonzeros 55..95
    check_split(ip, CH, cap=4)


def test_baseline_shapes():
    """The power-law and dense-row BASELINE patterns at the shipped range sizes."""
    from tilegen_amd.matrices import make_baseline
    for case, scale in (("c3a", 0.2), ("c3b", 0.5)):
        A = make_baseline(case, scale=scale)
        for CH in (256, 512, 1024):
            check_split(A.indptr, CH)


def test_emitted_geometry_matches_the_model():
    """The launcher's grid and the kernel's range size are the model's."""
    cfg = Config(tile_size=64, threads_per_row=4, unroll=2, block_size=256, balance="stream")
    g = generate(standard_kernels()["spmv"], cfg, "hip", write=False)
    geo = g.geometry
    assert geo.stream and geo.nnz_chunk == 512
    assert (geo.grid(0, 0), geo.grid(5, 0), geo.grid(5, 511), geo.grid(5, 512),
            geo.grid(5, 513)) == (0, 1, 1, 2, 2)
    assert "pa = pal + e * 512" in g.source
    assert "const tg_i64 pbase = tg_uniform(s_b[6]), pend = tg_uniform(s_b[7]);" in g.source
    # phase 1 runs first on the launch's own numbers, then again where they were wrong
    assert "const tg_i64 pa = e * 512, sb = 0, se = nnz;" in g.source
    assert "if (pbase != 0 || pend != nnz) {" in g.source
    assert "rows > 0 ? (nnz > 0 ? nnz : 0) / 512 + 1 : 0" in g.host_source
    assert "tg_launch_ordered" in g.host_source      # module scratch: ordered launches
    odd = generate(standard_kernels()["spmv"],
                   Config(tile_size=64, threads_per_row=64, unroll=3, block_size=1024,
                          balance="stream"), "hip", write=False)
    assert odd.geometry.nnz_chunk == 3072
    assert "2 * (" not in odd.source.split("1. this range")[1].split("if (threadIdx.x == 0)")[0]


def test_stream_schedule_checks():
    ok = Config(tile_size=64, threads_per_row=4, unroll=8, block_size=1024, balance="stream")
    generate(standard_kernels()["spmv"], ok, "hip", write=False)
    with pytest.raises(ValueError, match="stream ranges hold at most"):
        generate(standard_kernels()["spmv"],
                 Config(tile_size=64, threads_per_row=4, unroll=16, block_size=1024,
                        balance="stream"), "hip", write=False)
    with pytest.raises(ValueError, match="SpMV-shaped"):
        generate(standard_kernels()["spmm"],
                 Config(tile_size=64, threads_per_row=4, unroll=2, block_size=256,
                        balance="stream"), "hip", write=False)


def test_common_case_copy_has_no_general_case_code():
    """Phases 2-4 come twice: under indptr[0] = 0 and indptr[M] = nnz every range's
    staged positions end where its owned ones do (the model above: p1 == ps for every
    range when nnz is exact and the matrix starts at position 0), so that copy has no
    tail loads, no clamp of ranges past the grid and no partly-staged test; the copy for
    every other case keeps all three."""
    src = generate(standard_kernels()["spmv"], TUNED["c3a"], "hip", write=False).source
    body = src[src.index("__global__"):]
    i = body.index("if (pbase == 0 && pend == nnz) {")
    j = body.index("else {", i)
    fast, general = body[i:j], body[j:]
    assert "if (ps < p1)" not in fast and "NL - 1 ?" not in fast and "en <= qhi" not in fast
    assert general.count("if (ps < p1)") == 2 and "NL - 1 ?" in general and "en <= qhi" in general
    for M, nnz, CH in ((100, 4096 * 3 + 17, 4096), (7, 4096 * 2, 4096), (5, 0, 2048)):
        grid = nnz // CH + 1
        NR = (nnz + CH - 1) // CH if nnz > 0 else 1
        NL = min(NR, grid)
        for e in range(NL):
            pa = e * CH
            ps = min(pa + CH, nnz)
            p1 = nnz if e == NL - 1 else ps
            assert p1 == ps
