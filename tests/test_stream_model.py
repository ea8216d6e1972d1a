"""(CPU) The work split of the stream SpMV (``Config.balance == "stream"``) as a
model: which rows each range of nonzeros writes, which row pieces it commits
and which rows it sums whole, replayed from the same rules the emitted kernel
follows (``codegen._hip_stream_reduce``).

Range e holds nonzeros [e CH, (e+1) CH) and owns the rows from the row holding
its first nonzero (row 0 for e = 0) up to the row holding the next range's
first nonzero (M for the last range).  For every matrix below the model checks:

* every row is finished exactly once: written whole by the one range that owns
  it, or combined from pieces, or (past the scratch) summed whole by its first
  range;
* a combined row has exactly one piece in each range it spans, the pieces are
  disjoint and cover its nonzeros in range order, and their slots lie inside the
  scratch;
* a row written whole is covered by the owning range's own products.

The matrices put the rules at their edges: empty rows before, between and after
the nonzeros, rows ending exactly at a range boundary, one row holding every
nonzero, no nonzeros at all, a count of nonzeros that is a multiple of the range,
and a scratch so small that long rows take the whole-row path.
"""

from __future__ import annotations

import bisect
from collections import Counter, defaultdict

import numpy as np
import pytest

from tilegen_amd import codegen as cg
from tilegen_amd.codegen import Config, generate
from tilegen_amd.dsl import standard_kernels


def _row_holding(indptr, p):
    """The row r with indptr[r] <= p < indptr[r + 1] (what tg_mp_row returns)."""
    return bisect.bisect_right(indptr, p) - 1


def stream_split(indptr, CH, cap=cg.MERGE_CAP):
    """Replay the kernel's decisions.  Returns (writes, pieces, whole, grid):
    writes[r] = list of (range, lo, hi) covered by a whole-row write, pieces[r] =
    list of (range, lo, hi, slot) committed, whole[r] = ranges that sum r with
    their own loads."""
    indptr = [int(v) for v in indptr]
    M, nnz = len(indptr) - 1, indptr[-1]
    G = 0 if M == 0 else max(1, -(-nnz // CH))
    writes, pieces, whole = defaultdict(list), defaultdict(list), Counter()
    for e in range(G):
        p0, p1 = e * CH, min(e * CH + CH, nnz)
        if e == 0:
            ra, ra_s, ra_e = 0, 0, 0
        else:
            ra = _row_holding(indptr, p0)
            ra_s, ra_e = indptr[ra], indptr[ra + 1]
        if p1 < nnz:
            rb = _row_holding(indptr, p1)
            rb_s, rb_e = indptr[rb], indptr[rb + 1]
        else:
            rb, rb_s, rb_e = M, nnz, nnz
        ra_cut = e > 0 and ra < rb and ra_s < p0
        if ra_cut:
            ef, el = ra_s // CH, (ra_e - 1) // CH
            assert el == e
            if el < cap:
                pieces[ra].append((e, p0, ra_e, 2 * e + (1 if e == ef else 0)))
        if rb < M and rb_s < p1:
            ef, el = rb_s // CH, (rb_e - 1) // CH
            if el < cap:
                pieces[rb].append((e, max(rb_s, p0), p1, 2 * e + (1 if e == ef else 0)))
            elif ef == e:
                whole[rb] += 1
        for r in range(ra, rb):
            if r == ra and ra_cut:
                continue
            st, en = max(indptr[r], p0), indptr[r + 1]
            assert p0 <= st <= en <= p1 or (st == en), (e, r, st, en, p0, p1)
            writes[r].append((e, st, en))
    return writes, pieces, whole, G


def check_split(indptr, CH, cap=cg.MERGE_CAP):
    writes, pieces, whole, G = stream_split(indptr, CH, cap)
    M = len(indptr) - 1
    for r in range(M):
        s, t = int(indptr[r]), int(indptr[r + 1])
        ways = (len(writes[r]) > 0) + (len(pieces[r]) > 0) + (whole[r] > 0)
        assert ways == 1, "row %d finished %d ways" % (r, ways)
        if writes[r]:
            assert len(writes[r]) == 1, "row %d written %d times" % (r, len(writes[r]))
            _e, lo, hi = writes[r][0]
            assert (lo, hi) == (s, t) or s == t, (r, lo, hi, s, t)
        elif whole[r]:
            assert whole[r] == 1
            assert (t - 1) // CH >= cap
        else:
            wf, wl = s // CH, (t - 1) // CH
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
        assert G == (0 if M == 0 else max(1, -(-nnz // CH))), name


@pytest.mark.parametrize("seed", range(12))
def test_random_skew(seed):
    rng = np.random.default_rng(seed)
    M = int(rng.integers(1, 400))
    lengths = np.minimum(rng.zipf(1.6, size=M) - 1, 3000)
    lengths[rng.random(M) < 0.2] = 0
    CH = int(rng.choice([3, 16, 64, 256, 512]))
    check_split(_indptr(lengths), CH)


def test_scratch_edge_sends_long_rows_whole():
    """With room for only 4 ranges of slots, rows reaching past range 3 are
    summed whole by their first range and rows inside it are combined."""
    CH = 8
    ip = _indptr([3, 20, 2, 30, 0, 41, 5])
    writes, pieces, whole, _G = stream_split(ip, CH, cap=4)
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
    assert (geo.grid(0, 0), geo.grid(5, 0), geo.grid(5, 512), geo.grid(5, 513)) == (0, 1, 1, 2)
    assert "p0 = e * 512" in g.source
    assert "(nnz + 512 - 1) / 512 : 1) : 0" in g.host_source
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
