"""(CPU) The merge-path partition of the nnz-balanced SpMV kernels.

``mp_search`` restates the device search ``tg_mp_search`` lane for lane (64
probes per round ascending with the lane, the same first-round pattern,
clamping, and the bracket update from the ballot's first passing lane);
``partition`` restates the window set-up the emitter writes for every
workgroup (window bounds, first/last row, the pieces of rows longer than a
window, the rows summed whole).  The tests check them against what the
mathematics fixes, on skewed, empty-row, single-row and no-nonzero matrices
and on several grid sizes:

* the search returns the exact lower bound ``numpy.searchsorted`` gives, its
  probes stay inside the row-pointer array, and it ends within
  ``2 + ceil(log63(rows + 1))`` rounds;
* every nonzero of every row is summed exactly once: rows summed whole belong
  to exactly one window, and the pieces of a cut row tile its nonzeros with no
  gap or overlap, one piece per window from its first window to its last;
* no window holds two pieces of the same kind (its two scratch slots), and no
  window's work exceeds two windows' worth of items;
* rows that reach past the scratch capacity are summed whole by their first
  window and by no other.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from tests.util import ragged, range_edge_matrix
from tilegen_amd import codegen as cg
from tilegen_amd.codegen import Config
from tilegen_amd.matrices import make_baseline


def first_probes(g: int):
    """The first round's probe of each lane around the guess g (``tg_mp_probe``):
    8 rows at growing distances below, 48 consecutive, 8 at growing distances
    above, ascending with the lane."""
    return [g - 24 - (32 << (2 * (7 - l))) if l < 8 else
            (g - 32 + l if l < 56 else g + 24 + (32 << (2 * (l - 56)))) for l in range(64)]


def _ends(qs, passed):
    """The lanes the ballot names: the first that passes (None: none) and the
    one before it (None: the first lane passes).  The probes ascend with the
    lane and the test is monotone in the row, so the passing lanes are exactly
    the lanes from the first on."""
    assert all(qs[i] <= qs[i + 1] for i in range(63)), "probes must ascend with the lane"
    f = next((i for i, p in enumerate(passed) if p), None)
    assert f is None or all(passed[f:]), "the test must be monotone in the probed row"
    return f, (63 if f is None else (f - 1 if f > 0 else None))


def mp_search(indptr, R: int, t: int, X: int, base: int = 0):
    """Lane-for-lane model of ``tg_mp_search``: (answer, rounds, probed rows);
    items are counted from ``base`` = indptr[0]."""
    g = int(float(t) * (float(R) / float(X))) if X > 0 else 0
    qs = first_probes(g)
    lo, hi, rounds, probed = 0, R, 0, set()
    while True:
        rounds += 1
        qs = [min(max(q, lo), hi) for q in qs]
        probed.update(qs)
        f, fa = _ends(qs, [q + int(indptr[q]) - base >= t for q in qs])
        b = qs[f] if f is not None else hi
        a = qs[fa] if fa is not None else lo - 1
        lo, hi = a + 1, b
        if lo >= hi:
            return hi, rounds, probed
        s = (hi - lo + 62) // 63
        qs = [lo + l * s for l in range(64)]


def lower_bound(indptr, R: int, t: int) -> int:
    f = np.arange(R + 1, dtype=np.int64) + np.asarray(indptr[:R + 1], dtype=np.int64) \
        - int(indptr[0])
    return min(int(np.searchsorted(f, t, side="left")), R)


def partition(indptr, M: int, G: int, cap: int = cg.MERGE_CAP):
    """The emitter's per-workgroup window set-up for every workgroup: a list of
    (rows summed whole, pieces) with pieces as (row, begin, end, wf, wl, w).
    Items count from pbase = indptr[0] (a block of rows of a larger matrix)."""
    pbase = int(indptr[0])
    nnz = int(indptr[M]) - pbase
    X = M + nnz
    D = (X + G - 1) // G if X > G else 1
    ip = lambda r: int(indptr[r]) if r >= 0 else 0  # noqa: E731
    out = []
    for w in range(G):
        t0 = min(w * D, X)
        t1 = min(t0 + D, X)
        r0 = 0 if w == 0 else mp_search(indptr, M, t0, X, pbase)[0]
        r1 = M if w == G - 1 else mp_search(indptr, M, t1, X, pbase)[0]
        s2, s3, s4, s5 = ip(r0 - 1), ip(r0), ip(r1 - 1), ip(r1)
        pc_in = (r0 > 0 and s3 - s2 > D and (r0 - 1 + s3 - pbase - 1) // D < cap
                 and r0 - 1 + s3 - pbase > t0)
        pc_out = r1 > r0 and s5 - s4 > D and (r1 - 1 + s5 - pbase - 1) // D < cap
        r_own = r1 - 1 if pc_out else r1
        pieces = []
        for k, on in ((0, pc_in), (1, pc_out)):
            if not on:
                continue
            row = r0 - 1 if k == 0 else r1 - 1
            pb, pe = (s2, s3) if k == 0 else (s4, s5)
            c0 = t0 - row + pbase if k == 0 and t0 - row + pbase > pb else pb
            c1 = min(t1 - row + pbase, pe)
            pieces.append((row, c0, c1, (row + pb - pbase) // D, (row + pe - 1 - pbase) // D, w))
        out.append((range(r0, r_own), pieces, D))
    return out


def check_partition(indptr, M: int, G: int, cap: int = cg.MERGE_CAP) -> dict:
    parts = partition(indptr, M, G, cap)
    D = parts[0][2]
    whole = np.zeros(M, dtype=np.int64)
    cut = {}
    for w, (own, pieces, _) in enumerate(parts):
        for r in own:
            whole[r] += 1
        kinds = [p[3] == w for p in pieces]
        assert kinds.count(True) <= 1 and kinds.count(False) <= 1, (w, pieces)
        # rows past the scratch capacity are summed whole, so they are left out
        work = sum(int(indptr[r + 1] - indptr[r]) + 1 for r in own
                   if indptr[r + 1] - indptr[r] <= D)
        work += sum(p[2] - p[1] for p in pieces)
        assert work <= 2 * D + 1, (w, work, D)
        for p in pieces:
            cut.setdefault(p[0], []).append(p)
    for r, pcs in cut.items():
        assert whole[r] == 0, r
        rs, re = int(indptr[r]), int(indptr[r + 1])
        pcs.sort(key=lambda p: p[5])
        wf, wl = pcs[0][3], pcs[0][4]
        assert all(p[3] == wf and p[4] == wl for p in pcs), pcs
        assert [p[5] for p in pcs] == list(range(wf, wl + 1)), pcs
        assert wl < cap and wl > wf
        assert pcs[0][1] == rs and pcs[-1][2] == re, pcs
        for a, b in zip(pcs, pcs[1:]):
            assert a[2] == b[1] and a[1] < a[2], (a, b)
    lens = np.diff(np.asarray(indptr[:M + 1], dtype=np.int64))
    for r in range(M):
        if r not in cut:
            assert whole[r] == 1, (r, whole[r])
            if lens[r] > D:  # a long row kept whole: its windows reach past the scratch
                assert (r + int(indptr[r + 1]) - int(indptr[0]) - 1) // D >= cap
    return {"D": D, "cut": len(cut), "max_pieces": max((len(v) for v in cut.values()), default=0)}


def _cases():
    yield "power_law", make_baseline("c3a", scale=0.05)
    yield "dense_rows", make_baseline("c3b", scale=0.1)
    yield "uniform", make_baseline("c1", scale=0.02)
    yield "banded", make_baseline("c2", scale=0.02)
    yield "mostly_empty", ragged(3, 3000, 500, 3, empty_every=2, long_rows=[(7, 400)])
    yield "one_huge_row", ragged(4, 400, 30000, 2, long_rows=[(200, 25000)])
    yield "huge_first_and_last", ragged(5, 300, 9000, 5,
                                        long_rows=[(0, 8000), (299, 7000), (150, 6)])
    yield "no_nonzeros", ragged(6, 100, 10, 0)
    yield "single_row", ragged(7, 1, 5000, 0, long_rows=[(0, 4000)])


@pytest.mark.parametrize("T", [1, 4, 16, 64, 1024])
def test_partition_covers_every_nonzero_once(T):
    """Also as a block of rows of a larger matrix (indptr[0] > 0, odd and even)."""
    seen_cut = 0
    for label, A in _cases():
        M = A.shape[0]
        G = max(1, -(-M // T))
        info = check_partition(A.indptr, M, G)
        seen_cut += info["cut"]
        for off in (1, 6):
            view = check_partition(np.asarray(A.indptr, dtype=np.int64) + off, M, G)
            assert view == info, (label, off)
    if T <= 64:  # a window per 64 rows or fewer: the long rows above are cut
        assert seen_cut > 0


def test_search_is_the_exact_lower_bound():
    rng = np.random.default_rng(11)
    for label, A in _cases():
        M = A.shape[0]
        X = M + int(A.indptr[M])
        bound = 2 + math.ceil(math.log(M + 1, 63))
        for t in list(rng.integers(0, X + 2, size=60)) + [0, 1, X - 1, X, X + 1]:
            t = int(t)
            got, rounds, probed = mp_search(A.indptr, M, t, X)
            assert got == lower_bound(A.indptr, M, t), (label, t)
            assert min(probed) >= 0 and max(probed) <= M
            assert rounds <= bound, (label, t, rounds)


def test_uniform_rows_take_one_round():
    """Rows of equal length: the proportional guess lands within the 48
    consecutive probes, so a window's first row costs one row-pointer load."""
    for A in (make_baseline("c1", scale=0.05), make_baseline("c2", scale=0.05)):
        M = A.shape[0]
        X = M + int(A.indptr[M])
        G = -(-M // 16)
        D = -(-X // G)
        rounds = [mp_search(A.indptr, M, min(w * D, X), X)[1] for w in range(1, G)]
        assert max(rounds) == 1, max(rounds)


def test_rows_past_the_scratch_stay_whole():
    A = ragged(8, 500, 6000, 4, long_rows=[(20, 3000), (480, 5000)])
    full = check_partition(A.indptr, 500, 250)
    assert full["cut"] == 2
    small = check_partition(A.indptr, 500, 250, cap=100)  # only the first row's windows fit
    assert small["cut"] == 1


def test_config_balance_is_additive():
    """balance leaves every reference schedule's hash and dict as they were."""
    c = Config(tile_size=64, threads_per_row=8, unroll=2, block_size=512)
    assert "balance" not in c.to_dict()
    n = Config(tile_size=64, threads_per_row=8, unroll=2, block_size=512, balance="nnz")
    assert n.to_dict()["balance"] == "nnz" and n.hash() != c.hash()
    assert n.short() == c.short() + "/nnz"
    assert Config(**n.to_dict()) == n


def test_merge_source_and_refusals():
    from tilegen_amd import dsl
    ks = dsl.standard_kernels()
    cfg = Config(tile_size=64, threads_per_row=8, unroll=2, block_size=512, balance="nnz")
    for k in ("spmv", "fused_spmv_axpy"):
        g = cg.generate(ks[k], cfg, backend="hip", write=False)
        assert "tg_mp_search(indptr, row_lim, t0, X, pbase)" in g.source
        assert "tg_mp_commit(tg_part, wdx, wf, wl, t, &tot)" in g.source
        tiling = [e for e in cg._passes.run_pipeline(ks[k], cfg, backend="hip").pass_log
                  if e["pass"] == "tiling"][0]
        assert "merge path" in tiling["action"]
    # the row-tiled source is unchanged by the option's existence
    rows = cg.generate(ks["spmv"], Config(tile_size=64, threads_per_row=8, unroll=2,
                                          block_size=512), backend="hip", write=False)
    assert "tg_mp_" not in rows.source
    for k, c in (("spmm", Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=2,
                                 block_size=64, balance="nnz")),
                 ("spmv", Config(tile_size=1, threads_per_row=8, block_size=128,
                                 balance="nnz"))):
        with pytest.raises(ValueError, match="balance 'nnz'"):
            cg.generate(ks[k], c, backend="hip", write=False)
    # the CPU backend ignores it (like threads_per_row and block_size)
    cpu = cg.generate(ks["spmv"], cfg, backend="cpu", write=False)
    assert "tg_mp_" not in cpu.source


# --------------------------------------------------------------------------- #
# hybrid tiles: row tiles plus long-row workgroups over equal nonzero ranges
# --------------------------------------------------------------------------- #
def _row_at(indptr, R, P, pb, pe):
    """``tg_mp_row`` lane for lane: the row holding nonzero P, pb <= P < pe =
    indptr[R], pb = indptr[0], with its bounds, and the number of probe rounds
    it took."""
    qs = first_probes(int(float(P - pb) * (float(R) / float(pe - pb))))
    lo, hi, vlo, vhi = 0, R, pb, pe
    rounds = 0
    while True:
        rounds += 1
        qs = [min(max(q, lo), hi) for q in qs]
        vs = [int(indptr[q]) for q in qs]
        f, fa = _ends(qs, [v > P for v in vs])
        if f is not None:
            hi, vhi = qs[f], vs[f]
        if fa is not None:
            lo, vlo = qs[fa], vs[fa]
        if hi - lo <= 1:
            return lo, vlo, vhi, rounds
        s = (hi - lo + 61) // 63
        qs = [lo + 1 + l * s for l in range(64)]


def _range(indptr, M: int, CH: int, e: int):
    """Range e's positions [p0, p1): CH from (indptr[0] & ~1) + e CH, clipped to
    [indptr[0], indptr[M])."""
    pbase, pend = int(indptr[0]), int(indptr[M])
    pa = (pbase & ~1) + e * CH
    return max(pa, pbase), min(pa + CH, pend)


def _ranges(indptr, M: int, CH: int) -> int:
    """NR: the ranges the rows' nonzeros meet."""
    pbase, pend = int(indptr[0]), int(indptr[M])
    return -(-(pend - (pbase & ~1)) // CH) if pend > pbase else 0


def hybrid_listed(indptr, M: int, CH: int, e: int):
    """The long rows range e lists, as (row, start, end): the distinct rows
    longer than CH / 2 among those holding nonzeros p0, p0 + CH / 2 (p1 - 1 when
    that lies past the range) and p1 - 1."""
    pbase, pend = int(indptr[0]), int(indptr[M])
    LH = CH // 2
    p0, p1 = _range(indptr, M, CH, e)
    found = [_row_at(indptr, M, P, pbase, pend)[:3]
             for P in (p0, p0 + LH if p0 + LH < p1 else p1 - 1, p1 - 1)]
    out = []
    for k, (r, rs, re) in enumerate(found):
        if re - rs > LH and (k == 0 or r != found[k - 1][0]):
            out.append((r, rs, re))
    return out


def hybrid_pieces(indptr, M: int, CH: int, cap: int = cg.MERGE_CAP, nnz=None):
    """The long-row workgroups as the emitter writes them, for a launch with
    ``nnz`` (default: the rows' own count): for every range e that exists (the
    first NL = min(NR, GL), GL = floor(nnz / CH) + 1), the (row, begin, end, ef,
    el, e, cut) pieces it sums (the last range's piece of the row holding its
    last position runs to the row's end), the number of rows it listed, and
    the long rows the row tiles keep (their first range does not exist)."""
    pbase = int(indptr[0])
    pal = pbase & ~1
    if nnz is None:
        nnz = int(indptr[M]) - pbase
    GL = max(0, nnz) // CH + 1
    NL = min(_ranges(indptr, M, CH), GL)
    out, listed = [], []
    for e in range(NL):
        p0, p1 = _range(indptr, M, CH, e)
        last = e == NL - 1
        rows = hybrid_listed(indptr, M, CH, e)
        listed.append(len(rows))
        for row, rs, re in rows:
            ef, el = (rs - pal) // CH, min((re - 1 - pal) // CH, NL - 1)
            cut = el > ef and el < cap
            if not cut and ef != e:
                continue
            q0 = max(p0, rs) if cut else rs
            q1 = (re if last else min(p1, re)) if cut else re
            out.append((row, q0, q1, ef, el, e, cut))
    lens = np.diff(np.asarray(indptr[:M + 1], dtype=np.int64))
    starts = np.asarray(indptr[:M], dtype=np.int64)
    kept = set(np.nonzero((lens > CH // 2) & ((starts - pal) // CH >= NL))[0].tolist())
    return out, listed, kept


def test_row_search_finds_the_row_holding_a_nonzero():
    """The row search returns the row holding nonzero P (numpy searchsorted on
    the row pointers) and that row's two bounds, within a few rounds."""
    for label, A in _cases():
        ip = np.asarray(A.indptr, dtype=np.int64)
        M, nnz = A.shape[0], int(ip[-1])
        if nnz == 0:
            continue
        for t in sorted(set([0, nnz - 1, nnz // 2] + list(np.random.default_rng(1).integers(
                0, nnz, size=100)))):
            r, rs, re, rounds = _row_at(ip, M, int(t), 0, nnz)
            assert r == int(np.searchsorted(ip, t, side="right")) - 1, (label, t)
            assert (rs, re) == (int(ip[r]), int(ip[r + 1])) and rs <= t < re
            assert rounds <= 2 + int(np.ceil(np.log(max(M, 2)) / np.log(63))), (label, t, rounds)


def test_row_search_with_empty_rows_everywhere():
    """Runs of empty rows before, between and after the nonzeros: the row found
    is the nonempty one holding P."""
    lens = np.zeros(5000, dtype=np.int64)
    lens[[7, 8, 1999, 2000, 4990]] = [3, 1, 40, 2, 9]
    ip = np.concatenate([[0], np.cumsum(lens)])
    nnz = int(ip[-1])
    for t in range(nnz):
        r, rs, re, _ = _row_at(ip, len(lens), t, 0, nnz)
        assert lens[r] > 0 and rs <= t < re and (rs, re) == (ip[r], ip[r + 1])


@pytest.mark.parametrize("CH", [128, 512, 1536, 2048])
def test_ranges_list_every_long_row_meeting_them(CH):
    """The rows a range lists are exactly the rows longer than CH / 2 that meet
    [p0, p1), with their bounds, and never more than 3 of them; also on rows
    placed at the ranges' own edges (the GPU test's matrix)."""
    LH = CH // 2
    for label, A in list(_cases()) + [("range_edges", range_edge_matrix(CH, seed=CH))]:
        ip = np.asarray(A.indptr, dtype=np.int64)
        M, nnz = A.shape[0], int(ip[-1])
        lens = np.diff(ip)
        for off in (0, 1, CH + 5):
            v = ip + off
            for e in range(_ranges(v, M, CH)):
                p0, p1 = _range(v, M, CH, e)
                want = [int(r) for r in np.nonzero((lens > LH) & (v[1:] > p0) & (v[:-1] < p1))[0]]
                got = hybrid_listed(v, M, CH, e)
                assert [r for r, _, _ in got] == want and len(got) <= 3, (label, CH, e, off)
                assert all((rs, re) == (int(v[r]), int(v[r + 1])) for r, rs, re in got)


@pytest.mark.parametrize("CH", [128, 512, 2048, 4096])
def test_hybrid_long_rows_summed_once(CH):
    """Every row longer than CH / 2 is summed exactly once by the long-row
    workgroups (whole by one range, or as pieces that tile it, one per range
    from its first to its last), no range lists more than 3 such rows (the
    kernel's list holds 8), and no range holds two pieces of one kind."""
    LH = CH // 2
    for label, A, ip, nnz in _hybrid_launches(CH):
        M = A.shape[0]
        pieces, listed, kept = hybrid_pieces(ip, M, CH, nnz=nnz)
        assert max(listed, default=0) <= 3, (label, max(listed))
        lens = np.diff(A.indptr)
        by_row = {}
        for p in pieces:
            by_row.setdefault(p[0], []).append(p)
        assert not set(by_row) & kept, label
        assert set(by_row) | kept == set(np.nonzero(lens > LH)[0].tolist()), label
        own = int(ip[M] - ip[0])
        if nnz >= own:
            assert not kept, label  # nnz covers the rows: every long row has its ranges
        for row, ps in by_row.items():
            rs, re = int(ip[row]), int(ip[row + 1])
            if len(ps) == 1 and not ps[0][6]:
                assert (ps[0][1], ps[0][2]) == (rs, re)
                continue
            ps.sort(key=lambda p: p[5])
            ef, el = ps[0][3], ps[0][4]
            assert [p[5] for p in ps] == list(range(ef, el + 1)), (label, row)
            assert ps[0][1] == rs and ps[-1][2] == re
            assert all(a[2] == b[1] for a, b in zip(ps, ps[1:]))
        kinds = {}
        for p in pieces:
            if p[6]:
                k = (p[5], p[5] == p[3])
                assert k not in kinds, (label, k)
                kinds[k] = p[0]


def _hybrid_launches(CH):
    """(label, matrix, indptr, nnz) launches: the cases as given, as blocks of a
    larger matrix at odd and even offsets, and with nnz too large, zero and too
    small."""
    for label, A in _cases():
        ip = np.asarray(A.indptr, dtype=np.int64)
        own = int(ip[-1] - ip[0])
        yield label, A, ip, own
        for off in (1, 4, CH + 3):
            for nnz in (own, own + 3 * CH, 0, own // 3):
                yield "%s+%d/%d" % (label, off, nnz), A, ip + off, nnz


def test_hybrid_source_and_geometry():
    from tilegen_amd import dsl
    ks = dsl.standard_kernels()
    cfg = Config(tile_size=64, threads_per_row=8, unroll=2, block_size=512, balance="hybrid")
    g = cg.generate(ks["spmv"], cfg, backend="hip", write=False)
    assert "tg_mp_row(indptr, row_end, P, pbase, pend, &rs, &re)" in g.source
    assert "*grid += (nnz > 0 ? nnz : 0) / 2048 + 1;" in g.host_source
    assert g.geometry.grid(100000, 794591) == 1563 + 388
    assert g.geometry.grid(0, 5) == 0 and g.geometry.grid(10, 0) == 2
    assert cfg.short().endswith("/hybrid")


def test_hybrid_rows_past_the_scratch_stay_whole():
    """With a scratch of 4 ranges, a long row reaching range 4 or later is summed
    whole by its first range and by no other; one within the first 4 is cut."""
    A = ragged(12, 300, 4000, 3, long_rows=[(2, 300), (250, 900)])
    pieces, _, _ = hybrid_pieces(A.indptr, 300, 128, cap=4)
    by_row = {}
    for p in pieces:
        by_row.setdefault(p[0], []).append(p)
    assert len(by_row[2]) > 1 and all(p[6] for p in by_row[2])
    assert len(by_row[250]) == 1 and not by_row[250][0][6]
    rs, re = int(A.indptr[250]), int(A.indptr[251])
    assert by_row[250][0][1:3] == (rs, re) and by_row[250][0][5] == rs // 128
    # the same rows as a block of a larger matrix at an odd offset: ranges count from
    # the even position below indptr[0]
    off = 129
    pieces, _, _ = hybrid_pieces(np.asarray(A.indptr) + off, 300, 128, cap=4)
    by_row = {}
    for p in pieces:
        by_row.setdefault(p[0], []).append(p)
    assert len(by_row[250]) == 1 and by_row[250][0][5] == (rs + off - 128) // 128
