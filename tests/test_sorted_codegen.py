"""Row tiles whose first-step gathers are sorted in LDS (Config gather="sorted"),
checked on the CPU: the counting sort's steps replayed in numpy, the order in which
the emitted kernel issues its loads, and the bounds of its guessed loads.  The GPU
tests (test_gpu_sorted.py) check the kernels' bits against the direct gathers."""

from __future__ import annotations

import re

import numpy as np
import pytest

from tilegen_amd.autotune import enumerate_configs
from tilegen_amd.codegen import SORT_ZPAD, Config, generate, sort_buckets
from tilegen_amd.dsl import standard_kernels
from tilegen_amd.schedules import SORTED_TEST_SCHEDULES, TUNED


def _sort_model(cols, ok, nb, shift, rng):
    """The tile's sort as the kernel makes it: each item takes a rank in its bucket
    from an atomic add (in whatever order the atomics land: a random order here),
    the buckets' exclusive scan gives their bases, item i goes to base + rank as
    (col << 13 | slot), and sorted item s gathers its operand into s_x[slot]."""
    n = len(cols)
    key = np.where(ok, cols >> shift, 0)
    hist = np.zeros(nb, dtype=np.int64)
    rank = np.zeros(n, dtype=np.int64)
    for i in rng.permutation(n):
        if ok[i]:
            rank[i] = hist[key[i]]
            hist[key[i]] += 1
    base = np.concatenate([[0], np.cumsum(hist)[:-1]])
    nsort = int(hist.sum())
    ent = np.full(nsort, -1, dtype=np.int64)
    for i in range(n):
        if ok[i]:
            ent[base[key[i]] + rank[i]] = (int(cols[i]) << 13) | i
    return ent, nsort


@pytest.mark.parametrize("seed", range(4))
def test_counting_sort_model_gives_every_slot_its_operand(seed):
    rng = np.random.default_rng(seed)
    B, R, U = 512, 2, 4
    n = R * U * B
    N = int(rng.integers(1, 1 << 20))
    nb = sort_buckets(B)
    shift = max(0, int(N - 1).bit_length() - (nb.bit_length() - 1)) if N > nb else 0
    cols = rng.integers(0, N, n)
    ok = rng.random(n) < 0.9
    ent, nsort = _sort_model(cols, ok, nb, shift, rng)
    assert nsort == int(ok.sum()) and np.all(ent >= 0)          # a permutation of the items
    assert np.all(np.diff(ent >> 13 >> shift) >= 0)             # sorted by bucket
    x = rng.standard_normal(N)
    s_x = np.full(n, np.nan)
    s_x[ent & 8191] = x[ent >> 13]                              # the gathers
    assert np.array_equal(s_x[ok], x[cols[ok]])                 # every item's own operand
    assert np.all(np.isnan(s_x[~ok]))
    assert max(cols >> shift) < nb


def test_bucket_shift_keeps_buckets_under_the_count():
    """The kernel's shift, 64 - clz(N - 1) - log2(NB) for N > NB, maps 0..N-1 into
    fewer than NB buckets and is the smallest shift that does."""
    for nb in (64, 128, 512, 1024):
        for N in list(range(1, 5000, 37)) + [nb, nb + 1, 2 * nb, 100000, (1 << 20) + 3]:
            s = max(0, int(N - 1).bit_length() - (nb.bit_length() - 1)) if N > nb else 0
            assert (N - 1) >> s < nb
            assert s == 0 or (N - 1) >> (s - 1) >= nb


def test_row_pointers_load_before_the_guessed_loads():
    """Vector loads return in order: the tile's row pointers are loaded first, and
    the guessed first-step loads carry no branch, so the pointers' staging waits for
    their own load alone."""
    src = generate(standard_kernels()["spmv"], TUNED["c1"], "hip", write=False).source
    body = src[src.index("__global__"):]
    ptr = body.index("ptr0_ = __hip_atomic_load(")
    guess = body.index("(sidx_ + q)")
    stage = body.index("s_ptr[threadIdx.x] = ptr0_;")
    assert ptr < guess < stage
    assert "if (Ls > 0)" not in body[:stage]
    assert re.search(r"tg_i64 tg_zpad\[%d\];" % SORT_ZPAD, src)


def test_guessed_loads_stay_inside_the_zero_pad():
    """Without a guess the first-step loads read tg_zpad at the positions a row
    starting at 0 would take; for every legal sorted schedule those (and the second
    element of each 128-bit pair) lie inside the pad."""
    cfgs = [c for c, r in enumerate_configs("spmv") if c.gather == "sorted" and r is None]
    assert cfgs
    form = re.compile(r"\{ const tg_i64 q = \(\(gb\) & ~\(tg_i64\)1\) \+ "
                      r"(?:\(tg_i64\)lane \* (\d+)|(\d+) \* \(tg_i64\)lane) \+ (\d+);")
    checked = 0
    for c in cfgs + list(SORTED_TEST_SCHEDULES):
        src = generate(standard_kernels()["spmv"], c, "hip", write=False).source
        if "sidx_" not in src:
            continue  # odd unroll: no guessed loads
        offs = [(int(m.group(1) or m.group(2)), int(m.group(3))) for m in form.finditer(src)]
        assert len(offs) == c.unroll // 2, c.short()
        last = max(step * (c.threads_per_row - 1) + off + 1 for step, off in offs)
        assert last < SORT_ZPAD, (c.short(), last)
        checked += 1
    assert checked > 100


def test_sorted_needs_row_tiles():
    k = standard_kernels()["spmv"]
    with pytest.raises(ValueError, match="sorted"):
        generate(k, Config(tile_size=256, threads_per_row=4, unroll=4, block_size=512,
                           balance="stream", gather="sorted"), "hip", write=False)
    with pytest.raises(ValueError, match="sorted"):
        generate(k, Config(tile_size=256, threads_per_row=4, unroll=4, block_size=512,
                           balance="nnz", gather="sorted"), "hip", write=False)
