"""The hardware probes' host side (tilegen_amd/probes.py), on the CPU: the host
layouts keep every range's nonzeros, the expected outputs follow the kernel's
lane/pair layout, the line counts match a brute-force count, the LDS-sort shift
matches the sorted row tiles', and every probe compiles with hipRTC for gfx950."""

from __future__ import annotations

import numpy as np
import pytest

from tilegen_amd import probes


def _ranges(ind, val, ch):
    full = (len(ind) // ch) * ch
    return ind[:full].reshape(-1, ch), val[:full].reshape(-1, ch)


@pytest.mark.parametrize("order", ["line", "b9", "b0"])
def test_layout_permutes_each_range(order):
    rng = np.random.default_rng(1)
    blk, u = 128, 4
    nnz = 3 * blk * u + 77                    # three full ranges and a partial one
    ind = rng.integers(0, 5000, nnz)
    val = rng.standard_normal(nnz)
    li, lv = probes.flat_layout(ind, val, blk, u, order)
    for (a, b), (c, d) in zip(zip(*_ranges(ind, val, blk * u)), zip(*_ranges(li, lv, blk * u))):
        assert sorted(zip(a.tolist(), b.tolist())) == sorted(zip(c.tolist(), d.tolist()))
    tail = (nnz // (blk * u)) * blk * u
    assert np.array_equal(li[tail:], ind[tail:]) and np.array_equal(lv[tail:], val[tail:])
    # the sorted items are read in sorted order: gather instruction j, lane t
    shift = 4 if order == "line" else int(order[1:])
    pos = probes._slot_of_sorted(blk, u)
    first = li[:blk * u][pos]
    assert np.all(np.diff(first >> shift) >= 0)


def test_expected_output_is_the_lane_segment_sums():
    rng = np.random.default_rng(2)
    blk, u, seg = 64, 4, 4
    nnz = 2 * blk * u + 10
    ind = rng.integers(0, 300, nnz)
    val = rng.standard_normal(nnz)
    x = rng.standard_normal(300)
    got = probes.flat_expected(ind, val, x, blk, u, seg, "x")
    # brute force: lane t of range w owns positions 2 (k blk + t) + h
    ch = blk * u
    want = []
    for w in range(-(-nnz // ch)):
        lanes = np.zeros(blk)
        for t in range(blk):
            for k in range(u // 2):
                for h in range(2):
                    p = w * ch + 2 * (k * blk + t) + h
                    if p < nnz:
                        lanes[t] += val[p] * x[ind[p]]
        want += list(lanes.reshape(-1, seg).sum(axis=1))
    assert np.allclose(got, want, rtol=1e-13, atol=1e-13)


def test_gather_lines_matches_a_brute_force_count():
    rng = np.random.default_rng(3)
    blk, u = 128, 2
    ind = rng.integers(0, 4000, blk * u * 3)
    got = probes.gather_lines(ind, blk, u)
    pos = np.arange(len(ind)).reshape(-1, u // 2, blk // 64, 64, 2)
    lines = 0
    for r in range(pos.shape[0]):
        for k in range(u // 2):
            for wv in range(blk // 64):
                for h in range(2):
                    lines += len(set((ind[pos[r, k, wv, :, h]] >> 4).tolist()))
    assert got == pytest.approx(lines / len(ind))


def test_lsort_shift_is_the_sorted_tiles_shift():
    for nb in (64, 512):
        for N in (1, nb - 1, nb, nb + 1, 4097, 100000, 1 << 20):
            s = probes.lsort_shift(N, nb)
            kernel = max(0, int(N - 1).bit_length() - (nb.bit_length() - 1)) if N > nb else 0
            assert s == kernel, (N, nb)


def test_placement_records_decode():
    hw = (3 << 13) | (1 << 12) | (9 << 8) | (2 << 4) | 5   # se 3, sh 1, cu 9, simd 2, wave 5
    assert probes.placement_cu((6 << 32) | hw) == (6, (hw >> 8) & 0xFF)
    assert probes.placement_cu((6 << 32) | hw)[1] == probes.placement_cu(
        (6 << 32) | (hw & ~0xFF))[1]                           # the wave's slot does not count


def test_stream_probe_stays_in_its_padded_buffer():
    """Workgroup w reads pairs w BLK U + k BLK + t: for any grid the last pair read
    is the buffer's last, and the per-wave output has one slot per wave."""
    blk, u = probes.STREAM_BLOCK, probes.STREAM_UNROLL
    for grid in (1, 2, 7, 16384):
        n2 = grid * blk * u
        reads = {(w * blk * u + k * blk + t) for w in (0, grid - 1) for k in (0, u - 1)
                 for t in (0, blk - 1)}
        assert max(reads) == n2 - 1 and min(reads) == 0
        assert ((grid - 1) * blk + blk - 1) >> 6 == grid * blk // 64 - 1
    src = probes.stream_source("s")
    assert src.count("__builtin_nontemporal_load(") == u and "if (" not in src.split("v[0] =")[1].split("double s")[0]


def test_rowgather_probe_reads_inside_its_table():
    src = probes.rowgather_source("r")
    assert "if (row >= M) return;" in src
    assert "cols + row * %d" % probes.ROWGATHER_ROW_NNZ in src
    assert "(B + cc[k] * 64) + j" in src          # j < 32: 16 bytes of a 512-byte row


def test_gather_model_follows_the_kernel_hash():
    """The gather probe's numpy model replays the kernel's xorshift: every index is
    below n, inactive lanes add nothing, and one wave's sum is its lanes' sums."""
    x = np.arange(1000, dtype=np.float64)
    full = probes.gather_expected(1, 64, x)
    half = probes.gather_expected(1, 32, x)
    assert full.shape == (probes.GATHER_BLOCK // 64,)
    assert np.all(half <= full) and np.all(half > 0)
    src = probes.gather_source("g", 32)
    assert "(threadIdx.x & 63) < 32" in src and "x[h % n]" in src


def test_probes_compile_for_gfx950():
    name = "probe_placement_b1024_l45264"
    code = probes._code_object(name, probes.placement_source(name, 1024, 45264, 2000))
    assert code[:4] == b"\x7fELF"
    for nm, text in (("probe_stream_cpu", probes.stream_source("probe_stream_cpu")),
                     ("probe_rowgather_cpu", probes.rowgather_source("probe_rowgather_cpu"))):
        assert probes._code_object(nm, text)[:4] == b"\x7fELF"
    n = probes.build(orders=("matrix", "lsort"), shapes=((512, 8),), gathers=("x",),
                     others=False)
    assert n == 2
