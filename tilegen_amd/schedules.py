"""Named schedules: the tuned default per BASELINE case and the fixed set the
GPU parity tests sweep.

``TUNED`` holds the schedule each BASELINE case runs with unless a caller
passes its own (``bench.py --config``); values come from the CDNA4 search in
``autotune`` on an MI355X and are re-checked whenever the kernels change.
"""

from __future__ import annotations

from typing import Dict, List

from .codegen import Config

TUNED: Dict[str, Config] = {
    # winners of an exhaustive sweep of the legal CDNA4 space on one MI355X,
    # cold (rotated) inputs, GPU-event kernel time
    # 16 nonzeros per row, uniform random columns: tiles of 240 rows, one per
    # 4-lane group (15 waves, every nonzero of the tile one first-step item), the
    # tile's 3840 gathers sorted by column in LDS so that each gather
    # instruction's 64 lanes share cache lines of x.  11.4 us against 11.6 for
    # 256 rows on 1024 lanes, 11.7 for 224 rows on 512 lanes (two rows per
    # group), 12.6 for the best direct-gather tiles (T16/TPR8/U2/B128)
    # (interleaved repeats on one box; a sweep of all 307 legal sorted schedules
    # found the 1024-lane form first).  Two workgroups of 960 lanes share a CU
    # (62 VGPRs, 67.5 KB of LDS each); two of 832 or 896 lanes did not, and took
    # 15.6-15.8 us
    "c1": Config(tile_size=240, threads_per_row=4, unroll=4, vector_width=1, block_size=960,
                 gather="sorted"),
    # 7 nonzeros per row: 4 lanes x 2, two rows per lane group; tiles of 160 rows on
    # 320 lanes make 1250 workgroups, so the fullest CU holds 5 against a mean of 4.9
    # (tiles of 128 rows: 1563, 7 against 6.1). 6.44 us against 6.64-6.73 for
    # T128/TPR4/U2/B256, the fastest of the power-of-two space, 6.66 for T288/B576 and
    # 6.91-8.10 for other lane groups at 320 lanes (interleaved repeats on one box)
    "c2": Config(tile_size=160, threads_per_row=4, unroll=2, vector_width=1, block_size=320),
    # skewed rows, stream ranges: every workgroup takes an equal range of B x U
    # nonzeros and sums, from LDS, the rows that end in it.
    # c3a (power-law rows, half of them one nonzero long): ranges of 1024 (256 lanes
    # x 4), one lane per short row; 776 workgroups, all resident at once (three per
    # CU, four on eight of them: 20.6 KB of LDS each). Fastest of all 116 legal stream schedules: 11.25 us against 11.33 for 2-lane
    # groups at B256 and 11.37 for ranges of 4096 at 2-lane groups (T512/TPR2/U4/B1024),
    # 13.6-14.1 for the best hybrid tiles (T64/TPR4/U4/B256) and 17.4 for row tiles
    # alone (interleaved repeats on one box).
    # c3b (1% of rows 2000 long, the rest 4): ranges of 2048 (512 lanes x 4), one
    # lane per short row; 6.9-7.1 us against 7.4-7.7 for the best hybrid tiles
    # (T128/TPR4/U2/B512) and 10.6 for the best row tiles (T32/TPR32/U2/B1024)
    "c3a": Config(tile_size=256, threads_per_row=1, unroll=4, vector_width=1, block_size=256,
                  balance="stream"),
    "c3b": Config(tile_size=512, threads_per_row=1, unroll=4, vector_width=1, block_size=512,
                  balance="stream"),
    # K = 64: 8 lanes x 2 columns x 4 passes per row, 2 nonzeros' B rows in flight
    # (fastest of all 882 legal SpMM schedules in a verified sweep on c4; 102.1 us
    # against 103.8 for 16 lanes x 2 passes in three interleaved repeats)
    "c4": Config(tile_size=16, threads_per_row=8, unroll=2, vector_width=2, block_size=64),
    # K = 64 on the chunked SDDMM path: 8 lanes per row x 2 columns per load x 4
    # loads cover K; 8 adjacent rows per wave (two 4x4 block rows), chunks of 8
    # nonzeros, 4 V-row slices in flight per lane
    "c5": Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2, block_size=128),
    # c5x25 (100 nonzeros per row): the same schedule, fastest of all 228 legal
    # chunked-path schedules in a verified sweep on that matrix
    "c5x25": Config(tile_size=16, threads_per_row=8, unroll=4, vector_width=2, block_size=128),
}

# The schedule of launch_spmv_noalloc (include/tilegen_noalloc.h): hybrid tiles,
# row tiles of 128 rows on 4-lane groups plus long-row workgroups over ranges of
# 2048 nonzeros (c3b's tuned schedule before stream ranges took it over).
NOALLOC_SCHEDULE = Config(tile_size=128, threads_per_row=4, unroll=2, vector_width=1,
                          block_size=512, balance="hybrid")

# CPU-tuned OpenMP schedules per BASELINE case (``python -m tilegen_amd.cpu_tuned``:
# random search, budget 40, seed 0, on the GPU box's host); bench.py times them
# beside the reference default T32/TPR1/U1/V1/B128 as the CPU baseline's
# second OpenMP leg.
CPU_TUNED: Dict[str, Config] = {
    "c1": Config(tile_size=8, threads_per_row=32, unroll=2, vector_width=1, block_size=256),
    "c2": Config(tile_size=16, threads_per_row=16, unroll=2, vector_width=1, block_size=128),
    "c3a": Config(tile_size=16, threads_per_row=16, unroll=8, vector_width=1, block_size=128),
    "c3b": Config(tile_size=8, threads_per_row=32, unroll=2, vector_width=1, block_size=256),
    "c4": Config(tile_size=8, threads_per_row=16, unroll=1, vector_width=1, block_size=128),
    "c5": Config(tile_size=2, threads_per_row=4, unroll=2, vector_width=2, block_size=64),
    "c5x25": Config(tile_size=2, threads_per_row=8, unroll=4, vector_width=1, block_size=64),
}

# Swept by the GPU parity tests for every kernel: every threads_per_row the
# wave allows, tiles below/at/above the lane-group count, unroll 1..8, both
# vector widths, and an untiled schedule (reference tests/test_cuda_gpu.py:34-44
# covers the same dimensions for its CUDA emitter).
TEST_SCHEDULES: List[Config] = [
    Config(tile_size=32, threads_per_row=1, unroll=1, vector_width=1, block_size=128),
    Config(tile_size=64, threads_per_row=2, unroll=2, vector_width=1, block_size=128),
    Config(tile_size=64, threads_per_row=4, unroll=4, vector_width=2, block_size=256),
    Config(tile_size=128, threads_per_row=8, unroll=2, vector_width=2, block_size=512),
    Config(tile_size=32, threads_per_row=16, unroll=3, vector_width=1, block_size=256),
    Config(tile_size=16, threads_per_row=32, unroll=8, vector_width=2, block_size=512),
    Config(tile_size=4, threads_per_row=64, unroll=4, vector_width=1, block_size=256),
    Config(tile_size=1, threads_per_row=4, unroll=1, vector_width=1, block_size=64),
    Config(tile_size=256, threads_per_row=1, unroll=4, vector_width=1, block_size=256),
    Config(tile_size=1024, threads_per_row=8, unroll=2, vector_width=2, block_size=1024),
]

TEST_KERNELS = ["spmv", "spmm", "sddmm", "fused_spmv_axpy", "axpy"]

# Block sizes of 3, 5 and 7 waves: lane-group counts (3, 40, 28, 96) that are
# not powers of two, for every combine across lane groups or waves.
ODD_BLOCK_SCHEDULES: List[Config] = [
    Config(tile_size=12, threads_per_row=64, unroll=1, vector_width=1, block_size=192),
    Config(tile_size=40, threads_per_row=8, unroll=2, vector_width=2, block_size=320),
    Config(tile_size=28, threads_per_row=16, unroll=4, vector_width=2, block_size=448),
    Config(tile_size=96, threads_per_row=2, unroll=2, vector_width=1, block_size=192),
]

# Swept by the GPU parity tests of the merge-path (balance "nnz") SpMV and
# fused_spmv_axpy: one wave (both window searches in one wave) and sixteen,
# windows of about 2 to 256 rows, every lane-group width tier.
MERGE_TEST_SCHEDULES: List[Config] = [
    Config(tile_size=16, threads_per_row=8, unroll=2, block_size=128, balance="nnz"),
    Config(tile_size=64, threads_per_row=8, unroll=2, block_size=512, balance="nnz"),
    Config(tile_size=32, threads_per_row=32, unroll=2, block_size=1024, balance="nnz"),
    Config(tile_size=2, threads_per_row=4, unroll=1, block_size=64, balance="nnz"),
    Config(tile_size=128, threads_per_row=1, unroll=1, block_size=64, balance="nnz"),
    Config(tile_size=256, threads_per_row=64, unroll=4, block_size=256, balance="nnz"),
    Config(tile_size=8, threads_per_row=16, unroll=3, block_size=256, balance="nnz"),
]

# The same for hybrid tiles (row tiles plus long-row workgroups over nonzero
# ranges of 2 x block x unroll): ranges of 128 to 4096 nonzeros.
HYBRID_TEST_SCHEDULES: List[Config] = [
    Config(**{**c.to_dict(), "balance": "hybrid"}) for c in MERGE_TEST_SCHEDULES]


# The same for stream ranges (an equal range of block x unroll nonzeros per
# workgroup, rows summed from LDS): one wave (both row searches in one wave) and
# sixteen, ranges of 64 to 8192 nonzeros, odd and even unroll, every lane-group
# width tier, and blocks of 3 and 7 waves (legal, though the tuner offers powers
# of two only).  The tile size is not used by this form.
STREAM_TEST_SCHEDULES: List[Config] = [
    Config(tile_size=64, threads_per_row=4, unroll=2, block_size=256, balance="stream"),
    Config(tile_size=64, threads_per_row=1, unroll=1, block_size=64, balance="stream"),
    Config(tile_size=16, threads_per_row=64, unroll=3, block_size=1024, balance="stream"),
    Config(tile_size=128, threads_per_row=8, unroll=8, block_size=1024, balance="stream"),
    Config(tile_size=8, threads_per_row=16, unroll=4, block_size=128, balance="stream"),
    Config(tile_size=256, threads_per_row=2, unroll=1, block_size=512, balance="stream"),
    Config(tile_size=24, threads_per_row=8, unroll=2, block_size=192, balance="stream"),
    Config(tile_size=224, threads_per_row=2, unroll=4, block_size=448, balance="stream"),
]


# Row tiles whose first-step gathers are sorted in LDS (gather "sorted"): one to
# eight rows per lane group, odd and even unroll, lane groups of 1 to 64 lanes,
# blocks of 1, 3, 8 and 16 waves (64 to 1024 buckets), 384 to 8192 sorted items, and
# the largest LDS footprint the space allows (151,760 B: 8192 items, 1025 pointers).
SORTED_TEST_SCHEDULES: List[Config] = [
    Config(tile_size=256, threads_per_row=8, unroll=2, block_size=512, gather="sorted"),
    Config(tile_size=64, threads_per_row=4, unroll=2, block_size=256, gather="sorted"),
    Config(tile_size=128, threads_per_row=1, unroll=1, block_size=64, gather="sorted"),
    Config(tile_size=32, threads_per_row=16, unroll=3, block_size=256, gather="sorted"),
    Config(tile_size=8, threads_per_row=64, unroll=8, block_size=512, gather="sorted"),
    Config(tile_size=24, threads_per_row=8, unroll=2, block_size=192, gather="sorted"),
    Config(tile_size=512, threads_per_row=8, unroll=2, block_size=1024, gather="sorted"),
    Config(tile_size=1024, threads_per_row=2, unroll=4, block_size=1024, gather="sorted"),
]


def schedule_id(c: Config) -> str:
    return "T%d-TPR%d-U%d-V%d-B%d%s%s" % (c.tile_size, c.threads_per_row, c.unroll,
                                          c.vector_width, c.block_size,
                                          "" if c.balance == "rows" else "-" + c.balance,
                                          "" if c.gather == "direct" else "-" + c.gather)
