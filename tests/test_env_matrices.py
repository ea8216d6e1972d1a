"""Probe and inputs: the reference corpus restatement is pinned by the
reference's manifest (tests/golden/manifest_stats.json, from
data/matrices/manifest.json), the BASELINE generators by their stated
properties, the TGM1 format by a byte-level round trip."""

from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest

from tilegen_amd.env import probe, pretty
from tilegen_amd.matrices import (baseline_case, baseline_ids, baseline_operands,
                                  build_corpus, compulsory_bytes, corpus_classes,
                                  export_matrix_bin, load_csr_npz, load_matrix_bin,
                                  make_baseline, make_matrix, matrix_stats)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_probe_keys():
    info = probe()
    for key in ["has_hiprtc", "hip_version", "has_gpu", "gpu_name", "gfx_arch", "cpu_name",
                "num_cores", "physical_cores", "backend", "has_nvcc", "nvcc_version",
                "compute_capability", "sm_arch"]:
        assert key in info
    assert info["backend"] in ("hip", "cpu")
    assert isinstance(info["num_cores"], int) and info["num_cores"] >= 1
    assert info["has_nvcc"] is False
    assert "backend" in pretty(info)


def test_corpus_matches_reference_manifest():
    with open(os.path.join(GOLDEN, "manifest_stats.json")) as fh:
        ref = {m["class_name"]: m for m in json.load(fh)["matrices"]}
    assert sorted(ref) == sorted(corpus_classes())
    for name in corpus_classes():
        stats = matrix_stats(name, make_matrix(name))
        for key, want in ref[name].items():
            assert stats[key] == want, (name, key, stats[key], want)


def test_corpus_roundtrip(tmp_path):
    manifest = build_corpus(str(tmp_path))
    assert manifest["seed"] == 1234 and len(manifest["matrices"]) == 6
    for entry in manifest["matrices"]:
        name = entry["class_name"]
        m = load_csr_npz(str(tmp_path / ("%s.npz" % name)))
        assert m.shape[0] == entry["rows"] and m.nnz == entry["nnz"]
        b = load_matrix_bin(str(tmp_path / ("%s.bin" % name)))
        assert np.array_equal(b.indptr, m.indptr) and np.array_equal(b.indices, m.indices)
        assert b.data.tobytes() == m.data.tobytes()


def test_tgm1_layout(tmp_path):
    from tests.util import csr
    A = csr(2, 3, [0, 1, 3], [2, 0, 1], [1.5, -2.0, 4.0])
    path = str(tmp_path / "a.bin")
    export_matrix_bin(path, A)
    raw = open(path, "rb").read()
    assert struct.unpack("<Iqqq", raw[:28]) == (0x54474D31, 2, 3, 3)
    assert np.frombuffer(raw[28:52], "<i8").tolist() == [0, 1, 3]
    assert np.frombuffer(raw[52:76], "<i8").tolist() == [2, 0, 1]
    assert np.frombuffer(raw[76:100], "<f8").tolist() == [1.5, -2.0, 4.0]
    open(path, "wb").write(b"XXXX" + raw[4:])
    with pytest.raises(ValueError):
        load_matrix_bin(path)


def test_determinism_and_imbalance():
    a, b = make_matrix("uniform_random"), make_matrix("uniform_random")
    assert np.array_equal(a.indptr, b.indptr) and np.array_equal(a.indices, b.indices)
    assert np.array_equal(a.data, b.data)
    stats = matrix_stats("dense_rows", make_matrix("dense_rows"))
    assert stats["imbalance_ratio"] > 10.0


def _canonical(m):
    for r in range(0, m.shape[0], max(1, m.shape[0] // 997)):
        cols = m.indices[m.indptr[r]:m.indptr[r + 1]]
        assert (np.diff(cols) > 0).all() and (cols >= 0).all() and (cols < m.shape[1]).all()
    assert m.indptr.dtype == np.int64 and m.indices.dtype == np.int64


def test_baseline_cases_have_stated_shapes():
    assert baseline_ids() == ["c1", "c2", "c3a", "c3b", "c4", "c5", "c5x25"]
    c1 = make_baseline("c1")
    assert c1.shape == (100000, 100000) and c1.nnz == 1600000
    assert (np.diff(c1.indptr) == 16).all()
    assert compulsory_bytes("spmv", 100000, 100000, c1.nnz) == 28000008
    assert (np.abs(c1.data) < 1).all()
    _canonical(c1)
    c2 = make_baseline("c2")
    assert c2.shape == (200000, 200000) and c2.nnz == 1399988  # pinned by the manifest
    assert np.abs(c2.indices - np.repeat(np.arange(200000), np.diff(c2.indptr))).max() == 3
    _canonical(c2)
    c3a = make_baseline("c3a")
    L = np.diff(c3a.indptr)
    assert L.min() >= 1 and L.max() == 5000 and 700000 < c3a.nnz < 900000
    _canonical(c3a)
    c3b = make_baseline("c3b")
    L = np.diff(c3b.indptr)
    assert c3b.nnz == 479200 and (L == 2000).sum() == 200 and (L == 4).sum() == 19800
    _canonical(c3b)
    c5 = make_baseline("c5")
    assert c5.nnz == 1600000 and baseline_case("c5").K == 64
    # 4x4 blocks: each block row's 4 rows share one column set made of 4 whole blocks
    for br in (0, 1234, 24999):
        rows = [c5.indices[c5.indptr[r]:c5.indptr[r + 1]] for r in range(4 * br, 4 * br + 4)]
        assert all(np.array_equal(rows[0], r) for r in rows)
        assert (rows[0].reshape(4, 4) % 4 == np.arange(4)).all()
    _canonical(c5)


def test_baseline_operands_deterministic():
    a = baseline_operands("sddmm", 10, 8, 4)
    b = baseline_operands("sddmm", 10, 8, 4)
    assert a["U"].shape == (10, 4) and a["V"].shape == (8, 4)
    assert np.array_equal(a["U"], b["U"]) and (np.abs(a["V"]) < 1).all()
