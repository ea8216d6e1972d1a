"""GPU parity at the BASELINE configs' full sizes, with their tuned schedules.

Each case runs the tuned variant through ``launch_<name>`` and checks it
against the C oracle (normwise <= 1e-10) and size-independent properties:
indptr/indices byte-identical after the launch, and linearity in the dense
operand (scaling it by 2 doubles every output bit-exactly, because the kernel's
summation order does not depend on the values).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.util import rel_2, rel_inf
from tilegen_amd.matrices import baseline_case, baseline_operands, make_baseline
from tilegen_amd.schedules import TUNED
from tilegen_amd.variant import Variant

pytestmark = pytest.mark.gpu

TOL = 1e-10


@pytest.mark.parametrize("case_id", ["c1", "c2", "c3a", "c3b", "c4", "c5", "c5x25"])
def test_baseline_case_parity(case_id, hip_ready):
    case = baseline_case(case_id)
    A = make_baseline(case_id)
    M, N = A.shape
    ops = baseline_operands(case.kernel, M, N, case.K)
    v = Variant(case.kernel, TUNED[case_id])
    print("[gpu] %s %s %s nnz=%d" % (case_id, case.kernel, TUNED[case_id].short(), A.nnz),
          flush=True)
    out = v.run(A, **ops)
    want = oracle.compute(case.kernel, A, ops)
    assert rel_inf(out, want) <= TOL and rel_2(out, want) <= TOL, (
        case_id, rel_inf(out, want), rel_2(out, want))
    # linearity: scaling the dense operand by 2 is exact in binary floating point
    doubled = {k: 2.0 * val for k, val in ops.items()}
    if case.kernel == "sddmm":
        doubled = {"U": 2.0 * ops["U"], "V": ops["V"]}
    out2 = v.run(A, **doubled)
    assert np.array_equal(out2, 2.0 * out), case_id


@pytest.mark.parametrize("case_id", ["c1", "c2", "c3a", "c3b", "c4", "c5", "c5x25"])
def test_baseline_case_matches_scipy_and_openmp(case_id, hip_ready, tmp_path):
    """The parity gate as stated for the path: the tuned HIP variant against
    float64 SciPy (the reference's own oracle, ``_reference``) and against this
    build's OpenMP backend at the reference default schedule, both <= 1e-10
    normwise.  The OpenMP variant is compiled here with g++ -O3 -march=native
    -fopenmp, for the CPU it then runs on."""
    from tilegen_amd.autotune import BASELINE, _make_caller
    from tilegen_amd.codegen import generate
    from tilegen_amd.dsl import standard_kernels
    from tilegen_amd.verify import _reference, compile_generated

    case = baseline_case(case_id)
    A = make_baseline(case_id)
    M, N = A.shape
    ops = baseline_operands(case.kernel, M, N, case.K)
    out = Variant(case.kernel, TUNED[case_id]).run(A, **ops)
    data = (ops.get("x"), None, ops.get("B"), ops.get("U"), ops.get("V"), 1.0, 0.0)
    sci = np.asarray(_reference(case.kernel, A, data), dtype=np.float64).reshape(out.shape)
    gen = generate(standard_kernels()[case.kernel], BASELINE, "cpu", outdir=str(tmp_path))
    so, log = compile_generated(gen, "cpu", str(tmp_path))
    assert "fopenmp" in log
    caller, _out, _keep = _make_caller(so, case.kernel, A, data, case.K, "cpu")
    omp = np.asarray(caller(), dtype=np.float64).reshape(out.shape)
    for name, ref in (("scipy", sci), ("openmp", omp)):
        assert rel_inf(out, ref) <= TOL and rel_2(out, ref) <= TOL, (
            case_id, name, rel_inf(out, ref), rel_2(out, ref))
