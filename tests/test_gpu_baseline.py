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
