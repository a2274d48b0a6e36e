"""The correctness report on the GPU: every reference kernel, called through its
reference name with host buffers, passes on the reference's golden inputs."""

import io

import pytest

import parity_report as pr

pytestmark = pytest.mark.gpu


def test_every_reference_kernel_passes(hip):
    kernels = pr.KERNELS + [pr.EXTRA["avx512"], pr.EXTRA["sve2"]]
    out = io.StringIO()
    rep = pr.run_report(kernels=kernels, out=out)
    print(out.getvalue())
    status = {r[0]: r[1] for r in rep["rows"]}
    assert status.pop("matmul_q4_sve2") == "NOT IMPLEMENTED"  # an ARM64 kernel: no symbol here
    assert set(status.values()) == {"PASS"}, out.getvalue()
    assert rep["counts"] == {"PASS": 11, "FAIL": 0, "NOT IMPLEMENTED": 1}
    assert pr.exit_status(rep, len(kernels))[0] == 0
