"""The correctness report's own logic (no GPU): missing library or symbols are
NOT IMPLEMENTED, wrong outputs FAIL, right outputs PASS, and the exit status
follows the reference runner (test_runner.py:510-520)."""

import ctypes
import io

import numpy as np
import pytest

import parity_report as pr


class _Stub:
    """A ctypes-like function: argtypes set, body given in Python."""

    def __init__(self, body):
        self.argtypes = [ctypes.c_void_p]
        self.body = body

    def __call__(self, *args):
        self.body(*args)


def _arr(addr, n, dtype=np.float32):
    return np.ctypeslib.as_array(ctypes.cast(addr, ctypes.POINTER(np.ctypeslib.as_ctypes_type(dtype))), (n,))


def test_no_library_is_not_implemented_everywhere():
    out = io.StringIO()
    rep = pr.run_report(lib=None, out=out)
    assert rep["counts"] == {"PASS": 0, "FAIL": 0, "NOT IMPLEMENTED": 10}
    code, msg = pr.exit_status(rep, 10)
    assert code == 0 and "zero false passes" in msg
    assert "Summary: PASS: 0 | FAIL: 0 | NOT IMPLEMENTED: 10" in out.getvalue()


def test_wrong_output_fails_and_right_output_passes(golden, oracle):
    class Lib:
        pass

    lib = Lib()

    def zeros(q, s, x, y, M, K):  # leaves y at zero
        pass

    def right(q, s, x, y, M, K):
        qv = _arr(q, M * (K // 32) * 16, np.uint8).reshape(M, K // 32, 16)
        sv = _arr(s, M * (K // 32)).reshape(M, K // 32)
        _arr(y, M)[:] = oracle.matmul_q4(qv, sv, _arr(x, K))

    lib.asm_matmul_q4 = _Stub(right)
    lib.asm_matmul_q8 = _Stub(zeros)
    rep = pr.run_report(kernels=[k for k in pr.KERNELS if k[0] in ("matmul_q4", "matmul_q8", "rope")], lib=lib,
                        out=io.StringIO())
    status = {r[0]: r[1] for r in rep["rows"]}
    assert status == {"matmul_q4": "PASS", "matmul_q8": "FAIL", "rope": "NOT IMPLEMENTED"}
    assert pr.exit_status(rep, 3)[0] == 1


def test_fixture_is_the_reference_recipe(golden):
    assert sorted(pr.load_golden()) == sorted(golden)


def test_every_report_kernel_is_bound(oracle):
    from asmllm_amd import native

    for name, _tol, _ in pr.KERNELS + [pr.EXTRA["avx512"]]:
        assert f"asm_{name}" in native.SIGNATURES
        assert f"asm_{name}" in native.header_symbols()
