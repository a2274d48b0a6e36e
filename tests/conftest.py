import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN_DIR = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libasmllm.so")


@pytest.fixture(scope="session")
def oracle():
    from oracle import native

    native.lib()
    return native


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN_DIR / "reference_gen_seed42.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.fixture(scope="session")
def hip():
    """The HIP library on a GPU.  A GPU test fails (never skips) when the
    library or the device is missing."""
    from asmllm_amd import native

    lib = native.lib()
    n = lib.asmhip_device_count()
    if n < 1:
        pytest.fail("no HIP device visible to libasmllm.so")
    return lib


def assert_matvec_close(y, y_ref, w_fp32, x, rel=1e-4):
    """|y - y_ref| <= rel * sum_k |w[m,k]| |x[k]| for every row."""
    l1 = np.abs(w_fp32.astype(np.float64)) @ np.abs(np.asarray(x, np.float64))
    err = np.abs(np.asarray(y, np.float64) - np.asarray(y_ref, np.float64))
    bad = err > rel * l1 + 1e-30
    assert not bad.any(), (
        f"{bad.sum()} rows out of tolerance; worst row {int(np.argmax(err / (l1 + 1e-30)))} "
        f"err {err.max():.3e}, max err/L1 {np.max(err / (l1 + 1e-30)):.3e} (bar {rel:.0e})"
    )
    return float(np.max(err / (l1 + 1e-30)))
