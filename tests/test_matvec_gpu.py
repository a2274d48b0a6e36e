"""GPU parity of the Q4_0 / Q8_0 matvec (through the C ABI) against the CPU oracle.

Bar: dequantized values bit-exact; every output row within
1e-4 x sum_k |w[m,k]| |x[k]| of the oracle's restatement of the reference
kernel on the same bytes; the reference's own golden inputs within its
tolerances (tests/correctness/test_runner.py:33-36).
"""

import ctypes

import numpy as np
import pytest

from asmllm_amd import gguf
from asmllm_amd.device import DeviceBuffer, synchronize
from conftest import assert_matvec_close
from oracle import golden as golden_mod
from oracle import ops_ref

pytestmark = pytest.mark.gpu
NT = 16  # oracle threads


def _weights(seed, M, K, qt="q4"):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((M, K), dtype=np.float32) * np.float32(0.02))
    x = rng.standard_normal(K, dtype=np.float32)
    blocks = gguf.quantize_q4_0(w) if qt == "q4" else gguf.quantize_q8_0(w)
    return blocks, x


def _gguf_matvec(hip, qt, blocks, x):
    M, K = blocks.shape[0], blocks.shape[1] * 32
    db, dx, dy = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    fn = hip.asmhip_matmul_q4_0 if qt == "q4" else hip.asmhip_matmul_q8_0
    rc = fn(db.ptr, dx.ptr, dy.ptr, M, K, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dy.download(np.float32, M)


def _host_call(fn, *arrays_and_ints):
    args = [a.ctypes.data if isinstance(a, np.ndarray) else a for a in arrays_and_ints]
    fn(*args)


# ---- the reference's golden vectors through the reference-named entry points -----

def test_golden_q4_host_pointers(hip, golden, oracle):
    q, s, x = golden["q4_matmul_qweights"], golden["q4_matmul_scales"], golden["q4_matmul_x"]
    y = np.zeros(4, np.float32)
    _host_call(hip.asm_matmul_q4, q, s, x, y, 4, 64)
    assert np.abs(y - golden["q4_matmul_expected"]).max() <= golden_mod.TOLERANCE_Q4
    assert_matvec_close(y, oracle.matmul_q4(q, s, x), ops_ref.dequantize_q4_0(q, s), x)


def test_golden_q8_host_pointers(hip, golden, oracle):
    q, s, x = golden["q8_matmul_qweights"], golden["q8_matmul_scales"], golden["q8_matmul_x"]
    y = np.zeros(4, np.float32)
    _host_call(hip.asm_matmul_q8, q, s, x, y, 4, 64)
    assert np.abs(y - golden["q8_matmul_expected"]).max() <= golden_mod.TOLERANCE_Q8
    assert_matvec_close(y, oracle.matmul_q8(q, s, x), ops_ref.dequantize_q8_0(q, s), x)


def test_avx512_alias_and_mt_variants_bitwise(hip, oracle):
    rng = np.random.default_rng(31)
    M, K = 1000, 4096
    q = rng.integers(0, 256, (M, K // 32, 16), dtype=np.uint8)
    s = rng.uniform(0.05, 0.25, (M, K // 32)).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    ref = np.zeros(M, np.float32)
    _host_call(hip.asm_matmul_q4, q, s, x, ref, M, K)
    assert_matvec_close(ref, oracle.matmul_q4(q, s, x), ops_ref.dequantize_q4_0(q, s), x)
    y = np.zeros(M, np.float32)
    _host_call(hip.asm_matmul_q4_avx512, q, s, x, y, M, K)
    np.testing.assert_array_equal(y, ref)
    for nt in (1, 2, 4, 8, 16):
        y = np.zeros(M, np.float32)
        _host_call(hip.asm_matmul_q4_mt, q, s, x, y, M, K, nt)
        np.testing.assert_array_equal(y, ref)
    assert hip.asm_threadpool_get_num_threads() == 16


def test_threadpool_lifecycle_and_q8_dispatch(hip, oracle):
    rng = np.random.default_rng(32)
    M, K = 300, 512
    q = rng.integers(-128, 128, (M, K // 32, 32), dtype=np.int8)
    s = rng.uniform(0.05, 0.25, (M, K // 32)).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    hip.asm_threadpool_init(4)
    assert hip.asm_threadpool_get_num_threads() == 4
    hip.asm_threadpool_init(1000)
    assert hip.asm_threadpool_get_num_threads() == 64  # threadpool.c:346 clamp
    ref = np.zeros(M, np.float32)
    _host_call(hip.asm_matmul_q8, q, s, x, ref, M, K)
    assert_matvec_close(ref, oracle.matmul_q8(q, s, x), ops_ref.dequantize_q8_0(q, s), x)
    for call in ("asm_threadpool_dispatch_q8",):
        y = np.zeros(M, np.float32)
        _host_call(getattr(hip, call), q, s, x, y, M, K)
        np.testing.assert_array_equal(y, ref)
    y = np.zeros(M, np.float32)
    _host_call(hip.asm_matmul_q8_mt, q, s, x, y, M, K, 8)
    np.testing.assert_array_equal(y, ref)
    assert hip.asm_threadpool_get_num_threads() == 8
    y = np.zeros(31, np.float32)
    _host_call(hip.asm_matmul_q8_mt, q[:31], s[:31], x, y, 31, K, 3)  # M < 32 leaves the pool alone
    np.testing.assert_array_equal(y, ref[:31])
    assert hip.asm_threadpool_get_num_threads() == 8
    hip.asm_threadpool_shutdown()
    assert hip.asm_threadpool_get_num_threads() == 0
    y = np.zeros(M, np.float32)
    _host_call(hip.asm_matmul_q8, q, s, x, y, M, K)  # works again after shutdown
    np.testing.assert_array_equal(y, ref)


# ---- device-resident GGUF blocks at the configuration shapes ---------------------------

CONFIG_SHAPES = [
    ("q4", 4096, 4096), ("q4", 11008, 4096), ("q4", 4096, 11008),
    ("q4", 1024, 4096), ("q4", 14336, 4096), ("q4", 4096, 14336),
    ("q8", 4096, 4096),
]


@pytest.mark.parametrize("qt,M,K", CONFIG_SHAPES)
def test_gguf_config_shapes(hip, oracle, qt, M, K):
    blocks, x = _weights(M + K, M, K, qt)
    y = _gguf_matvec(hip, qt, blocks, x)
    if qt == "q4":
        y_ref = oracle.matmul_q4_0_gguf(blocks, x, NT)
        w = oracle.dequantize_q4_0(blocks)
    else:
        y_ref = oracle.matmul_q8_0_gguf(blocks, x, NT)
        w = oracle.dequantize_q8_0(blocks)
    worst = assert_matvec_close(y, y_ref, w, x)
    print(f"{qt} {M}x{K}: max err / row L1 = {worst:.2e}")


@pytest.mark.parametrize("qt", ["q4", "q8"])
def test_dequantize_bit_exact(hip, oracle, qt):
    blocks, _ = _weights(41, 300, 4096, qt)
    rows, K = blocks.shape[0], blocks.shape[1] * 32
    db, dw = DeviceBuffer.from_numpy(blocks), DeviceBuffer(rows * K * 4)
    fn = hip.asmhip_dequantize_q4_0 if qt == "q4" else hip.asmhip_dequantize_q8_0
    assert fn(db.ptr, dw.ptr, rows, K, None) == 0
    synchronize()
    got = dw.download(np.float32, (rows, K))
    ref = oracle.dequantize_q4_0(blocks) if qt == "q4" else oracle.dequantize_q8_0(blocks)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


# ---- edge cases -------------------------------------------------------------------------

@pytest.mark.parametrize("qt", ["q4", "q8"])
@pytest.mark.parametrize("M,K", [(1, 32), (3, 64), (17, 96), (4097, 4096), (5, 8192), (33, 352)])
def test_ragged_shapes(hip, oracle, qt, M, K):
    blocks, x = _weights(M * 7 + K, M, K, qt)
    y = _gguf_matvec(hip, qt, blocks, x)
    if qt == "q4":
        assert_matvec_close(y, oracle.matmul_q4_0_gguf(blocks, x), oracle.dequantize_q4_0(blocks), x)
    else:
        assert_matvec_close(y, oracle.matmul_q8_0_gguf(blocks, x), oracle.dequantize_q8_0(blocks), x)


def test_all_eight_nibbles_give_zero(hip):
    blocks = np.zeros((64, 128, 18), np.uint8)
    blocks[..., 0:2] = np.float16(0.37).view(np.uint8)
    blocks[..., 2:] = 0x88
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    assert np.all(_gguf_matvec(hip, "q4", blocks, x) == 0.0)


def test_zero_scale_gives_zero(hip):
    blocks, x = _weights(2, 64, 4096)
    blocks[..., 0:2] = 0
    assert np.all(_gguf_matvec(hip, "q4", blocks, x) == 0.0)


@pytest.mark.parametrize("qt", ["q4", "q8"])
@pytest.mark.parametrize("col", [0, 1, 15, 16, 31, 32, 33, 63, 4095])
def test_one_hot_x_picks_column_exactly(hip, oracle, qt, col):
    blocks, _ = _weights(3, 40, 4096, qt)
    x = np.zeros(4096, np.float32)
    x[col] = 1.0
    w = oracle.dequantize_q4_0(blocks) if qt == "q4" else oracle.dequantize_q8_0(blocks)
    np.testing.assert_array_equal(_gguf_matvec(hip, qt, blocks, x), w[:, col])


def test_misaligned_blocks_take_the_generic_path(hip, oracle):
    blocks, x = _weights(5, 50, 4096)
    M, K = 50, 4096
    raw = np.zeros(blocks.nbytes + 2, np.uint8)
    db = DeviceBuffer(raw.nbytes)
    db.upload(blocks.reshape(-1), offset=2)  # rows start 2 bytes past a dword boundary
    dx, dy = DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    assert hip.asmhip_matmul_q4_0(db.ptr + 2, dx.ptr, dy.ptr, M, K, None) == 0
    synchronize()
    assert_matvec_close(dy.download(np.float32, M), oracle.matmul_q4_0_gguf(blocks, x),
                        oracle.dequantize_q4_0(blocks), x)


def test_split_layout_device_pointers(hip, oracle):
    blocks, x = _weights(6, 2048, 4096)
    qs, sc = gguf.split_q4_0(blocks)
    dq, ds, dx, dy = (DeviceBuffer.from_numpy(qs), DeviceBuffer.from_numpy(sc), DeviceBuffer.from_numpy(x),
                      DeviceBuffer(2048 * 4))
    assert hip.asmhip_matmul_q4_split(dq.ptr, ds.ptr, dx.ptr, dy.ptr, 2048, 4096, None) == 0
    synchronize()
    y = dy.download(np.float32, 2048)
    assert_matvec_close(y, oracle.matmul_q4(qs, sc, x, "avx2"), oracle.dequantize_q4_0(blocks), x)
    # the synchronous reference entry point accepts the same device pointers
    y2 = np.zeros(2048, np.float32)
    hip.asm_matmul_q4(dq.ptr, ds.ptr, dx.ptr, dy.ptr, 2048, 4096)
    np.testing.assert_array_equal(dy.download(np.float32, 2048), y)


def test_bad_arguments_are_rejected(hip):
    dx, dy, db = DeviceBuffer(4096 * 4), DeviceBuffer(64 * 4), DeviceBuffer(64 * 128 * 18)
    assert hip.asmhip_matmul_q4_0(db.ptr, dx.ptr, dy.ptr, 64, 4000, None) == -1
    assert "K % 32" in hip.asmhip_last_error().decode()
    assert hip.asmhip_matmul_q4_0(db.ptr, dx.ptr, dy.ptr, 0, 4096, None) == -1
    assert hip.asmhip_matmul_q4_0(None, dx.ptr, dy.ptr, 64, 4096, None) == -1
