"""GPU parity of the Q5_0 matvec (through the C ABI) against the CPU oracle.

The reference's Q5_0 kernel (src/kernels/x86_64/matmul_q5_avx2.asm, its
threadpool dispatch threadpool.c:667-787) reads the split layout ql / qh /
fp32 scales; the GPU also reads the same values as 22-byte GGUF Q5_0 blocks
in place.  Bar: dequantized values bit-exact; every output row within
1e-4 x sum_k |w[m,k]| |x[k]| of the oracle on the same bytes; the
reference's golden inputs within TOLERANCE_Q5 (test_runner.py:35).  GGUF
blocks with K % 256 == 0 take the int8-MFMA stream, everything else the fp32
VALU kernels.
"""

import numpy as np
import pytest

from asmllm_amd import gguf
from asmllm_amd.device import DeviceBuffer, synchronize
from conftest import assert_matvec_close
from oracle import golden as golden_mod
from oracle import ops_ref

pytestmark = pytest.mark.gpu
NT = 16  # oracle threads


def _q5(seed, M, K):
    rng = np.random.default_rng(seed)
    ql = rng.integers(0, 256, (M, K // 32, 16), dtype=np.uint8)
    qh = rng.integers(0, 256, (M, K // 32, 4), dtype=np.uint8)
    d = (rng.uniform(0.002, 0.02, (M, K // 32)) * rng.choice([-1.0, 1.0], (M, K // 32))).astype(np.float16)
    x = rng.standard_normal(K, dtype=np.float32)
    return ql, qh, d, x


def _host_call(fn, *arrays_and_ints):
    fn(*[a.ctypes.data if isinstance(a, np.ndarray) else a for a in arrays_and_ints])


def _split_device(hip, ql, qh, s, x, qh_offset=0):
    M, K = ql.shape[0], x.shape[0]
    dl, dx, dy = DeviceBuffer.from_numpy(ql), DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    ds = DeviceBuffer.from_numpy(s)
    dh = DeviceBuffer(qh.nbytes + qh_offset)
    dh.upload(qh, offset=qh_offset)
    rc = hip.asmhip_matmul_q5_split(dl.ptr, dh.ptr + qh_offset, ds.ptr, dx.ptr, dy.ptr, M, K, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dy.download(np.float32, M)


def _gguf_device(hip, blocks, x):
    M, K = blocks.shape[0], x.shape[0]
    db, dx, dy = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    rc = hip.asmhip_matmul_q5_0(db.ptr, dx.ptr, dy.ptr, M, K, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dy.download(np.float32, M)


def test_golden_q5_host_pointers(hip, golden, oracle):
    ql, qh, s, x = (golden[k] for k in ("q5_matmul_ql", "q5_matmul_qh", "q5_matmul_scales", "q5_matmul_x"))
    y = np.zeros(4, np.float32)
    _host_call(hip.asm_matmul_q5, ql, qh, s, x, y, 4, 64)
    assert np.abs(y - golden["q5_matmul_expected"]).max() <= golden_mod.TOLERANCE_Q5
    assert_matvec_close(y, oracle.matmul_q5(ql, qh, s, x), ops_ref.dequantize_q5_0(ql, qh, s), x)
    y4 = np.zeros(4, np.float32)
    _host_call(hip.asm_matmul_q5_mt, ql, qh, s, x, y4, 4, 64, 4)  # test_runner.py:336-372 passes 4 threads
    np.testing.assert_array_equal(y4, y)


def test_q5_mt_and_dispatch_bitwise(hip, oracle):
    ql, qh, d, x = _q5(41, 1000, 4096)
    s = d.astype(np.float32)
    ref = np.zeros(1000, np.float32)
    _host_call(hip.asm_matmul_q5, ql, qh, s, x, ref, 1000, 4096)
    assert_matvec_close(ref, oracle.matmul_q5_mt(ql, qh, s, x, NT), ops_ref.dequantize_q5_0(ql, qh, s), x)
    for nt in (1, 2, 4, 16):
        y = np.zeros(1000, np.float32)
        _host_call(hip.asm_matmul_q5_mt, ql, qh, s, x, y, 1000, 4096, nt)
        np.testing.assert_array_equal(y, ref)
    assert hip.asm_threadpool_get_num_threads() == 16
    y = np.zeros(1000, np.float32)
    _host_call(hip.asm_threadpool_dispatch_q5, ql, qh, s, x, y, 1000, 4096)
    np.testing.assert_array_equal(y, ref)
    # device pointers through the reference-named entry point (no staging)
    dl, dh, ds, dx, dy = (DeviceBuffer.from_numpy(a) for a in (ql, qh, s, x, np.zeros(1000, np.float32)))
    hip.asm_matmul_q5(dl.ptr, dh.ptr, ds.ptr, dx.ptr, dy.ptr, 1000, 4096)
    np.testing.assert_array_equal(dy.download(np.float32, 1000), ref)


# (M, K): pair kernel at R = 1, 2, 4 (rows per wave); odd K/32 and K too large
# for the LDS copy of x take the generic kernel.
SHAPES = [(1, 64), (7, 64), (33, 256), (64, 4096), (3000, 4096), (11008, 4096), (4096, 11008),
          (1, 32), (300, 2336), (5, 40000)]


@pytest.mark.parametrize("M,K", SHAPES)
def test_q5_split_and_gguf_match_oracle(hip, oracle, M, K):
    ql, qh, d, x = _q5(M * 31 + K, M, K)
    s = d.astype(np.float32)
    y_split = _split_device(hip, ql, qh, s, x)
    w = ops_ref.dequantize_q5_0(ql, qh, s)
    assert_matvec_close(y_split, oracle.matmul_q5_mt(ql, qh, s, x, NT), w, x)
    blocks = gguf.pack_q5_0(ql, qh, d)
    y_gguf = _gguf_device(hip, blocks, x)
    assert_matvec_close(y_gguf, oracle.matmul_q5_0_gguf(blocks, x, NT), w, x)
    # the same values in the two layouts (GGUF blocks take the int8-MFMA stream where
    # K % 256 == 0, the split planes the fp32 VALU kernel): within the bar of each other
    assert_matvec_close(y_gguf, y_split, w, x)


def test_q5_unaligned_qh_takes_the_generic_kernel(hip, oracle):
    ql, qh, d, x = _q5(42, 200, 1024)
    s = d.astype(np.float32)
    y_pairs = _split_device(hip, ql, qh, s, x)
    y_generic = _split_device(hip, ql, qh, s, x, qh_offset=4)  # qh only dword aligned
    w = ops_ref.dequantize_q5_0(ql, qh, s)
    ref = oracle.matmul_q5(ql, qh, s, x)
    assert_matvec_close(y_pairs, ref, w, x)
    assert_matvec_close(y_generic, ref, w, x)


@pytest.mark.parametrize("col", [0, 15, 16, 31, 32, 4095])
def test_q5_one_hot_column_is_exact(hip, col):
    """Full 11008 x 4096 shape: x = e_col must return column col of W exactly
    (each product and the scale multiply round once, as the dequant does)."""
    ql, qh, d, _ = _q5(43, 11008, 4096)
    x = np.zeros(4096, np.float32)
    x[col] = 1.0
    blocks = gguf.pack_q5_0(ql, qh, d)
    w_col = gguf.dequantize_q5_0(blocks)[:, col]
    np.testing.assert_array_equal(_gguf_device(hip, blocks, x), w_col)
    np.testing.assert_array_equal(_split_device(hip, ql, qh, d.astype(np.float32), x), w_col)


def test_q5_linear_in_x_at_full_size(hip):
    ql, qh, d, x1 = _q5(44, 11008, 4096)
    x2 = np.random.default_rng(45).standard_normal(4096, dtype=np.float32)
    blocks = gguf.pack_q5_0(ql, qh, d)
    y1, y2 = _gguf_device(hip, blocks, x1), _gguf_device(hip, blocks, x2)
    y12 = _gguf_device(hip, blocks, (x1 + x2).astype(np.float32))
    w = gguf.dequantize_q5_0(blocks)
    l1 = ops_ref.row_l1(w, np.abs(x1) + np.abs(x2))
    assert np.all(np.abs(y12.astype(np.float64) - y1 - y2) <= 2e-4 * l1)


@pytest.mark.parametrize("rows,K", [(1, 32), (37, 320), (4096, 4096)])
def test_q5_dequant_bit_exact(hip, oracle, rows, K):
    ql, qh, d, _ = _q5(rows + K, rows, K)
    blocks = gguf.pack_q5_0(ql, qh, d)
    db, dw = DeviceBuffer.from_numpy(blocks), DeviceBuffer(rows * K * 4)
    assert hip.asmhip_dequantize_q5_0(db.ptr, dw.ptr, rows, K, None) == 0, hip.asmhip_last_error()
    synchronize()
    got = dw.download(np.float32, rows * K).reshape(rows, K)
    np.testing.assert_array_equal(got.view(np.uint32), oracle.dequantize_q5_0(blocks).view(np.uint32))


def test_q5_errors(hip):
    buf = DeviceBuffer(1 << 16)
    p = buf.ptr
    assert hip.asmhip_matmul_q5_split(p, p, p, p, p, 4, 48, None) == -1  # K % 32 != 0
    assert hip.asmhip_matmul_q5_split(p, None, p, p, p, 4, 64, None) == -1
    assert hip.asmhip_matmul_q5_0(None, p, p, 4, 64, None) == -1
    assert hip.asmhip_matmul_q5_0(p, p, p, 0, 64, None) == -1
    assert hip.asmhip_dequantize_q5_0(p, p, 1, 33, None) == -1
    assert "K % 32" in hip.asmhip_last_error().decode() or "K %% 32" in hip.asmhip_last_error().decode()


@pytest.mark.parametrize("K", [2048, 4096])
def test_q5_split_rows_do_not_depend_on_tile_height(hip, oracle, K):
    """Split Q5 planes with at most one 8-row tile per compute unit run 8-row
    tiles; the leading m rows of a 4096-row matrix (16-row tiles) give bitwise its
    first m outputs, and the whole matrix stays within the bar of the oracle."""
    M = 4096
    ql, qh, d, x = _q5(K + 5, M, K)
    s = d.astype(np.float32)
    full = _split_device(hip, ql, qh, s, x)
    assert_matvec_close(full, oracle.matmul_q5_mt(ql, qh, s, x, NT), ops_ref.dequantize_q5_0(ql, qh, s), x)
    for m in (1, 7, 8, 9, 100, 1000, 2047, 2048, 2049):
        y = _split_device(hip, ql[:m], qh[:m], s[:m], x)
        np.testing.assert_array_equal(y.view(np.uint32), full[:m].view(np.uint32), err_msg=f"m={m}")
