"""GPU parity of the Q4_0 / Q8_0 matvec (through the C ABI) against the CPU oracle.

Bar: dequantized values bit-exact; every output row within
1e-4 x sum_k |w[m,k]| |x[k]| of the oracle's restatement of the reference
kernel on the same bytes; the reference's own golden inputs within its
tolerances (tests/correctness/test_runner.py:33-36).
"""

import ctypes

import numpy as np
import pytest

from asmllm_amd import gguf, native
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


@pytest.fixture
def q4_kernel(hip):
    """Selects the Q4_0 GGUF kernel for one test; auto selection is restored after."""
    def select(kernel):
        assert hip.asmhip_set_q4_kernel(kernel) == 0, hip.asmhip_last_error()
        assert hip.asmhip_get_q4_kernel() == kernel
    yield select
    hip.asmhip_set_q4_kernel(native.Q4_KERNEL_AUTO)


Q4_KERNELS = [native.Q4_KERNEL_FP32, native.Q4_KERNEL_MFMA]
Q4_KERNEL_IDS = ["fp32", "mfma"]


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


def _sweep_cases(n, seed):
    """Seeded random (qt, M, K): M in [1, 6000], K a multiple of 32 up to 12800,
    about half of them multiples of 256 (the shapes the MFMA stream takes)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        M = int(rng.integers(1, 6001))
        K = 256 * int(rng.integers(1, 51)) if i % 2 == 0 else 32 * int(rng.integers(1, 401))
        cases.append(("q4" if i % 3 else "q8", M, K))
    return cases


@pytest.mark.parametrize("qt,M,K", _sweep_cases(24, 2024))
def test_random_shape_sweep(hip, oracle, qt, M, K):
    blocks, x = _weights(M + 13 * K, M, K, qt)
    y = _gguf_matvec(hip, qt, blocks, x)
    if qt == "q4":
        assert_matvec_close(y, oracle.matmul_q4_0_gguf(blocks, x, NT), oracle.dequantize_q4_0(blocks), x)
    else:
        assert_matvec_close(y, oracle.matmul_q8_0_gguf(blocks, x, NT), oracle.dequantize_q8_0(blocks), x)


def test_all_eight_nibbles_give_zero(hip):
    blocks = np.zeros((64, 128, 18), np.uint8)
    blocks[..., 0:2] = np.array([0.37], np.float16).view(np.uint8)
    blocks[..., 2:] = 0x88
    x = np.random.default_rng(1).standard_normal(4096).astype(np.float32)
    assert np.all(_gguf_matvec(hip, "q4", blocks, x) == 0.0)


def test_near_constant_rows_keep_relative_accuracy(hip, oracle):
    """Rows whose nibbles are all 8 but one, against an x with one small entry
    where the weight is nonzero and large entries elsewhere: the row's L1 is
    tiny, so any cancellation between large terms would break the bar."""
    M, K = 64, 4096
    blocks = np.zeros((M, K // 32, 18), np.uint8)
    blocks[..., 0:2] = np.array([0.01], np.float16).view(np.uint8)
    blocks[..., 2:] = 0x88
    rng = np.random.default_rng(77)
    cols = rng.integers(0, K, M)
    for m, c in enumerate(cols):
        b, j = divmod(int(c), 32)
        byte = 2 + (j % 16)
        blocks[m, b, byte] = (blocks[m, b, byte] & (0x0F if j >= 16 else 0xF0)) | ((9 << 4) if j >= 16 else 9)
    x = (rng.standard_normal(K) * 1e4).astype(np.float32)
    x[cols] = 1e-3
    y = _gguf_matvec(hip, "q4", blocks, x)
    assert_matvec_close(y, oracle.matmul_q4_0_gguf(blocks, x), oracle.dequantize_q4_0(blocks), x)


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


@pytest.mark.parametrize("M,K", [(1, 256), (300, 2304), (2048, 4096), (11008, 4096), (4096, 11008), (64, 16384),
                                 (33, 2080)])
def test_split_layout_both_kernels(hip, oracle, q4_kernel, M, K):
    """The reference's split layout through asmhip_matmul_q4_split: the int8-MFMA
    stream (K % 256 == 0, planes 16-byte aligned) and the fp32 VALU kernel
    (forced, and for K = 2080) both within the bar of the oracle's AVX2 kernel."""
    blocks, x = _weights(M + K, M, K)
    qs, sc = gguf.split_q4_0(blocks)
    ref = oracle.matmul_q4_mt(qs, sc, x, NT)
    w = oracle.dequantize_q4_0(blocks)
    dq, ds, dx, dy = (DeviceBuffer.from_numpy(qs), DeviceBuffer.from_numpy(sc), DeviceBuffer.from_numpy(x),
                      DeviceBuffer(M * 4))
    for kernel in (native.Q4_KERNEL_AUTO, native.Q4_KERNEL_FP32):
        q4_kernel(kernel)
        assert hip.asmhip_matmul_q4_split(dq.ptr, ds.ptr, dx.ptr, dy.ptr, M, K, None) == 0, hip.asmhip_last_error()
        synchronize()
        assert_matvec_close(dy.download(np.float32, M), ref, w, x)


@pytest.mark.parametrize("M,K", [(1, 256), (300, 2304), (4096, 4096), (11008, 4096), (64, 16384), (33, 2080)])
def test_q8_gguf_and_split_both_kernels(hip, oracle, q4_kernel, M, K):
    """Q8_0 GGUF blocks (asmhip_matmul_q8_0) and the split layout
    (asmhip_matmul_q8_split): the int8-MFMA stream where K % 256 == 0 and the
    fp32 VALU kernel (forced, and for K = 2080) within the bar of the oracle."""
    blocks, x = _weights(M * 3 + K, M, K, qt="q8")
    qs, sc = gguf.split_q8_0(blocks)
    ref = oracle.matmul_q8_0_gguf(blocks, x, NT)
    w = oracle.dequantize_q8_0(blocks)
    db, dq, ds = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(qs), DeviceBuffer.from_numpy(sc)
    dx, dy = DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)
    for kernel in (native.Q4_KERNEL_AUTO, native.Q4_KERNEL_FP32):
        q4_kernel(kernel)
        assert hip.asmhip_matmul_q8_0(db.ptr, dx.ptr, dy.ptr, M, K, None) == 0, hip.asmhip_last_error()
        synchronize()
        assert_matvec_close(dy.download(np.float32, M), ref, w, x)
        assert hip.asmhip_matmul_q8_split(dq.ptr, ds.ptr, dx.ptr, dy.ptr, M, K, None) == 0, hip.asmhip_last_error()
        synchronize()
        assert_matvec_close(dy.download(np.float32, M), ref, w, x)


TILE_HEIGHT_ROWS = [1, 2, 3, 5, 16, 17, 31, 64, 100, 255, 256, 513, 1000, 1024, 2047, 2048, 4095]


@pytest.mark.parametrize("fmt", ["q4", "q8", "q4s", "q8s"])
@pytest.mark.parametrize("K", [2048, 4096, 11008])
def test_rows_do_not_depend_on_tile_height(hip, oracle, fmt, K):
    """The MFMA stream runs 16-row tiles, and 8-row tiles (MFMA rows 8-15 loading
    zeros) for Q8_0 and the split layouts when at most one 8-row tile falls to each
    compute unit (M <= 2048 on 256 CUs).  A row's value must not depend on the tile
    height or on which rows share its tile: the leading m rows of a 4096-row
    matrix (16-row tiles) give bitwise its first m outputs, for every m from 1 up
    (8-row tiles where the format takes them, partial tiles at ragged m); the
    whole matrix stays within the bar of the oracle."""
    M = 4096
    blocks, x = _weights(K + len(fmt), M, K, qt=fmt[:2])
    split = fmt.endswith("s")
    if fmt == "q4s":
        planes, fn = gguf.split_q4_0(blocks), hip.asmhip_matmul_q4_split
    elif fmt == "q8s":
        planes, fn = gguf.split_q8_0(blocks), hip.asmhip_matmul_q8_split
    else:
        planes, fn = (blocks,), hip.asmhip_matmul_q4_0 if fmt == "q4" else hip.asmhip_matmul_q8_0
    dev = [DeviceBuffer.from_numpy(np.ascontiguousarray(p)) for p in planes]
    dx, dy = DeviceBuffer.from_numpy(x), DeviceBuffer(M * 4)

    def run(m):
        # a prefix of rows is a prefix of every plane
        assert fn(*[d.ptr for d in dev], dx.ptr, dy.ptr, m, K, None) == 0, hip.asmhip_last_error()
        synchronize()
        return dy.download(np.float32, m)

    full = run(M)
    if fmt[:2] == "q4":
        w = oracle.dequantize_q4_0(blocks)
        ref = oracle.matmul_q4_mt(*gguf.split_q4_0(blocks), x, NT)
    else:
        w = oracle.dequantize_q8_0(blocks)
        ref = oracle.matmul_q8_0_gguf(blocks, x, NT)
    assert_matvec_close(full, ref, w, x)
    for m in TILE_HEIGHT_ROWS:
        np.testing.assert_array_equal(run(m).view(np.uint32), full[:m].view(np.uint32), err_msg=f"m={m}")


def test_bad_arguments_are_rejected(hip):
    dx, dy, db = DeviceBuffer(4096 * 4), DeviceBuffer(64 * 4), DeviceBuffer(64 * 128 * 18)
    assert hip.asmhip_matmul_q4_0(db.ptr, dx.ptr, dy.ptr, 64, 4010, None) == -1
    assert "K % 32" in hip.asmhip_last_error().decode()
    assert hip.asmhip_matmul_q4_0(db.ptr, dx.ptr, dy.ptr, 0, 4096, None) == -1
    assert hip.asmhip_matmul_q4_0(None, dx.ptr, dy.ptr, 64, 4096, None) == -1


# ---- both Q4_0 GGUF kernels, selected explicitly ------------------------------------------

@pytest.mark.parametrize("kernel", Q4_KERNELS, ids=Q4_KERNEL_IDS)
@pytest.mark.parametrize("M,K", [s[1:] for s in CONFIG_SHAPES if s[0] == "q4"] +
                         [(16, 256), (40, 16384), (12288, 4096), (22016, 4096), (32000, 4096), (300, 2304),
                          (1, 4096), (255, 4096), (257, 4096), (5000, 4096)])
def test_q4_kernels_at_config_shapes(hip, oracle, q4_kernel, kernel, M, K):
    q4_kernel(kernel)
    blocks, x = _weights(3 * M + K, M, K)
    y = _gguf_matvec(hip, "q4", blocks, x)
    worst = assert_matvec_close(y, oracle.matmul_q4_0_gguf(blocks, x, NT), oracle.dequantize_q4_0(blocks), x)
    print(f"kernel {kernel} {M}x{K}: max err / row L1 = {worst:.2e}")


@pytest.mark.parametrize("kernel", Q4_KERNELS, ids=Q4_KERNEL_IDS)
def test_q4_kernels_edge_cases(hip, oracle, q4_kernel, kernel):
    q4_kernel(kernel)
    test_all_eight_nibbles_give_zero(hip)
    test_near_constant_rows_keep_relative_accuracy(hip, oracle)
    test_zero_scale_gives_zero(hip)
    for col in (0, 15, 16, 31, 4064, 4095):
        test_one_hot_x_picks_column_exactly(hip, oracle, "q4", col)


@pytest.mark.parametrize("kernel", [native.Q4_KERNEL_MFMA], ids=["mfma"])
@pytest.mark.parametrize("K", [4096, 11008])
def test_mfma_kernel_wide_dynamic_range_of_x(hip, oracle, q4_kernel, kernel, K):
    """x spanning up to 2^40 inside a block, with zero weights placed on the
    largest entries of some rows: the two-level fixed point keeps every row
    within the bar (K = 4096: x in registers; K = 11008: each wave digitizes its
    own units' x)."""
    q4_kernel(kernel)
    rng = np.random.default_rng(90)
    M = 256
    blocks, _ = _weights(91, M, K)
    x = (rng.standard_normal(K) * 2.0 ** rng.integers(-20, 21, K)).astype(np.float32)
    big = np.argsort(-np.abs(x).reshape(-1, 32), axis=1)[:, 0] + 32 * np.arange(K // 32)
    for m in range(0, M, 2):  # even rows: weight 0 (nibble 8) at each block's largest |x|
        for c in big:
            b, j = divmod(int(c), 32)
            byte = 2 + (j % 16)
            blocks[m, b, byte] = (blocks[m, b, byte] & (0x0F if j >= 16 else 0xF0)) | ((8 << 4) if j >= 16 else 8)
    y = _gguf_matvec(hip, "q4", blocks, x)
    worst = assert_matvec_close(y, oracle.matmul_q4_0_gguf(blocks, x, NT), oracle.dequantize_q4_0(blocks), x)
    assert worst < 1e-6


@pytest.mark.parametrize("qt", ["q4", "q8"])
@pytest.mark.parametrize("kernel", Q4_KERNELS, ids=Q4_KERNEL_IDS)
@pytest.mark.parametrize("bad", ["nan", "inf", "-inf"])
@pytest.mark.parametrize("K", [4096, 11008])
def test_non_finite_x_propagates(hip, oracle, q4_kernel, qt, kernel, bad, K):
    """A NaN or infinite activation makes every row it touches non-finite, as
    in the reference's fp32 arithmetic: no kernel may turn it into a finite
    number.  Where the fp32 sum is +-inf (an infinite x times a nonzero weight)
    the int8-MFMA stream returns NaN instead: it prepares x as fixed point per
    32-block and gives a block holding a NaN or an infinity a NaN scale, so an
    infinity is not carried with its sign (a stated difference; the fp32 VALU
    kernel keeps the reference's +-inf)."""
    q4_kernel(kernel)
    M = 300
    blocks, x = _weights(44, M, K, qt)
    x[1234] = {"nan": np.nan, "inf": np.inf, "-inf": -np.inf}[bad]
    y = _gguf_matvec(hip, qt, blocks, x)
    with np.errstate(invalid="ignore", over="ignore"):
        ref = oracle.matmul_q4_0_gguf(blocks, x) if qt == "q4" else oracle.matmul_q8_0_gguf(blocks, x)
    assert np.all(~np.isfinite(ref))  # the weight column at 1234 has no zero row here or NaN follows anyway
    np.testing.assert_array_equal(~np.isfinite(y), ~np.isfinite(ref))
    mfma = kernel != native.Q4_KERNEL_FP32  # the selection applies to Q4_0 and Q8_0 alike
    if bad == "nan" or not mfma:
        np.testing.assert_array_equal(np.isnan(y), np.isnan(ref))
        np.testing.assert_array_equal(y[np.isinf(ref)], ref[np.isinf(ref)])  # same infinities, same signs
    else:
        assert np.any(np.isinf(ref))  # the fp32 sum is +-inf on rows with a nonzero weight there
        assert np.all(np.isnan(y))
    # the other blocks still count: a finite x with the same bytes stays finite
    x[1234] = 0.5
    assert np.all(np.isfinite(_gguf_matvec(hip, qt, blocks, x)))


def test_forcing_mfma_on_an_ineligible_shape_is_an_error(hip, q4_kernel):
    q4_kernel(native.Q4_KERNEL_MFMA)
    blocks, x = _weights(8, 16, 96)
    db, dx, dy = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(x), DeviceBuffer(16 * 4)
    assert hip.asmhip_matmul_q4_0(db.ptr, dx.ptr, dy.ptr, 16, 96, None) == native.ERR_UNSUPPORTED
    assert "MFMA" in hip.asmhip_last_error().decode()
    assert hip.asmhip_set_q4_kernel(7) == -1


# ---- fused pre-ops and accumulation ---------------------------------------------------------

def _fused(hip, qtype, blocks, x, pre, arg, eps, y0):
    M, K = blocks.shape[0], blocks.shape[1] * 32
    db, dx = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(x)
    da = DeviceBuffer.from_numpy(arg) if arg is not None else None
    dy = DeviceBuffer.from_numpy(y0) if y0 is not None else DeviceBuffer(M * 4)
    rc = hip.asmhip_matmul_fused(qtype, db.ptr, dx.ptr, dy.ptr, M, K, pre, da.ptr if da else None, eps,
                                 int(y0 is not None), None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dy.download(np.float32, M)


@pytest.mark.parametrize("qt,kernel", [("q4", native.Q4_KERNEL_FP32), ("q4", native.Q4_KERNEL_MFMA),
                                       ("q8", native.Q4_KERNEL_AUTO), ("q8", native.Q4_KERNEL_FP32)],
                         ids=["q4-fp32", "q4-mfma", "q8", "q8-fp32"])
@pytest.mark.parametrize("pre", ["none", "rmsnorm", "swiglu", "rmsnorm-k11008", "none-k11008"])
@pytest.mark.parametrize("accumulate", [False, True])
def test_fused_matvec(hip, oracle, q4_kernel, qt, kernel, pre, accumulate):
    """The matvec with its pre-op fused into the read of x, overwriting or
    accumulating.  K = 11008 takes the stream where each wave digitizes only its
    own units' x (Q4_0 MFMA; with RMSNorm the waves' sums of squares meet after
    the stream)."""
    pre, _, kk = pre.partition("-k")
    M, K = 1000, int(kk) if kk else 4096 if pre != "swiglu" else 11008
    q4_kernel(kernel)
    blocks, x = _weights(17 + K, M, K, qt)
    rng = np.random.default_rng(5)
    arg = None
    x_eff = x
    if pre == "rmsnorm":
        arg = rng.uniform(0.5, 1.5, K).astype(np.float32)
        x_eff = oracle.rmsnorm(x, arg, 1e-6)
    elif pre == "swiglu":
        arg = rng.standard_normal(K).astype(np.float32)
        x_eff = oracle.silu_hadamard(x, arg)
    y0 = rng.standard_normal(M).astype(np.float32) if accumulate else None
    code = {"none": native.PRE_NONE, "rmsnorm": native.PRE_RMSNORM, "swiglu": native.PRE_SWIGLU}[pre]
    y = _fused(hip, native.Q4_0 if qt == "q4" else native.Q8_0, blocks, x, code, arg, 1e-6, y0)
    if qt == "q4":
        ref, w = oracle.matmul_q4_0_gguf(blocks, x_eff, NT), oracle.dequantize_q4_0(blocks)
    else:
        ref, w = oracle.matmul_q8_0_gguf(blocks, x_eff, NT), oracle.dequantize_q8_0(blocks)
    if accumulate:
        ref = ref + y0
        # the residual's own rounding: half an ulp of |y0| on top of the matvec bar
        l1 = np.abs(w.astype(np.float64)) @ np.abs(x_eff.astype(np.float64))
        err = np.abs(y.astype(np.float64) - ref.astype(np.float64))
        assert np.all(err <= 1e-4 * l1 + 2.0 ** -23 * np.abs(ref.astype(np.float64)))
    else:
        assert_matvec_close(y, ref, w, x_eff)


# ---- gate/up matvec with silu(gate) * up formed as it writes y ------------------------------

def _swiglu(hip, qtype, gu, x, pre, arg, eps):
    H, K = gu.shape[0] // 2, gu.shape[1] * 32
    db, dx = DeviceBuffer.from_numpy(gu), DeviceBuffer.from_numpy(x)
    da = DeviceBuffer.from_numpy(arg) if arg is not None else None
    dh, work = DeviceBuffer(H * 4), DeviceBuffer(2 * H * 4)
    rc = hip.asmhip_matmul_swiglu(qtype, db.ptr, dx.ptr, dh.ptr, H, K, pre, da.ptr if da else None, eps, work.ptr,
                                  None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dh.download(np.float32, H)


@pytest.mark.parametrize("qt,kernel,H,K,pre", [
    ("q4", native.Q4_KERNEL_AUTO, 5504, 4096, "rmsnorm"),   # the 7B FFN: one MFMA-stream launch
    ("q4", native.Q4_KERNEL_FP32, 5504, 4096, "rmsnorm"),   # fp32 kernel into work, then the pairs kernel
    ("q4", native.Q4_KERNEL_AUTO, 768, 288, "none"),        # stories15M: K = 288 is no MFMA-stream shape
    ("q4", native.Q4_KERNEL_AUTO, 1000, 2048, "none"),      # 125 tiles, the general (K != 4096) stream
    ("q8", native.Q4_KERNEL_AUTO, 1000, 4096, "none"),
], ids=["q4-7b-mfma", "q4-7b-fp32", "q4-k288", "q4-k2048", "q8"])
def test_matmul_swiglu(hip, oracle, q4_kernel, qt, kernel, H, K, pre):
    from asmllm_amd.engine import interleave_gate_up

    q4_kernel(kernel)
    gate, x = _weights(31 + H, H, K, qt)
    up, _ = _weights(77 + H, H, K, qt)
    gu = interleave_gate_up(gate, up)
    rng = np.random.default_rng(H)
    arg, x_eff, code = None, x, native.PRE_NONE
    if pre == "rmsnorm":
        arg = rng.uniform(0.5, 1.5, K).astype(np.float32)
        x_eff, code = oracle.rmsnorm(x, arg, 1e-6), native.PRE_RMSNORM
    qtype = native.Q4_0 if qt == "q4" else native.Q8_0
    h = _swiglu(hip, qtype, gu, x, code, arg, 1e-6)

    # exactly the two-step result on the GPU: the same 2H rows without the
    # epilogue, de-interleaved, then asmhip_silu_hadamard
    y = _fused(hip, qtype, gu, x, code, arg, 1e-6, None).reshape(H // 8, 2, 8)
    dg, du = DeviceBuffer.from_numpy(y[:, 0].reshape(H)), DeviceBuffer.from_numpy(y[:, 1].reshape(H))
    assert hip.asmhip_silu_hadamard(dg.ptr, du.ptr, H, None) == 0, hip.asmhip_last_error()
    synchronize()
    np.testing.assert_array_equal(h, dg.download(np.float32, H))

    # and the reference's sequence (two matvecs, silu_hadamard) within the matvec bar
    # carried through silu(g) u: |d/dg| <= 1.1 |u|, |d/du| = |silu(g)|
    mv, dq = ((oracle.matmul_q4_0_gguf, oracle.dequantize_q4_0) if qt == "q4"
              else (oracle.matmul_q8_0_gguf, oracle.dequantize_q8_0))
    g_ref, u_ref = mv(gate, x_eff, NT), mv(up, x_eff, NT)
    h_ref = oracle.silu_hadamard(g_ref, u_ref).astype(np.float64)
    ax = np.abs(x_eff.astype(np.float64))
    l1g, l1u = np.abs(dq(gate).astype(np.float64)) @ ax, np.abs(dq(up).astype(np.float64)) @ ax
    silu = np.abs(h_ref / np.where(u_ref == 0, 1, u_ref))
    bound = 1.1 * np.abs(u_ref) * 1e-4 * l1g + silu * 1e-4 * l1u + 4 * 2.0 ** -23 * np.abs(h_ref) + 1e-30
    assert np.all(np.abs(h.astype(np.float64) - h_ref) <= bound)


@pytest.mark.parametrize("H,K", [(8, 256), (24, 4096), (1000, 768), (2048, 2560), (4096, 8192), (136, 96),
                                 (8, 4096), (2056, 4096), (11008, 4096)])
def test_matmul_swiglu_shapes(hip, H, K):
    """Bitwise the two-step result (matvec of the same rows, then asmhip_silu_hadamard)
    at shapes from one tile to several tiles per workgroup, MFMA stream and not."""
    from asmllm_amd.engine import interleave_gate_up

    gate, x = _weights(5 + H + K, H, K)
    up, _ = _weights(9 + H + K, H, K)
    gu = interleave_gate_up(gate, up)
    h = _swiglu(hip, native.Q4_0, gu, x, native.PRE_NONE, None, 0.0)
    y = _fused(hip, native.Q4_0, gu, x, native.PRE_NONE, None, 0.0, None).reshape(H // 8, 2, 8)
    dg, du = DeviceBuffer.from_numpy(y[:, 0].reshape(H)), DeviceBuffer.from_numpy(y[:, 1].reshape(H))
    assert hip.asmhip_silu_hadamard(dg.ptr, du.ptr, H, None) == 0, hip.asmhip_last_error()
    synchronize()
    np.testing.assert_array_equal(h, dg.download(np.float32, H))


def test_matmul_swiglu_rejects_bad_arguments(hip):
    blocks, x = _weights(9, 32, 4096)
    db, dx, dh, work = (DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(x), DeviceBuffer(16 * 4),
                        DeviceBuffer(32 * 4))
    f = hip.asmhip_matmul_swiglu
    assert f(native.Q4_0, db.ptr, dx.ptr, dh.ptr, 12, 4096, 0, None, 0.0, work.ptr, None) == -1  # H % 8
    assert f(native.Q4_0, db.ptr, dx.ptr, dh.ptr, 16, 4096, 0, None, 0.0, None, None) == -1      # no work
    assert f(native.Q4_0, db.ptr, dx.ptr, dh.ptr, 16, 4096, native.PRE_RMSNORM, None, 1e-6, work.ptr, None) == -1
    assert f(5, db.ptr, dx.ptr, dh.ptr, 16, 4096, 0, None, 0.0, work.ptr, None) == -1
    assert f(native.Q4_0, db.ptr, dx.ptr, dh.ptr, 16, 4096, 0, None, 0.0, work.ptr, None) == 0
    synchronize()


def test_fused_pre_op_needs_its_argument(hip):
    blocks, x = _weights(9, 16, 4096)
    db, dx, dy = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(x), DeviceBuffer(16 * 4)
    assert hip.asmhip_matmul_fused(native.Q4_0, db.ptr, dx.ptr, dy.ptr, 16, 4096, native.PRE_RMSNORM, None,
                                   1e-6, 0, None) == -1
    assert hip.asmhip_matmul_fused(5, db.ptr, dx.ptr, dy.ptr, 16, 4096, 0, None, 0.0, 0, None) == -1
