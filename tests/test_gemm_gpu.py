"""GPU parity of the Q8_0 x Q8_0 prefill GEMM (through the C ABI) against the CPU oracle.

The oracle applies the reference's quantized-activation recipe per block in order
(int32 dot, product of the two fp16 scales, fma into fp32; matmul_q4_neon.S:190-255).
Bar: every output within 1e-4 x sum_k |a_deq[t,k]| |w_deq[j,k]| of the oracle on the
same blocks; activation quantization on the GPU bit-exact with the oracle's.
"""

import numpy as np
import pytest

from asmllm_amd import gguf, native
from asmllm_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu
NT = 16


def _problem(seed, T, M, K):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    a = rng.standard_normal((T, K)).astype(np.float32)
    return gguf.quantize_q8_0(w), gguf.quantize_q8_0(a)


def _gemm(hip, w_blocks, a_blocks):
    M, T, K = w_blocks.shape[0], a_blocks.shape[0], w_blocks.shape[1] * 32
    dw, da, dc = DeviceBuffer.from_numpy(w_blocks), DeviceBuffer.from_numpy(a_blocks), DeviceBuffer(T * M * 4)
    rc = hip.asmhip_gemm_q8_0(dw.ptr, da.ptr, dc.ptr, T, M, K, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dc.download(np.float32, (T, M))


def _assert_close(c, c_ref, w_blocks, a_blocks, oracle, rel=1e-4):
    wd = np.abs(oracle.dequantize_q8_0(w_blocks).astype(np.float64))
    ad = np.abs(oracle.dequantize_q8_0(a_blocks).astype(np.float64))
    l1 = ad @ wd.T
    err = np.abs(c.astype(np.float64) - c_ref.astype(np.float64))
    ratio = err / (l1 + 1e-30)
    assert np.all(err <= rel * l1 + 1e-30), f"max err/L1 {ratio.max():.3e} at {np.unravel_index(ratio.argmax(), ratio.shape)}"
    return float(ratio.max()), float(np.mean(c == c_ref))


@pytest.mark.parametrize("T,M,K", [(64, 128, 128), (512, 11008, 4096), (1, 1, 32), (7, 31, 96), (33, 200, 160),
                                   (100, 129, 4096), (65, 257, 224)])
def test_gemm_matches_oracle(hip, oracle, T, M, K):
    w_blocks, a_blocks = _problem(T * 7 + M + K, T, M, K)
    c = _gemm(hip, w_blocks, a_blocks)
    c_ref = oracle.gemm_q8_0(w_blocks, a_blocks, NT)
    worst, same = _assert_close(c, c_ref, w_blocks, a_blocks, oracle)
    print(f"GEMM {T}x{M}x{K}: max err/L1 {worst:.2e}, bitwise-equal outputs {same:.4f}")


def test_gemm_from_fp32_activations(hip, oracle):
    """fp32 activations -> GPU Q8_0 quantizer -> GEMM, against the oracle's
    quantizer and GEMM on the same fp32 input."""
    T, M, K = 96, 384, 1024
    rng = np.random.default_rng(3)
    a = rng.standard_normal((T, K)).astype(np.float32)
    a[5, :64] = 0.0  # all-zero blocks: scale 0
    w_blocks = gguf.quantize_q8_0((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    d_a, d_ab = DeviceBuffer.from_numpy(a), DeviceBuffer(T * (K // 32) * 34)
    assert hip.asmhip_quantize(native.Q8_0, d_a.ptr, d_ab.ptr, T, K, None) == 0
    dw, dc = DeviceBuffer.from_numpy(w_blocks), DeviceBuffer(T * M * 4)
    assert hip.asmhip_gemm_q8_0(dw.ptr, d_ab.ptr, dc.ptr, T, M, K, None) == 0
    synchronize()
    a_blocks = oracle.quantize_q8_0(a)
    np.testing.assert_array_equal(d_ab.download(np.uint8, a_blocks.shape), a_blocks)
    _assert_close(dc.download(np.float32, (T, M)), oracle.gemm_q8_0(w_blocks, a_blocks, NT), w_blocks, a_blocks,
                  oracle)


def test_gemm_one_hot_activation_picks_dequantized_weights(hip, oracle):
    T, M, K = 32, 96, 256
    w_blocks, _ = _problem(11, 1, M, K)
    a = np.zeros((T, K), np.float32)
    for t in range(T):
        a[t, (37 * t) % K] = 1.0
    a_blocks = gguf.quantize_q8_0(a)  # d = 1/127, q = 127 at the one-hot position
    c = _gemm(hip, w_blocks, a_blocks)
    c_ref = oracle.gemm_q8_0(w_blocks, a_blocks, 1)
    np.testing.assert_array_equal(c, c_ref)
    wd = oracle.dequantize_q8_0(w_blocks)
    d_a = np.float32(np.array([1.0 / 127], np.float16)[0])
    for t in range(T):
        np.testing.assert_allclose(c[t], wd[:, (37 * t) % K] * np.float32(127) * d_a, rtol=1e-6)


def test_gemm_subnormal_and_extreme_scales(hip, oracle):
    """fp16 scales that are subnormal (below 2^-14) or near the fp16 maximum:
    the scale product must stay exact, as the oracle's fp32 product is."""
    T, M, K = 64, 128, 512
    w_blocks, a_blocks = _problem(13, T, M, K)
    rng = np.random.default_rng(14)
    sub = np.array([2.0 ** -24, 3 * 2.0 ** -20, 2.0 ** -15, 6.0e-5], np.float16).view(np.uint8).reshape(-1, 2)
    big = np.array([60000.0, 1024.5, 0.5], np.float16).view(np.uint8).reshape(-1, 2)
    for blocks, pool in ((w_blocks, sub), (a_blocks, np.concatenate([sub, big]))):
        pick = rng.integers(0, len(pool), blocks.shape[:2])
        mask = rng.random(blocks.shape[:2]) < 0.3
        blocks[mask, 0:2] = pool[pick[mask]]
    c = _gemm(hip, w_blocks, a_blocks)
    c_ref = oracle.gemm_q8_0(w_blocks, a_blocks, NT)
    np.testing.assert_array_equal(c, c_ref)


def test_gemm_zero_scales_give_zero(hip):
    w_blocks, a_blocks = _problem(12, 64, 128, 256)
    w_blocks[..., 0:2] = 0
    assert np.all(_gemm(hip, w_blocks, a_blocks) == 0.0)


def test_gemm_rejects_bad_arguments(hip):
    d = DeviceBuffer(1 << 16)
    assert hip.asmhip_gemm_q8_0(d.ptr, d.ptr, d.ptr, 4, 4, 40, None) == native.ERR_INVALID_ARGUMENT
    assert hip.asmhip_gemm_q8_0(d.ptr, d.ptr, d.ptr, 0, 4, 32, None) == native.ERR_INVALID_ARGUMENT
    assert hip.asmhip_gemm_q8_0(None, d.ptr, d.ptr, 4, 4, 32, None) == native.ERR_INVALID_ARGUMENT


# ---- split layout: int8 qs planes + fp32 scale planes (asm_matmul_q8's operands) ----------

def _gemm_split(hip, wq, ws, aq, as_):
    M, T = wq.shape[0], aq.shape[0]
    K = wq.size // M
    bufs = [DeviceBuffer.from_numpy(np.ascontiguousarray(v)) for v in (wq, ws, aq, as_)]
    dc = DeviceBuffer(T * M * 4)
    rc = hip.asmhip_gemm_q8_split(bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, bufs[3].ptr, dc.ptr, T, M, K, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dc.download(np.float32, (T, M))


@pytest.mark.parametrize("T,M,K", [(64, 128, 128), (512, 11008, 4096), (1, 1, 32), (7, 31, 96), (33, 200, 160),
                                   (100, 129, 4096), (65, 257, 224)])
def test_gemm_split_matches_block_gemm_and_oracle(hip, oracle, T, M, K):
    """Scales widened from fp16: bitwise the block-form GEMM on the same blocks, and
    bitwise the oracle (all rows at the small shapes, 8 rows of the 512-row one)."""
    w_blocks, a_blocks = _problem(T * 7 + M + K + 1, T, M, K)
    wq, ws = oracle.split_q8_0(w_blocks)
    aq, as_ = oracle.split_q8_0(a_blocks)
    c = _gemm_split(hip, wq, ws, aq, as_)
    np.testing.assert_array_equal(c, _gemm(hip, w_blocks, a_blocks))
    rows = slice(0, min(T, 8)) if T * M * K > 1e9 else slice(0, T)
    np.testing.assert_array_equal(c[rows], oracle.gemm_q8_split(wq, ws, aq[rows], as_[rows], NT))


def test_gemm_split_arbitrary_fp32_scales(hip, oracle):
    """fp32 scales that no fp16 holds (U(0.5, 1.5), times 2^-30..2^30 on the
    activations): each block's scale is the fp32 product, rounded once, as the
    oracle's fmul; outputs bitwise the oracle's."""
    rng = np.random.default_rng(21)
    T, M, K = 96, 256, 1056
    nb = K // 32
    wq = rng.integers(-128, 128, (M, nb, 32)).astype(np.int8)
    aq = rng.integers(-128, 128, (T, nb, 32)).astype(np.int8)
    ws = rng.uniform(0.5, 1.5, (M, nb)).astype(np.float32)
    as_ = (rng.uniform(0.5, 1.5, (T, nb)) * 2.0 ** rng.integers(-30, 30, (T, nb))).astype(np.float32)
    np.testing.assert_array_equal(_gemm_split(hip, wq, ws, aq, as_), oracle.gemm_q8_split(wq, ws, aq, as_, NT))


def test_gemm_split_subnormal_scale_products(hip, oracle):
    """Scale products below the fp32 normal range (2^-140, 2^-145) and outputs that
    are subnormal or just normal: the matrix pipe keeps them, bitwise the oracle's."""
    rng = np.random.default_rng(25)
    T, M, K = 64, 160, 256
    nb = K // 32
    wq = rng.integers(-128, 128, (M, nb, 32)).astype(np.int8)
    aq = rng.integers(-128, 128, (T, nb, 32)).astype(np.int8)
    ws = (2.0 ** rng.integers(-75, -60, (M, nb)) * rng.uniform(1, 2, (M, nb))).astype(np.float32)
    as_ = (2.0 ** rng.integers(-75, -60, (T, nb)) * rng.uniform(1, 2, (T, nb))).astype(np.float32)
    assert np.any(ws[None, :, :] * as_[:, None, :] < np.finfo(np.float32).tiny)
    np.testing.assert_array_equal(_gemm_split(hip, wq, ws, aq, as_), oracle.gemm_q8_split(wq, ws, aq, as_, NT))


def test_quantize_q8_split_matches_block_quantizer(hip, oracle):
    """The split-output quantizer writes the block quantizer's quants and its fp16 d
    widened to fp32 (an all-zero row and large values included)."""
    rng = np.random.default_rng(22)
    T, K = 37, 4128
    a = rng.standard_normal((T, K)).astype(np.float32)
    a[3] = 0.0
    a[5, :64] *= 1e4
    da, db = DeviceBuffer.from_numpy(a), DeviceBuffer(gguf.q8_0_nbytes(T, K))
    dq, ds = DeviceBuffer(T * K), DeviceBuffer(T * K // 32 * 4)
    assert hip.asmhip_quantize_q8_split(da.ptr, dq.ptr, ds.ptr, T, K, None) == 0, hip.asmhip_last_error()
    assert hip.asmhip_quantize(native.Q8_0, da.ptr, db.ptr, T, K, None) == 0, hip.asmhip_last_error()
    synchronize()
    blocks = db.download(np.uint8, (T, K // 32, 34))
    np.testing.assert_array_equal(blocks, oracle.quantize_q8_0(a))
    qs_ref, sc_ref = oracle.split_q8_0(blocks)
    np.testing.assert_array_equal(dq.download(np.int8, (T, K // 32, 32)), qs_ref)
    np.testing.assert_array_equal(ds.download(np.float32, (T, K // 32)), sc_ref)


def test_gemm_split_from_fp32_activations(hip, oracle):
    """fp32 activations -> split quantizer -> split GEMM, bitwise the block path."""
    T, M, K = 96, 384, 1024
    rng = np.random.default_rng(23)
    a = rng.standard_normal((T, K)).astype(np.float32)
    w_blocks, _ = _problem(24, 1, M, K)
    wq, ws = oracle.split_q8_0(w_blocks)
    da = DeviceBuffer.from_numpy(a)
    dq, ds = DeviceBuffer(T * K), DeviceBuffer(T * K // 32 * 4)
    dwq, dws, dc = DeviceBuffer.from_numpy(wq), DeviceBuffer.from_numpy(ws), DeviceBuffer(T * M * 4)
    assert hip.asmhip_quantize_q8_split(da.ptr, dq.ptr, ds.ptr, T, K, None) == 0
    assert hip.asmhip_gemm_q8_split(dwq.ptr, dws.ptr, dq.ptr, ds.ptr, dc.ptr, T, M, K, None) == 0
    synchronize()
    a_blocks = oracle.quantize_q8_0(a)
    np.testing.assert_array_equal(dc.download(np.float32, (T, M)), oracle.gemm_q8_0(w_blocks, a_blocks, NT))


def test_gemm_split_against_asm_matmul_q8_on_fp32_activations(hip, oracle):
    """What a caller of asm_matmul_q8 (matmul_q8_avx2.asm:51-194: int8 weights times
    fp32 x) gets from the GEMM instead: the fp32 activations are quantized to int8
    first, so each output differs from T calls of asm_matmul_q8 (the oracle's
    restatement, on the unquantized rows) by the activations' rounding, at most half
    a block step d_a = amax/127 per element: |C - ref| <= sum_k |w_k| d_a(k) / 2
    (+ 1e-5 of the row's L1 norm for fp32 rounding).  The measured difference is
    printed as a fraction of that bound and of the L1 norm."""
    T, M, K = 32, 256, 2048
    rng = np.random.default_rng(41)
    a = rng.standard_normal((T, K)).astype(np.float32)
    w_blocks, _ = _problem(42, 1, M, K)
    wq, ws = oracle.split_q8_0(w_blocks)
    da = DeviceBuffer.from_numpy(a)
    dq, ds = DeviceBuffer(T * K), DeviceBuffer(T * K // 32 * 4)
    dwq, dws, dc = DeviceBuffer.from_numpy(wq), DeviceBuffer.from_numpy(ws), DeviceBuffer(T * M * 4)
    assert hip.asmhip_quantize_q8_split(da.ptr, dq.ptr, ds.ptr, T, K, None) == 0
    assert hip.asmhip_gemm_q8_split(dwq.ptr, dws.ptr, dq.ptr, ds.ptr, dc.ptr, T, M, K, None) == 0
    synchronize()
    c = dc.download(np.float32, (T, M)).astype(np.float64)
    d_a = ds.download(np.float32, (T, K // 32)).astype(np.float64)
    wabs = np.abs(oracle.dequantize_q8_0(w_blocks).astype(np.float64))       # [M][K]
    ref = np.stack([oracle.matmul_q8(wq, ws, a[t]) for t in range(T)]).astype(np.float64)
    step = np.repeat(d_a, 32, axis=1) / 2                                     # [T][K]
    bound = step @ wabs.T                                                     # sum_k |w_k| d_a(k) / 2
    l1 = np.abs(a.astype(np.float64)) @ wabs.T
    err = np.abs(c - ref)
    assert np.all(err <= bound + 1e-5 * l1), f"max err / bound {np.max(err / (bound + 1e-30)):.3f}"
    print(f"GEMM vs asm_matmul_q8 on fp32 x: max err/bound {np.max(err / bound):.3f}, "
          f"max err/L1 {np.max(err / l1):.2e}")


def test_gemm_split_rejects_bad_arguments(hip):
    d = DeviceBuffer(1 << 16)
    p = d.ptr
    bad = native.ERR_INVALID_ARGUMENT
    assert hip.asmhip_gemm_q8_split(p, p, p, p, p, 4, 4, 40, None) == bad      # K % 32
    assert hip.asmhip_gemm_q8_split(p, p, p, p, p, 0, 4, 32, None) == bad      # T = 0
    assert hip.asmhip_gemm_q8_split(p + 4, p, p, p, p, 4, 4, 32, None) == bad  # qs not 16-byte aligned
    assert hip.asmhip_gemm_q8_split(p, None, p, p, p, 4, 4, 32, None) == bad
    assert hip.asmhip_quantize_q8_split(p, p + 8, p, 4, 32, None) == bad
    assert hip.asmhip_quantize_q8_split(p, p, p, 4, 40, None) == bad


# ---- GEMM tile layout: the same blocks arranged so a workgroup's K step is contiguous --------

def tile_layout(blocks, R):
    """The GEMM tile layout by reshaping: rows padded with zeros to a multiple of R,
    then [tile][K step of two blocks][row of the tile][68 bytes]."""
    rows, nb, _ = blocks.shape
    padded = -(-rows // R) * R
    b = np.zeros((padded, nb, 34), np.uint8)
    b[:rows] = blocks
    return np.ascontiguousarray(b.reshape(padded // R, R, nb // 2, 68).transpose(0, 2, 1, 3)).reshape(-1)


def _tiled(hip, w_blocks, a_blocks):
    M, T, K = w_blocks.shape[0], a_blocks.shape[0], w_blocks.shape[1] * 32
    dwb, dab = DeviceBuffer.from_numpy(w_blocks), DeviceBuffer.from_numpy(a_blocks)
    dw = DeviceBuffer(hip.asmhip_gemm_q8_0_tiled_weight_bytes(M, K))
    da = DeviceBuffer(hip.asmhip_gemm_q8_0_tiled_activation_bytes(T, K))
    assert hip.asmhip_gemm_q8_0_tile_weights(dwb.ptr, dw.ptr, M, K, None) == 0, hip.asmhip_last_error()
    assert hip.asmhip_gemm_q8_0_tile_activations(dab.ptr, da.ptr, T, K, None) == 0, hip.asmhip_last_error()
    dc = DeviceBuffer(T * M * 4)
    rc = hip.asmhip_gemm_q8_0_tiled(dw.ptr, da.ptr, dc.ptr, T, M, K, None)
    assert rc == 0, hip.asmhip_last_error()
    synchronize()
    return dc.download(np.float32, (T, M)), dw.download(np.uint8, dw.nbytes), da.download(np.uint8, da.nbytes)


@pytest.mark.parametrize("T,M,K", [(512, 11008, 4096), (64, 128, 128), (1, 1, 64), (7, 33, 64), (100, 1000, 1024),
                                   (65, 257, 192), (130, 300, 320)])
def test_gemm_tiled_equals_block_gemm(hip, oracle, T, M, K):
    """Same blocks in the tile layout: C bitwise equal to asmhip_gemm_q8_0's, which the
    oracle bounds; the tiling kernels equal the reshape form of the layout, padding zero."""
    w_blocks, a_blocks = _problem(T * 5 + M + K, T, M, K)
    c, wt, at = _tiled(hip, w_blocks, a_blocks)
    np.testing.assert_array_equal(wt, tile_layout(w_blocks, 128))
    np.testing.assert_array_equal(at, tile_layout(a_blocks, 64))
    np.testing.assert_array_equal(c, _gemm(hip, w_blocks, a_blocks))
    if T * M <= 200_000:
        _assert_close(c, oracle.gemm_q8_0(w_blocks, a_blocks, NT), w_blocks, a_blocks, oracle)


def test_gemm_tiled_subnormal_and_extreme_scales(hip, oracle):
    T, M, K = 64, 128, 512
    w_blocks, a_blocks = _problem(13, T, M, K)
    rng = np.random.default_rng(15)
    sub = np.array([2.0 ** -24, 3 * 2.0 ** -20, 2.0 ** -15, 6.0e-5], np.float16).view(np.uint8).reshape(-1, 2)
    big = np.array([60000.0, 1024.5, 0.5], np.float16).view(np.uint8).reshape(-1, 2)
    for blocks, pool in ((w_blocks, sub), (a_blocks, np.concatenate([sub, big]))):
        pick = rng.integers(0, len(pool), blocks.shape[:2])
        mask = rng.random(blocks.shape[:2]) < 0.3
        blocks[mask, 0:2] = pool[pick[mask]]
    np.testing.assert_array_equal(_tiled(hip, w_blocks, a_blocks)[0], oracle.gemm_q8_0(w_blocks, a_blocks, NT))


def test_quantize_tiled_equals_quantize_then_tile(hip):
    T, K = 70, 256
    x = np.random.default_rng(21).standard_normal((T, K)).astype(np.float32)
    dx, db = DeviceBuffer.from_numpy(x), DeviceBuffer(gguf.q8_0_nbytes(T, K))
    n = hip.asmhip_gemm_q8_0_tiled_activation_bytes(T, K)
    dt = DeviceBuffer.from_numpy(np.full(n, 0xA5, np.uint8))
    assert hip.asmhip_quantize(native.Q8_0, dx.ptr, db.ptr, T, K, None) == 0
    assert hip.asmhip_quantize_q8_0_tiled(dx.ptr, dt.ptr, T, K, None) == 0, hip.asmhip_last_error()
    synchronize()
    blocks = db.download(np.uint8, (T, K // 32, 34))
    got = dt.download(np.uint8, n).reshape(-1, K // 64, 64, 68)  # [tile][step][row][68]
    want = tile_layout(blocks, 64).reshape(got.shape)
    rows = np.arange(got.shape[0] * 64).reshape(-1, 64)          # global row of each tile row
    live = rows < T
    np.testing.assert_array_equal(got.transpose(0, 2, 1, 3)[live], want.transpose(0, 2, 1, 3)[live])
    assert np.all(got.transpose(0, 2, 1, 3)[~live] == 0xA5)      # padding rows are not written


def test_gemm_tiled_rejects_bad_arguments(hip):
    d = DeviceBuffer(1 << 20)
    p = d.ptr
    bad = native.ERR_INVALID_ARGUMENT
    assert hip.asmhip_gemm_q8_0_tiled(p, p, p, 4, 4, 96, None) == bad       # K % 64
    assert hip.asmhip_gemm_q8_0_tiled(p, p, p, 0, 4, 64, None) == bad       # T = 0
    assert hip.asmhip_gemm_q8_0_tiled(p + 4, p, p, 4, 4, 64, None) == bad   # not 16-byte aligned
    assert hip.asmhip_gemm_q8_0_tiled(p, None, p, 4, 4, 64, None) == bad
    assert hip.asmhip_gemm_q8_0_tile_weights(p, p, 4, 96, None) == bad
    assert hip.asmhip_gemm_q8_0_tile_activations(p + 2, p, 4, 64, None) == bad
    assert hip.asmhip_quantize_q8_0_tiled(p, p, 4, 32, None) == bad
