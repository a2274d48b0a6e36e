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
