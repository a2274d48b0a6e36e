"""Host-side logic (no GPU): GGUF layouts and quantizers, the C-ABI library's
exports, and the Python binding's coverage of the public header."""

import ctypes

import numpy as np
import pytest

from asmllm_amd import gguf, native
from conftest import GOLDEN_DIR


def test_numpy_quantizers_match_oracle_bitwise(oracle):
    rng = np.random.default_rng(21)
    w = (rng.standard_normal((257, 512)) * 0.02).astype(np.float32)
    w[3, :32] = 0.0                  # all-zero block
    w[4, 40] = -w[4, 32:64].__abs__().max() * 2  # negative peak
    np.testing.assert_array_equal(gguf.quantize_q4_0(w), oracle.quantize_q4_0(w))
    np.testing.assert_array_equal(gguf.quantize_q8_0(w), oracle.quantize_q8_0(w))


def test_numpy_quantizers_known_answers():
    with np.load(GOLDEN_DIR / "quant_known_answers.npz") as f:
        np.testing.assert_array_equal(gguf.quantize_q4_0(f["q4_w"]), f["q4_blocks"])
        np.testing.assert_array_equal(gguf.quantize_q8_0(f["q8_w"]), f["q8_blocks"])


def test_split_and_dequant_match_oracle(oracle):
    rng = np.random.default_rng(22)
    w = (rng.standard_normal((33, 256)) * 0.02).astype(np.float32)
    b4, b8 = gguf.quantize_q4_0(w), gguf.quantize_q8_0(w)
    for mine, theirs in zip(gguf.split_q4_0(b4), oracle.split_q4_0(b4)):
        np.testing.assert_array_equal(mine, theirs)
    for mine, theirs in zip(gguf.split_q8_0(b8), oracle.split_q8_0(b8)):
        np.testing.assert_array_equal(mine, theirs)
    np.testing.assert_array_equal(gguf.dequantize_q4_0(b4), oracle.dequantize_q4_0(b4))
    np.testing.assert_array_equal(gguf.dequantize_q8_0(b8), oracle.dequantize_q8_0(b8))


def test_quantize_rejects_ragged_k():
    with pytest.raises(ValueError):
        gguf.quantize_q4_0(np.zeros((2, 33), np.float32))


def test_library_exports_every_header_symbol():
    lib = native.try_load_native_library()
    assert lib is not None, f"{native.LIB_PATH} not built (python -m asmllm_amd.build)"
    declared = native.header_symbols()
    assert len(declared) >= 30
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, f"declared in include/asmllm_hip.h but not exported: {missing}"


def test_binding_covers_header_exactly():
    assert sorted(native.SIGNATURES) == sorted(native.header_symbols())


def test_reference_argtypes_mirrored():
    # test_runner.py:94-101 (matvec) and :199-207 (_mt) argtypes
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    assert native.SIGNATURES["asm_matmul_q4"] == (None, [P, P, P, P, I64, I64])
    assert native.SIGNATURES["asm_matmul_q8"] == (None, [P, P, P, P, I64, I64])
    assert native.SIGNATURES["asm_matmul_q4_mt"] == (None, [P, P, P, P, I64, I64, ctypes.c_int])


def test_7b_decode_byte_budget():
    """Bytes one 7B-shape token step streams: 32 layers of Q4_0 q/k/v/o,
    gate/up/down (113,836,032 B each) plus the 32000x4096 lm-head."""
    from asmllm_amd.engine import LLAMA_7B

    assert LLAMA_7B.layer_weight_bytes() == 113_836_032
    assert LLAMA_7B.weight_bytes() == 3_716_481_024
    assert LLAMA_7B.kv_bytes_per_position() == 524_288
    assert LLAMA_7B.head_dim == 128 and LLAMA_7B.qkv_rows == 3 * 4096


def test_gate_up_interleave_round_trip():
    """The engine's gate/up row order (8 gate rows, the same 8 up rows, ...)."""
    from asmllm_amd.engine import interleave_gate_up, split_gate_up

    rng = np.random.default_rng(3)
    gate = rng.integers(0, 256, (24, 3, 18), dtype=np.uint8)
    up = rng.integers(0, 256, (24, 3, 18), dtype=np.uint8)
    gu = interleave_gate_up(gate, up)
    assert gu.shape == (48, 3, 18)
    for g in range(3):
        np.testing.assert_array_equal(gu[16 * g:16 * g + 8], gate[8 * g:8 * g + 8])
        np.testing.assert_array_equal(gu[16 * g + 8:16 * g + 16], up[8 * g:8 * g + 8])
    g2, u2 = split_gate_up(gu)
    np.testing.assert_array_equal(g2, gate)
    np.testing.assert_array_equal(u2, up)
    with pytest.raises(ValueError):
        interleave_gate_up(gate[:20], up[:20])


def test_gemm_tiled_sizes():
    """Tile-layout sizes: rows padded to 128 (weights) or 64 (activations), K/32 blocks
    of 34 bytes a row; 0 for shapes the tiled GEMM does not take."""
    lib = native.try_load_native_library()
    assert lib is not None
    assert lib.asmhip_gemm_q8_0_tiled_weight_bytes(11008, 4096) == 11008 * 128 * 34
    assert lib.asmhip_gemm_q8_0_tiled_weight_bytes(1000, 64) == 1024 * 2 * 34
    assert lib.asmhip_gemm_q8_0_tiled_activation_bytes(512, 4096) == 512 * 128 * 34
    assert lib.asmhip_gemm_q8_0_tiled_activation_bytes(65, 128) == 128 * 4 * 34
    for bad in ((0, 64), (4, 96), (4, 0), (-1, 64)):
        assert lib.asmhip_gemm_q8_0_tiled_weight_bytes(*bad) == 0
        assert lib.asmhip_gemm_q8_0_tiled_activation_bytes(*bad) == 0


def test_bench_trace_filters_name_built_kernels():
    """bench.py picks the headline matvec and the GEMM forms out of rocprofv3 traces by
    kernel name: every name it filters on is an instantiation the library holds."""
    import shutil
    import subprocess

    import bench

    if shutil.which("nm") is None or not native.LIB_PATH.exists():
        pytest.skip("nm or the built library missing")
    names = subprocess.run(["nm", "-C", str(native.LIB_PATH)], capture_output=True, text=True, check=True).stdout
    assert bench.HEADLINE_KERNEL + "(" in names
    for fragment in ("gemm_q8_0_tiled<", "gemm_q8_0_coalesced<", "gemm_q8_split("):
        assert fragment in names, fragment


def test_single_workgroup_ops_refuse_lengths_near_int_max():
    """The one-workgroup decode ops step an int index by up to 32768 while it is
    below the length; lengths that close to 2^31 are refused on the host before
    anything is launched (the pointers below are never dereferenced)."""
    lib = native.lib()
    p, big = ctypes.c_void_p(256), 2 ** 31 - 1
    calls = {
        "rmsnorm": lambda: lib.asmhip_rmsnorm(p, p, p, big, 1e-6, None),
        "softmax": lambda: lib.asmhip_softmax(p, p, big, None),
        "silu_hadamard": lambda: lib.asmhip_silu_hadamard(p, p, big, None),
        "attention": lambda: lib.asmhip_attention(p, p, p, p, 1, big, 1.0, None),
        "argmax": lambda: lib.asmhip_argmax(p, big, p, None, None),
    }
    for name, call in calls.items():
        assert call() == -1, name
        assert name in native.last_error(), (name, native.last_error())
