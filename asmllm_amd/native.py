"""ctypes binding of libasmllm.so.

Mirrors the reference's loader (tests/correctness/test_runner.py:52-68) and the
argtypes its callers set (test_runner.py:94-101, 199-207, 384-390, 408-414,
430, 448-456; src/runtime/generate.py:221-250).  The reference loads
``build/libasmllm.so``; this package loads ``asmllm_amd/lib/libasmllm.so``.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int64, c_size_t, c_uint64, c_void_p, c_char_p, POINTER
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "lib" / "libasmllm.so"
HEADER_PATH = PKG.parent / "include" / "asmllm_hip.h"

_P = c_void_p

# Values of the header's #defines.
Q4_0 = 2
Q5_0 = 6
Q8_0 = 8
PRE_NONE, PRE_RMSNORM, PRE_SWIGLU = 0, 1, 2
Q4_KERNEL_AUTO, Q4_KERNEL_FP32, Q4_KERNEL_MFMA = 0, 1, 2
OK, ERR_INVALID_ARGUMENT, ERR_HIP, ERR_UNSUPPORTED, ERR_NO_DEVICE = 0, -1, -2, -3, -4
# name -> (restype, argtypes)
SIGNATURES: dict[str, tuple] = {
    # reference-named entry points
    "asm_matmul_q4": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "asm_matmul_q4_avx512": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "asm_matmul_q8": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "asm_matmul_q4_mt": (None, [_P, _P, _P, _P, c_int64, c_int64, c_int]),
    "asm_matmul_q8_mt": (None, [_P, _P, _P, _P, c_int64, c_int64, c_int]),
    "asm_threadpool_dispatch_q8": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "asm_matmul_q5": (None, [_P, _P, _P, _P, _P, c_int64, c_int64]),
    "asm_matmul_q5_mt": (None, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int]),
    "asm_threadpool_dispatch_q5": (None, [_P, _P, _P, _P, _P, c_int64, c_int64]),
    "asm_threadpool_init": (None, [c_int]),
    "asm_threadpool_shutdown": (None, []),
    "asm_threadpool_get_num_threads": (c_int, []),
    "asm_rmsnorm": (None, [_P, _P, _P, c_int64, c_float]),
    "asm_rope": (None, [_P, _P, c_int64, c_int64, c_float]),
    "asm_softmax": (None, [_P, _P, c_int64]),
    "asm_silu_hadamard": (None, [_P, _P, c_int64]),
    "asm_attention": (None, [_P, _P, _P, _P, c_int64, c_int64, c_float]),
    # device entry points
    "asmhip_matmul_q4_0": (c_int, [_P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_matmul_q8_0": (c_int, [_P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_matmul_q4_split": (c_int, [_P, _P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_matmul_q8_split": (c_int, [_P, _P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_matmul_q5_split": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_matmul_q5_0": (c_int, [_P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_dequantize_q5_0": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "asmhip_dequantize_q4_0": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "asmhip_dequantize_q8_0": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "asmhip_matmul_fused": (c_int, [c_int, _P, _P, _P, c_int64, c_int64, c_int, _P, c_float, c_int, _P]),
    "asmhip_matmul_swiglu": (c_int, [c_int, _P, _P, _P, c_int64, c_int64, c_int, _P, c_float, _P, _P]),
    "asmhip_gemm_q8_0": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, _P]),
    "asmhip_gemm_q8_split": (c_int, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int64, _P]),
    "asmhip_gemm_q8_0_tiled_weight_bytes": (c_int64, [c_int64, c_int64]),
    "asmhip_gemm_q8_0_tiled_activation_bytes": (c_int64, [c_int64, c_int64]),
    "asmhip_gemm_q8_0_tile_weights": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "asmhip_gemm_q8_0_tile_activations": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "asmhip_quantize_q8_0_tiled": (c_int, [_P, _P, c_int64, c_int64, _P]),
    "asmhip_gemm_q8_0_tiled": (c_int, [_P, _P, _P, c_int64, c_int64, c_int64, _P]),
    "asmhip_set_q4_kernel": (c_int, [c_int]),
    "asmhip_get_q4_kernel": (c_int, []),
    "asmhip_quantize": (c_int, [c_int, _P, _P, c_int64, c_int64, _P]),
    "asmhip_quantize_q8_split": (c_int, [_P, _P, _P, c_int64, c_int64, _P]),
    "asmhip_random_blocks": (c_int, [c_int, _P, c_int64, c_int64, c_uint64, c_float, _P]),
    "asmhip_random_f16": (c_int, [_P, c_int64, c_uint64, c_float, _P]),
    "asmhip_fill_f32": (c_int, [_P, c_int64, c_float, _P]),
    "asmhip_rmsnorm": (c_int, [_P, _P, _P, c_int64, c_float, _P]),
    "asmhip_rope": (c_int, [_P, _P, c_int64, c_int64, c_int64, _P, c_int64, c_float, _P]),
    "asmhip_softmax": (c_int, [_P, _P, c_int64, _P]),
    "asmhip_silu_hadamard": (c_int, [_P, _P, c_int64, _P]),
    "asmhip_attention": (c_int, [_P, _P, _P, _P, c_int64, c_int64, c_float, _P]),
    "asmhip_rope_kv_write": (c_int, [_P, _P, _P, c_int, c_int, c_int, _P, c_int, c_float, _P]),
    "asmhip_attention_decode_workspace": (c_int64, [c_int, c_int, c_int]),
    "asmhip_attention_decode": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, _P, c_int, _P]),
    "asmhip_attention_decode_rope": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, _P, c_int, c_float, _P]),
    "asmhip_rope_table": (c_int, [_P, c_int, c_int, c_float, _P]),
    "asmhip_attention_decode_rope_table": (c_int, [_P, _P, _P, _P, _P, c_int, c_int, c_int, _P, c_int, _P, _P]),
    "asmhip_attention_decode_partials_rope_table": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P, c_int, _P, _P]),
    "asmhip_matmul_attn_output": (c_int, [c_int, _P, _P, _P, _P, c_int64, c_int, c_int, c_int, c_int, _P]),
    "asmhip_stream_read": (c_int, [_P, c_int64, _P, _P]),
    "asmhip_stream_read_shaped": (c_int, [_P, c_int64, _P, c_int, _P, c_int64, c_int, c_int, _P, _P]),
    "asmhip_empty_launch": (c_int, [c_int, c_int, c_int, _P]),
    "asmhip_matmul_q4_0_stamped": (c_int, [_P, _P, _P, c_int64, c_int64, _P, c_int64, _P]),
    "asmhip_grid_barrier": (c_int, [_P, c_int, _P, _P]),
    "asmhip_attention_decode_noalloc_max_floats": (c_int64, []),
    "asmhip_attention_decode_rope_noalloc": (c_int, [_P, _P, _P, _P, c_int, c_int, c_int, _P, c_int, c_float, _P]),
    "asmhip_embed_q4_0": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "asmhip_embed_q8_0": (c_int, [_P, _P, _P, c_int, c_int, _P]),
    "asmhip_argmax": (c_int, [_P, c_int, _P, _P, _P]),
    "asmhip_argmax_history": (c_int, [_P, c_int, _P, _P, _P, c_int, _P]),
    # plumbing
    "asmhip_device_count": (c_int, []),
    "asmhip_device_info": (c_int, [c_char_p, c_size_t, POINTER(c_int), POINTER(c_int), POINTER(c_size_t)]),
    "asmhip_malloc": (c_void_p, [c_size_t]),
    "asmhip_free": (c_int, [_P]),
    "asmhip_memcpy": (c_int, [_P, _P, c_size_t, c_int]),
    "asmhip_synchronize": (c_int, []),
    "asmhip_stream_create": (c_void_p, []),
    "asmhip_stream_destroy": (c_int, [_P]),
    "asmhip_stream_synchronize": (c_int, [_P]),
    "asmhip_event_create": (c_void_p, []),
    "asmhip_event_create_timing": (c_void_p, []),
    "asmhip_event_destroy": (c_int, [_P]),
    "asmhip_event_record": (c_int, [_P, _P]),
    "asmhip_event_synchronize": (c_int, [_P]),
    "asmhip_event_elapsed_ms": (c_int, [_P, _P, POINTER(c_float)]),
    "asmhip_stream_begin_capture": (c_int, [_P]),
    "asmhip_stream_end_capture": (c_int, [_P, POINTER(c_void_p)]),
    "asmhip_graph_launch": (c_int, [_P, _P]),
    "asmhip_graph_destroy": (c_int, [_P]),
    "asmhip_last_error": (c_char_p, []),
}


class NativeError(RuntimeError):
    """A libasmllm entry point returned a non-zero status."""


def declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def try_load_native_library() -> ctypes.CDLL | None:
    """Returns the loaded library, or None when it has not been built
    (the reference's "NOT IMPLEMENTED" convention, test_runner.py:52-68)."""
    if not LIB_PATH.exists():
        return None
    try:
        return declare(ctypes.CDLL(str(LIB_PATH)))
    except OSError:
        return None


_LIB: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it is missing (no silent fallback)."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m asmllm_amd.build`")
        _LIB = declare(ctypes.CDLL(str(LIB_PATH)))
    return _LIB


def last_error() -> str:
    msg = lib().asmhip_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str = "") -> None:
    if status != 0:
        raise NativeError(f"{what or 'libasmllm call'} failed ({status}): {last_error()}")


def header_symbols(path: Path = HEADER_PATH) -> list[str]:
    """Every function the public header declares."""
    import re

    text = path.read_text()
    return re.findall(r"ASMHIP_API\s+[\w\s\*]+?\b(\w+)\s*\(", text)
