"""ctypes binding of oracle/liboracle.so (test infrastructure only)."""

from __future__ import annotations

import ctypes
import subprocess
from ctypes import c_float, c_int, c_int64, c_uint16, c_void_p
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"

_P = c_void_p
_SIGS = {
    "oracle_matmul_q4_avx2": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q4_lanes": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q4_avx512": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q4_avx512_lanes": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q8_avx2": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q8_lanes": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q5_avx2": (None, [_P, _P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q5_lanes": (None, [_P, _P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q5_mt": (None, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int]),
    "oracle_threadpool_dispatch_q5": (None, [_P, _P, _P, _P, _P, c_int64, c_int64]),
    "oracle_matmul_q5_0_gguf": (None, [_P, _P, _P, c_int64, c_int64, c_int]),
    "oracle_split_q5_0": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_dequantize_q5_0": (None, [_P, _P, c_int64, c_int64]),
    "oracle_matmul_q4_0_gguf": (None, [_P, _P, _P, c_int64, c_int64, c_int]),
    "oracle_matmul_q8_0_gguf": (None, [_P, _P, _P, c_int64, c_int64, c_int]),
    "oracle_split_q4_0": (None, [_P, _P, _P, c_int64, c_int64]),
    "oracle_split_q8_0": (None, [_P, _P, _P, c_int64, c_int64]),
    "oracle_dequantize_q4_0": (None, [_P, _P, c_int64, c_int64]),
    "oracle_dequantize_q8_0": (None, [_P, _P, c_int64, c_int64]),
    "oracle_quantize_q4_0": (None, [_P, _P, c_int64, c_int64]),
    "oracle_quantize_q8_0": (None, [_P, _P, c_int64, c_int64]),
    "oracle_threadpool_init": (None, [c_int]),
    "oracle_threadpool_shutdown": (None, []),
    "oracle_threadpool_get_num_threads": (c_int, []),
    "oracle_tile_rows": (c_int64, [c_int64, c_int]),
    "oracle_matmul_q4_mt": (None, [_P, _P, _P, _P, c_int64, c_int64, c_int, c_int]),
    "oracle_matmul_q8_mt": (None, [_P, _P, _P, _P, c_int64, c_int64, c_int]),
    "oracle_threadpool_dispatch_q8": (None, [_P, _P, _P, _P, c_int64, c_int64]),
    "oracle_gemm_q8_0": (None, [_P, _P, _P, c_int64, c_int64, c_int64, c_int]),
    "oracle_gemm_q8_split": (None, [_P, _P, _P, _P, _P, c_int64, c_int64, c_int64, c_int]),
    "oracle_rmsnorm": (None, [_P, _P, _P, c_int64, c_float]),
    "oracle_rope": (None, [_P, _P, c_int64, c_int64, c_float]),
    "oracle_softmax": (None, [_P, _P, c_int64]),
    "oracle_silu_hadamard": (None, [_P, _P, c_int64]),
    "oracle_attention": (None, [_P, _P, _P, _P, c_int64, c_int64, c_float]),
    "oracle_attention_decode_f16": (None, [_P, _P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, c_int]),
    "oracle_f32_to_f16": (c_uint16, [c_float]),
    "oracle_f16_to_f32": (c_float, [c_uint16]),
    "oracle_has_avx512": (c_int, []),
}

_LIB = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        cdll = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(cdll, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = cdll
    return _LIB


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


# ---- split-layout kernels (a1/a2/a3) ----------------------------------------

def matmul_q4(qweights, scales, x, kernel: str = "avx2") -> np.ndarray:
    q, s, xv = _c(qweights, np.uint8), _c(scales, np.float32), _c(x, np.float32)
    M, K = q.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    fn = {
        "avx2": lib().oracle_matmul_q4_avx2,
        "lanes": lib().oracle_matmul_q4_lanes,
        "avx512": lib().oracle_matmul_q4_avx512,
        "avx512_lanes": lib().oracle_matmul_q4_avx512_lanes,
    }[kernel]
    fn(_ptr(q), _ptr(s), _ptr(xv), _ptr(y), M, K)
    return y


def matmul_q8(qweights, scales, x, kernel: str = "avx2") -> np.ndarray:
    q, s, xv = _c(qweights, np.int8), _c(scales, np.float32), _c(x, np.float32)
    M, K = q.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    fn = {"avx2": lib().oracle_matmul_q8_avx2, "lanes": lib().oracle_matmul_q8_lanes}[kernel]
    fn(_ptr(q), _ptr(s), _ptr(xv), _ptr(y), M, K)
    return y


def matmul_q4_mt(qweights, scales, x, nt: int, variant: int = 0) -> np.ndarray:
    q, s, xv = _c(qweights, np.uint8), _c(scales, np.float32), _c(x, np.float32)
    M, K = q.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    lib().oracle_matmul_q4_mt(_ptr(q), _ptr(s), _ptr(xv), _ptr(y), M, K, nt, variant)
    return y


def matmul_q8_mt(qweights, scales, x, nt: int) -> np.ndarray:
    q, s, xv = _c(qweights, np.int8), _c(scales, np.float32), _c(x, np.float32)
    M, K = q.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    lib().oracle_matmul_q8_mt(_ptr(q), _ptr(s), _ptr(xv), _ptr(y), M, K, nt)
    return y


def matmul_q5(ql, qh, scales, x, kernel: str = "avx2") -> np.ndarray:
    l, h, s, xv = _c(ql, np.uint8), _c(qh, np.uint8), _c(scales, np.float32), _c(x, np.float32)
    M, K = l.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    fn = {"avx2": lib().oracle_matmul_q5_avx2, "lanes": lib().oracle_matmul_q5_lanes}[kernel]
    fn(_ptr(l), _ptr(h), _ptr(s), _ptr(xv), _ptr(y), M, K)
    return y


def matmul_q5_mt(ql, qh, scales, x, nt: int) -> np.ndarray:
    l, h, s, xv = _c(ql, np.uint8), _c(qh, np.uint8), _c(scales, np.float32), _c(x, np.float32)
    M, K = l.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    lib().oracle_matmul_q5_mt(_ptr(l), _ptr(h), _ptr(s), _ptr(xv), _ptr(y), M, K, nt)
    return y


def tile_rows(M: int, nt: int) -> int:
    return int(lib().oracle_tile_rows(M, nt))


# ---- GGUF block kernels -------------------------------------------------------

def matmul_q4_0_gguf(blocks, x, nt: int = 1) -> np.ndarray:
    b, xv = _c(blocks, np.uint8), _c(x, np.float32)
    M, K = b.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    lib().oracle_matmul_q4_0_gguf(_ptr(b), _ptr(xv), _ptr(y), M, K, nt)
    return y


def matmul_q8_0_gguf(blocks, x, nt: int = 1) -> np.ndarray:
    b, xv = _c(blocks, np.uint8), _c(x, np.float32)
    M, K = b.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    lib().oracle_matmul_q8_0_gguf(_ptr(b), _ptr(xv), _ptr(y), M, K, nt)
    return y


def matmul_q5_0_gguf(blocks, x, nt: int = 1) -> np.ndarray:
    b, xv = _c(blocks, np.uint8), _c(x, np.float32)
    M, K = b.shape[0], xv.shape[0]
    y = np.zeros(M, np.float32)
    lib().oracle_matmul_q5_0_gguf(_ptr(b), _ptr(xv), _ptr(y), M, K, nt)
    return y


def quantize_q4_0(w) -> np.ndarray:
    wv = _c(w, np.float32)
    rows, K = wv.shape
    out = np.empty((rows, K // 32, 18), np.uint8)
    lib().oracle_quantize_q4_0(_ptr(wv), _ptr(out), rows, K)
    return out


def quantize_q8_0(w) -> np.ndarray:
    wv = _c(w, np.float32)
    rows, K = wv.shape
    out = np.empty((rows, K // 32, 34), np.uint8)
    lib().oracle_quantize_q8_0(_ptr(wv), _ptr(out), rows, K)
    return out


def dequantize_q4_0(blocks) -> np.ndarray:
    b = _c(blocks, np.uint8)
    rows, nb = b.shape[0], b.shape[1]
    out = np.empty((rows, nb * 32), np.float32)
    lib().oracle_dequantize_q4_0(_ptr(b), _ptr(out), rows, nb * 32)
    return out


def dequantize_q8_0(blocks) -> np.ndarray:
    b = _c(blocks, np.uint8)
    rows, nb = b.shape[0], b.shape[1]
    out = np.empty((rows, nb * 32), np.float32)
    lib().oracle_dequantize_q8_0(_ptr(b), _ptr(out), rows, nb * 32)
    return out


def dequantize_q5_0(blocks) -> np.ndarray:
    b = _c(blocks, np.uint8)
    rows, nb = b.shape[0], b.shape[1]
    out = np.empty((rows, nb * 32), np.float32)
    lib().oracle_dequantize_q5_0(_ptr(b), _ptr(out), rows, nb * 32)
    return out


def split_q5_0(blocks):
    """GGUF Q5_0 blocks [rows][nb][22] -> (ql [rows][nb][16], qh [rows][nb][4], fp32 scales)."""
    b = _c(blocks, np.uint8)
    rows, nb = b.shape[0], b.shape[1]
    ql = np.empty((rows, nb, 16), np.uint8)
    qh = np.empty((rows, nb, 4), np.uint8)
    sc = np.empty((rows, nb), np.float32)
    lib().oracle_split_q5_0(_ptr(b), _ptr(ql), _ptr(qh), _ptr(sc), rows, nb * 32)
    return ql, qh, sc


def split_q4_0(blocks):
    b = _c(blocks, np.uint8)
    rows, nb = b.shape[0], b.shape[1]
    qs = np.empty((rows, nb, 16), np.uint8)
    sc = np.empty((rows, nb), np.float32)
    lib().oracle_split_q4_0(_ptr(b), _ptr(qs), _ptr(sc), rows, nb * 32)
    return qs, sc


def split_q8_0(blocks):
    b = _c(blocks, np.uint8)
    rows, nb = b.shape[0], b.shape[1]
    qs = np.empty((rows, nb, 32), np.int8)
    sc = np.empty((rows, nb), np.float32)
    lib().oracle_split_q8_0(_ptr(b), _ptr(qs), _ptr(sc), rows, nb * 32)
    return qs, sc


def gemm_q8_0(w_blocks, a_blocks, nt: int = 1) -> np.ndarray:
    w, a = _c(w_blocks, np.uint8), _c(a_blocks, np.uint8)
    M, T, K = w.shape[0], a.shape[0], w.shape[1] * 32
    c = np.zeros((T, M), np.float32)
    lib().oracle_gemm_q8_0(_ptr(w), _ptr(a), _ptr(c), T, M, K, nt)
    return c


def gemm_q8_split(w_qs, w_scales, a_qs, a_scales, nt: int = 1) -> np.ndarray:
    """Split operands: qs int8 [rows][K/32][32] (or [rows][K]), scales fp32 [rows][K/32]."""
    wq, aq = _c(w_qs, np.int8), _c(a_qs, np.int8)
    ws, as_ = _c(w_scales, np.float32), _c(a_scales, np.float32)
    M, T = wq.shape[0], aq.shape[0]
    K = wq.size // M
    c = np.zeros((T, M), np.float32)
    lib().oracle_gemm_q8_split(_ptr(wq), _ptr(ws), _ptr(aq), _ptr(as_), _ptr(c), T, M, K, nt)
    return c


# ---- decode ops -------------------------------------------------------------------

def rmsnorm(x, w, eps: float) -> np.ndarray:
    xv, wv = _c(x, np.float32), _c(w, np.float32)
    y = np.zeros_like(xv)
    lib().oracle_rmsnorm(_ptr(xv), _ptr(wv), _ptr(y), xv.shape[0], eps)
    return y


def rope(q, k, head_dim: int, pos: int, theta: float):
    qv, kv = _c(q, np.float32).copy(), _c(k, np.float32).copy()
    lib().oracle_rope(_ptr(qv), _ptr(kv), head_dim, pos, theta)
    return qv, kv


def softmax(x) -> np.ndarray:
    xv = _c(x, np.float32)
    y = np.zeros_like(xv)
    lib().oracle_softmax(_ptr(xv), _ptr(y), xv.shape[0])
    return y


def silu_hadamard(gate, up) -> np.ndarray:
    g, u = _c(gate, np.float32).copy(), _c(up, np.float32)
    lib().oracle_silu_hadamard(_ptr(g), _ptr(u), g.shape[0])
    return g


def attention(q, k, v, scale: float) -> np.ndarray:
    qv, kv, vv = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    y = np.zeros_like(qv)
    lib().oracle_attention(_ptr(qv), _ptr(kv), _ptr(vv), _ptr(y), qv.shape[0], qv.shape[1], scale)
    return y


def attention_decode_f16(q, k_cache, v_cache, n_pos: int, n_kv_heads: int, nt: int = 1) -> np.ndarray:
    """q [n_heads, hd] float32; caches [max_pos, n_kv_heads, hd] as uint16 fp16 bits."""
    qv = _c(q, np.float32)
    kc, vc = _c(k_cache, np.uint16), _c(v_cache, np.uint16)
    n_heads, hd = qv.shape
    out = np.zeros_like(qv)
    lib().oracle_attention_decode_f16(_ptr(qv), _ptr(kc), _ptr(vc), _ptr(out), n_heads, n_kv_heads, hd, n_pos,
                                      n_kv_heads * hd, nt)
    return out


def f32_to_f16(f: float) -> int:
    return int(lib().oracle_f32_to_f16(f))


def f16_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(h))


def has_avx512() -> bool:
    return bool(lib().oracle_has_avx512())


def threadpool_init(n: int) -> None:
    lib().oracle_threadpool_init(n)


def threadpool_shutdown() -> None:
    lib().oracle_threadpool_shutdown()


def threadpool_size() -> int:
    return int(lib().oracle_threadpool_get_num_threads())
