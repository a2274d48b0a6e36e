"""numpy restatement of the reference oracle tests/reference/ops.py (test
infrastructure only), plus float64 closed forms used to pin it.

The float32 functions keep ops.py's dtypes and operation order so that they
produce what the reference's own correctness runner compares against.
"""

from __future__ import annotations

import math

import numpy as np


# ---- ops.py:16-30 / 33-41 ------------------------------------------------------

def dequantize_q4_0(qblocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """(rows, nb, 16) nibbles + (rows, nb) fp32 scales -> (rows, nb*32);
    low nibbles are weights 0..15, high nibbles 16..31."""
    rows, nb, width = qblocks.shape
    assert width == 16
    low = (qblocks & 0x0F).astype(np.float32) - 8.0
    high = ((qblocks >> 4) & 0x0F).astype(np.float32) - 8.0
    w = np.concatenate([low, high], axis=-1) * scales[:, :, None]
    return w.reshape(rows, nb * 32)


def q4_matmul(qweights: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    return dequantize_q4_0(qweights, scales) @ x


# ---- ops.py:44-64 ----------------------------------------------------------------

def dequantize_q8_0(qweights: np.ndarray, scales: np.ndarray) -> np.ndarray:
    rows, nb, width = qweights.shape
    assert width == 32
    return (qweights.astype(np.float32) * scales[:, :, None]).reshape(rows, nb * 32)


def q8_matmul(qweights: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    return dequantize_q8_0(qweights, scales) @ x


# ---- ops.py:67-99 ------------------------------------------------------------------

def dequantize_q5_0(ql: np.ndarray, qh: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """(rows, nb, 16) nibbles + (rows, nb, 4) high-bit planes + (rows, nb)
    fp32 scales -> (rows, nb*32).  Weight j's fifth bit is bit j % 8 of qh
    byte j // 8; value ((nibble | bit << 4) - 16) * scale in float32."""
    rows, nb, width = ql.shape
    assert width == 16 and qh.shape == (rows, nb, 4)
    nib = np.concatenate([ql & 0x0F, ql >> 4], axis=-1).astype(np.int32)
    bits = np.unpackbits(qh, axis=-1, bitorder="little").astype(np.int32)
    w = (nib | (bits << 4)).astype(np.float32) - np.float32(16.0)
    return (w * scales[:, :, None]).reshape(rows, nb * 32)


def q5_matmul(ql: np.ndarray, qh: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    return dequantize_q5_0(ql, qh, scales) @ x


# ---- ops.py:103-170 ----------------------------------------------------------------

def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    x32 = x.astype(np.float32)
    rms = np.sqrt(np.mean(x32 ** 2, axis=-1, keepdims=True) + eps)
    return ((x32 / rms) * weight).astype(x.dtype)


def rope(q: np.ndarray, k: np.ndarray, head_dim: int, pos: int, theta: float = 10000.0):
    """Interleaved pairs (2p, 2p+1) rotated by pos * theta^(-2p/hd)."""
    assert head_dim % 2 == 0
    freqs = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float32) / head_dim))
    ang = pos * freqs
    c, s = np.cos(ang), np.sin(ang)

    def rot(v):
        v32 = v.astype(np.float32)
        a, b = v32[..., 0::2], v32[..., 1::2]
        out = np.empty_like(v32)
        out[..., 0::2] = a * c - b * s
        out[..., 1::2] = a * s + b * c
        return out.astype(v.dtype)

    return rot(q), rot(k)


def softmax(x: np.ndarray) -> np.ndarray:
    e = np.exp(x - np.max(x, axis=-1, keepdims=True))
    return e / np.sum(e, axis=-1, keepdims=True)


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float | None = None) -> np.ndarray:
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[1])
    return softmax((q @ k.T) * scale) @ v


def silu_hadamard(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """generate.py:370: gate / (1 + exp(-gate)) * up."""
    return (gate / (1.0 + np.exp(-gate))) * up


# ---- float64 closed forms ------------------------------------------------------------

def q4_matvec_f64(qweights: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[m] = sum_b s[m,b] * sum_j (n - 8) x[32b+j], every term in float64,
    built element by element (no shared helper with dequantize_q4_0)."""
    M, nb, _ = qweights.shape
    n = np.empty((M, nb, 32), np.float64)
    for j in range(16):
        n[:, :, j] = (qweights[:, :, j] % 16).astype(np.float64) - 8.0
        n[:, :, 16 + j] = (qweights[:, :, j] // 16).astype(np.float64) - 8.0
    xb = x.astype(np.float64).reshape(nb, 32)
    per_block = np.einsum("mbj,bj->mb", n, xb)
    return (per_block * scales.astype(np.float64)).sum(axis=1)


def q8_matvec_f64(qweights: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    M, nb, _ = qweights.shape
    xb = x.astype(np.float64).reshape(nb, 32)
    per_block = np.einsum("mbj,bj->mb", qweights.astype(np.float64), xb)
    return (per_block * scales.astype(np.float64)).sum(axis=1)


def q5_matvec_f64(ql: np.ndarray, qh: np.ndarray, scales: np.ndarray, x: np.ndarray) -> np.ndarray:
    """y[m] = sum_b s[m,b] * sum_j ((n_j + 16 h_j) - 16) x[32b+j] in float64,
    with n_j and h_j read element by element (ql byte j % 16, low nibble for
    j < 16; bit j % 8 of qh byte j // 8), not through dequantize_q5_0."""
    M, nb, _ = ql.shape
    w = np.empty((M, nb, 32), np.float64)
    for j in range(32):
        n = (ql[:, :, j % 16] % 16) if j < 16 else (ql[:, :, j % 16] // 16)
        h = (qh[:, :, j // 8] // (1 << (j % 8))) % 2
        w[:, :, j] = n.astype(np.float64) + 16.0 * h.astype(np.float64) - 16.0
    xb = x.astype(np.float64).reshape(nb, 32)
    return (np.einsum("mbj,bj->mb", w, xb) * scales.astype(np.float64)).sum(axis=1)


def row_l1(w_fp32: np.ndarray, x: np.ndarray) -> np.ndarray:
    """sum_k |w[m,k]| |x[k]|, the scale of the matvec tolerance."""
    return np.abs(w_fp32.astype(np.float64)) @ np.abs(x.astype(np.float64))
