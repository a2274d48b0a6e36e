"""GGUF Q4_0 / Q8_0 / Q5_0 block layouts on the host (numpy).

Block layouts (32 weights per block):
  * Q4_0, 18 bytes: fp16 d, then 16 bytes; byte j holds weight j in its low
    nibble and weight j+16 in its high nibble; value = (nibble - 8) * d.
  * Q8_0, 34 bytes: fp16 d, then 32 int8; value = q * d.
  * Q5_0, 22 bytes: fp16 d, qh[4], qs[16]; qs as in Q4_0, and bit j of the
    little-endian word qh is weight j's fifth bit; value =
    ((nibble | bit << 4) - 16) * d (tests/reference/ops.py:67-92, whose
    split layout ql/qh/scales is these three fields pulled apart).

The split conversion mirrors src/runtime/generate.py:91-119 (qs split out,
fp16 d widened exactly to fp32).  The quantizers produce the synthetic
weights of the benchmark configurations; the CPU oracle and the GPU
quantizer kernels produce the same bytes.
"""

from __future__ import annotations

import numpy as np

QK = 32
Q4_0_BYTES = 18
Q8_0_BYTES = 34
Q5_0_BYTES = 22


def _blocks(w: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.float32)
    if w.ndim != 2 or w.shape[1] % QK:
        raise ValueError(f"expected [rows, K] with K % 32 == 0, got {w.shape}")
    return w.reshape(w.shape[0], w.shape[1] // QK, QK)


def quantize_q4_0(w: np.ndarray) -> np.ndarray:
    """[rows, K] float32 -> [rows, K/32, 18] uint8.

    d = m / -8 with m the first element of largest magnitude; id = 1/d
    (0 if d == 0); q = min(15, trunc(w*id + 8.5)); d stored as fp16 (RNE).
    """
    v = _blocks(w)
    a = np.abs(v)
    amax = a.max(axis=-1)
    idx = a.argmax(axis=-1)
    mx = np.take_along_axis(v, idx[..., None], axis=-1)[..., 0]
    mx = np.where(amax > 0, mx, np.float32(0.0)).astype(np.float32)
    d = (mx / np.float32(-8.0)).astype(np.float32)
    inv = np.zeros_like(d)
    np.divide(np.float32(1.0), d, out=inv, where=d != 0)
    x = (v * inv[..., None]).astype(np.float32)
    q = np.minimum((x + np.float32(8.5)).astype(np.int32), 15).astype(np.uint8)
    out = np.empty(v.shape[:2] + (Q4_0_BYTES,), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(d.shape + (2,))
    out[..., 2:] = q[..., :16] | (q[..., 16:] << 4)
    return out


def quantize_q8_0(w: np.ndarray) -> np.ndarray:
    """[rows, K] float32 -> [rows, K/32, 34] uint8.

    d = amax / 127, inv = 127 / amax (0 if amax == 0), q = saturate(rint(w*inv))
    with ties to even -- the reference's activation quantizer
    (src/kernels/arm64/matmul_q4_neon.S:80-135) -- and d stored as fp16.
    """
    v = _blocks(w)
    amax = np.abs(v).max(axis=-1).astype(np.float32)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.zeros_like(amax)
    np.divide(np.float32(127.0), amax, out=inv, where=amax != 0)
    t = (v * inv[..., None]).astype(np.float32)
    q = np.clip(np.rint(t), -128, 127).astype(np.int8)
    out = np.empty(v.shape[:2] + (Q8_0_BYTES,), dtype=np.uint8)
    out[..., 0:2] = d.astype(np.float16).view(np.uint8).reshape(d.shape + (2,))
    out[..., 2:] = q.view(np.uint8)
    return out


def split_q4_0(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """GGUF Q4_0 blocks -> (qs [rows, nb, 16] uint8, scales [rows, nb] float32);
    generate.py:91-99."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0].astype(np.float32)
    return np.ascontiguousarray(b[..., 2:]), np.ascontiguousarray(scales)


def split_q8_0(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """GGUF Q8_0 blocks -> (qs [rows, nb, 32] int8, scales [rows, nb] float32);
    generate.py:109-117."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0].astype(np.float32)
    return np.ascontiguousarray(b[..., 2:]).view(np.int8), np.ascontiguousarray(scales)


def dequantize_q4_0(blocks: np.ndarray) -> np.ndarray:
    """Exact fp32 weights [rows, K]; generate.py:100-105."""
    qs, scales = split_q4_0(blocks)
    lo = (qs & 0x0F).astype(np.float32) - np.float32(8.0)
    hi = (qs >> 4).astype(np.float32) - np.float32(8.0)
    w = np.concatenate([lo, hi], axis=-1) * scales[..., None]
    return w.reshape(qs.shape[0], -1).astype(np.float32)


def dequantize_q8_0(blocks: np.ndarray) -> np.ndarray:
    """Exact fp32 weights [rows, K]; generate.py:117-118."""
    qs, scales = split_q8_0(blocks)
    w = qs.astype(np.float32) * scales[..., None]
    return w.reshape(qs.shape[0], -1).astype(np.float32)


def q4_0_nbytes(rows: int, K: int) -> int:
    return rows * (K // QK) * Q4_0_BYTES


def q8_0_nbytes(rows: int, K: int) -> int:
    return rows * (K // QK) * Q8_0_BYTES


def q5_0_nbytes(rows: int, K: int) -> int:
    return rows * (K // QK) * Q5_0_BYTES


def pack_q5_0(ql: np.ndarray, qh: np.ndarray, d: np.ndarray) -> np.ndarray:
    """Split Q5_0 (ql [rows, nb, 16], qh [rows, nb, 4], d [rows, nb] as
    float16) -> GGUF blocks [rows, nb, 22]."""
    ql = np.ascontiguousarray(ql, dtype=np.uint8)
    rows, nb, _ = ql.shape
    out = np.empty((rows, nb, Q5_0_BYTES), np.uint8)
    out[..., 0:2] = np.ascontiguousarray(d, dtype=np.float16).reshape(rows, nb, 1).view(np.uint8)
    out[..., 2:6] = qh
    out[..., 6:] = ql
    return out


def split_q5_0(blocks: np.ndarray) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """GGUF Q5_0 blocks -> (ql [rows, nb, 16], qh [rows, nb, 4], scales
    [rows, nb] float32), the layout asm_matmul_q5 reads."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    scales = np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0].astype(np.float32)
    return np.ascontiguousarray(b[..., 6:]), np.ascontiguousarray(b[..., 2:6]), np.ascontiguousarray(scales)


def dequantize_q5_0(blocks: np.ndarray) -> np.ndarray:
    """Exact fp32 weights [rows, K]."""
    ql, qh, scales = split_q5_0(blocks)
    nib = np.concatenate([ql & 0x0F, ql >> 4], axis=-1).astype(np.int32)
    word = qh.astype(np.uint32)
    word = word[..., 0] | (word[..., 1] << 8) | (word[..., 2] << 16) | (word[..., 3] << 24)
    bits = ((word[..., None] >> np.arange(32, dtype=np.uint32)) & 1).astype(np.int32)
    w = (nib | (bits << 4)).astype(np.float32) - np.float32(16.0)
    return (w * scales[..., None]).reshape(ql.shape[0], -1).astype(np.float32)
