"""The reference's golden inputs (test infrastructure only).

Restates tools/reference_gen.py:31-112: one np.random.RandomState(seed)
stream drawn in the reference's order, so the inputs are the ones the
reference's correctness runner feeds its kernels.  Expected outputs follow
tests/reference/ops.py (restated in oracle/ops_ref.py), as the reference
computes them at test time (test_runner.py:493).
"""

from __future__ import annotations

import numpy as np

from . import ops_ref

# tests/correctness/test_runner.py:33-36
TOLERANCE_Q4 = 0.5
TOLERANCE_Q8 = 1e-2
TOLERANCE_Q5 = 1e-2
TOLERANCE_FP32 = 1e-5


def generate_reference_data(seed: int = 42) -> dict[str, np.ndarray]:
    rng = np.random.RandomState(seed)
    d: dict[str, np.ndarray] = {}

    # reference_gen.py:39-49 -- Q4, M=4 K=64
    q4 = rng.randint(0, 256, size=(4, 2, 16), dtype=np.uint8)
    q4s = rng.uniform(0.1, 1.5, size=(4, 2)).astype(np.float32)
    x = rng.randn(64).astype(np.float32)
    d["q4_matmul_qweights"], d["q4_matmul_scales"], d["q4_matmul_x"] = q4, q4s, x
    d["q4_matmul_expected"] = ops_ref.q4_matmul(q4, q4s, x)

    # :51-59 -- Q8, same x
    q8 = rng.randint(-128, 128, size=(4, 2, 32), dtype=np.int8)
    q8s = rng.uniform(0.1, 1.5, size=(4, 2)).astype(np.float32)
    d["q8_matmul_qweights"], d["q8_matmul_scales"], d["q8_matmul_x"] = q8, q8s, x
    d["q8_matmul_expected"] = ops_ref.q8_matmul(q8, q8s, x)

    # :61-71 -- Q5, same x
    q5l = rng.randint(0, 256, size=(4, 2, 16), dtype=np.uint8)
    q5h = rng.randint(0, 256, size=(4, 2, 4), dtype=np.uint8)
    q5s = rng.uniform(0.1, 1.5, size=(4, 2)).astype(np.float32)
    d["q5_matmul_ql"], d["q5_matmul_qh"], d["q5_matmul_scales"], d["q5_matmul_x"] = q5l, q5h, q5s, x
    d["q5_matmul_expected"] = ops_ref.q5_matmul(q5l, q5h, q5s, x)

    # :73-81 -- RMSNorm, dim 64, eps 1e-5
    xn = rng.randn(64).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, size=(64,)).astype(np.float32)
    d["rmsnorm_x"], d["rmsnorm_weight"] = xn, wn
    d["rmsnorm_eps"] = np.array(1e-5, dtype=np.float32)
    d["rmsnorm_expected"] = ops_ref.rmsnorm(xn, wn, eps=1e-5)

    # :83-92 -- RoPE, head_dim 32, pos 5
    qr = rng.randn(32).astype(np.float32)
    kr = rng.randn(32).astype(np.float32)
    d["rope_q"], d["rope_k"] = qr, kr
    d["rope_pos"] = np.array(5, dtype=np.int32)
    d["rope_q_expected"], d["rope_k_expected"] = ops_ref.rope(qr, kr, head_dim=32, pos=5, theta=10000.0)

    # :94-99 -- softmax, dim 64
    xs = rng.randn(64).astype(np.float32) * 2.0
    d["softmax_x"] = xs
    d["softmax_expected"] = ops_ref.softmax(xs)

    # :101-110 -- attention, seq 8, head_dim 16
    qa = rng.randn(8, 16).astype(np.float32)
    ka = rng.randn(8, 16).astype(np.float32)
    va = rng.randn(8, 16).astype(np.float32)
    d["attention_q"], d["attention_k"], d["attention_v"] = qa, ka, va
    d["attention_expected"] = ops_ref.attention(qa, ka, va)
    return d
