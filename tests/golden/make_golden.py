"""Writes the golden fixtures under tests/golden/.

reference_gen_seed42.npz: the reference's golden inputs, drawn with
np.random.RandomState(42) in the order of tools/reference_gen.py:31-112
(restated in oracle/golden.py), with the expected outputs the reference's
runner computes from tests/reference/ops.py (restated in oracle/ops_ref.py).

quant_known_answers.npz: hand-constructed Q4_0 / Q8_0 blocks whose bytes
follow from the quantization rule by hand; the expected bytes below are
literals, not recomputed.

stories15m_m2_tokens.json: the prompt and greedy tokens of the reference's
end-to-end stories15M run, read from its log (tests/results/m2_generation.log).

Run: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.golden import generate_reference_data  # noqa: E402


def _pack4(d_bits: int, q: list[int]) -> np.ndarray:
    q = np.asarray(q, np.uint8)
    out = np.empty(18, np.uint8)
    out[0], out[1] = d_bits & 0xFF, d_bits >> 8
    out[2:] = q[:16] | (q[16:] << 4)
    return out


def _pack8(d_bits: int, q: list[int]) -> np.ndarray:
    out = np.empty(34, np.uint8)
    out[0], out[1] = d_bits & 0xFF, d_bits >> 8
    out[2:] = np.asarray(q, np.int8).view(np.uint8)
    return out


def quant_known_answers() -> dict[str, np.ndarray]:
    # Q4_0, rule: d = m/-8 (m = first element of largest magnitude), id = 1/d,
    # q = min(15, trunc(w*id + 8.5)).
    # Block 0: w_j = (j - 16)/4.  m = w_0 = -4, d = 0.5 (fp16 0x3800), id = 2,
    # w*id + 8.5 = j/2 + 0.5, so q_j = floor(j/2 + 0.5), clamped to 15 at j = 31.
    w0 = (np.arange(32, dtype=np.float32) - 16) / np.float32(4)
    q0 = [0, 1, 1, 2, 2, 3, 3, 4, 4, 5, 5, 6, 6, 7, 7, 8, 8, 9, 9, 10, 10, 11, 11, 12, 12, 13, 13, 14, 14, 15, 15, 15]
    # Block 1: zeros except w_5 = 3: d = -0.375 (0xB600), id = -8/3,
    # q_5 = trunc(-8 + 8.5) = 0, all others trunc(8.5) = 8.
    w1 = np.zeros(32, np.float32)
    w1[5] = 3.0
    q1 = [8] * 32
    q1[5] = 0
    # Block 2: all zeros: m = 0, d = 0/-8 = -0.0 (0x8000), id = 0, q = 8.
    w2 = np.zeros(32, np.float32)
    q2 = [8] * 32
    q4_w = np.concatenate([w0, w1, w2]).reshape(1, 96)
    q4_blocks = np.stack([_pack4(0x3800, q0), _pack4(0xB600, q1), _pack4(0x8000, q2)]).reshape(1, 3, 18)

    # Q8_0, rule: d = amax/127, inv = 127/amax, q = rint(w*inv) (ties to even).
    # Block 0: w_j = j - 16, w_31 = 127: amax = 127, d = 1 (0x3C00), inv = 1, q = w.
    w8 = np.arange(32, dtype=np.float32) - 16
    w8[31] = 127.0
    q8 = list(range(-16, 15)) + [127]
    # Block 1: w_0 = 127 and exact ties: rint gives the even neighbour.
    w9 = np.zeros(32, np.float32)
    w9[:8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]
    q9 = [127, 0, 2, 2, 0, -2, -2, 126] + [0] * 24
    # Block 2: all zeros: d = 0 (0x0000), inv = 0, q = 0.
    w10 = np.zeros(32, np.float32)
    q10 = [0] * 32
    # Block 3: amax = 254: d = 2 (0x4000), inv = 0.5, q = rint(w/2).
    w11 = np.zeros(32, np.float32)
    w11[:6] = [254.0, 3.0, 5.0, -3.0, 1.0, 7.0]
    q11 = [127, 2, 2, -2, 0, 4] + [0] * 26
    q8_w = np.concatenate([w8, w9, w10, w11]).reshape(1, 128)
    q8_blocks = np.stack([_pack8(0x3C00, q8), _pack8(0x3C00, q9), _pack8(0x0000, q10),
                          _pack8(0x4000, q11)]).reshape(1, 4, 34)
    return {"q4_w": q4_w, "q4_blocks": q4_blocks, "q8_w": q8_w, "q8_blocks": q8_blocks}


M2_LOG = Path("/root/reference/tests/results/m2_generation.log")


def m2_tokens(log_text: str) -> dict:
    """The prompt and the 30 greedy token ids of the reference's end-to-end
    run on stories15M (m2_generation.log:5, 10-39), read from the log's text."""
    import re

    prompt = [int(t) for t in re.search(r"Prompt Tokens: \[([\d, ]+)\]", log_text).group(1).split(",")]
    rows = re.findall(r"^(\d+)\s+(\d+)\s+'.*?'\s+(\d+)\s+(\w+)", log_text, re.M)
    assert [int(r[0]) for r in rows] == list(range(1, len(rows) + 1))
    assert all(r[1] == r[2] and r[3] == "YES" for r in rows)  # the reference's own check passed
    return {"source": "tests/results/m2_generation.log (asmllm), stories15M-q4_0.gguf greedy decode",
            "prompt": prompt, "generated": [int(r[1]) for r in rows]}


def main() -> None:
    import json

    data = generate_reference_data(42)
    np.savez_compressed(HERE / "reference_gen_seed42.npz", **data)
    np.savez_compressed(HERE / "quant_known_answers.npz", **quant_known_answers())
    if M2_LOG.exists():  # the reference tree is only present where the fixtures are made
        (HERE / "stories15m_m2_tokens.json").write_text(json.dumps(m2_tokens(M2_LOG.read_text()), indent=1) + "\n")
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")) + sorted(p.name for p in HERE.glob("*.json")))


if __name__ == "__main__":
    main()
