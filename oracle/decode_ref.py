"""CPU single-token decode, composed from the oracle's decode ops (TEST INFRASTRUCTURE ONLY).

Restates ``AsmEngineForward.forward_token`` (src/runtime/generate.py:261-326)
step for step, with the two storage choices of the GPU engine made explicit:
the KV cache holds fp16 values (k after RoPE and v, rounded to nearest even
when written), head-major [n_kv_heads][max_ctx][head_dim]; and heads may be
grouped (n_heads / n_kv_heads query heads per kv head; the reference has
n_heads == n_kv_heads).  ``kv_dtype="f32"`` keeps the cache in fp32 as the
reference does (generate.py:252-253), and ``attention="f64"`` evaluates the
per-head QK^T/sqrt(hd) -> softmax -> PV in float64 over either cache, so the
two storage choices can be compared with nothing else changed.  Every arithmetic step calls an oracle function that
tests/test_oracle.py pins on its own:

  * matvecs: oracle_matmul_q4_0_gguf (matmul_q4_avx2.asm:110-178 over GGUF
    blocks, scale widened from fp16 as generate.py:91-106 does);
  * rmsnorm (rmsnorm_avx2.asm:63-151), rope (rope_avx2.asm:52-146),
    silu_hadamard (swiglu_avx2.asm:45-81);
  * attention over the fp16 cache: oracle_attention_decode_f16, the
    reference's per-head QK^T/sqrt(hd) -> softmax -> PV (generate.py:291-296).
"""

from __future__ import annotations

import numpy as np

from . import native as o


class DecodeRef:
    """Host copy of a decode model: GGUF Q4_0 blocks ([rows][K/32][18] uint8;
    the embedding and lm-head may be Q8_0, [rows][K/32][34]),
    fp32 norm weights, fp16 caches given head-major [n_kv][max_ctx][hd] as
    uint16 bits (stored position-major in k_caches / v_caches)."""

    def __init__(self, *, dim, n_heads, n_kv_heads, hidden_dim, vocab, eps, theta, embed, final_norm, output,
                 layers, k_caches, v_caches, nt: int = 1, kv_dtype: str = "f16", attention: str = "oracle"):
        self.dim, self.n_heads, self.n_kv_heads = dim, n_heads, n_kv_heads
        self.hidden_dim, self.vocab, self.eps, self.theta = hidden_dim, vocab, eps, theta
        self.hd = dim // n_heads
        self.embed, self.final_norm, self.output = embed, final_norm, output
        self.layers = layers            # dicts: attn_norm wq wk wv wo ffn_norm w_gate w_up w_down
        if kv_dtype not in ("f16", "f32") or attention not in ("oracle", "f64"):
            raise ValueError(f"kv_dtype {kv_dtype!r} / attention {attention!r}")
        if kv_dtype == "f32" and attention == "oracle":
            raise ValueError("the oracle's decode attention reads an fp16 cache; use attention='f64'")
        self.kv_dtype, self.attention = kv_dtype, attention
        # kept position-major [max_ctx][n_kv][hd], the oracle kernel's layout, so a
        # step slices the cache without copying it (fp16 as uint16 bits, or fp32)
        store = np.uint16 if kv_dtype == "f16" else np.float32
        self.k_caches = [np.ascontiguousarray(np.asarray(k, store).transpose(1, 0, 2)) for k in k_caches]
        self.v_caches = [np.ascontiguousarray(np.asarray(v, store).transpose(1, 0, 2)) for v in v_caches]
        self.nt = nt

    def _mv(self, blocks, x):
        if blocks.shape[-1] == 34:  # Q8_0 blocks (an lm-head; generate.py:177-180)
            return o.matmul_q8_0_gguf(blocks, x, self.nt)
        return o.matmul_q4_0_gguf(blocks, x, self.nt)

    def _rope_heads(self, v, n):
        """RoPE on n heads of v (rope_avx2.asm rotates one q head and one k head per call)."""
        out = v.reshape(n, self.hd).copy()
        for h in range(n):
            out[h], _ = o.rope(out[h], out[h], self.hd, self._pos, self.theta)
        return out.reshape(-1)

    def _store(self, vals: np.ndarray) -> np.ndarray:
        return vals.astype(np.float16).view(np.uint16) if self.kv_dtype == "f16" else vals.astype(np.float32)

    def _attend(self, q: np.ndarray, kc: np.ndarray, vc: np.ndarray, n_pos: int) -> np.ndarray:
        """Per query head: softmax(q . K^T / sqrt(hd)) . V over positions 0..n_pos-1
        (generate.py:291-296); query head h reads kv head h // (n_heads / n_kv_heads)."""
        if self.attention == "oracle":
            return o.attention_decode_f16(q, kc, vc, n_pos, self.n_kv_heads, self.nt)
        def wide(c):
            return (c.view(np.float16) if self.kv_dtype == "f16" else c).astype(np.float64)
        K, V = wide(kc[:n_pos]), wide(vc[:n_pos])               # [pos][n_kv][hd]
        group = self.n_heads // self.n_kv_heads
        out = np.empty((self.n_heads, self.hd), np.float64)
        for h in range(self.n_heads):
            s = K[:, h // group] @ q[h].astype(np.float64) / np.sqrt(self.hd)
            p = np.exp(s - s.max())
            out[h] = (p / p.sum()) @ V[:, h // group]
        return out.astype(np.float32)

    def forward_token(self, token_id: int, pos: int) -> np.ndarray:
        """Logits of token_id at pos; writes cache row pos (generate.py:261-326)."""
        self._pos = pos
        hd, nh, nkv = self.hd, self.n_heads, self.n_kv_heads
        row = self.embed[token_id:token_id + 1]
        x = (o.dequantize_q8_0(row) if row.shape[-1] == 34 else o.dequantize_q4_0(row))[0].copy()  # :262
        for li, ly in enumerate(self.layers):
            xn = o.rmsnorm(x, ly["attn_norm"], self.eps)                          # :268-272
            q = self._mv(ly["wq"], xn)                                            # :278-280
            k = self._mv(ly["wk"], xn)
            v = self._mv(ly["wv"], xn)
            q = self._rope_heads(q, nh)                                           # :282-285
            k = self._rope_heads(k, nkv)
            kc, vc = self.k_caches[li], self.v_caches[li]                         # :289-290
            kc[pos] = self._store(k.reshape(nkv, hd))
            vc[pos] = self._store(v.reshape(nkv, hd))
            attn = self._attend(q.reshape(nh, hd), kc, vc, pos + 1)               # :291-296
            x = x + self._mv(ly["wo"], attn.reshape(-1))                          # :298-300
            xn = o.rmsnorm(x, ly["ffn_norm"], self.eps)                           # :302-306
            gate = self._mv(ly["w_gate"], xn)                                     # :308-311
            up = self._mv(ly["w_up"], xn)
            g = o.silu_hadamard(gate, up)                                         # :313
            x = x + self._mv(ly["w_down"], g)                                     # :315-317
        xn = o.rmsnorm(x, self.final_norm, self.eps)                              # :319-323
        return self._mv(self.output, xn)                                          # :325
