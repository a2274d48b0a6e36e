"""Single-token decode of a Llama-shaped model with every tensor resident in HBM.

GPU counterpart of ``AsmEngineForward`` (src/runtime/generate.py:208-326).
The reference sequences one token as embed row -> per layer [RMSNorm, q/k/v
matvecs, RoPE per head, KV-cache write, per-head QK^T -> softmax -> PV, o
matvec + residual, RMSNorm, gate/up matvecs, SiLU*up, down matvec + residual]
-> final RMSNorm -> lm-head (generate.py:261-326), with numpy arrays between
native calls.  Here the same sequence is a fixed list of launches on one
stream, so it can be captured once into a HIP graph and replayed per token:

  * q, k and v weights are stacked into one [q; k; v] Q4_0 matrix (rows are
    independent, so y is the same as three separate matvecs), and gate/up
    into one matrix whose rows interleave the two in groups of 8, so that one
    matvec launch also forms silu(gate) * up as it writes its outputs
    (asmhip_matmul_swiglu); the RMSNorms are fused into the read of x by the
    matvec that follows them, and both residual adds into the o and down
    matvecs (accumulate);
  * the token id and the position live in device ints: the embedding kernel
    reads the token, RoPE / the KV write / attention read the position, and
    the argmax kernel writes the next token, records it in a device history
    indexed by position and advances the position, so a replayed graph of one
    or many token steps walks the sequence without host involvement and keeps
    every token it chose;
  * RoPE and the KV-cache write are fused into the attention launch
    (asmhip_attention_decode_partials_rope_table), its cos/sin read from a
    table of every position's angles formed once at set-up
    (asmhip_rope_table); the attention leaves its splits' (384 or 512
    positions) softmax states in a workspace, and the o matvec merges them as it reads
    its x (asmhip_matmul_attn_output), so attention + o take two launches;
  * the KV cache is fp16, head-major [n_kv_heads][max_ctx][head_dim] per layer
    (the reference keeps fp32 [128][heads][head_dim], generate.py:252-253);
  * head_dim 48 (the reference's stories15M demo model, dim 288), 64 or 128;
    where dim is not a multiple of 64 the RMSNorm runs as its own launch
    before the matvec instead of inside it.

All weights are Q4_0 GGUF blocks, including the token embedding and the
lm-head (generate.py:182-184 loads both through get_tensor).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import native
from .device import DeviceBuffer, Graph, Stream
from .gguf import q4_0_nbytes, q8_0_nbytes
from .native import check


@dataclass(frozen=True)
class LlamaShape:
    """Model hyper-parameters (generate.py:123-141 reads the same fields from GGUF metadata)."""

    dim: int = 4096
    n_layers: int = 32
    n_heads: int = 32
    n_kv_heads: int = 32
    hidden_dim: int = 11008
    vocab: int = 32000
    eps: float = 1e-6
    theta: float = 10000.0

    @property
    def head_dim(self) -> int:
        return self.dim // self.n_heads

    @property
    def kv_dim(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def qkv_rows(self) -> int:
        return self.dim + 2 * self.kv_dim

    def layer_weight_bytes(self) -> int:
        d, h = self.dim, self.hidden_dim
        return (q4_0_nbytes(self.qkv_rows, d) + q4_0_nbytes(d, d) + q4_0_nbytes(2 * h, d) +
                q4_0_nbytes(d, h))

    def weight_bytes(self) -> int:
        """Q4_0 bytes one token step reads: every layer plus the lm-head
        (the embedding table contributes one row)."""
        return self.n_layers * self.layer_weight_bytes() + q4_0_nbytes(self.vocab, self.dim)

    def kv_bytes_per_position(self) -> int:
        return self.n_layers * 2 * self.kv_dim * 2


LLAMA_7B = LlamaShape()
# The reference's end-to-end demo model (generate.py:122-164: stories15M, 6 layers,
# dim 288, 6 heads of 48, FFN 768, vocab 32000, eps 1e-5).
STORIES_15M = LlamaShape(dim=288, n_layers=6, n_heads=6, n_kv_heads=6, hidden_dim=768, vocab=32000, eps=1e-5)


def shape_from_gguf(g) -> LlamaShape:
    """LlamaShape from a GGUFFile's llama.* metadata (the fields generate.py:123-141
    fixes for its model); the vocabulary size from the token embedding."""
    md = g.metadata
    arch = md.get("general.architecture", "llama")

    def get(key, default=None):
        v = md.get(f"{arch}.{key}", default)
        if v is None:
            raise ValueError(f"{g.path}: metadata {arch}.{key} missing")
        return v

    n_heads = int(get("attention.head_count"))
    emb = g.tensors.get("token_embd.weight")
    if emb is None:
        raise ValueError(f"{g.path}: no token_embd.weight")
    return LlamaShape(dim=int(get("embedding_length")), n_layers=int(get("block_count")), n_heads=n_heads,
                      n_kv_heads=int(get("attention.head_count_kv", n_heads)),
                      hidden_dim=int(get("feed_forward_length")), vocab=int(emb.dims[1]),
                      eps=float(get("attention.layer_norm_rms_epsilon", 1e-5)),
                      theta=float(get("rope.freq_base", 10000.0)))


def interleave_gate_up(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    """[gate; up] block rows ([H][nb][bytes] each, H % 8 == 0) in the order
    asmhip_matmul_swiglu reads them: 8 gate rows, then the same 8 up rows."""
    if gate.shape != up.shape or gate.shape[0] % 8:
        raise ValueError(f"gate {gate.shape} / up {up.shape}: need equal shapes and a multiple of 8 rows")
    H = gate.shape[0]
    g = gate.reshape(H // 8, 1, 8, *gate.shape[1:])
    u = up.reshape(H // 8, 1, 8, *up.shape[1:])
    return np.concatenate([g, u], axis=1).reshape(2 * H, *gate.shape[1:])


def split_gate_up(gu: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Inverse of interleave_gate_up."""
    H = gu.shape[0] // 2
    v = gu.reshape(H // 8, 2, 8, *gu.shape[1:])
    return v[:, 0].reshape(H, *gu.shape[1:]), v[:, 1].reshape(H, *gu.shape[1:])


class _Layer:
    def __init__(self, s: LlamaShape, max_ctx: int):
        d, h = s.dim, s.hidden_dim
        self.attn_norm = DeviceBuffer(4 * d)
        self.ffn_norm = DeviceBuffer(4 * d)
        self.wqkv = DeviceBuffer(q4_0_nbytes(s.qkv_rows, d))
        self.wo = DeviceBuffer(q4_0_nbytes(d, d))
        self.wgu = DeviceBuffer(q4_0_nbytes(2 * h, d))
        self.wdown = DeviceBuffer(q4_0_nbytes(d, h))
        self.k_cache = DeviceBuffer(2 * s.n_kv_heads * max_ctx * s.head_dim)
        self.v_cache = DeviceBuffer(2 * s.n_kv_heads * max_ctx * s.head_dim)


class DecodeEngine:
    """Greedy single-token decode on one GPU (AsmEngineForward, generate.py:208-326).

    ``init_random`` fills the model the way the synthetic benchmark model is
    specified: linear weights N(0, stddev^2) quantized to Q4_0 on the GPU, norm
    weights 1, KV cache N(0, 1) in fp16.  ``load_*`` methods take host GGUF
    blocks instead.
    """

    def __init__(self, shape: LlamaShape = LLAMA_7B, max_ctx: int = 2176, stream: Stream | None = None,
                 embed_type: int = native.Q4_0, output_type: int = native.Q4_0):
        s = shape
        if embed_type not in (native.Q4_0, native.Q8_0) or output_type not in (native.Q4_0, native.Q8_0):
            raise ValueError("the token embedding and the lm-head must be Q4_0 or Q8_0")
        if s.dim % s.n_heads or s.n_heads % s.n_kv_heads:
            raise ValueError("dim must split into heads, and heads into kv groups")
        if s.head_dim not in (48, 64, 128):
            raise ValueError("head_dim must be 48, 64 or 128")
        if s.dim % 32 or s.hidden_dim % 32:
            raise ValueError("dim and hidden_dim must be multiples of 32 (Q4_0 blocks)")
        self.shape = s
        self.max_ctx = int(max_ctx)
        self.stream = stream or Stream()
        self.lib = native.lib()
        self.layers = [_Layer(s, self.max_ctx) for _ in range(s.n_layers)]
        self.embed_type, self.output_type = embed_type, output_type
        nbytes = {native.Q4_0: q4_0_nbytes, native.Q8_0: q8_0_nbytes}
        self.embed = DeviceBuffer(nbytes[embed_type](s.vocab, s.dim))
        self.final_norm = DeviceBuffer(4 * s.dim)
        self.output = DeviceBuffer(nbytes[output_type](s.vocab, s.dim))
        # activations
        self.x = DeviceBuffer(4 * s.dim)
        self.qkv = DeviceBuffer(4 * s.qkv_rows)
        self.attn = DeviceBuffer(4 * s.dim)
        self.gu = DeviceBuffer(4 * 2 * s.hidden_dim)  # work buffer of asmhip_matmul_swiglu
        self.ffn = DeviceBuffer(4 * s.hidden_dim)     # silu(gate) * up
        self.logits = DeviceBuffer(4 * s.vocab)
        # The matvecs fuse RMSNorm into their read of x when K % 64 == 0;
        # otherwise (stories15M: dim 288) it runs as its own launch first.
        self.fuse_norm = s.dim % 64 == 0
        self.xn = None if self.fuse_norm else DeviceBuffer(4 * s.dim)
        ws = self.lib.asmhip_attention_decode_workspace(s.n_heads, s.head_dim, self.max_ctx)
        self.workspace = DeviceBuffer(4 * max(int(ws), 1))
        # cos/sin of every RoPE angle, formed once instead of in every attention launch
        self.rope_table = DeviceBuffer(4 * self.max_ctx * s.head_dim)
        check(self.lib.asmhip_rope_table(self.rope_table.ptr, s.head_dim, self.max_ctx, ctypes.c_float(s.theta),
                                         self.stream.handle), "rope table")
        self.token = DeviceBuffer(4)
        self.pos = DeviceBuffer(4)
        # history[p] = the greedy token chosen at position p (written by the argmax launch)
        self.history = DeviceBuffer(4 * self.max_ctx)
        self.vocab: list[str] = []
        self._graph: Graph | None = None
        self._multi: dict[int, Graph] = {}

    # ---- model data ---------------------------------------------------------------

    def init_random(self, seed: int = 42, stddev: float = 0.02, kv_stddev: float = 1.0) -> None:
        s, L, st = self.shape, self.lib, self.stream.handle
        d, h = s.dim, s.hidden_dim

        def blocks(buf, rows, K, tag, qtype=native.Q4_0):
            check(L.asmhip_random_blocks(qtype, buf.ptr, rows, K, seed * 1000003 + tag, stddev, st),
                  "random weights")

        for i, ly in enumerate(self.layers):
            base = 16 * (i + 1)
            blocks(ly.wqkv, s.qkv_rows, d, base + 0)
            blocks(ly.wo, d, d, base + 1)
            blocks(ly.wgu, 2 * h, d, base + 2)
            blocks(ly.wdown, d, h, base + 3)
            for buf in (ly.attn_norm, ly.ffn_norm):
                check(L.asmhip_fill_f32(buf.ptr, d, 1.0, st), "norm weights")
            n_kv = s.n_kv_heads * self.max_ctx * s.head_dim
            check(L.asmhip_random_f16(ly.k_cache.ptr, n_kv, seed * 1000003 + base + 4, kv_stddev, st), "kv")
            check(L.asmhip_random_f16(ly.v_cache.ptr, n_kv, seed * 1000003 + base + 5, kv_stddev, st), "kv")
        blocks(self.embed, s.vocab, d, 1, self.embed_type)
        blocks(self.output, s.vocab, d, 2, self.output_type)
        check(L.asmhip_fill_f32(self.final_norm.ptr, d, 1.0, st), "norm weights")
        self.stream.synchronize()

    def load_layer(self, i: int, *, attn_norm, wq, wk, wv, wo, ffn_norm, w_gate, w_up, w_down) -> None:
        """Host GGUF Q4_0 blocks ([rows][K/32][18] uint8) and fp32 norm weights
        of layer i (the tensors generate.py:186-205 collects per layer)."""
        ly = self.layers[i]
        ly.attn_norm.upload(np.asarray(attn_norm, np.float32))
        ly.ffn_norm.upload(np.asarray(ffn_norm, np.float32))
        ly.wqkv.upload(np.concatenate([wq, wk, wv], axis=0))
        ly.wo.upload(wo)
        ly.wgu.upload(interleave_gate_up(np.asarray(w_gate), np.asarray(w_up)))
        ly.wdown.upload(w_down)

    def gate_up_blocks(self, i: int) -> tuple[np.ndarray, np.ndarray]:
        """The gate and up matrices of layer i as host GGUF blocks [hidden_dim][dim/32][18]."""
        s = self.shape
        gu = self.layers[i].wgu.download(np.uint8, (2 * s.hidden_dim, s.dim // 32, 18))
        return split_gate_up(gu)

    def load_globals(self, *, embed, final_norm, output) -> None:
        """Token embedding and lm-head as host GGUF blocks of the engine's
        embed_type / output_type, final norm weights fp32."""
        for name, arr, buf in (("embedding", embed, self.embed), ("lm-head", output, self.output)):
            if np.asarray(arr).nbytes != buf.nbytes:
                raise ValueError(f"{name}: {np.asarray(arr).nbytes} bytes, the engine holds {buf.nbytes}")
        self.embed.upload(embed)
        self.final_norm.upload(np.asarray(final_norm, np.float32))
        self.output.upload(output)

    @classmethod
    def from_gguf(cls, path, max_ctx: int = 2048, stream: Stream | None = None) -> "DecodeEngine":
        """Engine for a Llama GGUF model, every tensor uploaded once to HBM
        (the tensor names of generate.py:182-205; the shape from the llama.*
        metadata).  Layer weights must be Q4_0; the token embedding and the
        lm-head Q4_0 or Q8_0 (generate.py:169-180 reads both types); norm
        weights F32.  A model without output.weight uses the token embedding
        as its lm-head."""
        from .gguf_file import F32, Q4_0, Q8_0, GGUFFile

        g = GGUFFile(path)
        try:
            shape = shape_from_gguf(g)
            out_name = "output.weight" if "output.weight" in g.tensors else "token_embd.weight"
            types = {}
            for name in ("token_embd.weight", out_name):
                t = g.tensors.get(name)
                if t is None:
                    raise KeyError(f"{path}: no tensor {name!r}")
                if t.type not in (Q4_0, Q8_0):
                    raise ValueError(f"{name}: tensor type {t.type}; the engine takes Q4_0 ({Q4_0}) or Q8_0 ({Q8_0})")
                types[name] = native.Q4_0 if t.type == Q4_0 else native.Q8_0
            eng = cls(shape, max_ctx=max_ctx, stream=stream, embed_type=types["token_embd.weight"],
                      output_type=types[out_name])

            def q4(name):
                t = g.tensors.get(name)
                if t is None:
                    raise KeyError(f"{path}: no tensor {name!r}")
                if t.type != Q4_0:
                    raise ValueError(f"{name}: tensor type {t.type}; the engine takes Q4_0 ({Q4_0}) weights")
                return g.tensor(name)

            def f32(name):
                t = g.tensors.get(name)
                if t is None or t.type != F32:
                    raise ValueError(f"{name}: missing or not F32")
                return g.tensor(name)

            for i in range(shape.n_layers):
                b = f"blk.{i}."
                eng.load_layer(i, attn_norm=f32(b + "attn_norm.weight"), wq=q4(b + "attn_q.weight"),
                               wk=q4(b + "attn_k.weight"), wv=q4(b + "attn_v.weight"), wo=q4(b + "attn_output.weight"),
                               ffn_norm=f32(b + "ffn_norm.weight"), w_gate=q4(b + "ffn_gate.weight"),
                               w_up=q4(b + "ffn_up.weight"), w_down=q4(b + "ffn_down.weight"))
            eng.load_globals(embed=g.tensor("token_embd.weight"), final_norm=f32("output_norm.weight"),
                             output=g.tensor(out_name))
            eng.vocab = g.vocab()
        finally:
            g.close()
        return eng

    def load_kv(self, i: int, k_cache: np.ndarray, v_cache: np.ndarray) -> None:
        """fp16 caches of layer i as [n_kv_heads][max_ctx][head_dim] (uint16 bits or float16)."""
        s = self.shape
        want = (s.n_kv_heads, self.max_ctx, s.head_dim)
        for buf, arr in ((self.layers[i].k_cache, k_cache), (self.layers[i].v_cache, v_cache)):
            a = np.ascontiguousarray(arr).view(np.uint16)
            if a.shape != want:
                raise ValueError(f"cache shape {a.shape} != {want}")
            buf.upload(a)

    # ---- one token ------------------------------------------------------------------

    def enqueue_step(self) -> None:
        """Launches one token step on the engine's stream: logits for the token
        in ``token`` at position ``pos``, then token <- argmax, pos += 1."""
        for _kind, _layer, launch in self.step_launches():
            launch()

    def step_launches(self):
        """The launches of one token step in order, as (kind, layer or None,
        launch): kinds embed, qkv, attention, o, gate_up, down, lm_head, argmax."""
        s, L, st = self.shape, self.lib, self.stream.handle
        d, h, hd = s.dim, s.hidden_dim, s.head_dim
        eps = ctypes.c_float(s.eps)
        Q4, RMS, NONE = native.Q4_0, native.PRE_RMSNORM, native.PRE_NONE

        def mv(w, x, y, M, K, pre, arg, acc, what, qtype=Q4):
            check(L.asmhip_matmul_fused(qtype, w.ptr, x, y, M, K, pre, arg, eps, acc, st), what)

        def norm_in(norm):  # (x, pre-op, argument) that give the matvec rmsnorm(x; norm)
            if self.fuse_norm:
                return self.x.ptr, RMS, norm.ptr
            check(L.asmhip_rmsnorm(self.x.ptr, norm.ptr, self.xn.ptr, d, eps, st), "rmsnorm")
            return self.xn.ptr, NONE, None

        def normed(norm, M, w, y, what, qtype=Q4):  # y = W rmsnorm(x; norm)
            xin, pre, arg = norm_in(norm)
            mv(w, xin, y, M, d, pre, arg, 0, what, qtype)

        def attention(ly):
            check(L.asmhip_attention_decode_partials_rope_table(self.qkv.ptr, ly.k_cache.ptr, ly.v_cache.ptr,
                                                                self.workspace.ptr, s.n_heads, s.n_kv_heads, hd,
                                                                self.pos.ptr, self.max_ctx, self.rope_table.ptr, st),
                  "rope + attention")

        def gate_up(ly):
            xin, pre, arg = norm_in(ly.ffn_norm)
            check(L.asmhip_matmul_swiglu(Q4, ly.wgu.ptr, xin, self.ffn.ptr, h, d, pre, arg, eps, self.gu.ptr, st),
                  "gate/up matvec + swiglu")

        embed = L.asmhip_embed_q8_0 if self.embed_type == native.Q8_0 else L.asmhip_embed_q4_0
        yield "embed", None, lambda: check(embed(self.embed.ptr, self.token.ptr, self.x.ptr, s.vocab, d, st),
                                           "embed")
        for i, ly in enumerate(self.layers):
            yield "qkv", i, lambda ly=ly: normed(ly.attn_norm, s.qkv_rows, ly.wqkv, self.qkv.ptr, "qkv matvec")
            yield "attention", i, lambda ly=ly: attention(ly)
            yield "o", i, lambda ly=ly: check(L.asmhip_matmul_attn_output(Q4, ly.wo.ptr, self.workspace.ptr,
                                                                           self.attn.ptr, self.x.ptr, d, s.n_heads,
                                                                           hd, self.max_ctx, 1, st),
                                               "merge + o matvec")
            yield "gate_up", i, lambda ly=ly: gate_up(ly)
            yield "down", i, lambda ly=ly: mv(ly.wdown, self.ffn.ptr, self.x.ptr, d, h, NONE, None, 1, "down matvec")
        yield "lm_head", None, lambda: normed(self.final_norm, s.vocab, self.output, self.logits.ptr,
                                              "lm-head matvec", self.output_type)
        yield "argmax", None, lambda: check(L.asmhip_argmax_history(self.logits.ptr, s.vocab, self.token.ptr,
                                                                    self.pos.ptr, self.history.ptr, self.max_ctx,
                                                                    st), "argmax")

    def set_position(self, token_id: int, pos: int) -> None:
        if not 0 <= pos < self.max_ctx:
            raise ValueError(f"position {pos} outside the cache (max_ctx {self.max_ctx})")
        if not 0 <= token_id < self.shape.vocab:
            raise ValueError(f"token {token_id} outside the vocabulary")
        self.token.upload(np.array([token_id], np.int32))
        self.pos.upload(np.array([pos], np.int32))

    def forward_token(self, token_id: int, pos: int) -> np.ndarray:
        """Logits of ``token_id`` at ``pos`` (generate.py:261-326); the KV cache
        row ``pos`` of every layer is written as a side effect."""
        self.set_position(token_id, pos)
        self.enqueue_step()
        self.stream.synchronize()
        return self.logits.download(np.float32, (self.shape.vocab,))

    def capture(self) -> Graph:
        """One token step as a HIP graph (captured once, replayed per token)."""
        if self._graph is None:
            self._graph = Graph.capture(self.stream, self.enqueue_step)
        return self._graph

    def capture_steps(self, n_steps: int) -> Graph:
        """n_steps consecutive token steps as one HIP graph (the caller closes it).
        Each step reads the token and position the previous one left on the GPU
        and records its token in `history`, so one replay decodes n_steps tokens
        with one graph launch instead of n_steps (a graph launch costs ~7 us
        before its first kernel starts)."""
        if n_steps < 1:
            raise ValueError("n_steps must be >= 1")
        return Graph.capture(self.stream, lambda: [self.enqueue_step() for _ in range(n_steps)])

    STEPS_PER_GRAPH = 16

    def enqueue_generate(self, n_steps: int, use_graph: bool = True) -> None:
        """Enqueues n_steps token steps from the token and position on the GPU
        (no synchronization): replays of a cached graph of STEPS_PER_GRAPH steps,
        then one-step replays for the rest; or direct launches."""
        if not use_graph:
            for _ in range(n_steps):
                self.enqueue_step()
            return
        per = self.STEPS_PER_GRAPH
        if n_steps >= per and per not in self._multi:
            self._multi[per] = self.capture_steps(per)
        for _ in range(n_steps // per):
            self._multi[per].launch(self.stream)
        rest = n_steps % per
        if rest:
            one = self.capture()
            for _ in range(rest):
                one.launch(self.stream)

    def read_history(self, pos: int, n: int) -> list[int]:
        """The greedy tokens chosen at positions pos .. pos + n - 1."""
        if pos < 0 or pos + n > self.max_ctx:
            raise ValueError("history range outside the cache")
        return [int(t) for t in self.history.download(np.int32, (n,), offset=4 * pos)]

    def generate(self, token_id: int, pos: int, n_steps: int, use_graph: bool = True) -> list[int]:
        """Greedy decode of n_steps tokens starting from token_id at pos
        (the loop of generate.py:411-430, argmax on the GPU).  Every step is
        enqueued before the host waits: the tokens come back from the device
        history in one copy at the end."""
        if pos + n_steps > self.max_ctx:
            raise ValueError("decode would run past the KV cache")
        self.set_position(token_id, pos)
        self.enqueue_generate(n_steps, use_graph)
        self.stream.synchronize()
        return self.read_history(pos, n_steps)

    def read_position(self) -> int:
        return int(self.pos.download(np.int32, (1,))[0])

    def close(self) -> None:
        if self._graph is not None:
            self._graph.close()
            self._graph = None
        for g in self._multi.values():
            g.close()
        self._multi.clear()
