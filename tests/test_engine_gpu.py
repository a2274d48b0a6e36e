"""GPU decode engine (asmllm_amd.engine) against the oracle's composed decode step.

The engine's weights and caches are read back from HBM, so both sides run on
the same bytes.  Bar: logits within 2e-4 of the largest logit magnitude (the
per-op fp32 tolerance, 1e-5 at test_runner.py:36, accumulated over the
layers and the lm-head), and the greedy token equal whenever the oracle's
top-2 margin is above that bar.  A graph replay of the step must reproduce
the eager launches bit for bit.
"""

import numpy as np
import pytest

from asmllm_amd import native
from asmllm_amd.engine import LLAMA_7B, STORIES_15M, DecodeEngine, LlamaShape
from asmllm_amd.gguf import q4_0_nbytes

pytestmark = pytest.mark.gpu
LOGIT_TOL = 2e-4


def _blocks(buf, rows, K, qtype=native.Q4_0):
    return buf.download(np.uint8, (rows, K // 32, 34 if qtype == native.Q8_0 else 18))


def _oracle_model(eng: DecodeEngine, nt: int):
    from oracle.decode_ref import DecodeRef

    s = eng.shape
    d, h, kv = s.dim, s.hidden_dim, s.kv_dim
    layers, kcs, vcs = [], [], []
    for i, ly in enumerate(eng.layers):
        qkv = _blocks(ly.wqkv, s.qkv_rows, d)
        gate, up = eng.gate_up_blocks(i)
        layers.append({
            "attn_norm": ly.attn_norm.download(np.float32, d), "ffn_norm": ly.ffn_norm.download(np.float32, d),
            "wq": qkv[:d], "wk": qkv[d:d + kv], "wv": qkv[d + kv:],
            "wo": _blocks(ly.wo, d, d), "w_gate": gate, "w_up": up, "w_down": _blocks(ly.wdown, d, h),
        })
        shape = (s.n_kv_heads, eng.max_ctx, s.head_dim)
        kcs.append(ly.k_cache.download(np.uint16, shape))
        vcs.append(ly.v_cache.download(np.uint16, shape))
    return DecodeRef(dim=d, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, hidden_dim=h, vocab=s.vocab, eps=s.eps,
                     theta=s.theta, embed=_blocks(eng.embed, s.vocab, d, eng.embed_type),
                     final_norm=eng.final_norm.download(np.float32, d),
                     output=_blocks(eng.output, s.vocab, d, eng.output_type),
                     layers=layers, k_caches=kcs, v_caches=vcs, nt=nt)


def _check_logits(got, ref, what):
    scale = float(np.abs(ref).max())
    err = float(np.abs(got.astype(np.float64) - ref).max())
    assert err <= LOGIT_TOL * scale, f"{what}: max |err| {err:.3e} > {LOGIT_TOL:.0e} x max|logit| {scale:.3e}"
    top2 = np.sort(ref)[-2:]
    if top2[1] - top2[0] > 2 * LOGIT_TOL * scale:
        assert int(np.argmax(got)) == int(np.argmax(ref)), what
    return err / scale


SMALL = [
    LlamaShape(dim=256, n_layers=2, n_heads=4, n_kv_heads=4, hidden_dim=512, vocab=1000),
    LlamaShape(dim=512, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=1408, vocab=777, eps=1e-5),
    LlamaShape(dim=512, n_layers=3, n_heads=8, n_kv_heads=8, hidden_dim=1024, vocab=4096, theta=5e5),
]
# (shape, embedding type, lm-head type): the stories15M shape (head_dim 48, dim 288: RMSNorm not
# fused) with a Q8_0 lm-head, and a Q8_0 embedding at a fused shape.
CASES = [(SMALL[0], native.Q4_0, native.Q4_0), (SMALL[1], native.Q4_0, native.Q4_0),
         (SMALL[2], native.Q4_0, native.Q4_0), (STORIES_15M, native.Q4_0, native.Q8_0),
         (SMALL[1], native.Q8_0, native.Q8_0)]


@pytest.mark.parametrize("shape,embed_type,output_type", CASES,
                         ids=["mha", "gqa", "hd64", "stories15m_q8_head", "q8_embed_head"])
def test_decode_steps_match_oracle(shape, embed_type, output_type):
    eng = DecodeEngine(shape, max_ctx=48, embed_type=embed_type, output_type=output_type)
    eng.init_random(seed=7)
    ref = _oracle_model(eng, nt=4)
    token, pos0 = 5, 29
    for step in range(4):
        pos = pos0 + step
        got = eng.forward_token(token, pos)
        want = ref.forward_token(token, pos)
        rel = _check_logits(got, want, f"step {step} pos {pos}")
        print(f"step {step}: max err / max|logit| {rel:.2e}")
        token = int(np.argmax(want))
    # the caches agree after the steps: k within one fp16 rounding, v likewise
    s = eng.shape
    for li, ly in enumerate(eng.layers):
        kc = ly.k_cache.download(np.uint16, (s.n_kv_heads, eng.max_ctx, s.head_dim))
        for p in range(pos0, pos0 + 4):
            a = kc[:, p].view(np.float16).astype(np.float32)
            b = ref.k_caches[li][p].view(np.float16).astype(np.float32)   # oracle keeps [pos][kv][hd]
            np.testing.assert_allclose(a, b, rtol=2 ** -9, atol=1e-3)
    eng.close()


def test_graph_replay_matches_eager_launches():
    shape = SMALL[0]
    eng = DecodeEngine(shape, max_ctx=64)
    eng.init_random(seed=3)
    eager = eng.generate(11, 40, 6, use_graph=False)
    logits_eager = eng.logits.download(np.float32, shape.vocab)
    assert eng.read_position() == 46
    graphed = eng.generate(11, 40, 6, use_graph=True)   # same start: rewrites the same cache rows
    assert graphed == eager
    np.testing.assert_array_equal(eng.logits.download(np.float32, shape.vocab), logits_eager)
    assert eng.read_position() == 46
    again = eng.generate(11, 40, 6, use_graph=True)     # replays of one captured graph
    assert again == eager
    eng.close()


@pytest.mark.parametrize("max_ctx,pos0", [(800, 381), (3100, 1021)], ids=["384-splits", "512-splits"])
def test_steps_across_attention_split_boundaries(max_ctx, pos0):
    """Steps whose positions cross a split boundary of the decode attention
    (max_ctx 800: 384-position splits, 3 of them; max_ctx 3100: 512-position
    splits, 7): every step within the bar of the oracle, and a graph replay of
    the same steps equal to the eager launches bit for bit."""
    eng = DecodeEngine(SMALL[1], max_ctx=max_ctx)
    eng.init_random(seed=11)
    ref = _oracle_model(eng, nt=4)
    token = 3
    for step in range(5):
        pos = pos0 + step
        got = eng.forward_token(token, pos)
        want = ref.forward_token(token, pos)
        _check_logits(got, want, f"max_ctx {max_ctx} pos {pos}")
        token = int(np.argmax(want))
    eager = eng.generate(3, pos0, 5, use_graph=False)
    logits_eager = eng.logits.download(np.float32, SMALL[1].vocab)
    graphed = eng.generate(3, pos0, 5, use_graph=True)
    assert graphed == eager
    np.testing.assert_array_equal(eng.logits.download(np.float32, SMALL[1].vocab), logits_eager)
    eng.close()


def test_multi_step_graph_matches_single_step_replays():
    """A graph of 5 consecutive token steps (capture_steps) leaves the same
    token, position and logits, bit for bit, as 5 replays of the one-step graph."""
    shape = SMALL[2]
    eng = DecodeEngine(shape, max_ctx=64)
    eng.init_random(seed=5)
    single = eng.generate(7, 20, 5, use_graph=True)
    logits_single = eng.logits.download(np.float32, shape.vocab)
    assert eng.read_position() == 25
    multi = eng.capture_steps(5)
    eng.set_position(7, 20)
    multi.launch(eng.stream)
    eng.stream.synchronize()
    assert eng.read_position() == 25
    assert int(eng.token.download(np.int32, (1,))[0]) == single[-1]
    # every step of the graph recorded its token, not only the last one
    assert eng.read_history(20, 5) == single
    np.testing.assert_array_equal(eng.logits.download(np.float32, shape.vocab), logits_single)
    multi.close()
    eng.close()


def test_generate_through_multi_step_graphs_keeps_every_token():
    """generate() with more steps than one graph holds (16 + 16 + 3: two replays
    of the 16-step graph, then one-step replays) returns the same tokens, bit for
    bit the same final logits, as launching every step directly and reading the
    token after each one."""
    shape = SMALL[0]
    eng = DecodeEngine(shape, max_ctx=96)
    eng.init_random(seed=9)
    n, pos0 = 35, 30
    step_by_step = []
    eng.set_position(4, pos0)
    for _ in range(n):
        eng.enqueue_step()
        eng.stream.synchronize()
        step_by_step.append(int(eng.token.download(np.int32, (1,))[0]))
    logits_eager = eng.logits.download(np.float32, shape.vocab)
    graphed = eng.generate(4, pos0, n, use_graph=True)
    assert graphed == step_by_step
    assert eng.read_position() == pos0 + n
    np.testing.assert_array_equal(eng.logits.download(np.float32, shape.vocab), logits_eager)
    assert eng.generate(4, pos0, n, use_graph=False) == step_by_step
    eng.close()


def test_engine_rejects_positions_outside_the_cache():
    eng = DecodeEngine(SMALL[0], max_ctx=16)
    with pytest.raises(ValueError):
        eng.forward_token(1, 16)
    with pytest.raises(ValueError):
        eng.generate(1, 10, 7)
    with pytest.raises(ValueError):
        eng.forward_token(SMALL[0].vocab, 0)


def test_7b_shape_step_at_context_2048_matches_oracle():
    """One token of the 32-layer 7B-shape model at position 2048 (cache
    prefilled with N(0,1) fp16), the benchmark's decode workload."""
    eng = DecodeEngine(LLAMA_7B, max_ctx=2176)
    eng.init_random(seed=42)
    assert eng.layers[0].wqkv.nbytes == q4_0_nbytes(3 * 4096, 4096)
    got = eng.forward_token(1, 2048)
    ref = _oracle_model(eng, nt=16)
    want = ref.forward_token(1, 2048)
    rel = _check_logits(got, want, "7B step")
    print(f"7B step: max err / max|logit| {rel:.2e}")
    eng.close()


def _write_llama_gguf(path, s: LlamaShape, seed: int, tied: bool, output_q8: bool = False):
    from asmllm_amd import gguf
    from asmllm_amd import gguf_file as gf

    rng = np.random.default_rng(seed)

    def q4(rows, K):
        return gguf.quantize_q4_0((rng.standard_normal((rows, K)) * 0.05).astype(np.float32))

    d, h, kv = s.dim, s.hidden_dim, s.kv_dim
    t = {"token_embd.weight": (gf.Q4_0, (d, s.vocab), q4(s.vocab, d)),
         "output_norm.weight": (gf.F32, (d,), rng.uniform(0.5, 1.5, d).astype(np.float32))}
    if not tied:
        if output_q8:
            w = gguf.quantize_q8_0((rng.standard_normal((s.vocab, d)) * 0.05).astype(np.float32))
            t["output.weight"] = (gf.Q8_0, (d, s.vocab), w)
        else:
            t["output.weight"] = (gf.Q4_0, (d, s.vocab), q4(s.vocab, d))
    for i in range(s.n_layers):
        b = f"blk.{i}."
        t[b + "attn_norm.weight"] = (gf.F32, (d,), rng.uniform(0.5, 1.5, d).astype(np.float32))
        t[b + "ffn_norm.weight"] = (gf.F32, (d,), rng.uniform(0.5, 1.5, d).astype(np.float32))
        for name, rows, K in (("attn_q", d, d), ("attn_k", kv, d), ("attn_v", kv, d), ("attn_output", d, d),
                              ("ffn_gate", h, d), ("ffn_up", h, d), ("ffn_down", d, h)):
            t[b + name + ".weight"] = (gf.Q4_0, (K, rows), q4(rows, K))
    meta = {"general.architecture": (gf.T_STRING, "llama"),
            "llama.embedding_length": (gf.T_UINT32, d), "llama.block_count": (gf.T_UINT32, s.n_layers),
            "llama.feed_forward_length": (gf.T_UINT32, h), "llama.attention.head_count": (gf.T_UINT32, s.n_heads),
            "llama.attention.head_count_kv": (gf.T_UINT32, s.n_kv_heads),
            "llama.attention.layer_norm_rms_epsilon": (gf.T_FLOAT32, s.eps),
            "llama.rope.freq_base": (gf.T_FLOAT32, s.theta),
            "tokenizer.ggml.tokens": (gf.T_ARRAY, (gf.T_STRING, [f"t{i}" for i in range(s.vocab)]))}
    gf.write_gguf(path, meta, t, alignment=64)


TINY = LlamaShape(dim=256, n_layers=2, n_heads=4, n_kv_heads=2, hidden_dim=512, vocab=500,
                  eps=float(np.float32(1e-5)))  # as the file stores it
STORIES_FILE = LlamaShape(**{**STORIES_15M.__dict__, "eps": float(np.float32(1e-5))})


@pytest.mark.parametrize("s,tied,output_q8", [(TINY, False, False), (TINY, True, False), (STORIES_FILE, False, True)],
                         ids=["lm_head", "tied_embedding", "stories15m_shape_q8_head"])
def test_engine_from_gguf_matches_oracle(tmp_path, s, tied, output_q8):
    """A GGUF Llama (generate.py:182-205 tensor names) loaded once into HBM
    decodes as the oracle's forward_token on the file's own tensors; the last
    case has the reference demo model's architecture (synthetic weights)."""
    from asmllm_amd import gguf_file as gf
    from oracle.decode_ref import DecodeRef

    path = tmp_path / "tiny.gguf"
    _write_llama_gguf(path, s, seed=11, tied=tied, output_q8=output_q8)
    max_ctx = 32
    eng = DecodeEngine.from_gguf(path, max_ctx=max_ctx)
    assert eng.shape == s and eng.vocab[:2] == ["t0", "t1"]
    with gf.GGUFFile(path) as g:
        T = lambda n: np.array(g.tensor(n))
        layers = [{"attn_norm": T(f"blk.{i}.attn_norm.weight"), "ffn_norm": T(f"blk.{i}.ffn_norm.weight"),
                   "wq": T(f"blk.{i}.attn_q.weight"), "wk": T(f"blk.{i}.attn_k.weight"),
                   "wv": T(f"blk.{i}.attn_v.weight"), "wo": T(f"blk.{i}.attn_output.weight"),
                   "w_gate": T(f"blk.{i}.ffn_gate.weight"), "w_up": T(f"blk.{i}.ffn_up.weight"),
                   "w_down": T(f"blk.{i}.ffn_down.weight")} for i in range(s.n_layers)]
        embed = T("token_embd.weight")
        ref = DecodeRef(dim=s.dim, n_heads=s.n_heads, n_kv_heads=s.n_kv_heads, hidden_dim=s.hidden_dim,
                        vocab=s.vocab, eps=s.eps, theta=s.theta, embed=embed,
                        final_norm=T("output_norm.weight"), output=embed if tied else T("output.weight"),
                        layers=layers,
                        k_caches=[np.zeros((s.n_kv_heads, max_ctx, s.head_dim), np.uint16)] * s.n_layers,
                        v_caches=[np.zeros((s.n_kv_heads, max_ctx, s.head_dim), np.uint16)] * s.n_layers)
    token = 1
    for pos in range(6):  # from position 0: every cache row read was written by an earlier step
        got = eng.forward_token(token, pos)
        want = ref.forward_token(token, pos)
        _check_logits(got, want, f"pos {pos}")
        token = int(np.argmax(want))
    eng.close()


M2_FIXTURE = "stories15m_m2_tokens.json"


def _stories15m_path():
    import os
    from pathlib import Path

    for cand in (os.environ.get("ASMLLM_STORIES15M", ""), "models/stories15M-q4_0.gguf", "stories15M-q4_0.gguf"):
        if cand and Path(cand).is_file() and Path(cand).stat().st_size >= 1024:
            return Path(cand)
    return None


def test_stories15m_greedy_matches_reference_log():
    """The reference's end-to-end check (generate.py:382-430): prompt
    [1, 9038, 2501, 263, 931] fed token by token, then 30 greedy tokens, which
    must equal the tokens in the reference's own log (m2_generation.log:10-39,
    kept in tests/golden).  Needs the published stories15M-q4_0.gguf, which
    is not available offline: set ASMLLM_STORIES15M or place it in models/."""
    import json

    from conftest import GOLDEN_DIR

    path = _stories15m_path()
    if path is None:
        pytest.skip("stories15M-q4_0.gguf not present (no network to fetch it)")
    want = json.loads((GOLDEN_DIR / M2_FIXTURE).read_text())
    eng = DecodeEngine.from_gguf(path, max_ctx=64)
    assert eng.shape.dim == 288 and eng.shape.head_dim == 48
    prompt = want["prompt"]
    for pos, tok in enumerate(prompt[:-1]):
        eng.forward_token(tok, pos)
    got = eng.generate(prompt[-1], len(prompt) - 1, len(want["generated"]), use_graph=True)
    assert got == want["generated"]
    eng.close()
