"""GPU parity of the decode-step ops, the GPU quantizers and the synthetic
model generators (through the C ABI) against the CPU oracle.

Bar: the reference's fp32 tolerance for these ops (1e-5, test_runner.py:36),
fp16 cache entries within one fp16 rounding, quantized bytes bit-exact.
"""

import numpy as np
import pytest

from asmllm_amd import gguf, native
from asmllm_amd.device import DeviceBuffer, synchronize

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _host(fn, *args):
    fn(*[a.ctypes.data if isinstance(a, np.ndarray) else a for a in args])


def _ok(hip, rc):
    assert rc == 0, hip.asmhip_last_error()


# ---- reference-named ops on host buffers ---------------------------------------------------

@pytest.mark.parametrize("dim", [1, 33, 4096, 11008])
def test_rmsnorm(hip, oracle, dim):
    rng = np.random.default_rng(dim)
    x = rng.standard_normal(dim).astype(np.float32)
    w = rng.uniform(0.5, 1.5, dim).astype(np.float32)
    for eps in (1e-5, 1e-6):
        y = np.zeros(dim, np.float32)
        _host(hip.asm_rmsnorm, x, w, y, dim, eps)
        np.testing.assert_allclose(y, oracle.rmsnorm(x, w, eps), rtol=TOL, atol=TOL)


@pytest.mark.parametrize("hd", [64, 128])
@pytest.mark.parametrize("pos", [0, 1, 17, 2047, 2175, 100000])
def test_rope(hip, oracle, hd, pos):
    rng = np.random.default_rng(hd + pos)
    q = rng.standard_normal(hd).astype(np.float32)
    k = rng.standard_normal(hd).astype(np.float32)
    q_ref, k_ref = oracle.rope(q, k, hd, pos, 10000.0)
    _host(hip.asm_rope, q, k, hd, pos, 10000.0)
    np.testing.assert_allclose(q, q_ref, rtol=TOL, atol=TOL)
    np.testing.assert_allclose(k, k_ref, rtol=TOL, atol=TOL)


def test_rope_position_zero_is_identity(hip):
    q = np.arange(128, dtype=np.float32)
    k = -np.arange(128, dtype=np.float32)
    q0, k0 = q.copy(), k.copy()
    _host(hip.asm_rope, q, k, 128, 0, 10000.0)
    np.testing.assert_array_equal(q, q0)
    np.testing.assert_array_equal(k, k0)


@pytest.mark.parametrize("dim", [1, 7, 2049, 32000])
def test_softmax(hip, oracle, dim):
    rng = np.random.default_rng(dim)
    x = (rng.standard_normal(dim) * 4).astype(np.float32)
    y = np.zeros(dim, np.float32)
    _host(hip.asm_softmax, x, y, dim)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(y, e / e.sum(), rtol=TOL, atol=1e-12)
    # the reference sums exp() sequentially in fp32 (softmax_avx2.asm:65-97): its
    # result carries up to (dim - 1) roundings of the sum on top of the bar
    np.testing.assert_allclose(y, oracle.softmax(x), rtol=TOL + dim * 2.0 ** -24, atol=1e-12)
    assert abs(float(y.astype(np.float64).sum()) - 1.0) < 1e-5
    inplace = x.copy()
    _host(hip.asm_softmax, inplace, inplace, dim)  # x == y (attention_avx2.asm:141-142)
    np.testing.assert_array_equal(inplace, y)


@pytest.mark.parametrize("dim", [1, 100, 11008])
def test_silu_hadamard(hip, oracle, dim):
    rng = np.random.default_rng(dim)
    g = (rng.standard_normal(dim) * 3).astype(np.float32)
    u = rng.standard_normal(dim).astype(np.float32)
    ref = oracle.silu_hadamard(g, u)
    _host(hip.asm_silu_hadamard, g, u, dim)
    np.testing.assert_allclose(g, ref, rtol=TOL, atol=1e-7)


@pytest.mark.parametrize("seq,hd", [(1, 64), (7, 64), (128, 128), (300, 128)])
def test_attention(hip, oracle, seq, hd):
    rng = np.random.default_rng(seq * hd)
    q, k, v = (rng.standard_normal((seq, hd)).astype(np.float32) for _ in range(3))
    scale = float(1.0 / np.sqrt(hd))
    y = np.zeros((seq, hd), np.float32)
    _host(hip.asm_attention, q, k, v, y, seq, hd, scale)
    s64 = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    p64 = np.exp(s64 - s64.max(axis=1, keepdims=True))
    ref64 = (p64 / p64.sum(axis=1, keepdims=True)) @ v.astype(np.float64)
    np.testing.assert_allclose(y, ref64, rtol=TOL, atol=TOL)
    # the reference's sequential fp32 softmax sum adds up to seq roundings
    np.testing.assert_allclose(y, oracle.attention(q, k, v, scale), rtol=TOL + seq * 2.0 ** -24, atol=TOL)


# ---- device forms used by the decode step ----------------------------------------------------

def test_multi_head_rope_reads_position_on_device(hip, oracle):
    n_q, n_k, hd, pos = 32, 8, 128, 1234
    rng = np.random.default_rng(3)
    q = rng.standard_normal((n_q, hd)).astype(np.float32)
    k = rng.standard_normal((n_k, hd)).astype(np.float32)
    dq, dk = DeviceBuffer.from_numpy(q), DeviceBuffer.from_numpy(k)
    dpos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    _ok(hip, hip.asmhip_rope(dq.ptr, dk.ptr, n_q, n_k, hd, dpos.ptr, 0, 10000.0, None))
    synchronize()
    gq, gk = dq.download(np.float32, (n_q, hd)), dk.download(np.float32, (n_k, hd))
    for h in range(n_q):
        rq, rk = oracle.rope(q[h], k[h % n_k], hd, pos, 10000.0)
        np.testing.assert_allclose(gq[h], rq, rtol=TOL, atol=TOL)
        if h < n_k:
            np.testing.assert_allclose(gk[h], rk, rtol=TOL, atol=TOL)


def _random_attention_cases(n, seed):
    """Seeded random head layouts, cache lengths and positions."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        hd = int(rng.choice([48, 64, 128]))
        n_kv = int(rng.choice([1, 2, 4, 8]))
        n_heads = n_kv * int(rng.choice([1, 2, 4]))
        max_ctx = int(rng.integers(1, 4097))
        cases.append((n_heads, n_kv, hd, int(rng.integers(0, max_ctx)), max_ctx))
    return cases


@pytest.mark.parametrize("n_heads,n_kv,hd,pos,max_ctx", [
    (32, 32, 128, 0, 256), (32, 32, 128, 2047, 2176), (32, 8, 128, 700, 1024), (8, 2, 64, 129, 130),
    (32, 8, 128, 128, 300), (4, 4, 128, 127, 128), (8, 8, 64, 8191, 8192),
    # head_dim 48 (stories15M): one split, several, and 64 splits (more than the merge's 48 threads)
    (6, 6, 48, 5, 64), (6, 6, 48, 300, 2048), (6, 2, 48, 8000, 8192),
    # split (384 positions up to max_ctx 3072, 512 above) and chunk (64 / 128
    # positions) boundaries, a split holding only pos, the most splits a matvec
    # merges (8), and a cache of 64 splits (the most the merge launch takes)
    (4, 4, 128, 383, 600), (4, 2, 128, 384, 600), (4, 4, 128, 385, 800), (6, 6, 48, 767, 800),
    (8, 4, 64, 768, 1000), (4, 4, 128, 3071, 3072), (4, 4, 128, 511, 3073), (4, 2, 128, 512, 3200),
    (4, 4, 128, 513, 4096), (4, 4, 128, 511, 600), (4, 4, 128, 513, 1100), (4, 4, 128, 63, 64),
    (4, 4, 128, 64, 130), (8, 4, 64, 127, 1024), (6, 6, 48, 1535, 1537), (2, 1, 128, 32767, 32768),
] + _random_attention_cases(8, 77))
def test_rope_kv_write_and_decode_attention(hip, oracle, n_heads, n_kv, hd, pos, max_ctx):
    rng = np.random.default_rng(n_heads * 1000 + pos)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * hd).astype(np.float32)
    # caches head-major [n_kv][max_ctx][hd]; positions < pos hold earlier tokens
    kc = np.zeros((n_kv, max_ctx, hd), np.float16)
    vc = np.zeros((n_kv, max_ctx, hd), np.float16)
    kc[:, :pos] = rng.standard_normal((n_kv, pos, hd))
    vc[:, :pos] = rng.standard_normal((n_kv, pos, hd))
    dqkv, dkc, dvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
    dpos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    ws = hip.asmhip_attention_decode_workspace(n_heads, hd, max_ctx)
    assert ws > 0
    dws, dout = DeviceBuffer(ws * 4), DeviceBuffer(n_heads * hd * 4)
    # the fused form on copies of the same inputs
    fqkv, fkc, fvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
    fout = DeviceBuffer(n_heads * hd * 4)
    _ok(hip, hip.asmhip_attention_decode_rope(fqkv.ptr, fkc.ptr, fvc.ptr, dws.ptr, fout.ptr, n_heads, n_kv, hd,
                                              dpos.ptr, max_ctx, 10000.0, None))
    # and with the angles from a table formed once
    tqkv, tkc, tvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
    tout, table = DeviceBuffer(n_heads * hd * 4), DeviceBuffer(max_ctx * hd * 4)
    _ok(hip, hip.asmhip_rope_table(table.ptr, hd, max_ctx, 10000.0, None))
    _ok(hip, hip.asmhip_attention_decode_rope_table(tqkv.ptr, tkc.ptr, tvc.ptr, dws.ptr, tout.ptr, n_heads, n_kv,
                                                    hd, dpos.ptr, max_ctx, table.ptr, None))
    _ok(hip, hip.asmhip_rope_kv_write(dqkv.ptr, dkc.ptr, dvc.ptr, n_heads, n_kv, hd, dpos.ptr, max_ctx, 10000.0,
                                      None))
    _ok(hip, hip.asmhip_attention_decode(dqkv.ptr, dkc.ptr, dvc.ptr, dws.ptr, dout.ptr, n_heads, n_kv, hd,
                                         dpos.ptr, max_ctx, None))
    synchronize()

    q = qkv[: n_heads * hd].reshape(n_heads, hd)
    k = qkv[n_heads * hd: (n_heads + n_kv) * hd].reshape(n_kv, hd)
    v = qkv[(n_heads + n_kv) * hd:].reshape(n_kv, hd)
    q_rot = np.stack([oracle.rope(q[h], k[0], hd, pos, 10000.0)[0] for h in range(n_heads)])
    k_rot = np.stack([oracle.rope(q[0], k[h], hd, pos, 10000.0)[1] for h in range(n_kv)])
    got_q = dqkv.download(np.float32, n_heads * hd).reshape(n_heads, hd)
    np.testing.assert_allclose(got_q, q_rot, rtol=TOL, atol=TOL)
    got_kc = dkc.download(np.float16, (n_kv, max_ctx, hd))
    got_vc = dvc.download(np.float16, (n_kv, max_ctx, hd))
    np.testing.assert_array_equal(got_vc[:, pos], v.astype(np.float16))
    np.testing.assert_allclose(got_kc[:, pos].astype(np.float32), k_rot, rtol=2 ** -10, atol=1e-6)
    np.testing.assert_array_equal(got_kc[:, :pos], kc[:, :pos])  # earlier positions untouched
    if pos + 1 < max_ctx:
        assert not got_kc[:, pos + 1:].any()

    # oracle cache layout [pos][kv_head][hd], fp16 bits; the GPU's own k entry
    kc_o = np.ascontiguousarray(got_kc.transpose(1, 0, 2)).view(np.uint16)
    vc_o = np.ascontiguousarray(got_vc.transpose(1, 0, 2)).view(np.uint16)
    ref = oracle.attention_decode_f16(got_q, kc_o, vc_o, pos + 1, n_kv, 8)
    out = dout.download(np.float32, (n_heads, hd))
    np.testing.assert_allclose(out, ref, rtol=TOL, atol=TOL)
    # fused = rope_kv_write then attention, bit for bit (same rotation, same fp16 row)
    np.testing.assert_array_equal(fout.download(np.float32, (n_heads, hd)), out)
    np.testing.assert_array_equal(fkc.download(np.float16, (n_kv, max_ctx, hd)), got_kc)
    np.testing.assert_array_equal(fvc.download(np.float16, (n_kv, max_ctx, hd)), got_vc)
    np.testing.assert_array_equal(fqkv.download(np.float32, qkv.size), qkv)  # q left unrotated
    np.testing.assert_array_equal(tout.download(np.float32, (n_heads, hd)), out)
    np.testing.assert_array_equal(tkc.download(np.float16, (n_kv, max_ctx, hd)), got_kc)
    np.testing.assert_array_equal(tvc.download(np.float16, (n_kv, max_ctx, hd)), got_vc)
    np.testing.assert_array_equal(tqkv.download(np.float32, qkv.size), qkv)


@pytest.mark.parametrize("hd,max_ctx,theta", [(128, 2176, 10000.0), (64, 300, 500000.0), (48, 8192, 10000.0)])
def test_rope_table_angles(hip, hd, max_ctx, theta):
    """table[p][2i], [2i + 1] = cos, sin of p * theta^(-2i / hd): the exponent a
    float32 quotient (divss in rope_avx2.asm), the angle and its cos / sin in
    float64, rounded to float32 (to within an ulp of numpy's float64 math)."""
    table = DeviceBuffer(max_ctx * hd * 4)
    _ok(hip, hip.asmhip_rope_table(table.ptr, hd, max_ctx, theta, None))
    synchronize()
    got = table.download(np.float32, (max_ctx, hd // 2, 2))
    e = (np.float32(-2) * np.arange(hd // 2, dtype=np.float32)) / np.float32(hd)
    ang = np.power(np.float64(np.float32(theta)), e.astype(np.float64))[None, :] * np.arange(max_ctx)[:, None]
    np.testing.assert_allclose(got[..., 0], np.cos(ang).astype(np.float32), rtol=0, atol=2e-7)
    np.testing.assert_allclose(got[..., 1], np.sin(ang).astype(np.float32), rtol=0, atol=2e-7)
    assert np.array_equal(got[0, :, 0], np.ones(hd // 2, np.float32)) and not got[0, :, 1].any()



def test_embed_row_and_argmax(hip, oracle):
    n_vocab, dim = 1000, 256
    rng = np.random.default_rng(4)
    table = gguf.quantize_q4_0(rng.standard_normal((n_vocab, dim)).astype(np.float32))
    dt = DeviceBuffer.from_numpy(table)
    dtok = DeviceBuffer.from_numpy(np.array([417], np.int32))
    dx = DeviceBuffer(dim * 4)
    _ok(hip, hip.asmhip_embed_q4_0(dt.ptr, dtok.ptr, dx.ptr, n_vocab, dim, None))
    synchronize()
    np.testing.assert_array_equal(dx.download(np.float32, dim), oracle.dequantize_q4_0(table[417:418])[0])
    t8 = gguf.quantize_q8_0(rng.standard_normal((n_vocab, 288)).astype(np.float32))
    dt8, dx8 = DeviceBuffer.from_numpy(t8), DeviceBuffer(288 * 4)
    _ok(hip, hip.asmhip_embed_q8_0(dt8.ptr, dtok.ptr, dx8.ptr, n_vocab, 288, None))
    synchronize()
    np.testing.assert_array_equal(dx8.download(np.float32, 288), oracle.dequantize_q8_0(t8[417:418])[0])

    logits = rng.standard_normal(32000).astype(np.float32)
    logits[[123, 31000]] = 9.0  # tie: the first index wins, as numpy.argmax
    dl = DeviceBuffer.from_numpy(logits)
    dpos = DeviceBuffer.from_numpy(np.array([41], np.int32))
    _ok(hip, hip.asmhip_argmax(dl.ptr, 32000, dtok.ptr, dpos.ptr, None))
    synchronize()
    assert int(dtok.download(np.int32, 1)[0]) == int(np.argmax(logits)) == 123
    assert int(dpos.download(np.int32, 1)[0]) == 42


def test_argmax_history_records_each_position(hip):
    """asmhip_argmax_history: history[pos] = the token, then pos + 1; a position
    outside [0, history_len) advances without writing."""
    rng = np.random.default_rng(3)
    n, hl = 32000, 8
    dl, dtok, dpos = DeviceBuffer(4 * n), DeviceBuffer(4), DeviceBuffer(4)
    dhist = DeviceBuffer(4 * hl)
    dhist.upload(np.full(hl, -1, np.int32))
    want = []
    for p in (0, 3, 7):
        logits = rng.standard_normal(n).astype(np.float32)
        dl.upload(logits)
        dpos.upload(np.array([p], np.int32))
        _ok(hip, hip.asmhip_argmax_history(dl.ptr, n, dtok.ptr, dpos.ptr, dhist.ptr, hl, None))
        synchronize()
        assert int(dpos.download(np.int32, 1)[0]) == p + 1
        want.append((p, int(np.argmax(logits))))
    hist = dhist.download(np.int32, hl)
    for p, t in want:
        assert hist[p] == t
    assert all(hist[p] == -1 for p in range(hl) if p not in (0, 3, 7))
    dpos.upload(np.array([hl], np.int32))  # past the history: no write
    _ok(hip, hip.asmhip_argmax_history(dl.ptr, n, dtok.ptr, dpos.ptr, dhist.ptr, hl, None))
    synchronize()
    assert int(dpos.download(np.int32, 1)[0]) == hl + 1
    np.testing.assert_array_equal(dhist.download(np.int32, hl), hist)
    assert hip.asmhip_argmax_history(dl.ptr, n, dtok.ptr, None, dhist.ptr, hl, None) != 0


@pytest.mark.parametrize("n", [1, 5, 36, 1024, 32000, 32768, 32769, 128256])
def test_argmax_sizes_and_ties(hip, n):
    """One pass (n <= 32768) and several (the Llama-3 vocabulary), with 16-byte
    loads (n % 4 == 0) and single floats; a tie across passes and lanes resolves
    to the first index, as numpy.argmax."""
    rng = np.random.default_rng(n)
    logits = rng.standard_normal(n).astype(np.float32)
    if n > 2:
        a, b = sorted(rng.choice(n, 2, replace=False))
        logits[[a, b]] = 9.0
    dl = DeviceBuffer.from_numpy(logits)
    dtok = DeviceBuffer.from_numpy(np.array([-1], np.int32))
    _ok(hip, hip.asmhip_argmax(dl.ptr, n, dtok.ptr, None, None))
    synchronize()
    assert int(dtok.download(np.int32, 1)[0]) == int(np.argmax(logits))


# ---- GPU quantizers and synthetic weights -----------------------------------------------------

@pytest.mark.parametrize("qt", ["q4", "q8"])
def test_gpu_quantizer_bit_exact(hip, oracle, qt):
    rng = np.random.default_rng(12)
    rows, K = 513, 4096
    w = (rng.standard_normal((rows, K)) * 0.02).astype(np.float32)
    w[0, :32] = 0.0                       # all-zero block
    w[1, :32] = np.float32(0.5)           # constant block
    w[2, :32] = np.linspace(-1, 1, 32)    # exact ties
    m = float(np.abs(w[3, :32]).max())
    w[3, 5], w[3, 9] = -m, m              # repeated magnitude: the first one sets the sign of d
    dw, db = DeviceBuffer.from_numpy(w), DeviceBuffer(rows * (K // 32) * (18 if qt == "q4" else 34))
    code = native.Q4_0 if qt == "q4" else native.Q8_0
    _ok(hip, hip.asmhip_quantize(code, dw.ptr, db.ptr, rows, K, None))
    synchronize()
    bpb = 18 if qt == "q4" else 34
    got = db.download(np.uint8, (rows, K // 32, bpb))
    ref = oracle.quantize_q4_0(w) if qt == "q4" else oracle.quantize_q8_0(w)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, f"mismatched bytes at {bad[:8].tolist()}: got {got[tuple(bad[:8].T)]}, want {ref[tuple(bad[:8].T)]}"
    np.testing.assert_array_equal(ref, gguf.quantize_q4_0(w) if qt == "q4" else gguf.quantize_q8_0(w))


@pytest.mark.parametrize("qt", ["q4", "q8"])
def test_random_blocks_are_deterministic_and_distributed(hip, oracle, qt):
    rows, K, std = 256, 4096, 0.02
    code, bpb = (native.Q4_0, 18) if qt == "q4" else (native.Q8_0, 34)
    a, b, c = (DeviceBuffer(rows * (K // 32) * bpb) for _ in range(3))
    _ok(hip, hip.asmhip_random_blocks(code, a.ptr, rows, K, 7, std, None))
    _ok(hip, hip.asmhip_random_blocks(code, b.ptr, rows, K, 7, std, None))
    _ok(hip, hip.asmhip_random_blocks(code, c.ptr, rows, K, 8, std, None))
    synchronize()
    ba, bb, bc = (d.download(np.uint8, (rows, K // 32, bpb)) for d in (a, b, c))
    np.testing.assert_array_equal(ba, bb)
    assert (ba != bc).mean() > 0.5
    w = oracle.dequantize_q4_0(ba) if qt == "q4" else oracle.dequantize_q8_0(ba)
    assert abs(float(w.mean())) < 1e-3
    assert 0.8 * std < float(w.std()) < 1.2 * std

    h = DeviceBuffer(100001 * 2)
    _ok(hip, hip.asmhip_random_f16(h.ptr, 100001, 3, 1.0, None))
    f = DeviceBuffer(1000 * 4)
    _ok(hip, hip.asmhip_fill_f32(f.ptr, 1000, 1.5, None))
    synchronize()
    v = h.download(np.float16, 100001).astype(np.float64)
    assert abs(v.mean()) < 0.02 and 0.97 < v.std() < 1.03
    assert np.all(f.download(np.float32, 1000) == 1.5)


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("pos", [-1, 256, 1 << 20])
def test_decode_attention_outside_the_cache_is_zero(hip, pos, rope):
    """A position outside [0, max_ctx) (a replayed graph past the cache end) reads and
    writes no cache row and leaves a defined zero output rather than 0 / 0."""
    n_heads, n_kv, hd, max_ctx = 8, 4, 128, 256
    rng = np.random.default_rng(5)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * hd).astype(np.float32)
    kc = rng.standard_normal((n_kv, max_ctx, hd)).astype(np.float16)
    vc = rng.standard_normal((n_kv, max_ctx, hd)).astype(np.float16)
    dqkv, dkc, dvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
    dpos = DeviceBuffer.from_numpy(np.array([pos], np.int32))
    dws = DeviceBuffer(hip.asmhip_attention_decode_workspace(n_heads, hd, max_ctx) * 4)
    dout = DeviceBuffer.from_numpy(np.full(n_heads * hd, 7.0, np.float32))
    fn = hip.asmhip_attention_decode_rope if rope else hip.asmhip_attention_decode
    args = (dqkv.ptr, dkc.ptr, dvc.ptr, dws.ptr, dout.ptr, n_heads, n_kv, hd, dpos.ptr, max_ctx)
    _ok(hip, fn(*args, 10000.0, None) if rope else fn(*args, None))
    synchronize()
    assert np.all(dout.download(np.float32, n_heads * hd) == 0.0)
    np.testing.assert_array_equal(dkc.download(np.float16, kc.shape), kc)
    np.testing.assert_array_equal(dvc.download(np.float16, vc.shape), vc)
    np.testing.assert_array_equal(dqkv.download(np.float32, qkv.size), qkv)


@pytest.mark.parametrize("n", [5, 1024, 32000, 32769])
@pytest.mark.parametrize("case", ["all-nan", "one-nan", "two-nan", "all-neg-inf", "neg-inf-and-one", "two-pos-inf"])
def test_argmax_non_finite_as_numpy(hip, n, case):
    """numpy.argmax semantics on non-finite logits: a NaN ranks first (the first NaN
    wins), and an all -inf vector gives index 0 rather than no index at all."""
    rng = np.random.default_rng(n)
    logits = rng.standard_normal(n).astype(np.float32)
    a, b = sorted(rng.choice(n, 2, replace=False))
    if case == "all-nan":
        logits[:] = np.nan
    elif case == "one-nan":
        logits[b] = np.nan
    elif case == "two-nan":
        logits[[a, b]] = np.nan
    elif case == "all-neg-inf":
        logits[:] = -np.inf
    elif case == "neg-inf-and-one":
        logits[:] = -np.inf
        logits[b] = -1e30
    else:
        logits[[a, b]] = np.inf
    dl = DeviceBuffer.from_numpy(logits)
    dtok = DeviceBuffer.from_numpy(np.array([-1], np.int32))
    _ok(hip, hip.asmhip_argmax(dl.ptr, n, dtok.ptr, None, None))
    synchronize()
    assert int(dtok.download(np.int32, 1)[0]) == int(np.argmax(logits))


@pytest.mark.parametrize("qtype", [native.Q4_0, native.Q8_0])
@pytest.mark.parametrize("n_heads,n_kv,hd,pos,max_ctx,M", [
    (32, 32, 128, 2048, 2176, 4096),   # the 7B step: the merge inside the int8-MFMA matvec
    (8, 2, 64, 300, 1024, 384),        # K = 512: the MFMA stream with its x from LDS
    (16, 4, 128, 5000, 6000, 200),     # 12 splits: more than are requested up front
    (16, 16, 128, 3071, 3072, 1024),   # 8 splits of 384 positions: the most the matvec merges
    (16, 16, 128, 3072, 3073, 1024),   # past 3072: 7 splits of 512
    (16, 16, 64, 0, 100, 32),          # one position, one split
    (6, 6, 48, 100, 256, 288),         # K = 288 (stories15M): merge launch + matvec
])
def test_attention_partials_and_fused_attn_output(hip, qtype, n_heads, n_kv, hd, pos, max_ctx, M):
    """asmhip_attention_decode_partials_rope_table + asmhip_matmul_attn_output (the
    merge of the split states inside the o matvec's read of x) equal, bit for bit,
    asmhip_attention_decode_rope_table (split launch + merge launch) followed by
    asmhip_matmul_fused on its output, accumulating and overwriting; the caches
    written the same way."""
    K = n_heads * hd
    rng = np.random.default_rng(pos + M)
    qkv = rng.standard_normal((n_heads + 2 * n_kv) * hd).astype(np.float32)
    kc = np.zeros((n_kv, max_ctx, hd), np.float16)
    vc = np.zeros((n_kv, max_ctx, hd), np.float16)
    kc[:, :pos] = rng.standard_normal((n_kv, pos, hd))
    vc[:, :pos] = rng.standard_normal((n_kv, pos, hd))
    w = (rng.standard_normal((M, K)) * 0.02).astype(np.float32)
    blocks = gguf.quantize_q4_0(w) if qtype == native.Q4_0 else gguf.quantize_q8_0(w)
    y0 = rng.standard_normal(M).astype(np.float32)
    db, dpos = DeviceBuffer.from_numpy(blocks), DeviceBuffer.from_numpy(np.array([pos], np.int32))
    table = DeviceBuffer(max_ctx * hd * 4)
    _ok(hip, hip.asmhip_rope_table(table.ptr, hd, max_ctx, 10000.0, None))
    ws_n = hip.asmhip_attention_decode_workspace(n_heads, hd, max_ctx)
    outs = {}
    for fused in (False, True):
        dqkv, dkc, dvc = DeviceBuffer.from_numpy(qkv), DeviceBuffer.from_numpy(kc), DeviceBuffer.from_numpy(vc)
        dws, dattn = DeviceBuffer(ws_n * 4), DeviceBuffer(K * 4)
        ya, yo = DeviceBuffer.from_numpy(y0), DeviceBuffer(M * 4)
        if fused:
            _ok(hip, hip.asmhip_attention_decode_partials_rope_table(dqkv.ptr, dkc.ptr, dvc.ptr, dws.ptr, n_heads,
                                                                     n_kv, hd, dpos.ptr, max_ctx, table.ptr, None))
            for y, acc in ((ya, 1), (yo, 0)):
                _ok(hip, hip.asmhip_matmul_attn_output(qtype, db.ptr, dws.ptr, dattn.ptr, y.ptr, M, n_heads, hd,
                                                       max_ctx, acc, None))
        else:
            _ok(hip, hip.asmhip_attention_decode_rope_table(dqkv.ptr, dkc.ptr, dvc.ptr, dws.ptr, dattn.ptr, n_heads,
                                                            n_kv, hd, dpos.ptr, max_ctx, table.ptr, None))
            for y, acc in ((ya, 1), (yo, 0)):
                _ok(hip, hip.asmhip_matmul_fused(qtype, db.ptr, dattn.ptr, y.ptr, M, K, native.PRE_NONE, None,
                                                 0.0, acc, None))
        synchronize()
        outs[fused] = (ya.download(np.float32, M), yo.download(np.float32, M),
                       dkc.download(np.float16, kc.shape), dvc.download(np.float16, vc.shape))
    for a, b in zip(outs[True], outs[False]):
        np.testing.assert_array_equal(a.view(np.uint16 if a.dtype == np.float16 else np.uint32),
                                      b.view(np.uint16 if b.dtype == np.float16 else np.uint32))
    assert np.all(np.isfinite(outs[True][0]))
    # and the values themselves: y0 + W attn against the oracle's fp16-cache attention
    from oracle import native as oracle
    q = qkv[: n_heads * hd].reshape(n_heads, hd)
    k = qkv[n_heads * hd: (n_heads + n_kv) * hd].reshape(n_kv, hd)
    q_rot = np.stack([oracle.rope(q[h], k[0], hd, pos, 10000.0)[0] for h in range(n_heads)])
    kc_o = np.ascontiguousarray(outs[True][2].transpose(1, 0, 2)).view(np.uint16)
    vc_o = np.ascontiguousarray(outs[True][3].transpose(1, 0, 2)).view(np.uint16)
    attn = oracle.attention_decode_f16(q_rot, kc_o, vc_o, pos + 1, n_kv, 8).reshape(K).astype(np.float32)
    wq = gguf.dequantize_q4_0(blocks) if qtype == native.Q4_0 else gguf.dequantize_q8_0(blocks)
    ref = wq.astype(np.float64) @ attn.astype(np.float64)
    l1 = np.abs(wq.astype(np.float64)) @ np.abs(attn.astype(np.float64))
    assert np.all(np.abs(outs[True][1] - ref) <= 1e-4 * l1 + 1e-6)
