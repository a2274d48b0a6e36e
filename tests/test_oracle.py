"""Pins the CPU oracle (test infrastructure) before it is trusted as the checker.

Each restated function is checked against at least one of: the reference's
golden inputs with its own tolerances (tests/correctness/test_runner.py:33-36),
a float64 closed form, an exact special case, or a second independently
written per-lane model of the same SIMD arithmetic.
"""

import numpy as np
import pytest

from conftest import GOLDEN_DIR, assert_matvec_close
from oracle import golden as golden_mod
from oracle import ops_ref


def _rand_q4(rng, M, K):
    q = rng.integers(0, 256, size=(M, K // 32, 16), dtype=np.uint8)
    s = rng.uniform(0.05, 0.25, size=(M, K // 32)).astype(np.float32)
    return q, s


def _rand_q8(rng, M, K):
    q = rng.integers(-128, 128, size=(M, K // 32, 32), dtype=np.int8)
    s = rng.uniform(0.05, 0.25, size=(M, K // 32)).astype(np.float32)
    return q, s


# ---- golden vectors (reference_gen.py recipe, test_runner.py tolerances) ----------

def test_golden_fixture_matches_recipe(golden):
    fresh = golden_mod.generate_reference_data(42)
    assert sorted(fresh) == sorted(golden)
    for k in golden:
        np.testing.assert_array_equal(fresh[k], golden[k], err_msg=k)


@pytest.mark.parametrize("kernel", ["avx2", "lanes", "avx512", "avx512_lanes"])
def test_q4_golden(oracle, golden, kernel):
    y = oracle.matmul_q4(golden["q4_matmul_qweights"], golden["q4_matmul_scales"], golden["q4_matmul_x"], kernel)
    err = np.abs(y - golden["q4_matmul_expected"]).max()
    assert err <= golden_mod.TOLERANCE_Q4
    assert err <= 1e-4  # fp32 reassociation only


@pytest.mark.parametrize("kernel", ["avx2", "lanes"])
def test_q8_golden(oracle, golden, kernel):
    y = oracle.matmul_q8(golden["q8_matmul_qweights"], golden["q8_matmul_scales"], golden["q8_matmul_x"], kernel)
    err = np.abs(y - golden["q8_matmul_expected"]).max()
    assert err <= golden_mod.TOLERANCE_Q8


def test_golden_q4_expected_against_float64(golden):
    y64 = ops_ref.q4_matvec_f64(golden["q4_matmul_qweights"], golden["q4_matmul_scales"], golden["q4_matmul_x"])
    np.testing.assert_allclose(golden["q4_matmul_expected"], y64, rtol=0, atol=1e-4)


def test_decode_ops_golden(oracle, golden):
    tol = golden_mod.TOLERANCE_FP32
    y = oracle.rmsnorm(golden["rmsnorm_x"], golden["rmsnorm_weight"], float(golden["rmsnorm_eps"]))
    assert np.abs(y - golden["rmsnorm_expected"]).max() <= tol
    q, k = oracle.rope(golden["rope_q"], golden["rope_k"], 32, int(golden["rope_pos"]), 10000.0)
    assert max(np.abs(q - golden["rope_q_expected"]).max(), np.abs(k - golden["rope_k_expected"]).max()) <= tol
    y = oracle.softmax(golden["softmax_x"])
    assert np.abs(y - golden["softmax_expected"]).max() <= tol
    a = oracle.attention(golden["attention_q"], golden["attention_k"], golden["attention_v"], 1.0 / np.sqrt(16))
    assert np.abs(a - golden["attention_expected"]).max() <= tol


# ---- SIMD restatements against their per-lane models (bitwise) ----------------------

@pytest.mark.parametrize("M,K", [(1, 32), (7, 64), (33, 256), (64, 4096)])
def test_q4_avx2_equals_lane_model(oracle, M, K):
    rng = np.random.default_rng(M * 1000 + K)
    q, s = _rand_q4(rng, M, K)
    x = rng.standard_normal(K).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_q4(q, s, x, "avx2"), oracle.matmul_q4(q, s, x, "lanes"))
    np.testing.assert_array_equal(oracle.matmul_q4(q, s, x, "avx512"), oracle.matmul_q4(q, s, x, "avx512_lanes"))


@pytest.mark.parametrize("M,K", [(1, 32), (9, 128), (64, 4096)])
def test_q8_avx2_equals_lane_model(oracle, M, K):
    rng = np.random.default_rng(M + K)
    q, s = _rand_q8(rng, M, K)
    x = rng.standard_normal(K).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_q8(q, s, x, "avx2"), oracle.matmul_q8(q, s, x, "lanes"))


def test_avx2_and_avx512_orders_differ_but_agree(oracle):
    rng = np.random.default_rng(5)
    q, s = _rand_q4(rng, 256, 4096)
    x = rng.standard_normal(4096).astype(np.float32)
    a, b = oracle.matmul_q4(q, s, x, "avx2"), oracle.matmul_q4(q, s, x, "avx512")
    assert_matvec_close(a, b, ops_ref.dequantize_q4_0(q, s), x, rel=1e-6)


# ---- float64 closed forms -----------------------------------------------------------

@pytest.mark.parametrize("M,K", [(16, 4096), (8, 11008)])
def test_q4_against_float64(oracle, M, K):
    rng = np.random.default_rng(K)
    q, s = _rand_q4(rng, M, K)
    x = rng.standard_normal(K).astype(np.float32)
    y64 = ops_ref.q4_matvec_f64(q, s, x)
    for kern in ("avx2", "avx512"):
        assert_matvec_close(oracle.matmul_q4(q, s, x, kern), y64, ops_ref.dequantize_q4_0(q, s), x, rel=1e-6)


def test_q8_against_float64(oracle):
    rng = np.random.default_rng(8)
    q, s = _rand_q8(rng, 16, 4096)
    x = rng.standard_normal(4096).astype(np.float32)
    assert_matvec_close(oracle.matmul_q8(q, s, x), ops_ref.q8_matvec_f64(q, s, x), ops_ref.dequantize_q8_0(q, s), x,
                        rel=1e-6)


def test_closed_form_catches_swapped_nibbles(oracle):
    """A plausible mistake -- low/high nibble halves swapped -- must fail the bar."""
    rng = np.random.default_rng(11)
    q, s = _rand_q4(rng, 8, 256)
    x = rng.standard_normal(256).astype(np.float32)
    swapped = ((q & 0x0F) << 4) | (q >> 4)
    y_bad = oracle.matmul_q4(swapped, s, x)
    l1 = np.abs(ops_ref.dequantize_q4_0(q, s).astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert np.any(np.abs(y_bad - ops_ref.q4_matvec_f64(q, s, x)) > 1e-4 * l1)


# ---- exact special cases ---------------------------------------------------------------

def test_q4_all_eight_is_zero(oracle):
    q = np.full((5, 4, 16), 0x88, np.uint8)
    s = np.ones((5, 4), np.float32)
    x = np.random.default_rng(1).standard_normal(128).astype(np.float32)
    assert np.all(oracle.matmul_q4(q, s, x) == 0.0)


def test_q4_zero_scale_is_zero(oracle):
    rng = np.random.default_rng(2)
    q, _ = _rand_q4(rng, 5, 128)
    x = rng.standard_normal(128).astype(np.float32)
    assert np.all(oracle.matmul_q4(q, np.zeros((5, 4), np.float32), x) == 0.0)


@pytest.mark.parametrize("col", [0, 5, 16, 31, 63])
def test_q4_one_hot_picks_column(oracle, col):
    rng = np.random.default_rng(col)
    q, s = _rand_q4(rng, 6, 64)
    x = np.zeros(64, np.float32)
    x[col] = 1.0
    w = ops_ref.dequantize_q4_0(q, s)
    np.testing.assert_array_equal(oracle.matmul_q4(q, s, x), w[:, col])


@pytest.mark.parametrize("col", [0, 17, 40])
def test_q8_one_hot_picks_column(oracle, col):
    rng = np.random.default_rng(col)
    q, s = _rand_q8(rng, 6, 64)
    x = np.zeros(64, np.float32)
    x[col] = 1.0
    np.testing.assert_array_equal(oracle.matmul_q8(q, s, x), ops_ref.dequantize_q8_0(q, s)[:, col])


# ---- a4: threadpool tiling ------------------------------------------------------------

@pytest.mark.parametrize("M,nt,tile", [(4096, 4, 1024), (100, 3, 48), (33, 8, 16), (4096, 64, 64), (1000, 7, 144)])
def test_tile_rule(oracle, M, nt, tile):
    # threadpool.c:408-410: round_up(ceil(M/nt), 16)
    assert oracle.tile_rows(M, nt) == tile


@pytest.mark.parametrize("variant", [0, 1])
def test_q4_mt_bitwise_independent_of_threads(oracle, variant):
    rng = np.random.default_rng(3)
    q, s = _rand_q4(rng, 1000, 256)
    x = rng.standard_normal(256).astype(np.float32)
    ref = oracle.matmul_q4(q, s, x, "avx2" if variant == 0 else "avx512")
    for nt in (1, 2, 3, 4, 7, 8):
        np.testing.assert_array_equal(oracle.matmul_q4_mt(q, s, x, nt, variant), ref)
    assert oracle.threadpool_size() == 8


def test_q8_mt_bitwise_and_small_m_fallback(oracle):
    rng = np.random.default_rng(4)
    q, s = _rand_q8(rng, 300, 128)
    x = rng.standard_normal(128).astype(np.float32)
    ref = oracle.matmul_q8(q, s, x)
    for nt in (2, 5):
        np.testing.assert_array_equal(oracle.matmul_q8_mt(q, s, x, nt), ref)
    oracle.threadpool_init(3)
    y = oracle.matmul_q8_mt(q[:31], s[:31], x, 16)  # M < 32: single thread, pool untouched
    np.testing.assert_array_equal(y, ref[:31])
    assert oracle.threadpool_size() == 3


# ---- GGUF blocks, fp16, quantizers -------------------------------------------------------

def test_fp16_widen_matches_numpy_everywhere(oracle):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([oracle.f16_to_f32(int(v)) for v in h[::7]], np.float32)
    np.testing.assert_array_equal(got.view(np.uint32)[~np.isnan(got)], ref[::7].view(np.uint32)[~np.isnan(got)])


def test_fp16_narrow_matches_numpy(oracle):
    rng = np.random.default_rng(6)
    vals = np.concatenate([
        rng.standard_normal(3000).astype(np.float32) * 10.0 ** rng.integers(-9, 6, 3000),
        np.array([0.0, -0.0, 65504, 65519.99, 65520, 1e9, 2 ** -24, 2 ** -25, 3 * 2 ** -26, 6.1e-5], np.float32),
    ]).astype(np.float32)
    got = np.array([oracle.f32_to_f16(float(v)) for v in vals], np.uint16)
    with np.errstate(over="ignore"):
        ref = vals.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, ref)


def test_quantize_known_answers(oracle):
    with np.load(GOLDEN_DIR / "quant_known_answers.npz") as f:
        np.testing.assert_array_equal(oracle.quantize_q4_0(f["q4_w"]), f["q4_blocks"])
        np.testing.assert_array_equal(oracle.quantize_q8_0(f["q8_w"]), f["q8_blocks"])


def test_q4_gguf_equals_split_path(oracle):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((96, 256)) * 0.02).astype(np.float32)
    blocks = oracle.quantize_q4_0(w)
    qs, sc = oracle.split_q4_0(blocks)
    x = rng.standard_normal(256).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_q4_0_gguf(blocks, x), oracle.matmul_q4(qs, sc, x))
    np.testing.assert_array_equal(oracle.matmul_q4_0_gguf(blocks, x, nt=4), oracle.matmul_q4(qs, sc, x))
    np.testing.assert_array_equal(oracle.dequantize_q4_0(blocks), ops_ref.dequantize_q4_0(qs, sc))


def test_q8_gguf_equals_split_path(oracle):
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    blocks = oracle.quantize_q8_0(w)
    qs, sc = oracle.split_q8_0(blocks)
    x = rng.standard_normal(512).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_q8_0_gguf(blocks, x), oracle.matmul_q8(qs, sc, x))
    np.testing.assert_array_equal(oracle.dequantize_q8_0(blocks), ops_ref.dequantize_q8_0(qs, sc))


def test_quantizers_reconstruct_within_half_step(oracle):
    rng = np.random.default_rng(10)
    w = (rng.standard_normal((64, 512)) * 0.02).astype(np.float32)
    b4 = oracle.quantize_q4_0(w)
    _, s4 = oracle.split_q4_0(b4)
    # Q4_0 spans [-8d, 7d]: the element opposite the peak clamps from 8d to 7d,
    # so the bound is |d| (plus the fp16 rounding of d, at most 8 |d| 2^-11).
    err4 = np.abs(oracle.dequantize_q4_0(b4) - w).reshape(64, 16, 32).max(-1)
    assert np.all(err4 <= np.abs(s4) * (1 + 8 * 2 ** -11) + 1e-12)
    b8 = oracle.quantize_q8_0(w)
    _, s8 = oracle.split_q8_0(b8)
    # half a step, plus |q| <= 127 times the fp16 rounding of d
    err8 = np.abs(oracle.dequantize_q8_0(b8) - w).reshape(64, 16, 32).max(-1)
    assert np.all(err8 <= np.abs(s8) * (0.5 + 127 * 2 ** -11) + 1e-12)


# ---- a8: GEMM recipe ---------------------------------------------------------------------

def test_gemm_against_exact_integer_form(oracle):
    rng = np.random.default_rng(12)
    T, M, K = 5, 7, 256
    wb = oracle.quantize_q8_0((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    ab = oracle.quantize_q8_0(rng.standard_normal((T, K)).astype(np.float32))
    c = oracle.gemm_q8_0(wb, ab)
    wq, ws = oracle.split_q8_0(wb)
    aq, as_ = oracle.split_q8_0(ab)
    idot = np.einsum("mbj,tbj->tmb", wq.astype(np.int64), aq.astype(np.int64))
    exact = (idot.astype(np.float64) * ws[None].astype(np.float64) * as_[:, None].astype(np.float64)).sum(-1)
    l1 = np.abs(oracle.dequantize_q8_0(ab).astype(np.float64)) @ np.abs(oracle.dequantize_q8_0(wb).astype(np.float64)).T
    assert np.all(np.abs(c - exact) <= 1e-6 * l1 + 1e-30)
    np.testing.assert_array_equal(oracle.gemm_q8_0(wb, ab, nt=3), c)


def test_gemm_split_equals_block_form_on_widened_scales(oracle):
    """With scales widened from the blocks' fp16 d, the split-operand GEMM is the
    block-form GEMM bit for bit (the same products, roundings and order)."""
    rng = np.random.default_rng(15)
    T, M, K = 9, 13, 320
    wb = oracle.quantize_q8_0((rng.standard_normal((M, K)) * 0.02).astype(np.float32))
    ab = oracle.quantize_q8_0(rng.standard_normal((T, K)).astype(np.float32))
    wq, ws = oracle.split_q8_0(wb)
    aq, as_ = oracle.split_q8_0(ab)
    c = oracle.gemm_q8_split(wq, ws, aq, as_)
    np.testing.assert_array_equal(c, oracle.gemm_q8_0(wb, ab))
    np.testing.assert_array_equal(oracle.gemm_q8_split(wq, ws, aq, as_, nt=4), c)


def _round_f32(fr):
    """The fp32 value nearest the rational fr, ties to even (no double rounding)."""
    from fractions import Fraction

    f = np.float32(float(fr))
    cands = [np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf))]
    return min(cands, key=lambda v: (abs(Fraction(float(v)) - fr), int(np.float32(v).view(np.uint32)) & 1))


def _gemm_split_exact_steps(wq, ws, aq, as_):
    """Brute force in exact rationals: per block the fp32 product of the two
    scales, then acc = round_f32(dot * scale + acc) in block order."""
    from fractions import Fraction

    T, M, nb = aq.shape[0], wq.shape[0], ws.shape[1]
    c = np.zeros((T, M), np.float32)
    for t in range(T):
        for j in range(M):
            acc = np.float32(0)
            for b in range(nb):
                dot = int(np.dot(aq[t, b].astype(np.int64), wq[j, b].astype(np.int64)))
                sc = _round_f32(Fraction(float(ws[j, b])) * Fraction(float(as_[t, b])))
                acc = _round_f32(Fraction(dot) * Fraction(float(sc)) + Fraction(float(acc)))
            c[t, j] = acc
    return c


def test_gemm_split_matches_exact_rounding_brute_force(oracle):
    """Arbitrary fp32 scales (U(0.5, 1.5) as the reference's tests draw them, and
    wide exponents): every output equals the exact-rational evaluation of the
    recipe's roundings; a plausible slip, the scales of one block taken from the
    next, fails the same comparison."""
    rng = np.random.default_rng(16)
    T, M, nb = 3, 5, 4
    wq = rng.integers(-128, 128, (M, nb, 32)).astype(np.int8)
    aq = rng.integers(-128, 128, (T, nb, 32)).astype(np.int8)
    ws = rng.uniform(0.5, 1.5, (M, nb)).astype(np.float32)
    as_ = (rng.uniform(0.5, 1.5, (T, nb)) * 2.0 ** rng.integers(-40, 40, (T, nb))).astype(np.float32)
    exact = _gemm_split_exact_steps(wq, ws, aq, as_)
    np.testing.assert_array_equal(oracle.gemm_q8_split(wq, ws, aq, as_), exact)
    slipped = oracle.gemm_q8_split(wq, np.roll(ws, 1, axis=1), aq, as_)
    assert not np.array_equal(slipped, exact)


# ---- decode attention over fp16 KV -----------------------------------------------------------

def test_attention_decode_f16_against_numpy(oracle):
    rng = np.random.default_rng(13)
    n_heads, n_kv, hd, n_pos, max_pos = 8, 2, 64, 37, 40
    q = rng.standard_normal((n_heads, hd)).astype(np.float32)
    kc = rng.standard_normal((max_pos, n_kv, hd)).astype(np.float16)
    vc = rng.standard_normal((max_pos, n_kv, hd)).astype(np.float16)
    got = oracle.attention_decode_f16(q, kc.view(np.uint16), vc.view(np.uint16), n_pos, n_kv)
    got_mt = oracle.attention_decode_f16(q, kc.view(np.uint16), vc.view(np.uint16), n_pos, n_kv, nt=4)
    np.testing.assert_array_equal(got, got_mt)
    for h in range(n_heads):
        kv = h // (n_heads // n_kv)
        k = kc[:n_pos, kv].astype(np.float64)
        v = vc[:n_pos, kv].astype(np.float64)
        s = k @ q[h].astype(np.float64) / np.sqrt(hd)
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ v
        np.testing.assert_allclose(got[h], ref, rtol=0, atol=1e-6)


# ---- Q5_0 (matmul_q5_avx2.asm, ops.py:67-99, threadpool.c:667-787) -------------------------

def _rand_q5(rng, M, K):
    ql = rng.integers(0, 256, size=(M, K // 32, 16), dtype=np.uint8)
    qh = rng.integers(0, 256, size=(M, K // 32, 4), dtype=np.uint8)
    s = rng.uniform(0.05, 0.25, size=(M, K // 32)).astype(np.float32)
    return ql, qh, s


@pytest.mark.parametrize("kernel", ["avx2", "lanes"])
def test_q5_golden(oracle, golden, kernel):
    y = oracle.matmul_q5(golden["q5_matmul_ql"], golden["q5_matmul_qh"], golden["q5_matmul_scales"],
                         golden["q5_matmul_x"], kernel)
    err = np.abs(y - golden["q5_matmul_expected"]).max()
    assert err <= golden_mod.TOLERANCE_Q5
    assert err <= 1e-4  # fp32 reassociation only


def test_golden_q5_expected_against_float64(golden):
    y64 = ops_ref.q5_matvec_f64(golden["q5_matmul_ql"], golden["q5_matmul_qh"], golden["q5_matmul_scales"],
                                golden["q5_matmul_x"])
    np.testing.assert_allclose(golden["q5_matmul_expected"], y64, rtol=0, atol=1e-4)


def test_q5_dequant_known_answers():
    # Block 0: ql byte j = j (low nibble j, high nibble 0); qh = 0x0000FFFF, so
    # weights 0..15 get their fifth bit (j + 16 - 16 = j) and 16..31 do not (0 - 16).
    ql = np.zeros((1, 2, 16), np.uint8)
    qh = np.zeros((1, 2, 4), np.uint8)
    ql[0, 0] = np.arange(16)
    qh[0, 0] = [0xFF, 0xFF, 0x00, 0x00]
    # Block 1: ql byte j = 0xF0 | 0x0F (both nibbles 15); qh = 0x80000001: weight 0
    # (15 + 16 - 16 = 15) and weight 31 (15) high, the rest 15 - 16 = -1.
    ql[0, 1] = 0xFF
    qh[0, 1] = [0x01, 0x00, 0x00, 0x80]
    s = np.array([[1.0, 0.5]], np.float32)
    w = ops_ref.dequantize_q5_0(ql, qh, s)
    expect0 = list(range(16)) + [-16] * 16
    expect1 = [15] + [-1] * 30 + [15]
    np.testing.assert_array_equal(w[0, :32], np.array(expect0, np.float32))
    np.testing.assert_array_equal(w[0, 32:], np.array(expect1, np.float32) * np.float32(0.5))


@pytest.mark.parametrize("M,K", [(1, 32), (7, 64), (33, 256), (64, 4096)])
def test_q5_avx2_equals_lane_model(oracle, M, K):
    rng = np.random.default_rng(M * 7 + K)
    ql, qh, s = _rand_q5(rng, M, K)
    x = rng.standard_normal(K).astype(np.float32)
    np.testing.assert_array_equal(oracle.matmul_q5(ql, qh, s, x, "avx2"), oracle.matmul_q5(ql, qh, s, x, "lanes"))


@pytest.mark.parametrize("M,K", [(16, 4096), (8, 11008)])
def test_q5_against_float64(oracle, M, K):
    rng = np.random.default_rng(K + 5)
    ql, qh, s = _rand_q5(rng, M, K)
    x = rng.standard_normal(K).astype(np.float32)
    assert_matvec_close(oracle.matmul_q5(ql, qh, s, x), ops_ref.q5_matvec_f64(ql, qh, s, x),
                        ops_ref.dequantize_q5_0(ql, qh, s), x, rel=1e-6)


@pytest.mark.parametrize("mistake", ["bit_order_reversed", "high_bits_from_low_half", "offset_8"])
def test_q5_closed_form_catches_plausible_mistakes(oracle, mistake):
    """Inputs that model a plausible misreading of the format must fail the bar."""
    rng = np.random.default_rng(14)
    ql, qh, s = _rand_q5(rng, 8, 256)
    x = rng.standard_normal(256).astype(np.float32)
    y64 = ops_ref.q5_matvec_f64(ql, qh, s, x)
    l1 = ops_ref.row_l1(ops_ref.dequantize_q5_0(ql, qh, s), x)
    if mistake == "bit_order_reversed":  # bit 7 - j % 8 instead of bit j % 8
        reversed_bits = np.packbits(np.unpackbits(qh, axis=-1, bitorder="little"), axis=-1, bitorder="big")
        bad = oracle.matmul_q5(ql, reversed_bits, s, x)
    elif mistake == "high_bits_from_low_half":  # weights 16..31 reuse bits 0..15
        qh2 = qh.copy()
        qh2[..., 2:] = qh[..., :2]
        bad = oracle.matmul_q5(ql, qh2, s, x)
    else:  # (n | h << 4) - 8: the Q4 offset
        bad = oracle.matmul_q5(ql, qh, s, x) + 8.0 * (s.astype(np.float64) * x.astype(np.float64).reshape(-1, 32)
                                                      .sum(-1)).sum(-1)
    assert np.any(np.abs(bad - y64) > 1e-4 * l1)


def test_q5_special_cases(oracle):
    rng = np.random.default_rng(15)
    ql, qh, s = _rand_q5(rng, 6, 128)
    x = rng.standard_normal(128).astype(np.float32)
    # every weight 16: all nibbles 0 with the fifth bit set -> exactly zero
    assert np.all(oracle.matmul_q5(np.zeros_like(ql), np.full_like(qh, 0xFF), s, x) == 0.0)
    assert np.all(oracle.matmul_q5(ql, qh, np.zeros_like(s), x) == 0.0)
    w = ops_ref.dequantize_q5_0(ql, qh, s)
    for col in (0, 15, 16, 31, 32, 100):
        e = np.zeros(128, np.float32)
        e[col] = 1.0
        np.testing.assert_array_equal(oracle.matmul_q5(ql, qh, s, e), w[:, col])


def test_q5_mt_bitwise_and_small_m_fallback(oracle):
    rng = np.random.default_rng(16)
    ql, qh, s = _rand_q5(rng, 700, 256)
    x = rng.standard_normal(256).astype(np.float32)
    ref = oracle.matmul_q5(ql, qh, s, x)
    for nt in (2, 4, 7):
        np.testing.assert_array_equal(oracle.matmul_q5_mt(ql, qh, s, x, nt), ref)
    oracle.threadpool_init(3)
    np.testing.assert_array_equal(oracle.matmul_q5_mt(ql[:20], qh[:20], s[:20], x, 8), ref[:20])
    assert oracle.threadpool_size() == 3


def test_q5_gguf_equals_split_path(oracle):
    from asmllm_amd import gguf

    rng = np.random.default_rng(17)
    ql, qh, _ = _rand_q5(rng, 40, 320)
    d = (rng.standard_normal((40, 10)) * 0.01).astype(np.float16)
    blocks = gguf.pack_q5_0(ql, qh, d)
    l2, h2, sc = oracle.split_q5_0(blocks)
    np.testing.assert_array_equal(l2, ql)
    np.testing.assert_array_equal(h2, qh)
    np.testing.assert_array_equal(sc, d.astype(np.float32))
    for a, b in zip(gguf.split_q5_0(blocks), (ql, qh, d.astype(np.float32))):
        np.testing.assert_array_equal(a, b)
    x = rng.standard_normal(320).astype(np.float32)
    ref = oracle.matmul_q5(ql, qh, sc, x)
    np.testing.assert_array_equal(oracle.matmul_q5_0_gguf(blocks, x), ref)
    np.testing.assert_array_equal(oracle.matmul_q5_0_gguf(blocks, x, nt=4), ref)
    w = ops_ref.dequantize_q5_0(ql, qh, sc)
    np.testing.assert_array_equal(oracle.dequantize_q5_0(blocks), w)
    np.testing.assert_array_equal(gguf.dequantize_q5_0(blocks), w)


# ---- SiLU . up (swiglu_avx2.asm:45-81) against the mathematics ----------------------------

_ULP = 2.0 ** -23


def _silu_pins(fn) -> list[str]:
    """Every check of silu(g) * u that the mathematics fixes, run on `fn(gate, up)`;
    returns the names of the checks that fail (empty: pinned)."""
    failed = []
    f32 = np.float32
    # silu(0) = 0 exactly, whatever u is
    u = np.array([1.0, -3.5, 7.25, 1e30], f32)
    if not np.all(fn(np.zeros(4, f32), u) == 0.0):
        failed.append("silu(0) = 0")
    # g = ln 3: 1 + e^-g = 4/3, so silu(g) u = 0.75 g u (to the rounding of the fp32 steps)
    g = np.full(3, np.log(3.0), f32)
    u = np.array([1.0, 2.0, -0.5], f32)
    want = 0.75 * g.astype(np.float64) * u
    if not np.all(np.abs(fn(g, u) - want) <= 4 * _ULP * np.abs(want)):
        failed.append("silu(ln 3) = 0.75 ln 3")
    # silu(g) - silu(-g) = g sigma(g) + g sigma(-g) = g, over a sweep of g (u = 1)
    gs = np.concatenate([np.linspace(-30, 30, 4001), np.geomspace(1e-6, 1e3, 200)]).astype(f32)
    ones = np.ones_like(gs)
    pos, neg = fn(gs, ones).astype(np.float64), fn(-gs, ones).astype(np.float64)
    if not np.all(np.abs((pos - neg) - gs) <= 4 * _ULP * (np.abs(pos) + np.abs(neg)) + 1e-45):
        failed.append("silu(g) - silu(-g) = g")
    # large |g|: e^-g vanishes next to 1, so silu(g) u = g u exactly; the negative side is
    # g e^g to fp32 rounding, and past the fp32 range of 1 + e^-g (g < -88.7) the rounded
    # denominator is infinite and the result a signed zero, as in the reference's fstp dword
    big = np.array([20.0, 50.0, 88.0, 1e4], f32)
    u = np.array([1.5, -2.0, 0.25, 3.0], f32)
    if not np.array_equal(fn(big, u), big * u):
        failed.append("silu(g) = g for large g")
    gneg = np.array([-20.0, -50.0, -80.0], f32)
    want = gneg.astype(np.float64) / (1.0 + np.exp(-gneg.astype(np.float64)))
    if not np.all(np.abs(fn(gneg, np.ones(3, f32)) - want) <= 4 * _ULP * np.abs(want)):
        failed.append("silu(g) = g e^g for large -g")
    if not np.all(fn(np.array([-100.0, -1e4], f32), np.array([2.0, 1.0], f32)) == 0.0):
        failed.append("silu(g) = 0 where 1 + e^-g overflows fp32")
    # a float64 closed form over random g, u (three fp32 roundings: 1 + e^-g, /, *)
    rng = np.random.default_rng(11)
    g = (rng.standard_normal(20000) * 6).astype(f32)
    u = rng.standard_normal(20000).astype(f32)
    g64 = g.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u
    if not np.all(np.abs(fn(g, u) - want) <= 4 * _ULP * np.abs(want) + 1e-44):
        failed.append("float64 closed form")
    return failed


def test_silu_hadamard_pinned_by_the_mathematics(oracle):
    assert _silu_pins(oracle.silu_hadamard) == []


def test_silu_hadamard_agrees_with_the_python_reference_formula(oracle):
    """generate.py:370's numpy form (ops_ref.silu_hadamard) in fp32, within the rounding of
    the two fp32 evaluations of exp."""
    rng = np.random.default_rng(12)
    g = (rng.standard_normal(5000) * 8).astype(np.float32)
    u = rng.standard_normal(5000).astype(np.float32)
    with np.errstate(over="ignore"):
        ref = ops_ref.silu_hadamard(g, u).astype(np.float64)
    got = oracle.silu_hadamard(g, u).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 8 * _ULP * np.abs(ref) + 1e-44)


@pytest.mark.parametrize("mistake", ["exp(+g)", "g * (1 + exp(-g))", "sigmoid only", "up ignored"])
def test_silu_pins_catch_plausible_mistakes(mistake):
    """The checks above reject each plausible slip, so passing them means something."""
    def mutant(gate, up):
        g = gate.astype(np.float64)
        if mistake == "exp(+g)":
            r = g / (1.0 + np.exp(g))
        elif mistake == "g * (1 + exp(-g))":
            r = g * (1.0 + np.exp(-g))
        elif mistake == "sigmoid only":
            r = 1.0 / (1.0 + np.exp(-g))
        else:
            return (g / (1.0 + np.exp(-g))).astype(np.float32)
        return (r * up).astype(np.float32)

    with np.errstate(over="ignore", invalid="ignore"):
        assert _silu_pins(mutant) != []
