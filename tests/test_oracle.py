"""Pins the CPU oracle before it is trusted as the checker.

Each oracle function is checked against something that does not restate its own
formula: numpy's IEEE binary16 conversion; the published GGML dequantisation
algorithm (dequantize_row_q4_K / dequantize_row_q6_K, the algorithm of the
reference's oracle dependency `gguf`, pyproject.toml:12, gguf>=0.17, absent here)
written in its own 64-/128-value loop structure; hand-built known-answer blocks;
numpy float64 matmul; scipy's softmax; complex multiplication for RoPE; and
algebraic identities (split-K merge, constant values, single position).
"""
import numpy as np
import pytest
from scipy.special import softmax

import oracle as orc
from ggml_ref import ggml_q4k, ggml_q6k
from known_answers import known_answer_fields
from rta import synth


# ---------------------------------------------------------------- binary16 ----
def test_half_to_float_all_codes():
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_half_to_float(int(c)) for c in codes], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_float_to_half_round_nearest_even():
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e-8, 5.96e-8, 2.98e-8, 6.1e-5, np.inf, -np.inf],
                 dtype=np.float32)]).astype(np.float32)
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.lib().orc_float_to_half(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


def _bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q4k_dequant_matches_ggml_bitwise(seed):
    raw = synth.random_q4k(np.random.default_rng(seed), 24)
    got = orc.dequant(orc.Q4_K, raw, 24 * 256)
    assert np.array_equal(_bits(got), _bits(ggml_q4k(raw)))


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_q6k_dequant_matches_ggml_bitwise(seed):
    raw = synth.random_q6k(np.random.default_rng(seed), 24)
    got = orc.dequant(orc.Q6_K, raw, 24 * 256)
    assert np.array_equal(_bits(got), _bits(ggml_q6k(raw)))


def test_q4k_known_answers():
    n = 1
    q = (np.arange(256) * 7 % 16).astype(np.uint8)[None]
    # d = dmin = 0 -> all zeros
    raw = synth.pack_q4k(np.zeros(n), np.zeros(n), np.full((n, 8), 63), np.full((n, 8), 63), q)
    assert not orc.dequant(orc.Q4_K, raw, 256).any()
    # d = 1, sc = 1, m = 0 -> the quant itself
    raw = synth.pack_q4k(np.ones(n), np.ones(n), np.ones((n, 8)), np.zeros((n, 8)), q)
    assert np.array_equal(orc.dequant(orc.Q4_K, raw, 256), q[0].astype(np.float32))
    # every 6-bit code in every group position, across the g<4 / g>=4 packing split
    for code in range(64):
        for g in range(8):
            sc = np.zeros((1, 8), np.uint8)
            mn = np.zeros((1, 8), np.uint8)
            sc[0, g] = code
            mn[0, 7 - g] = 63 - code
            qq = np.ones((1, 256), np.uint8)
            raw = synth.pack_q4k(np.ones(1), np.full(1, 0.5), sc, mn, qq)
            v = orc.dequant(orc.Q4_K, raw, 256).reshape(8, 32)
            expect = np.array([(code if gg == g else 0) - 0.5 * ((63 - code) if gg == 7 - g else 0)
                               for gg in range(8)], dtype=np.float32)
            assert np.array_equal(v, np.repeat(expect[:, None], 32, 1)), (code, g)


def test_q6k_known_answers():
    q = (np.arange(256) % 64).astype(np.uint8)[None]
    raw = synth.pack_q6k(np.ones(1), np.ones((1, 16), np.int8), q)
    assert np.array_equal(orc.dequant(orc.Q6_K, raw, 256), q[0].astype(np.float32) - 32)
    sc = np.arange(-8, 8, dtype=np.int8)[None]  # negative int8 scales
    raw = synth.pack_q6k(np.full(1, 0.25), sc, q)
    expect = 0.25 * np.repeat(sc[0].astype(np.float32), 16) * (q[0].astype(np.float32) - 32)
    assert np.array_equal(orc.dequant(orc.Q6_K, raw, 256), expect.astype(np.float32))


def test_plain_formats():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(256).astype(np.float32)
    assert np.array_equal(orc.dequant(orc.F32, v.view(np.uint8), 256), v)
    h = v.astype(np.float16)
    assert np.array_equal(orc.dequant(orc.F16, h.view(np.uint8), 256), h.astype(np.float32))
    bf = (v.view(np.uint32) >> 16).astype(np.uint16)
    expect = (bf.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(orc.dequant(orc.BF16, bf.view(np.uint8), 256), expect)


def test_golden_fixtures():
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "dequant_golden.npz")
    assert np.array_equal(_bits(orc.dequant(orc.Q4_K, g["q4k_raw"], g["q4k_values"].size)), _bits(g["q4k_values"]))
    assert np.array_equal(_bits(orc.dequant(orc.Q6_K, g["q6k_raw"], g["q6k_values"].size)), _bits(g["q6k_values"]))


# --------------------------------------------------------------------- GEMV ----
@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
def test_gemv_matches_numpy_matmul(fmt):
    rng = np.random.default_rng(4)
    rows, cols = 48, 512
    w = synth.random_matrix(rng, fmt, rows, cols)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    dense = orc.dequant(fmt, w, rows * cols).reshape(rows, cols).astype(np.float64)
    ref = x.astype(np.float64) @ dense.T
    got = orc.gemv_f64(fmt, w, rows, cols, x)
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-12)
    got32 = orc.gemv_f32(fmt, w, rows, cols, x)
    assert np.allclose(got32, ref, rtol=1e-4, atol=1e-4)


def test_gemv_integer_exact():
    # d = 1, sc = 1, m = 0 and integer x: the contraction is an exact integer
    rng = np.random.default_rng(5)
    rows, cols = 8, 256
    q = rng.integers(0, 16, (rows, 256), dtype=np.uint8)
    w = synth.pack_q4k(np.ones(rows), np.zeros(rows), np.ones((rows, 8)), np.zeros((rows, 8)), q)
    x = rng.integers(-5, 6, (1, cols)).astype(np.float32)
    got = orc.gemv_f64(orc.Q4_K, w, rows, cols, x)
    assert np.array_equal(got[0], q.astype(np.int64) @ x[0].astype(np.int64))


# ---------------------------------------------------------------------- MLP ----
def test_mlp_closed_form():
    rng = np.random.default_rng(6)
    hidden, inter = 256, 512
    wg = synth.random_matrix(rng, orc.Q4_K, inter, hidden)
    wu = synth.random_matrix(rng, orc.Q4_K, inter, hidden)
    wd = synth.random_matrix(rng, orc.Q6_K, hidden, inter)
    x = rng.standard_normal((4, hidden)).astype(np.float32)
    x[1] = 0.0                       # zero row (verify_rt_mlp.py:64-67)
    x[2] = -x[0]
    act, y = orc.mlp_swiglu((orc.Q4_K, orc.Q4_K, orc.Q6_K), wg, wu, wd, hidden, inter, x)
    G = orc.dequant(orc.Q4_K, wg, inter * hidden).reshape(inter, hidden).astype(np.float64)
    U = orc.dequant(orc.Q4_K, wu, inter * hidden).reshape(inter, hidden).astype(np.float64)
    D = orc.dequant(orc.Q6_K, wd, hidden * inter).reshape(hidden, inter).astype(np.float64)
    g, u = x @ G.T, x @ U.T
    silu = g / (1.0 + np.exp(-g))
    assert np.allclose(act, silu * u, rtol=1e-12, atol=1e-15)
    assert not act[1].any() and not y[1].any()
    assert np.allclose(y, act.astype(np.float32).astype(np.float64) @ D.T, rtol=1e-12, atol=1e-12)
    act1, y1 = orc.mlp_swiglu((orc.Q4_K, orc.Q4_K, orc.Q6_K), wg, wu, wd, hidden, inter, x[:1])
    assert np.array_equal(act1[0], act[0]) and np.array_equal(y1[0], y[0])   # batch-prefix invariance


# ------------------------------------------------------------------- argmax ----
def test_argmax_margin_rule():
    a = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    assert orc.argmax_margin_f32(a, 0.0) == 1                  # exact tie -> lowest id
    b = np.array([0.0, 0.99995, 1.0], np.float32)
    assert orc.argmax_margin_f32(b, 1e-4) == 1                 # within 1e-4 relative
    assert orc.argmax_margin_f32(b, 0.0) == 2
    c = np.array([-2.0, -1.00005, -1.0], np.float32)
    assert orc.argmax_margin_f32(c, 1e-4) == 1                 # |M| for negative maxima
    d = np.array([np.nan, 5.0, np.nan], np.float32)
    assert orc.argmax_margin_f32(d, 1e-4) == 1
    rng = np.random.default_rng(7)
    for _ in range(50):
        v = rng.standard_normal(1000).astype(np.float32)
        assert orc.argmax_margin_f32(v, 0.0) == int(np.argmax(v))
        assert orc.argmax_margin_f64(v.astype(np.float64), 0.0) == int(np.argmax(v))


def test_lm_head_planted_winner():
    rng = np.random.default_rng(8)
    vocab, hidden = 300, 256
    w = synth.random_matrix(rng, orc.Q6_K, vocab, hidden)
    h = rng.standard_normal((2, hidden)).astype(np.float32)
    logits, ids = orc.lm_head(orc.Q6_K, w, vocab, hidden, h)
    dense = orc.dequant(orc.Q6_K, w, vocab * hidden).reshape(vocab, hidden).astype(np.float64)
    assert np.allclose(logits, h.astype(np.float64) @ dense.T, rtol=1e-12, atol=1e-12)
    assert list(ids) == [int(np.argmax(l)) for l in logits]


# -------------------------------------------------------------------- RoPE ----
def test_rope_matches_complex_rotation():
    rng = np.random.default_rng(9)
    heads, hd, theta = 3, 128, 1e6
    v = rng.standard_normal((heads, hd)).astype(np.float32)
    for t in (0, 1, 17, 32767):
        got = orc.rope(v, t, theta=theta)
        z = v[:, 0::2].astype(np.float64) + 1j * v[:, 1::2].astype(np.float64)
        ang = t * theta ** (-np.arange(hd // 2) / (hd // 2))
        r = z * np.exp(1j * ang)
        ref = np.stack([r.real, r.imag], -1).reshape(heads, hd).astype(np.float32)
        assert np.allclose(got, ref, rtol=1e-6, atol=1e-6)
        if t == 0:
            assert np.array_equal(got, v)
    part = orc.rope(v, 5, rotary=64, theta=theta)            # pairs >= rotary/2 untouched
    assert np.array_equal(part[:, 64:], v[:, 64:])


# --------------------------------------------------------------- attention ----
def _history(rng, n, hkv, hd, fmt_k, fmt_v):
    return synth.random_packets(rng, n, hkv * hd, fmt_k, fmt_v)


def _dense_reference(q, packets, fmt_k, fmt_v, L, hkv, hd):
    kvw = hkv * hd
    K = np.stack([[orc.lib().orc_packet_value(p.ctypes.data, kvw, fmt_k, fmt_v, 0, c) for c in range(kvw)]
                  for p in packets[:L]]).reshape(L, hkv, hd).astype(np.float64)
    V = np.stack([[orc.lib().orc_packet_value(p.ctypes.data, kvw, fmt_k, fmt_v, 1, c) for c in range(kvw)]
                  for p in packets[:L]]).reshape(L, hkv, hd).astype(np.float64)
    hq = q.shape[0]
    mapping = np.arange(hq) // (hq // hkv)
    s = np.einsum("hd,nhd->hn", q.astype(np.float64), K[:, mapping]) / np.sqrt(hd)
    w = softmax(s, axis=1)
    return np.einsum("hn,nhd->hd", w, V[:, mapping]), s.max(1), np.exp(s - s.max(1, keepdims=True)).sum(1)


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
def test_attention_matches_scipy_softmax(fmts):
    rng = np.random.default_rng(10)
    hq, hkv, hd, L = 8, 2, 128, 37
    packets = _history(rng, L, hkv, hd, *fmts)
    q = rng.standard_normal((1, hq, hd)).astype(np.float32)
    out, m, z = orc.decode_attention(q, packets, fmts[0], fmts[1], [0], [L], 1 << 20, hkv)
    ref, rm, rz = _dense_reference(q[0], packets, fmts[0], fmts[1], L, hkv, hd)
    assert np.allclose(out[0], ref, rtol=1e-10, atol=1e-12)
    assert np.allclose(m[0], rm) and np.allclose(z[0], rz)


def test_attention_identities():
    rng = np.random.default_rng(11)
    hq, hkv, hd = 4, 1, 128
    one = _history(rng, 1, hkv, hd, orc.Q4_K, orc.Q6_K)
    const = np.repeat(one, 9, axis=0)
    q = rng.standard_normal((1, hq, hd)).astype(np.float32)
    v0 = np.array([orc.lib().orc_packet_value(one[0].ctypes.data, hd, orc.Q4_K, orc.Q6_K, 1, c) for c in range(hd)])
    out, m, z = orc.decode_attention(q, one, orc.Q4_K, orc.Q6_K, [0], [1], 64, hkv)
    assert np.allclose(out[0], v0[None], rtol=1e-12) and np.allclose(z, 1.0)       # one position -> V0
    out, m, z = orc.decode_attention(q, const, orc.Q4_K, orc.Q6_K, [0], [9], 64, hkv)
    assert np.allclose(out[0], v0[None], rtol=1e-12) and np.allclose(z, 9.0)       # constant V -> V
    hist = _history(rng, 20, hkv, hd, orc.Q4_K, orc.Q6_K)
    zq = np.zeros((1, hq, hd), np.float32)
    out, m, z = orc.decode_attention(zq, hist, orc.Q4_K, orc.Q6_K, [0], [20], 64, hkv)
    V = np.array([[orc.lib().orc_packet_value(p.ctypes.data, hd, orc.Q4_K, orc.Q6_K, 1, c) for c in range(hd)]
                  for p in hist])
    assert np.allclose(out[0], V.mean(0)[None], rtol=1e-10)                        # zero q -> uniform
    assert np.allclose(z, 20.0) and np.allclose(m, 0.0)


def test_attention_split_merge_identity():
    # The split-K merge (resident_attention_runtime.inl:618-645; paper eq. 46):
    # two halves combined with M = max, Z = sum Z_i e^(m_i - M) equal the whole.
    rng = np.random.default_rng(12)
    hq, hkv, hd, L = 4, 1, 128, 50
    hist = _history(rng, L, hkv, hd, orc.Q4_K, orc.Q6_K)
    q = rng.standard_normal((1, hq, hd)).astype(np.float32)
    full, mf, zf = orc.decode_attention(q, hist, orc.Q4_K, orc.Q6_K, [0], [L], 1 << 20, hkv)
    # positions 20..49 in a ring of capacity 30 (slot = p % 30); the query at t = 49
    # sees exactly them.  Positions 0..19 are the other half.
    a, ma, za = orc.decode_attention(q, hist[:20], orc.Q4_K, orc.Q6_K, [0], [20], 1 << 20, hkv)
    ring = np.empty((30, hist.shape[1]), np.uint8)
    for p in range(20, L):
        ring[p % 30] = hist[p]
    b, mb, zb = orc.decode_attention(q, ring, orc.Q4_K, orc.Q6_K, [0], [L], 30, hkv)
    M = np.maximum(ma, mb)
    Z = za * np.exp(ma - M) + zb * np.exp(mb - M)
    merged = (a * (za * np.exp(ma - M))[..., None] + b * (zb * np.exp(mb - M))[..., None]) / Z[..., None]
    assert np.allclose(merged, full, rtol=1e-10, atol=1e-12)
    assert np.allclose(M, mf) and np.allclose(Z, zf)


# ------------------------------------------------------------------ packer ----
@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
def test_packer_round_trip(fmts):
    rng = np.random.default_rng(13)
    kvw = 512
    k = rng.normal(0, 0.25, kvw).astype(np.float32)
    v = rng.normal(0, 0.5, kvw).astype(np.float32)
    pk = orc.pack_history(k, v, *fmts)
    assert pk.size == 712
    kk = np.array([orc.lib().orc_packet_value(pk.ctypes.data, kvw, fmts[0], fmts[1], 0, c) for c in range(kvw)])
    vv = np.array([orc.lib().orc_packet_value(pk.ctypes.data, kvw, fmts[0], fmts[1], 1, c) for c in range(kvw)])
    # error within one quantisation step of each field's 16/32-value group
    for field, dec in ((k, kk), (v, vv)):
        step = np.abs(field).max() / 7.0
        assert np.max(np.abs(dec - field)) <= step, np.max(np.abs(dec - field))
    assert not pk[708:].any()                                  # 4 pad bytes stay zero


def test_packer_known_answer_bytes():
    """Packet bytes equal the hand-built GGUF blocks: d / dmin from /63 and /127 (a /64 or
    /128 changes the binary16 bytes), scale code 127 kept (no 63 clamp on Q6_K), codes
    rounded to nearest (not truncated), .5 ties to even, and the pad bytes zero."""
    k, v, expected = known_answer_fields()
    got = orc.pack_history(k, v, orc.Q4_K, orc.Q6_K)
    assert got.size == expected.size == 360
    diff = np.nonzero(got != expected)[0]
    assert diff.size == 0, f"bytes differ at {diff[:16]}"
    # the swapped field order puts V's Q6_K block first and K's Q4_K block second
    sw = orc.pack_history(v, k, orc.Q6_K, orc.Q4_K)
    assert np.array_equal(sw[:210], expected[144:354]) and np.array_equal(sw[210:354], expected[:144])


def test_packer_one_signed_groups_known_answer_bytes():
    """Q4_K groups entirely above or below zero keep lo / hi started at 0
    (resident_history_quant.glsl:14-15): all-positive groups get minimum code 0 and the span
    [0, max], all-negative ones the span [min, 0].  A packer taking the true group min / max
    changes the scale and minimum codes and fails."""
    from known_answers import one_signed_fields
    k, v, expected = one_signed_fields()
    got = orc.pack_history(k, v, orc.Q4_K, orc.Q6_K)
    diff = np.nonzero(got != expected)[0]
    assert diff.size == 0, f"bytes differ at {diff[:16]}"
    sw = orc.pack_history(v, k, orc.Q6_K, orc.Q4_K)
    assert np.array_equal(sw[:210], expected[144:354]) and np.array_equal(sw[210:354], expected[:144])


def test_packer_rounds_d_to_binary16_before_the_codes():
    """The block scale is rounded to binary16 before the group codes are formed
    (resident_history_quant.glsl:22 then :27): group ranges 1.0 and 0.5 give
    maxD / 63 = 0.0010582 -> binary16 0.00105857849, so the second group's code is
    round(0.5/15 / 0.00105857849) = round(31.489) = 31 (with the unrounded scale it
    would be round(31.500002) = 32)."""
    k = np.zeros(256, np.float32)
    k[0:32] = np.linspace(0.0, 1.0, 32, dtype=np.float32)
    k[32:64] = np.linspace(0.0, 0.5, 32, dtype=np.float32)
    pk = orc.pack_history(k, np.zeros(256, np.float32), orc.Q4_K, orc.Q6_K)
    assert pk[0:2].view(np.float16)[0] == np.float16(0.0010585784912109375)
    assert pk[2:4].view(np.uint16)[0] == 0                     # dmin = 0: every minimum is 0
    assert pk[4] & 63 == 63 and pk[5] & 63 == 31
    assert pk[6] & 63 == 0 and pk[8] & 63 == 0                  # empty groups, zero minima


# ------------------------------------------------------- decoder-step ops ----
def test_embed_rows_match_ggml_rows():
    rng = np.random.default_rng(14)
    vocab, hidden = 50, 512
    for fmt, ref in ((orc.Q4_K, ggml_q4k), (orc.Q6_K, ggml_q6k)):
        table = synth.random_matrix(rng, fmt, vocab, hidden)
        ids = np.array([3, 0, 49, 3], np.uint32)
        got = orc.embed(fmt, table, vocab, hidden, ids)
        for b, t in enumerate(ids):
            assert np.array_equal(_bits(got[b]), _bits(ref(table[t]))), (fmt, t)


def test_rmsnorm_known_answers():
    x = np.array([[3.0, 4.0], [-2.0, 0.0]], np.float32)
    out = orc.rmsnorm(x, np.array([1.0, 2.0], np.float32), eps=0.0)
    assert np.allclose(out[0], [3 / np.sqrt(12.5), 8 / np.sqrt(12.5)], rtol=1e-15)
    assert np.allclose(out[1], [-np.sqrt(2.0), 0.0], rtol=1e-15)
    rng = np.random.default_rng(15)
    y = rng.standard_normal((3, 4096)).astype(np.float32)
    o1 = orc.rmsnorm(y, np.ones(4096, np.float32), eps=0.0)
    assert np.allclose(np.mean(o1 ** 2, axis=1), 1.0, rtol=1e-12)          # unit RMS
    o2 = orc.rmsnorm(y * np.float32(8.0), np.ones(4096, np.float32), eps=0.0)
    assert np.allclose(o1, o2, rtol=1e-12)                                 # scale invariance


def test_head_norm_modes_and_gate():
    rng = np.random.default_rng(16)
    heads, hd = 3, 128
    x = rng.standard_normal((2, heads * hd)).astype(np.float32)
    rms = orc.head_norm(x, heads, hd, mean=True, eps=0.0).reshape(2, heads, hd)
    l2 = orc.head_norm(x, heads, hd, mean=False, eps=0.0).reshape(2, heads, hd)
    assert np.allclose(np.mean(rms ** 2, axis=2), 1.0, rtol=1e-12)
    assert np.allclose(np.sum(l2 ** 2, axis=2), 1.0, rtol=1e-12)
    assert np.allclose(rms, l2 * np.sqrt(hd), rtol=1e-12)
    g0 = np.zeros_like(x)
    assert not orc.head_norm(x, heads, hd, gate=g0).any()                  # silu(0) = 0
    g = np.full_like(x, 40.0)                                              # silu(40) = 40 (to 1e-17)
    assert np.allclose(orc.head_norm(x, heads, hd, gate=g), 40.0 * orc.head_norm(x, heads, hd), rtol=1e-15)


def test_delta_gates_closed_forms():
    z = np.zeros((1, 3), np.float32)
    a_log = np.array([0.0, np.log(2.0), 0.0], np.float32)
    b = np.array([[0.0, np.log(3.0), -np.log(3.0)]], np.float32)
    decay, beta = orc.delta_gates(z, b, a_log, np.zeros(3, np.float32))
    # softplus(0) = ln 2: exp(-1 * ln 2) = 1/2, exp(-2 ln 2) = 1/4
    assert np.allclose(decay, [[0.5, 0.25, 0.5]], rtol=1e-7)
    assert np.allclose(beta, [[0.5, 0.75, 0.25]], rtol=1e-7)


def test_short_conv_taps_and_state():
    rng = np.random.default_rng(17)
    heads, hd, batch = 2, 128, 2
    W3 = 3 * heads * hd
    raw = rng.standard_normal((batch, W3 + 5)).astype(np.float32)          # extra columns: row stride
    state = rng.standard_normal((batch, W3, 3)).astype(np.float32)
    silu = lambda s: s / (1.0 + np.exp(-s))
    for tap in range(4):
        w = np.zeros((W3, 4), np.float32)
        w[:, tap] = 1.0
        out, ns = orc.short_conv(raw, state, w, heads, hd, eps=0.0)
        src = (raw[:, :W3] if tap == 3 else state[:, :, tap]).astype(np.float64)
        y = silu(src)
        for part in range(2):                                              # q, k: unit L2 per head
            blk = y[:, part * heads * hd:(part + 1) * heads * hd].reshape(batch, heads, hd)
            y[:, part * heads * hd:(part + 1) * heads * hd] = (blk / np.sqrt((blk ** 2).sum(-1, keepdims=True))
                                                                ).reshape(batch, -1)
        assert np.allclose(out, y, rtol=1e-12, atol=1e-15), tap
        assert np.array_equal(ns[:, :, :2], state[:, :, 1:]) and np.array_equal(ns[:, :, 2], raw[:, :W3])


def test_delta_rule_recall_and_decay():
    rng = np.random.default_rng(18)
    heads, hd = 2, 128
    # orthonormal keys: writing (k_i, v_i) from S = 0 with decay 1, beta 1 stores
    # S = sum v_i k_i^T; querying k_j * sqrt(hd) returns v_j
    basis = np.linalg.qr(rng.standard_normal((hd, hd)))[0]
    S = np.zeros((1, heads, hd, hd))
    vs = []
    for i in range(5):
        k = np.tile(basis[:, i], heads)[None]
        v = rng.standard_normal((1, heads * hd))
        vs.append(v)
        S, _ = orc.delta_rule(S, np.zeros_like(v), k, v, np.ones((1, heads)), np.ones((1, heads)))
    for j in range(5):
        q = np.tile(basis[:, j], heads)[None] * np.sqrt(hd)
        zero = np.zeros((1, heads))
        _, o = orc.delta_rule(S, q, np.zeros_like(q), np.zeros_like(q), np.ones((1, heads)), zero)
        assert np.allclose(o, vs[j], atol=1e-12), j
    # beta = 0: the state only decays and the read is decay * S q / sqrt(hd)
    S0 = rng.standard_normal((1, heads, hd, hd))
    q = rng.standard_normal((1, heads * hd))
    S1, o = orc.delta_rule(S0, q, rng.standard_normal((1, heads * hd)), rng.standard_normal((1, heads * hd)),
                           np.full((1, heads), 0.9), np.zeros((1, heads)))
    assert np.allclose(S1, 0.9 * S0, rtol=1e-15)
    ref = np.einsum("hvk,hk->hv", 0.9 * S0[0], q.reshape(heads, hd)).reshape(1, -1) / np.sqrt(hd)
    assert np.allclose(o, ref, rtol=1e-12)


def test_delta_rule_rank_one_closed_form():
    """Decay, then predict, then write (resident_math.comp:144-146): from a rank-1 state
    S0 = a b^T ([value][key]) with decay l and beta t,
      S1 = l a b^T + t (v - l a (b.k)) k^T,   o = S1 q / sqrt(hd)
         = (l a (b.q) + t (v - l a (b.k)) (k.q)) / sqrt(hd).
    Predicting from the undecayed state (u = a (b.k)), a transposed state or a dropped
    decay each change the result."""
    rng = np.random.default_rng(19)
    hd = 128
    a, b, k, q, v = (rng.standard_normal(hd) for _ in range(5))
    lam, beta = 0.5, 0.75
    S0 = np.outer(a, b)[None, None]
    S1, o = orc.delta_rule(S0, q[None], k[None], v[None], np.array([[lam]]), np.array([[beta]]))
    err = v - lam * a * (b @ k)
    assert np.allclose(S1[0, 0], lam * np.outer(a, b) + beta * np.outer(err, k), rtol=1e-13, atol=1e-13)
    want = (lam * a * (b @ q) + beta * err * (k @ q)) / np.sqrt(hd)
    assert np.allclose(o[0], want, rtol=1e-12, atol=1e-13)
    wrong = (lam * a * (b @ q) + beta * (v - a * (b @ k)) * (k @ q)) / np.sqrt(hd)   # predict before decay
    assert not np.allclose(o[0], wrong, rtol=1e-6)


# --------------------------------------------------------- dense receipts ----
from receipt_check import bounds, merge, rows_heads   # noqa: E402


def _receipts(q, packets, base, ctx, cap, hkv, block, fmts=(orc.Q4_K, orc.Q6_K)):
    return orc.attention_receipts(q, packets, fmts[0], fmts[1], np.asarray(base, np.int64),
                                  np.asarray(ctx, np.int32), cap, hkv, block)


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
def test_receipts_merge_to_attention(fmts):
    """The records of each (row, head), merged as the reference's checker merges them
    (max, rescaled Z and U), give the whole-history attention of decode_attention."""
    rng = np.random.default_rng(40)
    hq, hkv, hd, cap, block = 4, 2, 128, 70, 32
    ctx = [1, 31, 32, 33, 70, 95]
    base = [0, 100, 200, 300, 400, 500]
    packets = _history(rng, 600, hkv, hd, *fmts)
    q = rng.standard_normal((len(ctx), hq, hd)).astype(np.float32)
    vals, words, tie = _receipts(q, packets, base, ctx, cap, hkv, block, fmts)
    index = rows_heads(ctx, cap, block, hq)
    assert len(vals) == len(index) == hq * sum((min(c, cap) + block - 1) // block for c in ctx)
    out, M, Z = merge(vals[:, 0], vals[:, 1], vals[:, 3:], index, len(ctx), hq)
    ref, m, z = orc.decode_attention(q, packets, fmts[0], fmts[1], base, ctx, cap, hkv)
    np.testing.assert_allclose(out, ref, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(M, m, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(Z, z, rtol=1e-10)
    bounds(words, index, block)
    assert not tie.all()


def test_receipts_groups_are_newest_first():
    """A group of one position holds exactly that position's (score, 1, V): the record of
    group g at block 32 for a history of 64 positions covers ages 32 g .. 32 g + 31."""
    rng = np.random.default_rng(41)
    hq, hkv, hd = 2, 1, 128
    packets = _history(rng, 65, hkv, hd, orc.Q4_K, orc.Q6_K)
    q = rng.standard_normal((1, hq, hd)).astype(np.float32)
    vals, words, _ = _receipts(q, packets, [0], [65], 1 << 20, hkv, 32)
    assert len(vals) == 3 * hq
    # the last group holds age 64 alone: position 0
    ref, m, z = orc.decode_attention(q, packets[:1], orc.Q4_K, orc.Q6_K, [0], [1], 1 << 20, hkv)
    for h in range(hq):
        np.testing.assert_allclose(vals[2 * hq + h, 3:], ref[0, h], rtol=1e-12)
        assert vals[2 * hq + h, 1] == 1.0 and words[2 * hq + h, 2] == 1
    # the first group: positions 64 .. 33 (newest first)
    ring = np.empty((32, packets.shape[1]), np.uint8)
    for p in range(33, 65):
        ring[p % 32] = packets[p]
    ref, m, z = orc.decode_attention(q, ring, orc.Q4_K, orc.Q6_K, [0], [65], 32, hkv)
    np.testing.assert_allclose(vals[:hq, 3:] / vals[:hq, 1:2], ref[0], rtol=1e-10, atol=1e-12)


def test_receipts_event_closed_forms():
    rng = np.random.default_rng(42)
    hq, hkv, hd, count = 1, 1, 128, 29
    one = _history(rng, 1, hkv, hd, orc.Q4_K, orc.Q6_K)
    q = rng.standard_normal((1, hq, hd)).astype(np.float32)
    # identical packets: one exp (every later weight reused), one value run
    _, words, tie = _receipts(q, np.repeat(one, count, 0), [0], [count], 1 << 20, hkv, 32)
    assert list(words[0, 2:8]) == [count, 1, 1, count, 2 + 2, 3 | 4 | 8] and not tie[0]
    # keys alpha_a * ones with alpha rising with age: each tile of four raises the running
    # maximum, so every weight and every later tile's rescale costs an exp (the reference
    # checker's upper bound count + ceil(count / 4) - 1); distinct values: count runs
    e = np.ones((1, hd), np.float32)
    k = [np.float32(1.0 + 0.25 * a) * e for a in range(count)][::-1]          # position p = count-1-age
    v = [rng.standard_normal((1, hd)).astype(np.float32) for _ in range(count)]
    pk = np.stack([orc.pack_history(k[p], v[p]) for p in range(count)])
    qe = np.ones((1, hq, hd), np.float32)
    vals, words, tie = _receipts(qe, pk, [0], [count], 1 << 20, hkv, 32)
    assert not tie[0]
    assert list(words[0, 2:8]) == [count, count + (count + 3) // 4 - 1, count, count, 4, 3]
    # keys falling with age: the first tile sets the maximum for good, no rescales
    pk2 = np.stack([orc.pack_history(k[count - 1 - p], v[p]) for p in range(count)])
    _, words, tie = _receipts(qe, pk2, [0], [count], 1 << 20, hkv, 32)
    assert not tie[0] and words[0, 3] == count
    # values repeating in runs of three along the ages: ceil(count / 3) runs
    vr = [v[(count - 1 - p) // 3] for p in range(count)]
    pk3 = np.stack([orc.pack_history(k[p], vr[p]) for p in range(count)])
    _, words, _ = _receipts(qe, pk3, [0], [count], 1 << 20, hkv, 32)
    assert words[0, 4] == (count + 2) // 3 and words[0, 7] & 8
