"""GPU parity: librta.so's HIP kernels against the CPU oracle on identical seeded
inputs.  Bars: dequantised values and argmax ids bit exact; float outputs within
max|gpu - ref| <= 1e-5 + 1e-3 * max|ref| per output tensor (fp64 oracle built
from the bit-exact fp32 dequantised weights)."""
import numpy as np
import pytest

import oracle as orc
from conftest import assert_close, check_margin_ids
from rta import ops, synth

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def to_dev(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _bits(a):
    return np.asarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- dequant ----
@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
def test_dequant_bit_exact(torch_dev, fmt):
    torch, dev = torch_dev
    rng = np.random.default_rng(100 + fmt)
    raw = synth.random_q4k(rng, 777) if fmt == orc.Q4_K else synth.random_q6k(rng, 777)
    n = 777 * 256
    got = ops.dequant(fmt, to_dev(torch, raw, dev), n).cpu().numpy()
    assert np.array_equal(_bits(got), _bits(orc.dequant(fmt, raw, n)))


def test_dequant_golden_and_plain(torch_dev):
    torch, dev = torch_dev
    from pathlib import Path
    g = np.load(Path(__file__).parent / "golden" / "dequant_golden.npz")
    for fmt, key in ((orc.Q4_K, "q4k"), (orc.Q6_K, "q6k")):
        raw, ref = g[key + "_raw"], g[key + "_values"]
        got = ops.dequant(fmt, to_dev(torch, raw, dev), ref.size).cpu().numpy()
        assert np.array_equal(_bits(got), _bits(ref)), key
    v = np.random.default_rng(5).standard_normal(4096).astype(np.float32)
    for fmt, raw in ((orc.F32, v.view(np.uint8)), (orc.F16, v.astype(np.float16).view(np.uint8)),
                     (orc.BF16, (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8))):
        got = ops.dequant(fmt, to_dev(torch, raw, dev), 4096).cpu().numpy()
        assert np.array_equal(_bits(got), _bits(orc.dequant(fmt, raw, 4096))), fmt


# ------------------------------------------------------------------- GEMV ----
GEMV_SHAPES = [(4096, 4096), (6144, 2048), (2048, 6144), (1000, 768), (37, 256), (5, 12288), (300, 1024), (64, 8192),
               (7, 16384)]


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("rows,cols", GEMV_SHAPES)
def test_gemv_parity(torch_dev, fmt, rows, cols):
    torch, dev = torch_dev
    rng = np.random.default_rng(rows * 7 + cols + fmt)
    w = synth.random_matrix(rng, fmt, rows, cols)
    wd = to_dev(torch, w, dev)
    for batch in (1, 2, 3, 5, 8, 11):
        x = rng.standard_normal((batch, cols)).astype(np.float32)
        got = ops.gemv(fmt, wd, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
        ref = orc.gemv_f64(fmt, w, rows, cols, x)
        for b in range(batch):
            assert_close(got[b], ref[b], f"fmt {fmt} {rows}x{cols} batch {batch} row {b}")


MMA_SHAPES = [(4096, 4096), (1000, 768), (37, 256), (300, 12288), (6144, 2048)]


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("rows,cols", MMA_SHAPES)
def test_gemv_matrix_core_parity(torch_dev, fmt, rows, cols):
    """Batches of >= 5 rows run on the matrix cores (prepared fp16 hi/lo x, exact integer
    weight operands, fixed-order K-slab reduce)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(rows * 13 + cols + fmt)
    w = synth.random_matrix(rng, fmt, rows, cols)
    wd = to_dev(torch, w, dev)
    for batch in (5, 7, 8, 9, 16, 17, 32, 33, 40):
        x = rng.standard_normal((batch, cols)).astype(np.float32)
        x[0] *= 1e3          # rows of very different magnitude (per-row binary16 scaling)
        x[-1] *= 1e-3
        got = ops.gemv(fmt, wd, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
        ref = orc.gemv_f64(fmt, w, rows, cols, x)
        for b in range(batch):
            assert_close(got[b], ref[b], f"fmt {fmt} {rows}x{cols} batch {batch} row {b}")


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
def test_gemv_small_batches_of_a_large_matrix(torch_dev, fmt):
    """12288 x 4096 (more than 2^25 weights) runs on the matrix cores from batch 3, on the
    vector ALUs at batch 2; both against the oracle, and the batch-3 rows bitwise equal to
    the same rows inside a batch of 4 (one path for both)."""
    torch, dev = torch_dev
    rows, cols = 12288, 4096
    rng = np.random.default_rng(92 + fmt)
    w = synth.random_matrix(rng, fmt, rows, cols)
    wd = to_dev(torch, w, dev)
    x = rng.standard_normal((4, cols)).astype(np.float32)
    ref = orc.gemv_f64(fmt, w, rows, cols, x)
    got = {}
    for batch in (2, 3, 4):
        got[batch] = ops.gemv(fmt, wd, rows, cols, to_dev(torch, x[:batch], dev)).cpu().numpy()
        for b in range(batch):
            assert_close(got[batch][b], ref[b], f"fmt {fmt} batch {batch} row {b}")
    assert np.array_equal(got[3], got[4][:3])


def test_matrix_core_large_q6k_scales(torch_dev):
    """Q6_K int8 scales beyond +-64 (products above 2048 round to 11 bits)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(91)
    rows, cols = 256, 1024
    n = rows * cols // 256
    d = (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float16)
    sc = rng.integers(-128, 128, (n, 16)).astype(np.int8)
    q = rng.integers(0, 64, (n, 256)).astype(np.uint8)
    w = synth.pack_q6k(d, sc, q).reshape(rows, -1)
    x = rng.standard_normal((16, cols)).astype(np.float32)
    got = ops.gemv(orc.Q6_K, to_dev(torch, w, dev), rows, cols, to_dev(torch, x, dev)).cpu().numpy()
    ref = orc.gemv_f64(orc.Q6_K, w, rows, cols, x)
    for b in range(16):
        assert_close(got[b], ref[b], f"row {b}")


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
def test_gemv_invariants(torch_dev, fmt):
    """Zero row -> exact zero; batch-prefix bitwise invariance (verify_rt_mlp.py:95-98)
    within each path: the VALU kernels (batches of <= 4 rows of this 512 x 4096 matrix)
    and the matrix-core kernels (>= 5 rows) each compute a row independently of the other
    rows; across the two paths results agree to tolerance.  x -> -x gives y -> -y exactly on the VALU
    path; on the matrix cores only to tolerance (the MFMA's multi-operand fp32
    accumulation is not sign-symmetric at the last bits)."""
    torch, dev = torch_dev
    rows, cols = 512, 4096
    rng = np.random.default_rng(33)
    w_host = synth.random_matrix(rng, fmt, rows, cols)
    w = to_dev(torch, w_host, dev)
    x = rng.standard_normal((40, cols)).astype(np.float32)
    x[1] = 0.0
    x[2] = -x[0]
    for n, prefixes, exact_sign in ((4, (1, 2, 3), True), (40, (5, 8, 16, 33), False)):
        y = ops.gemv(fmt, w, rows, cols, to_dev(torch, x[:n], dev)).cpu().numpy()
        assert not y[1].any()                              # zero row -> exact zero
        if exact_sign:
            assert np.array_equal(y[2], -y[0])             # x -> -x gives y -> -y exactly
        else:
            assert_close(y[2], -y[0], "sign symmetry (matrix cores)")
        for prefix in prefixes:
            yp = ops.gemv(fmt, w, rows, cols, to_dev(torch, x[:prefix], dev)).cpu().numpy()
            assert np.array_equal(yp, y[:prefix]), (n, prefix)
        base = rng.standard_normal((n, rows)).astype(np.float32)
        yacc = to_dev(torch, base, dev)
        ops.gemv(fmt, w, rows, cols, to_dev(torch, x[:n], dev), y=yacc, accumulate=True)
        assert np.array_equal(yacc.cpu().numpy(), (base + y).astype(np.float32))
    ref = orc.gemv_f64(fmt, w_host, rows, cols, x)
    y40 = ops.gemv(fmt, w, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
    y7 = ops.gemv(fmt, w, rows, cols, to_dev(torch, x[:7], dev)).cpu().numpy()
    for b in range(7):
        assert_close(y40[b], ref[b], f"matrix cores row {b}")
        assert_close(y7[b], ref[b], f"VALU row {b}")


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("batch", [4, 8, 32])
def test_readouts_tiny_and_huge_inputs(torch_dev, fmt, packed, batch):
    """Input rows whose superblocks hold fp32 subnormals only, or values near 1e30, beside
    ordinary rows: every path (vector ALUs below 8 rows, matrix cores from 8 rows and on
    packed weights) stays finite and within the bar per row."""
    from rta._lib import TILED
    torch, dev = torch_dev
    rows, cols = 320, 2048
    rng = np.random.default_rng(61 + batch + 2 * fmt)
    w = synth.random_matrix(rng, fmt, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    sub = (rng.standard_normal(cols) * 1e-40).astype(np.float32)     # fp32 subnormals
    x[0] = sub                                                      # a whole row of subnormals
    x[1, 256:512] = sub[:256]                                       # one subnormal superblock
    x[2, :256] *= np.float32(1e30)                                  # one superblock near 1e30
    x[3] = np.float32(-1e30) * np.sign(x[3])                        # a whole row at -+1e30
    assert np.all(np.abs(x[0][x[0] != 0]) < np.finfo(np.float32).tiny)
    wd = to_dev(torch, w, dev)
    f = fmt
    if packed:
        wd, f = ops.pack(fmt, wd, rows, cols), fmt | TILED
    got = ops.gemv(f, wd, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
    ref = orc.gemv_f64(fmt, w, rows, cols, x)
    assert np.isfinite(got).all()
    for b in range(batch):
        assert_close(got[b], ref[b], f"row {b}")
    assert ops.device_error() == 0


def test_gemv_plain_formats(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(44)
    rows, cols = 129, 520
    wf = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal((3, cols)).astype(np.float32)
    for fmt, raw in ((orc.F32, wf), (orc.F16, wf.astype(np.float16)),
                     (orc.BF16, (wf.view(np.uint32) >> 16).astype(np.uint16))):
        raw = raw.view(np.uint8).reshape(rows, -1)
        got = ops.gemv(fmt, to_dev(torch, raw, dev), rows, cols, to_dev(torch, x, dev)).cpu().numpy()
        assert_close(got, orc.gemv_f64(fmt, raw, rows, cols, x), f"plain fmt {fmt}")


# -------------------------------------------------------------------- MLP ----
@pytest.mark.parametrize("batch", [1, 7, 8, 17, 32, 40])
def test_mlp_swiglu_parity(torch_dev, batch):
    torch, dev = torch_dev
    hidden, inter = 2048, 6144
    rng = np.random.default_rng(20261111)
    wg = synth.random_matrix(rng, orc.Q4_K, inter, hidden)
    wu = synth.random_matrix(rng, orc.Q4_K, inter, hidden)
    wd = synth.random_matrix(rng, orc.Q6_K, hidden, inter)
    x = rng.normal(0, 1.0, (batch, hidden)).astype(np.float32)
    if batch >= 4:   # the reference verifier's special rows (verify_rt_mlp.py:64-67)
        x[1] = 0.0
        x[2] = -x[0]
        x[3] = np.where(np.arange(hidden) % 2, 0.5, -0.5)
    fm = (orc.Q4_K, orc.Q4_K, orc.Q6_K)
    act, y = ops.mlp_swiglu(fm, to_dev(torch, wg, dev), to_dev(torch, wu, dev), to_dev(torch, wd, dev), hidden,
                            inter, to_dev(torch, x, dev))
    ract, ry = orc.mlp_swiglu(fm, wg, wu, wd, hidden, inter, x)
    act, y = act.cpu().numpy(), y.cpu().numpy()
    for b in range(batch):
        assert_close(act[b], ract[b], f"activation row {b}")
        assert_close(y[b], ry[b], f"output row {b}")
    if batch >= 4:
        assert not act[1].any() and not y[1].any()


# --------------------------------------------------------------- LM head ----
@pytest.mark.parametrize("batch", [1, 4, 16, 33])
def test_lm_head_parity(torch_dev, batch):
    torch, dev = torch_dev
    vocab, hidden = (151936 if batch == 1 else 20011), 2048
    rng = np.random.default_rng(20261113 + batch)
    w = synth.random_matrix(rng, orc.Q6_K, vocab, hidden)
    h = (rng.standard_normal((batch, hidden)) * 2.0).astype(np.float32)
    logits, ids = ops.lm_head(orc.Q6_K, to_dev(torch, w, dev), vocab, hidden, to_dev(torch, h, dev), margin=1e-4)
    logits, ids = logits.cpu().numpy(), ids.cpu().numpy().view(np.uint32)
    ref = orc.gemv_f64(orc.Q6_K, w, vocab, hidden, h)
    for b in range(batch):
        assert_close(logits[b], ref[b], f"logits row {b}")
    check_margin_ids(logits, ids, ref, 1e-4)


def test_lm_head_planted_winner_and_ties(torch_dev):
    torch, dev = torch_dev
    vocab, hidden = 5000, 256
    rng = np.random.default_rng(77)
    w = synth.random_matrix(rng, orc.Q6_K, vocab, hidden)
    h = rng.standard_normal((3, hidden)).astype(np.float32)
    win = w[123].copy()
    w[4000] = win            # exact duplicate of row 123 later in the vocabulary: exact tie
    win6 = win.reshape(1, 210).copy()
    win6[0, 208:210] = (np.float16(np.abs(win6[0, 208:210].view(np.float16)[0]) * 4)).reshape(1).view(np.uint8)
    w[123] = win6.reshape(-1)
    w[4000] = win6.reshape(-1)
    wd = to_dev(torch, w, dev)
    for margin in (0.0, 1e-4):
        logits, ids = ops.lm_head(orc.Q6_K, wd, vocab, hidden, to_dev(torch, h, dev), margin=margin)
        logits, ids = logits.cpu().numpy(), ids.cpu().numpy().view(np.uint32)
        for b in range(3):
            assert logits[b, 123] == logits[b, 4000]
            assert int(ids[b]) == orc.argmax_margin_f32(logits[b], margin)
            if int(np.argmax(logits[b])) == 123:
                assert int(ids[b]) == 123           # the tie goes to the lower id


# ------------------------------------------------------------- attention ----
def _attention_case(torch, dev, seed, ctx, hq, hkv, fmts, capacity=None, gate=False):
    rng = np.random.default_rng(seed)
    hd = 128
    nseq = len(ctx)
    ctx = np.asarray(ctx, np.int32)
    cap = int(capacity or max(ctx))
    slots = np.array([min(int(c), cap) if capacity else int(c) for c in ctx])
    base = np.concatenate([[0], np.cumsum([cap if capacity else c for c in ctx])[:-1]]).astype(np.int64)
    total = int(base[-1] + (cap if capacity else ctx[-1]))
    packets = synth.random_packets(rng, total, hkv * hd, *fmts)
    q = rng.standard_normal((nseq, hq, hd)).astype(np.float32)
    g = rng.normal(0, 2.0, (nseq, hq, hd)).astype(np.float32) if gate else None
    max_ctx = int(min(ctx.max(), cap))
    out, m, z = ops.decode_attention(to_dev(torch, q, dev), to_dev(torch, packets, dev), fmts[0], fmts[1],
                                     to_dev(torch, base, dev), to_dev(torch, ctx, dev), cap, max_ctx, hkv,
                                     gate=None if g is None else to_dev(torch, g, dev))
    rout, rm, rz = orc.decode_attention(q, packets, fmts[0], fmts[1], base, ctx, cap, hkv, gate=g)
    assert ops.device_error() == 0
    assert_close(out.cpu().numpy(), rout, "attention output")
    assert_close(m.cpu().numpy(), rm, "attention max")
    assert_close(z.cpu().numpy(), rz, "attention Z")
    del slots


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
def test_attention_boundaries(torch_dev, fmts):
    torch, dev = torch_dev
    # history lengths around the 256-position chunk (verify_attention_receipts.py:215-218)
    ctx = [1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 513]
    _attention_case(torch, dev, 5, ctx, 16, 4, fmts)


@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 4), (16, 4), (32, 4), (32, 8), (8, 2), (4, 1), (24, 6)])
def test_attention_gqa_groups(torch_dev, hq, hkv):
    torch, dev = torch_dev
    _attention_case(torch, dev, 6, [700, 3, 1500], hq, hkv, (orc.Q4_K, orc.Q6_K), gate=True)


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K), (orc.Q4_K, orc.Q4_K)])
@pytest.mark.parametrize("max_ctx", [2100, 9000, 17000])
def test_attention_multi_tile_chunks(torch_dev, fmts, max_ctx):
    """64 sequences: the grid bound max_ctx (a host upper bound, above every context here) sets
    the tiles per chunk to 1, 2 and 4; contexts cover one to several chunks and partial tiles."""
    torch, dev = torch_dev
    rng = np.random.default_rng(max_ctx)
    ctx = rng.integers(1, 700, 64)
    ctx[:4] = [2047, 1025, 511, 64]
    rng2 = np.random.default_rng(11)
    nseq, hq, hkv, hd = 64, 8, 2, 128
    ctx = ctx.astype(np.int32)
    base = np.concatenate([[0], np.cumsum(ctx)[:-1]]).astype(np.int64)
    packets = synth.random_packets(rng2, int(ctx.sum()), hkv * hd, *fmts)
    q = rng2.standard_normal((nseq, hq, hd)).astype(np.float32)
    out, m, z = ops.decode_attention(to_dev(torch, q, dev), to_dev(torch, packets, dev), fmts[0], fmts[1],
                                     to_dev(torch, base, dev), to_dev(torch, ctx, dev), 1 << 20, max_ctx, hkv)
    rout, rm, rz = orc.decode_attention(q, packets, fmts[0], fmts[1], base, ctx, 1 << 20, hkv)
    assert ops.device_error() == 0
    assert_close(out.cpu().numpy(), rout, "attention output")
    assert_close(m.cpu().numpy(), rm, "attention max")
    assert_close(z.cpu().numpy(), rz, "attention Z")


def test_attention_ring_capacity(torch_dev):
    torch, dev = torch_dev
    _attention_case(torch, dev, 7, [600, 1000, 90], 16, 4, (orc.Q6_K, orc.Q4_K), capacity=300)


# ------------------------------------------------------------------- RoPE ----
def test_rope_parity(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(9)
    v = rng.standard_normal((6, 16, 128)).astype(np.float32)
    pos = np.array([0, 1, 511, 4095, 32767, 100000], np.int64)
    got = ops.rope(to_dev(torch, v, dev), to_dev(torch, pos, dev), theta=1e6).cpu().numpy()
    for r in range(6):
        ref = orc.rope(v[r], pos[r], theta=1e6)
        assert np.allclose(got[r], ref, rtol=0, atol=2e-6 * max(1.0, np.abs(ref).max())), r
