"""GPU parity of the packed (tiled) K-quant path: rta_pack's layout, and every
projection entry point over packed weights against the CPU oracle on the GGUF
matrix they were packed from (same bars as test_gpu_parity: floats within
max|gpu - ref| <= 1e-5 + 1e-3 max|ref|, ids exactly the margin rule)."""
import numpy as np
import pytest

import oracle as orc
from conftest import assert_close
from rta import ops, synth
from rta._lib import TILED

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def to_dev(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def scale_fields(q):
    """Bytes 4..15 of a packed Q4_K row header from the GGUF block's 12 scale bytes
    (q [..., 12]): the 6-bit scales and minima decoded as resident_quant.glsl:10-19 does
    and regrouped per lane segment s at bits 24 s + (0, 6, 12, 18) of a 96-bit field."""
    q = q.astype(np.uint64)
    field = np.zeros(q.shape[:-1], dtype=object)
    for g in range(8):
        j = g & 3
        if g < 4:
            sc, m = q[..., j] & 63, q[..., j + 4] & 63
        else:
            sc = (q[..., j + 8] & 15) | ((q[..., j] >> 6) << 4)
            m = (q[..., j + 8] >> 4) | ((q[..., j + 4] >> 6) << 4)
        s, k = g >> 1, g & 1
        field = field + (sc.astype(object) << (24 * s + 6 * k)) + (m.astype(object) << (24 * s + 12 + 6 * k))
    out = np.zeros(q.shape, np.uint8)
    for b in range(12):
        out[..., b] = np.vectorize(lambda f: (f >> (8 * b)) & 255, otypes=[np.uint8])(field)
    return out


def np_pack(fmt, w, rows, cols):
    """The tile layout, built field by field from the GGUF blocks (debugging aid;
    the parity tests below pin the packed path against the oracle)."""
    nsb, blk = cols // 256, (144 if fmt == orc.Q4_K else 210)
    nt = (rows + 15) // 16
    g = np.zeros((nt * 16, nsb, blk), np.uint8)
    g[:rows] = np.asarray(w, np.uint8).reshape(rows, nsb, blk)
    g = g.reshape(nt, 16, nsb, blk).transpose(0, 2, 1, 3)           # [tile][sb][row][block]
    if fmt == orc.Q4_K:
        hdr = g[..., :16].copy()
        hdr[..., 4:16] = scale_fields(g[..., 4:16])
        hdr = hdr.reshape(nt, nsb, 256)
        qs = g[..., 16:].reshape(nt, nsb, 16, 4, 2, 16)               # [..][row][s][k][16]
        lanes = qs.transpose(0, 1, 4, 3, 2, 5).reshape(nt, nsb, 2048)  # [k][s][row][16]
        out = np.concatenate([hdr, lanes], axis=2)
    else:
        ql, qh = g[..., :128], g[..., 128:192]
        sc, d = g[..., 192:208].reshape(nt, nsb, 256), g[..., 208:210].reshape(nt, nsb, 32)
        qlr = ql.reshape(nt, nsb, 16, 2, 2, 2, 16)                    # [row][h][ab][sg][16]
        qhr = qh.reshape(nt, nsb, 16, 2, 2, 16)                       # [row][h][sg][16]
        parts = []
        for ab in (0, 1):
            x = qlr[:, :, :, :, ab]                                    # [row][h][sg][16]
            parts.append(x.transpose(0, 1, 3, 4, 2, 5).reshape(nt, nsb, 1024))   # lane 16(2h+sg)+row
        parts.append(qhr.transpose(0, 1, 3, 4, 2, 5).reshape(nt, nsb, 1024))
        out = np.concatenate([sc, d] + parts, axis=2)
    return out.reshape(-1)


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("rows,cols", [(37, 512), (100, 256), (16, 1024)])
def test_pack_layout(torch_dev, fmt, rows, cols):
    torch, dev = torch_dev
    rng = np.random.default_rng(rows + cols + fmt)
    w = synth.random_matrix(rng, fmt, rows, cols)
    got = ops.pack(fmt, to_dev(torch, w, dev), rows, cols).cpu().numpy()
    assert got.size == ops.pack_bytes(fmt, rows, cols)
    assert np.array_equal(got, np_pack(fmt, w, rows, cols))


SHAPES = [(4096, 4096), (1000, 768), (37, 256), (300, 12288), (151936, 256), (6144, 2048)]


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_tiled_gemv_parity(torch_dev, fmt, rows, cols):
    torch, dev = torch_dev
    rng = np.random.default_rng(rows * 3 + cols + fmt)
    w = synth.random_matrix(rng, fmt, rows, cols)
    wp = ops.pack(fmt, to_dev(torch, w, dev), rows, cols)
    sub = min(rows, 2048)    # oracle rows checked (all of them below 2048)
    for batch in (1, 3, 8, 16, 17, 32, 40):
        x = rng.standard_normal((batch, cols)).astype(np.float32)
        got = ops.gemv(fmt | TILED, wp, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
        ref = orc.gemv_f64(fmt, w[:sub], sub, cols, x)
        for b in range(batch):
            assert_close(got[b, :sub], ref[b], f"fmt {fmt} {rows}x{cols} batch {batch} row {b}")


def test_tiled_large_q6k_scales(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(92)
    rows, cols = 256, 1024
    n = rows * cols // 256
    d = (np.abs(rng.standard_normal(n)) * 0.01).astype(np.float16)
    sc = rng.integers(-128, 128, (n, 16)).astype(np.int8)
    q = rng.integers(0, 64, (n, 256)).astype(np.uint8)
    w = synth.pack_q6k(d, sc, q).reshape(rows, -1)
    wp = ops.pack(orc.Q6_K, to_dev(torch, w, dev), rows, cols)
    x = rng.standard_normal((24, cols)).astype(np.float32)
    got = ops.gemv(orc.Q6_K | TILED, wp, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
    ref = orc.gemv_f64(orc.Q6_K, w, rows, cols, x)
    for b in range(24):
        assert_close(got[b], ref[b], f"row {b}")


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
def test_tiled_invariants(torch_dev, fmt):
    """Zero row -> exact zero; a row's result does not depend on the other rows of
    the call (bitwise, within one operand width: batch tiles of <= 16 and of 17..32
    rows are planned separately); accumulate adds exactly."""
    torch, dev = torch_dev
    rows, cols = 700, 4096
    rng = np.random.default_rng(34)
    w_host = synth.random_matrix(rng, fmt, rows, cols)
    wp = ops.pack(fmt, to_dev(torch, w_host, dev), rows, cols)
    x = rng.standard_normal((40, cols)).astype(np.float32)
    x[1] = 0.0
    for n, prefixes in ((16, (1, 5, 9)), (40, (17, 24, 33))):
        y = ops.gemv(fmt | TILED, wp, rows, cols, to_dev(torch, x[:n], dev)).cpu().numpy()
        assert not y[1].any()
        for prefix in prefixes:
            yp = ops.gemv(fmt | TILED, wp, rows, cols, to_dev(torch, x[:prefix], dev)).cpu().numpy()
            assert np.array_equal(yp, y[:prefix]), (n, prefix)
        base = rng.standard_normal((n, rows)).astype(np.float32)
        yacc = to_dev(torch, base, dev)
        ops.gemv(fmt | TILED, wp, rows, cols, to_dev(torch, x[:n], dev), y=yacc, accumulate=True)
        assert np.array_equal(yacc.cpu().numpy(), (base + y).astype(np.float32))


@pytest.mark.parametrize("hidden,inter,batch", [(2048, 6144, 1), (2048, 6144, 8), (2048, 6144, 32),
                                                (2048, 6144, 40), (256, 32768, 4)])
def test_tiled_mlp_parity(torch_dev, hidden, inter, batch):
    torch, dev = torch_dev
    rng = np.random.default_rng(20261121 + inter + batch)
    wg = synth.random_matrix(rng, orc.Q4_K, inter, hidden)
    wu = synth.random_matrix(rng, orc.Q4_K, inter, hidden)
    wd = synth.random_matrix(rng, orc.Q6_K, hidden, inter)
    x = rng.normal(0, 1.0, (batch, hidden)).astype(np.float32)
    if batch >= 4:
        x[1] = 0.0
        x[2] = -x[0]
    pg = ops.pack(orc.Q4_K, to_dev(torch, wg, dev), inter, hidden)
    pu = ops.pack(orc.Q4_K, to_dev(torch, wu, dev), inter, hidden)
    pd = ops.pack(orc.Q6_K, to_dev(torch, wd, dev), hidden, inter)
    fm = (orc.Q4_K | TILED, orc.Q4_K | TILED, orc.Q6_K | TILED)
    act, y = ops.mlp_swiglu(fm, pg, pu, pd, hidden, inter, to_dev(torch, x, dev))
    ract, ry = orc.mlp_swiglu((orc.Q4_K, orc.Q4_K, orc.Q6_K), wg, wu, wd, hidden, inter, x)
    act, y = act.cpu().numpy(), y.cpu().numpy()
    for b in range(batch):
        assert_close(act[b], ract[b], f"activation row {b}")
        assert_close(y[b], ry[b], f"output row {b}")
    if batch >= 4:
        assert not act[1].any() and not y[1].any()


@pytest.mark.parametrize("vocab,hidden,batch", [(20011, 2048, 1), (20011, 2048, 16), (20011, 2048, 33),
                                                (151936, 512, 3)])
def test_tiled_lm_head_parity(torch_dev, vocab, hidden, batch):
    torch, dev = torch_dev
    rng = np.random.default_rng(20261123 + batch + vocab)
    w = synth.random_matrix(rng, orc.Q6_K, vocab, hidden)
    h = (rng.standard_normal((batch, hidden)) * 2.0).astype(np.float32)
    wp = ops.pack(orc.Q6_K, to_dev(torch, w, dev), vocab, hidden)
    logits, ids = ops.lm_head(orc.Q6_K | TILED, wp, vocab, hidden, to_dev(torch, h, dev), margin=1e-4)
    logits, ids = logits.cpu().numpy(), ids.cpu().numpy().view(np.uint32)
    ref = orc.gemv_f64(orc.Q6_K, w, vocab, hidden, h)
    for b in range(batch):
        assert_close(logits[b], ref[b], f"logits row {b}")
        assert int(ids[b]) == orc.argmax_margin_f32(logits[b], 1e-4), b


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("batch", [1, 5, 32])
def test_swiglu_stage_alone(torch_dev, packed, batch):
    """rta_swiglu (the fused gate/up stage) equals rta_mlp_swiglu's activation bit for bit
    and meets the oracle's bar."""
    torch, dev = torch_dev
    hidden, inter = 4096, 1536
    rng = np.random.default_rng(20261130 + batch)
    wg, wu = (synth.random_matrix(rng, orc.Q4_K, inter, hidden) for _ in range(2))
    wd = synth.random_matrix(rng, orc.Q4_K, hidden, inter)
    x = rng.standard_normal((batch, hidden)).astype(np.float32)
    dg, du, dd = (to_dev(torch, w, dev) for w in (wg, wu, wd))
    f = orc.Q4_K
    if packed:
        dg, du, dd = ops.pack(f, dg, inter, hidden), ops.pack(f, du, inter, hidden), ops.pack(f, dd, hidden, inter)
        f |= TILED
    xd = to_dev(torch, x, dev)
    act = ops.swiglu(f, dg, du, hidden, inter, xd)
    act_mlp, _ = ops.mlp_swiglu((f, f, f), dg, du, dd, hidden, inter, xd)
    assert torch.equal(act, act_mlp)
    ract, _ = orc.mlp_swiglu((orc.Q4_K, orc.Q4_K, orc.Q4_K), wg, wu, wd, hidden, inter, x)
    act = act.cpu().numpy()
    for b in range(batch):
        assert_close(act[b], ract[b], f"activation row {b}")



@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("batch", [1, 5, 17, 32])
def test_image_readout_matches_oracle(torch_dev, fmt, batch):
    """rta_image_from_rows + rta_image_readout (the decode step's readout path) in every
    mode, with the RMSNorm factor, against the oracle on rmsnorm(x) * w."""
    torch, dev = torch_dev
    rng = np.random.default_rng(900 + 7 * batch + fmt)
    rows, cols, P = 300, 1024, fmt | TILED
    print(f"image readout: fmt {fmt} batch {batch} rows {rows} cols {cols}", flush=True)
    wg, wu = synth.random_matrix(rng, fmt, rows, cols), synth.random_matrix(rng, fmt, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    nw = (1.0 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    pg = ops.pack(fmt, to_dev(torch, wg, dev), rows, cols)
    pu = ops.pack(fmt, to_dev(torch, wu, dev), rows, cols)
    img, ss = ops.image_from_rows(P, to_dev(torch, x, dev), to_dev(torch, nw, dev))
    x64 = x.astype(np.float64)
    xn = (x64 / np.sqrt((x64 * x64).mean(1, keepdims=True) + 1e-6) * nw).astype(np.float32)
    g, u = orc.gemv_f64(fmt, wg, rows, cols, xn), orc.gemv_f64(fmt, wu, rows, cols, xn)
    y = torch.zeros(batch, rows, device=dev)
    assert ops.image_readout(P, 0, pg, None, rows, cols, img, batch, y, ss=ss) == 1
    assert_close(y.cpu().numpy(), g, "store")
    ops.image_readout(P, 1, pg, None, rows, cols, img, batch, y, ss=ss)
    assert_close(y.cpu().numpy(), 2 * g, "accumulate")
    act = torch.zeros(batch, rows, device=dev)
    ops.image_readout(P, ops.IMAGE_SWIGLU, pg, pu, rows, cols, img, batch, act, ss=ss)
    assert_close(act.cpu().numpy(), g * u / (1 + np.exp(-g)), "swiglu")
    # without ss: W (x * w); K slabs left in the workspace as [slab][32][rows] add up to it
    g0 = orc.gemv_f64(fmt, wg, rows, cols, (x * nw).astype(np.float32))
    ops.image_readout(P, 0, pg, None, rows, cols, img, batch, y)
    assert_close(y.cpu().numpy(), g0, "store, no norm")
    ws = torch.zeros(ops.image_readout_workspace_bytes(rows, cols, False), dtype=torch.uint8, device=dev)
    ns = ops.image_readout(P, 0, pg, None, rows, cols, img, batch, y, reduce=False, workspace=ws)
    if ns > 1:
        part = ws.view(torch.float32)[:ns * 32 * rows].view(ns, 32, rows)[:, :batch].sum(0)
        assert_close(part.cpu().numpy(), g0, "slabs")
    torch.cuda.synchronize()


@pytest.mark.parametrize("batch", [3, 32])
def test_swiglu_image_feeds_down_readout(torch_dev, batch):
    """The decode step's MLP through the image path: gate/up readout with K slabs left ->
    rta_image_from_swiglu -> down readout, against the oracle."""
    torch, dev = torch_dev
    rng = np.random.default_rng(950 + batch)
    fmt, D, FF = orc.Q4_K, 512, 768
    P = fmt | TILED
    print(f"swiglu image: batch {batch} D {D} FF {FF}", flush=True)
    wg, wu, wd = (synth.random_matrix(rng, fmt, FF, D), synth.random_matrix(rng, fmt, FF, D),
                  synth.random_matrix(rng, fmt, D, FF))
    x = rng.standard_normal((batch, D)).astype(np.float32)
    pg, pu, pd = (ops.pack(fmt, to_dev(torch, w, dev), r, c) for w, r, c in ((wg, FF, D), (wu, FF, D), (wd, D, FF)))
    img, _ = ops.image_from_rows(P, to_dev(torch, x, dev))
    ws = torch.zeros(ops.image_readout_workspace_bytes(FF, D, True), dtype=torch.uint8, device=dev)
    act = torch.zeros(batch, FF, device=dev)
    ns = ops.image_readout(P, ops.IMAGE_SWIGLU, pg, pu, FF, D, img, batch, act, reduce=False, workspace=ws)
    g, u = orc.gemv_f64(fmt, wg, FF, D, x), orc.gemv_f64(fmt, wu, FF, D, x)
    a = (g * u / (1 + np.exp(-g))).astype(np.float32)
    if ns == 1:
        pytest.skip("one K slab at this shape: no slabs to turn into an image")
    img2 = ops.image_from_swiglu(P, ws.view(torch.float32), ns, FF, batch)
    y = torch.zeros(batch, D, device=dev)
    ops.image_readout(P, 0, pd, None, D, FF, img2, batch, y)
    assert_close(y.cpu().numpy(), orc.gemv_f64(fmt, wd, D, FF, a), "down from the SwiGLU image")
    torch.cuda.synchronize()
