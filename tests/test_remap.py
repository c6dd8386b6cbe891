"""CPU pins of the oracle's row/axis remap (resident_quant.glsl:20-31 quantizedWeight,
modes assigned by compiler/export.py:96-98,108).

Each check is fixed by something other than the remap formula itself:
- the exporter's own permutation of the Q/K norm weights (export.py:100-101), which
  must agree with the rows the detector reads;
- the RoPE identity that motivates modes 1/3: rotating adjacent pairs of the
  remapped rows equals the half-split (NeoX) rotation of the original rows, permuted;
- mode 4 undoing mode 3 through a product (V rows remapped, O columns remapped);
- the Q|gate interleave: modes 1 and 2 partition the exported rows;
- the recurrent key repeat tiling the key heads like export.py:115-116's conv tile.
"""
import numpy as np
import pytest

import oracle as orc
from rta import synth


def _export_norm_perm(hd, r):
    """export.py:100-101: perm[:r] interleaves the two rotary halves."""
    perm = np.arange(hd)
    perm[:r] = np.stack((np.arange(r // 2), np.arange(r // 2) + r // 2), -1).ravel()
    return perm


@pytest.mark.parametrize("hd,r", [(128, 128), (128, 64), (256, 64), (64, 0), (16, 8)])
def test_rotary_source_is_the_exporters_norm_permutation(hd, r):
    perm = _export_norm_perm(hd, r)
    got = np.array([orc.lib().orc_rotary_source(i, r) for i in range(hd)])
    assert np.array_equal(got, perm)
    # mode 3 reads row (head, perm[i]) for logical row (head, i)
    for head in (0, 3):
        for i in (0, 1, r // 2 - 1 if r else 0, r, hd - 1):
            if 0 <= i < hd:
                assert orc.remap_row(3, hd, r, 0, head * hd + i) == head * hd + perm[i]


def _neox_rope(y, t, hd, r, theta):
    """Half-split rotation: pair (i, i + r/2) by t * theta^(-i / (r/2))."""
    y = y.astype(np.float64).reshape(-1, hd).copy()
    h = r // 2
    ang = t * theta ** (-np.arange(h) / h)
    c, s = np.cos(ang), np.sin(ang)
    a, b = y[:, :h].copy(), y[:, h:r].copy()
    y[:, :h] = a * c - b * s
    y[:, h:r] = a * s + b * c
    return y


@pytest.mark.parametrize("mode", [1, 3])
@pytest.mark.parametrize("hd,r", [(16, 16), (32, 16), (128, 128)])
def test_adjacent_rope_of_remapped_rows_is_neox_rope_of_the_original(mode, hd, r):
    rng = np.random.default_rng(hd + r + mode)
    heads, cols, theta, t = 3, 64, 1e4, 77
    src_rows = heads * hd * (2 if mode == 1 else 1)
    w = rng.standard_normal((src_rows, cols)).astype(np.float32)
    x = rng.standard_normal((1, cols)).astype(np.float32)
    y_src = (w.astype(np.float64) @ x[0].astype(np.float64))
    y_log = orc.gemv_remap_f64(orc.F32, w.view(np.uint8), src_rows, heads * hd, cols, mode, hd, r, 0, x)[0]
    # the query part of the exported rows, in the exporter's (half-split) order
    q_src = y_src.reshape(heads, -1)[:, :hd] if mode == 1 else y_src.reshape(heads, hd)
    rotated_src = _neox_rope(q_src, t, hd, r, theta)
    got = orc.rope(y_log.astype(np.float32).reshape(heads, hd), t, rotary=r, theta=theta).astype(np.float64)
    perm = _export_norm_perm(hd, r)
    assert np.allclose(got, rotated_src[:, perm], rtol=1e-5, atol=1e-4)


def test_query_and_gate_partition_the_interleaved_rows():
    hd, r, heads = 16, 8, 4
    q = [orc.remap_row(1, hd, r, 0, i) for i in range(heads * hd)]
    g = [orc.remap_row(2, hd, r, 0, i) for i in range(heads * hd)]
    assert sorted(q + g) == list(range(2 * heads * hd))
    assert all((s // hd) % 2 == 0 for s in q) and all((s // hd) % 2 == 1 for s in g)
    assert q[0] == 0 and q[1] == r // 2 and q[hd] == 2 * hd and g[0] == hd and g[hd + 1] == 3 * hd + r // 2


@pytest.mark.parametrize("hd,r", [(16, 16), (32, 8)])
def test_axis_remap_undoes_the_row_remap(hd, r):
    """O (mode 4 columns) after V (mode 3 rows) is O after V with neither remapped."""
    rng = np.random.default_rng(hd * 3 + r)
    heads, d = 2, 48
    v = rng.standard_normal((heads * hd, d)).astype(np.float32)
    o = rng.standard_normal((d, heads * hd)).astype(np.float32)
    x = rng.standard_normal((2, d)).astype(np.float32)
    vx = orc.gemv_remap_f64(orc.F32, v.view(np.uint8), heads * hd, heads * hd, d, 3, hd, r, 0, x)
    got = orc.gemv_remap_f64(orc.F32, o.view(np.uint8), d, d, heads * hd, 4, hd, r, 0, vx.astype(np.float32))
    plain = (o.astype(np.float64) @ (v.astype(np.float64) @ x.T.astype(np.float64))).T
    assert np.allclose(got, plain, rtol=1e-5, atol=1e-4)
    # and the remap is not the identity for these shapes
    assert not np.allclose(orc.gemv_remap_f64(orc.F32, o.view(np.uint8), d, d, heads * hd, 0, hd, r, 0,
                                              vx.astype(np.float32)), plain, rtol=1e-3, atol=1e-2)


def test_key_repeat_tiles_the_key_heads():
    key_rows, heads_rep = 256, 3
    assert [orc.remap_row(5, 0, 0, key_rows, i) for i in (0, 255, 256, 300, 767)] == [0, 255, 0, 44, 255]
    # the exporter's conv weights for the repeated q channels: np.tile(conv[:key], (repeat, 1))
    conv = np.arange(key_rows * 4).reshape(key_rows, 4)
    tiled = np.tile(conv, (heads_rep, 1))
    for c in (0, 17, 256, 511, 700):
        assert np.array_equal(tiled[c], conv[orc.remap_row(5, 0, 0, key_rows, c)])


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 4, 5])
def test_remapped_gemv_reads_the_remapped_coefficients(fmt, mode):
    """Brute force on a small quantised matrix: every weight from its remapped (row, axis)."""
    rng = np.random.default_rng(40 + mode + fmt)
    hd, r, key_rows, cols = 128, 64, 96, 256
    rows = 2 * hd
    src_rows = {1: 2 * rows, 2: 2 * rows, 5: key_rows}.get(mode, rows)
    w = synth.random_matrix(rng, fmt, src_rows, cols)
    dense = orc.dequant(fmt, w, src_rows * cols).reshape(src_rows, cols).astype(np.float64)
    x = rng.standard_normal((2, cols)).astype(np.float32)
    got = orc.gemv_remap_f64(fmt, w, src_rows, rows, cols, mode, hd, r, key_rows, x)
    ref = np.empty_like(got)
    for i in range(rows):
        sr = {1: (i // hd) * 2 * hd + _export_norm_perm(hd, r)[i % hd],
              2: (i // hd) * 2 * hd + hd + _export_norm_perm(hd, r)[i % hd],
              3: (i // hd) * hd + _export_norm_perm(hd, r)[i % hd],
              5: i % key_rows}.get(mode, i)
        row = dense[sr]
        if mode == 4:
            row = row[(np.arange(cols) // hd) * hd + _export_norm_perm(hd, r)[np.arange(cols) % hd]]
        ref[:, i] = x.astype(np.float64) @ row
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-9)


def test_remapped_gemv_rejects_rows_outside_the_matrix():
    w = np.zeros((4, 16), dtype=np.float32)
    x = np.zeros((1, 16), dtype=np.float32)
    with pytest.raises(AssertionError):
        orc.gemv_remap_f64(orc.F32, w.view(np.uint8), 4, 8, 16, 1, 4, 4, 0, x)
