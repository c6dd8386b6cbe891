"""GPU parity of the row/axis remap (rta_gemv_remap, rta_pack_remap) against the
oracle's quantizedWeight restatement (resident_quant.glsl:20-31).  Bars: packed
bytes bit exact; outputs within max|gpu - ref| <= 1e-5 + 1e-3 * max|ref| per row."""
import numpy as np
import pytest

import oracle as orc
from conftest import tolerance_ok
from rta import _lib, ops, synth

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5
HD, ROT = 128, 64   # head dim and a partial rotary dim (axes >= 64 stay in place)


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def to_dev(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _matrix(rng, fmt, rows, cols):
    if fmt in (orc.Q4_K, orc.Q6_K):
        return synth.random_matrix(rng, fmt, rows, cols)
    v = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    if fmt == orc.F32:
        return v.view(np.uint8)
    if fmt == orc.F16:
        return v.astype(np.float16).view(np.uint8)
    return (v.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8)


def _src_rows(mode, rows, key_rows):
    return {1: 2 * rows, 2: 2 * rows, 5: key_rows}.get(mode, rows)


def _check(got, ref, what):
    for b in range(ref.shape[0]):
        ok, frac = tolerance_ok(got[b], ref[b], REL, ABS)
        assert ok, f"{what} row {b}: max|err|/peak = {frac:.3e}"


@pytest.mark.parametrize("fmt", [orc.F32, orc.F16, orc.BF16, orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("mode", [1, 2, 3, 4, 5])
def test_gemv_remap_parity(torch_dev, fmt, mode):
    torch, dev = torch_dev
    rng = np.random.default_rng(300 + 10 * mode + fmt)
    rows, cols, key_rows = 4 * HD, 1024, 256
    src_rows = _src_rows(mode, rows, key_rows)
    w = _matrix(rng, fmt, src_rows, cols)
    wd = to_dev(torch, w, dev)
    rm = ops.remap(mode, HD, ROT, key_rows)
    for batch in (1, 3, 9, 32):
        x = rng.standard_normal((batch, cols)).astype(np.float32)
        ref = orc.gemv_remap_f64(fmt, w, src_rows, rows, cols, mode, HD, ROT, key_rows, x)
        got = ops.gemv_remap(fmt, wd, src_rows, rows, cols, rm, to_dev(torch, x, dev)).cpu().numpy()
        _check(got, ref, f"fmt {fmt} mode {mode} batch {batch}")
        y0 = rng.standard_normal((batch, rows)).astype(np.float32)
        yd = to_dev(torch, y0, dev)
        ops.gemv_remap(fmt, wd, src_rows, rows, cols, rm, to_dev(torch, x, dev), y=yd, accumulate=True)
        _check(yd.cpu().numpy(), ref + y0, f"fmt {fmt} mode {mode} batch {batch} accumulate")


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
@pytest.mark.parametrize("mode", [0, 1, 2, 3, 5])
def test_pack_remap_is_the_pack_of_the_gathered_rows(torch_dev, fmt, mode):
    """rta_pack_remap == rta_pack of the source rows gathered on the host, byte for byte;
    the packed readout of it matches the oracle."""
    torch, dev = torch_dev
    rng = np.random.default_rng(400 + mode + fmt)
    rows, cols, key_rows = 3 * HD, 512, 160
    src_rows = _src_rows(mode, rows, key_rows)
    w = synth.random_matrix(rng, fmt, src_rows, cols)
    wd = to_dev(torch, w, dev)
    rm = ops.remap(mode, HD, ROT, key_rows)
    got = ops.pack_remap(fmt, wd, src_rows, cols, rm, rows).cpu().numpy()
    order = [orc.remap_row(mode, HD, ROT, key_rows, r) for r in range(rows)]
    plain = ops.pack(fmt, to_dev(torch, w[order], dev), rows, cols).cpu().numpy()
    assert np.array_equal(got, plain)
    x = rng.standard_normal((32, cols)).astype(np.float32)
    ref = orc.gemv_remap_f64(fmt, w, src_rows, rows, cols, mode, HD, ROT, key_rows, x)
    y = ops.gemv(fmt | _lib.TILED, to_dev(torch, got, dev), rows, cols, to_dev(torch, x, dev)).cpu().numpy()
    _check(y, ref, f"packed fmt {fmt} mode {mode}")


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K])
def test_axis_remap_on_packed_matrix(torch_dev, fmt):
    """Mode 4 runs on a packed matrix through rta_gemv_remap (x permuted)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(500 + fmt)
    rows, cols = 1000, 4 * HD
    w = synth.random_matrix(rng, fmt, rows, cols)
    packed = ops.pack(fmt, to_dev(torch, w, dev), rows, cols)
    rm = ops.remap(4, HD, ROT, 0)
    for batch in (1, 17, 32):
        x = rng.standard_normal((batch, cols)).astype(np.float32)
        ref = orc.gemv_remap_f64(fmt, w, rows, rows, cols, 4, HD, ROT, 0, x)
        got = ops.gemv_remap(fmt | _lib.TILED, packed, rows, rows, cols, rm, to_dev(torch, x, dev)).cpu().numpy()
        _check(got, ref, f"packed fmt {fmt} mode 4 batch {batch}")


def test_packed_parts_at_row_offsets(torch_dev):
    """A fused Q | gate | K packed part by part (rta_pack_bytes(offset) into dst)."""
    torch, dev = torch_dev
    rng = np.random.default_rng(600)
    fmt, cols, heads, kv = orc.Q4_K, 512, 2, 1
    q_src = synth.random_matrix(rng, fmt, 2 * heads * HD, cols)   # interleaved Q | gate
    k_src = synth.random_matrix(rng, fmt, kv * HD, cols)
    rows = 2 * heads * HD + kv * HD
    dst = torch.empty(ops.pack_bytes(fmt, rows, cols), dtype=torch.uint8, device=dev)
    parts = [(q_src, 1, heads * HD, 0), (q_src, 2, heads * HD, heads * HD), (k_src, 3, kv * HD, 2 * heads * HD)]
    for src, mode, n, off in parts:
        view = dst[ops.pack_bytes(fmt, off, cols) if off else 0:]
        ops.pack_remap(fmt, to_dev(torch, src, dev), src.shape[0], cols, ops.remap(mode, HD, ROT, 0), n, out=view)
    x = rng.standard_normal((5, cols)).astype(np.float32)
    got = ops.gemv(fmt | _lib.TILED, dst, rows, cols, to_dev(torch, x, dev)).cpu().numpy()
    ref = np.concatenate([orc.gemv_remap_f64(fmt, src, src.shape[0], n, cols, mode, HD, ROT, 0, x)
                          for src, mode, n, _ in parts], axis=1)
    _check(got, ref, "fused parts")


def test_remap_argument_errors(torch_dev):
    torch, dev = torch_dev
    lib = _lib.load()
    import ctypes
    w = torch.zeros(16 * 1024, dtype=torch.float32, device=dev)   # covers every accepted call's source rows
    x = torch.zeros(1, 1024, dtype=torch.float32, device=dev)
    y = torch.zeros(1, 8, dtype=torch.float32, device=dev)
    ws = torch.empty(1 << 20, dtype=torch.uint8, device=dev)

    def call(mode, hd, rot, key, src_rows, rows, cols=1024):
        rm = ops.remap(mode, hd, rot, key)
        return lib.rta_gemv_remap(orc.F32, ctypes.c_void_p(w.data_ptr()), src_rows, rows, cols, ctypes.byref(rm),
                                  ctypes.c_void_p(x.data_ptr()), 1, ctypes.c_void_p(y.data_ptr()), 0,
                                  ctypes.c_void_p(ws.data_ptr()), ws.numel(), None)

    assert call(9, 4, 4, 0, 8, 8) == 7                # unknown mode: RANGE
    assert call(3, 4, 6, 0, 8, 8) == 7                # rotary > head dim
    assert call(3, 4, 3, 0, 8, 8) == 7                # odd rotary
    assert call(1, 4, 4, 0, 8, 8) == 2                # Q|gate needs 2 rows of source per row
    assert call(3, 3, 2, 0, 8, 8) == 2                # rows % head dim
    assert call(5, 0, 0, 0, 8, 8) == 7                # key_rows 0
    assert call(5, 0, 0, 4, 2, 8) == 2                # fewer source rows than key rows used
    assert call(3, 4, 4, 0, 8, 8) == 0
    assert call(1, 4, 4, 0, 16, 8) == 0
    torch.cuda.synchronize()
    assert lib.rta_pack_remap(orc.Q4_K, ctypes.c_void_p(w.data_ptr()), 4, 256, ctypes.byref(ops.remap(4, 128, 64, 0)),
                              4, ctypes.c_void_p(ws.data_ptr()), None) == 7   # axes cannot be packed
