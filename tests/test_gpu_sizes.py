"""GPU parity at the sizes the benchmarks run: the vocabulary readout over the full
151936-word vocabulary at batch 2, 4 and 16 (row and packed layouts; the row layout on
the matrix cores from batch 2 at this size) and the packed
151936 x 4096 LM head of the 9B decode step at batch 32; and the decode step itself at
the 9B widths (hidden 4096, 32 / 8 heads, 32 delta-net heads, FF 12288, vocab 151936,
contexts U[256, 8192]) with four layers (three recurrent, one full): at batch 32 over
packed weights, at batch 1 over GGUF rows (the RMSNorm fused into the readouts' x
staging, the 151936 x 4096 LM head with its group maxima), and at batch 32 with the
exporter's in-projection parts of uneven row counts.

Bars: logits within max|gpu - ref| <= 1e-5 + 1e-3 max|ref| per row against the fp64
oracle; ids exactly the margin rule on the kernel's logits and the oracle's id unless
a logit sits within rounding of the threshold."""
import numpy as np
import pytest

import oracle as orc
from conftest import assert_close, check_margin_ids
from rta import model, ops
from rta._lib import Q4_K, Q6_K, TILED
from step_reference import check_steps

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def _lm_head_case(torch, dev, vocab, hidden, batch, packed, seed):
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    w = model.random_kquant(Q6_K, vocab, hidden, gen, dev)
    h = torch.randn(batch, hidden, device=dev, generator=gen) * 2.0
    wk = ops.pack(Q6_K, w, vocab, hidden) if packed else w
    logits, ids = ops.lm_head(Q6_K | (TILED if packed else 0), wk, vocab, hidden, h, margin=1e-4)
    logits, ids = logits.cpu().numpy(), ids.cpu().numpy().view(np.uint32)
    assert ops.device_error() == 0
    ref = orc.gemv_f64(orc.Q6_K, w.cpu().numpy(), vocab, hidden, h.cpu().numpy())
    for b in range(batch):
        assert_close(logits[b], ref[b], f"logits row {b}")
    check_margin_ids(logits, ids, ref, 1e-4)


@pytest.mark.parametrize("packed", [False, True])
@pytest.mark.parametrize("batch", [2, 4, 16])
def test_lm_head_full_vocabulary(torch_dev, batch, packed):
    torch, dev = torch_dev
    _lm_head_case(torch, dev, 151936, 2048, batch, packed, 20261114 + batch)


def test_packed_lm_head_9b_width_batch32(torch_dev):
    torch, dev = torch_dev
    _lm_head_case(torch, dev, 151936, 4096, 32, True, 20261115)


def test_decode_step_9b_widths():
    shape = model.shape_9b(capacity=8448, packed=True)
    shape.layers = 4
    ctx = np.random.default_rng(20261115).integers(256, 8193, 32)
    m = model.DecodeModel(shape, 32, ctx.tolist(), seed=20261115, keep_gguf=True)
    check_steps(m, 2)


def test_decode_step_9b_widths_batch1():
    """The batch-1 step as the metric runs it: GGUF-row readouts (gemv_b1_kernel with the
    RMSNorm fused into x staging at 4096 columns, the 3-wave rows of the 12288-column down
    projection with the accumulate epilogue, the 151936 x 4096 LM head)."""
    shape = model.shape_9b(capacity=8448, packed=False)
    shape.layers = 4
    ctx = np.random.default_rng(20261116).integers(256, 8193, 1)
    m = model.DecodeModel(shape, 1, ctx.tolist(), seed=20261116, keep_gguf=True)
    check_steps(m, 2)


def test_decode_step_9b_widths_uneven_in_projection_parts():
    """In-projection parts of uneven row counts at the 9B widths and batch 32: the full
    layers' q | k | v | gate rows as 7168 Q4_K rows and 3072 Q6_K rows.  A 7168-row readout
    needs more workspace than the whole 10240-row one (fewer row tiles take more K slabs);
    the step's workspace covers every part row count."""
    shape = model.shape_9b(capacity=8448, packed=True)
    shape.layers, shape.attn_gate, shape.layer_formats = 4, 1, 1
    ctx = np.random.default_rng(20261117).integers(256, 8193, 32)
    fmts = lambda l, full: {"in": Q4_K | TILED, "o": Q4_K | TILED, "gate_up": Q4_K | TILED,  # noqa: E731
                            "down": Q4_K | TILED, "ab": Q4_K | TILED}
    parts = lambda l, full: [(7168, Q4_K), (3072, Q6_K)] if full else None  # noqa: E731
    m = model.DecodeModel(shape, 32, ctx.tolist(), seed=20261117, keep_gguf=True, layer_fmts=fmts,
                          in_parts=parts)
    check_steps(m, 1)


@pytest.mark.parametrize("batch", [1, 32])
def test_decode_step_9b_full_depth_against_the_cpu_step(batch):
    """All 32 layers of the 9B step, as the metric runs them (batch 32 on packed tiles, batch 1
    on GGUF rows), one step against the oracle's fp32 CPU step (oracle/rta_cpu_step.c, itself
    checked against the fp64 composition in tests/test_cpu_step.py) from the same state: the
    logits of every row to the float bar, the next tokens under the margin rule (and equal to
    the CPU step's unless a logit sits within rounding of the threshold), the updated
    recurrent state to the float bar and the shifted conv windows bit exactly."""
    shape = model.shape_9b(capacity=8448, packed=batch == 32)
    ctx = np.random.default_rng(20261118 + batch).integers(256, 8193, batch)
    m = model.DecodeModel(shape, batch, ctx.tolist(), seed=20261118 + batch, keep_gguf=True)
    st = dict(rec=np.ascontiguousarray(m.state_view("recurrent")), conv=np.ascontiguousarray(m.state_view("conv")),
              packets=np.ascontiguousarray(m.state_view("packets")), ctx=m.state_view("ctx"),
              tokens=m.tokens.cpu().numpy().view(np.uint32).copy())
    m.step(logits=True)
    got = m.logits.cpu().numpy()
    got_tokens = m.tokens.cpu().numpy().view(np.uint32)
    assert ops.device_error() == 0
    cpu = orc.CpuStep(shape, m.gguf)
    ref = np.empty((batch, shape.vocab), np.float32)
    cpu.step(batch, st["rec"], st["conv"], st["packets"], st["ctx"], st["tokens"], ref)
    for b in range(batch):
        assert_close(got[b], ref[b], f"logits row {b}")
    check_margin_ids(got, got_tokens, ref, 1e-4)
    conv = m.state_view("conv")
    assert np.array_equal(conv[..., :2], st["conv"][..., :2])
    assert_close(conv[..., 2], st["conv"][..., 2], "conv windows (new raw values)")
    assert_close(m.state_view("recurrent"), st["rec"], "recurrent state")


def test_decode_step_9b_full_depth_composition():
    """The whole 32-layer 9B step at batch 32 against the fp64 composition (one step): every
    layer's residual rows, the eight full layers' packed key / value rows and their history
    packets byte for byte (step_reference.check_steps)."""
    shape = model.shape_9b(capacity=8448, packed=True)
    ctx = np.random.default_rng(20261119).integers(256, 8193, 32)
    m = model.DecodeModel(shape, 32, ctx.tolist(), seed=20261119, keep_gguf=True)
    check_steps(m, 1)
