"""GPU parity at the sizes the benchmarks run: the vocabulary readout over the full
151936-word vocabulary at batch 4 and 16 (row and packed layouts) and the packed
151936 x 4096 LM head of the 9B decode step at batch 32; and the decode step itself at
the 9B widths (hidden 4096, 32 / 8 heads, 32 delta-net heads, FF 12288, vocab 151936,
batch 32, contexts U[256, 8192]) with four layers (three recurrent, one full).

Bars: logits within max|gpu - ref| <= 1e-5 + 1e-3 max|ref| per row against the fp64
oracle; ids exactly the margin rule on the kernel's logits and the oracle's id unless
a logit sits within rounding of the threshold."""
import numpy as np
import pytest

import oracle as orc
from conftest import check_margin_ids, tolerance_ok
from rta import model, ops
from rta._lib import Q4_K, Q6_K, TILED
from step_reference import check_steps

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def assert_close(got, ref, what):
    ok, frac = tolerance_ok(got, ref, REL, ABS)
    assert ok, f"{what}: max|err|/peak = {frac:.3e}"


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
@pytest.mark.parametrize("batch", [4, 16])
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
