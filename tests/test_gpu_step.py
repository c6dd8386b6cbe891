"""GPU parity of the decoder-step ops around the projections (embedding, RMSNorm,
per-head norms, delta-net gates, short convolution, delta rule, history packer)
against the CPU oracle: embedding rows, conv windows and packets bit exact; floats
within max|gpu - ref| <= 1e-5 + 1e-3 max|ref| per tensor."""
import numpy as np
import pytest

import oracle as orc
from conftest import assert_close
from rta import ops, synth

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def to_dev(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("fmt", [orc.Q4_K, orc.Q6_K, orc.F16])
def test_embed_bit_exact(torch_dev, fmt):
    torch, dev = torch_dev
    rng = np.random.default_rng(300 + fmt)
    vocab, hidden = 1000, 4096
    if fmt == orc.F16:
        table = rng.standard_normal((vocab, hidden)).astype(np.float16).view(np.uint8).reshape(vocab, -1)
    else:
        table = synth.random_matrix(rng, fmt, vocab, hidden)
    ids = rng.integers(0, vocab, 33).astype(np.uint32)
    got = ops.embed(fmt, to_dev(torch, table, dev), vocab, hidden, to_dev(torch, ids.view(np.int32), dev))
    ref = orc.embed(fmt, table, vocab, hidden, ids)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), ref.view(np.uint32))


def test_embed_bad_token(torch_dev):
    torch, dev = torch_dev
    ops.device_error(clear=True)
    table = synth.random_matrix(np.random.default_rng(1), orc.Q4_K, 10, 256)
    ids = np.array([3, 10], np.uint32)
    got = ops.embed(orc.Q4_K, to_dev(torch, table, dev), 10, 256, to_dev(torch, ids.view(np.int32), dev))
    assert not got[1].any().item()
    assert ops.device_error(clear=True) & 4096


def test_rmsnorm_parity(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(301)
    x = (rng.standard_normal((32, 4096)) * 3.0).astype(np.float32)
    w = rng.normal(1.0, 0.2, 4096).astype(np.float32)
    xd = to_dev(torch, x, dev)
    got = ops.rmsnorm(xd, to_dev(torch, w, dev), eps=1e-6).cpu().numpy()
    assert_close(got, orc.rmsnorm(x, w, 1e-6), "rmsnorm")
    ops.rmsnorm(xd, to_dev(torch, w, dev), eps=1e-6, out=xd)                 # in place (op 1 index 2)
    assert np.array_equal(xd.cpu().numpy(), got)


@pytest.mark.parametrize("mode", ["qk", "l2", "gated"])
def test_head_norm_parity(torch_dev, mode):
    torch, dev = torch_dev
    rng = np.random.default_rng(302)
    rows, heads, hd = 9, 32, 128
    big = (rng.standard_normal((rows, heads * hd + 77)) * 2).astype(np.float32)   # strided rows
    w = rng.normal(1.0, 0.3, heads * hd).astype(np.float32) if mode != "l2" else None
    gate = (rng.standard_normal((rows, heads * hd + 5)) * 2).astype(np.float32) if mode == "gated" else None
    xd = to_dev(torch, big, dev)[:, :heads * hd]
    gd = None if gate is None else to_dev(torch, gate, dev)[:, :heads * hd]
    ops.head_norm(xd, heads, hd, w=None if w is None else to_dev(torch, w, dev), gate=gd, mean=mode != "l2")
    ref = orc.head_norm(big, heads, hd, w=w, gate=gate, mean=mode != "l2")
    assert_close(xd.cpu().numpy(), ref, mode)


def test_delta_gates_parity(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(303)
    batch, heads = 32, 32
    ab = (rng.standard_normal((batch, 2 * heads + 3)) * 3).astype(np.float32)
    a_log = rng.uniform(-2, 1, heads).astype(np.float32)
    dt = rng.uniform(-1, 1, heads).astype(np.float32)
    abd = to_dev(torch, ab, dev)
    decay, beta = ops.delta_gates(abd[:, :heads], abd[:, heads:2 * heads], to_dev(torch, a_log, dev),
                                  to_dev(torch, dt, dev))
    rd, rb = orc.delta_gates(ab[:, :heads], ab[:, heads:2 * heads], a_log, dt)
    assert_close(decay.cpu().numpy(), rd, "decay")
    assert_close(beta.cpu().numpy(), rb, "beta")


def test_short_conv_parity(torch_dev):
    torch, dev = torch_dev
    rng = np.random.default_rng(304)
    batch, heads, hd = 8, 32, 128
    W3 = 3 * heads * hd
    raw = rng.standard_normal((batch, W3 + 4096 + 64)).astype(np.float32)        # z and a|b follow
    state = rng.standard_normal((batch, W3, 3)).astype(np.float32)
    w = rng.normal(0, 0.5, (W3, 4)).astype(np.float32)
    sd = to_dev(torch, state, dev)
    out = ops.short_conv(to_dev(torch, raw, dev), sd, to_dev(torch, w, dev), heads, hd)
    ref, ref_state = orc.short_conv(raw, state, w, heads, hd)
    assert_close(out.cpu().numpy(), ref, "conv out")
    assert np.array_equal(sd.cpu().numpy(), ref_state)


@pytest.mark.parametrize("fused", [False, True])
def test_delta_rule_parity(torch_dev, fused):
    torch, dev = torch_dev
    rng = np.random.default_rng(305 + fused)
    batch, heads, hd = 4, 32, 128
    W = heads * hd
    state = (rng.standard_normal((batch, heads, hd, hd)) * 0.1).astype(np.float32)
    qkv = rng.standard_normal((batch, 3 * W)).astype(np.float32)
    for part in range(2):                                       # unit-L2 q and k per head
        blk = qkv[:, part * W:(part + 1) * W].reshape(batch, heads, hd)
        qkv[:, part * W:(part + 1) * W] = (blk / np.linalg.norm(blk, axis=-1, keepdims=True)).reshape(batch, W)
    decay = rng.uniform(0.9, 0.999, (batch, heads)).astype(np.float32)
    beta = rng.uniform(0.0, 1.0, (batch, heads)).astype(np.float32)
    norm_w = rng.normal(1.0, 0.2, W).astype(np.float32)
    gate = rng.standard_normal((batch, W)).astype(np.float32)
    sd = to_dev(torch, state, dev)
    out = ops.delta_rule(sd, to_dev(torch, qkv, dev), to_dev(torch, decay, dev), to_dev(torch, beta, dev), heads, hd,
                         norm_w=to_dev(torch, norm_w, dev) if fused else None,
                         gate=to_dev(torch, gate, dev) if fused else None)
    q, k, v = (qkv[:, i * W:(i + 1) * W].astype(np.float64) for i in range(3))
    ref_state, ref = orc.delta_rule(state.astype(np.float64), q, k, v, decay.astype(np.float64),
                                    beta.astype(np.float64))
    if fused:
        ref = orc.head_norm(ref.astype(np.float32), heads, hd, w=norm_w, gate=gate, mean=True)
    assert_close(out.cpu().numpy(), ref, "delta rule out")
    assert_close(sd.cpu().numpy(), ref_state, "delta rule state")


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
@pytest.mark.parametrize("kvw", [1024, 512, 300])
def test_pack_history_bit_exact(torch_dev, fmts, kvw):
    torch, dev = torch_dev
    rng = np.random.default_rng(306 + kvw)
    batch = 12
    k = (rng.standard_normal((batch, kvw + 16)) * rng.uniform(0.01, 4, (batch, 1))).astype(np.float32)
    v = (rng.standard_normal((batch, kvw + 8)) * rng.uniform(0.01, 4, (batch, 1))).astype(np.float32)
    k[0] = 0.0                                              # all-zero field
    v[1, :100] = 0.0
    k[2] = np.abs(k[2])                                     # one-signed fields
    v[3] = -np.abs(v[3])
    stride = orc.history_bytes(kvw)
    n_slots = 40
    slots = rng.permutation(n_slots)[:batch].astype(np.int64)
    packets = torch.zeros(n_slots * stride, dtype=torch.uint8, device=dev)
    ops.pack_history(to_dev(torch, k, dev)[:, :kvw], to_dev(torch, v, dev)[:, :kvw], to_dev(torch, slots, dev),
                     packets, *fmts)
    got = packets.cpu().numpy().reshape(n_slots, stride)
    for b in range(batch):
        ref = orc.pack_history(k[b, :kvw], v[b, :kvw], *fmts)
        assert np.array_equal(got[slots[b]], ref), b
    untouched = np.setdiff1d(np.arange(n_slots), slots)
    assert not got[untouched].any()


def test_pack_history_bad_slot(torch_dev):
    torch, dev = torch_dev
    ops.device_error(clear=True)
    k = torch.ones(2, 512, device="cuda:0")
    packets = torch.zeros(3 * orc.history_bytes(512), dtype=torch.uint8, device="cuda:0")
    ops.pack_history(k, k, torch.tensor([1, 3], dtype=torch.int64, device="cuda:0"), packets)
    assert ops.device_error(clear=True) & 8
    got = packets.cpu().numpy().reshape(3, -1)
    assert got[1].any() and not got[0].any() and not got[2].any()


@pytest.mark.parametrize("which", ["mixed", "one_signed"])
@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
def test_pack_history_known_answer(torch_dev, fmts, which):
    """The HIP packer writes the hand-built packet bytes (exact d / dmin from /63 and /127,
    scale code 127, round to nearest with .5 ties to even; Q4_K groups entirely above or
    below zero with lo / hi started at 0) in both field orders."""
    from known_answers import known_answer_fields, one_signed_fields
    torch, dev = torch_dev
    k, v, expected = known_answer_fields() if which == "mixed" else one_signed_fields()
    if fmts[0] == orc.Q6_K:   # swapped: the Q6_K row is the K field
        k, v = v, k
        expected = np.concatenate([expected[144:354], expected[:144], expected[354:]])
    packets = torch.zeros(2 * 360, dtype=torch.uint8, device=dev)
    ops.pack_history(to_dev(torch, k[None], dev), to_dev(torch, v[None], dev),
                     to_dev(torch, np.array([1], np.int64), dev), packets, *fmts)
    got = packets.cpu().numpy().reshape(2, 360)
    assert not got[0].any()
    diff = np.nonzero(got[1] != expected)[0]
    assert diff.size == 0, f"bytes differ at {diff[:16]}"
