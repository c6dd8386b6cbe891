"""GPU parity of the dense attention receipts (rta_attention_receipts) against the
oracle's records: the standard backend's per-group (m, Z, U) and counters
(resident_attention_dense.comp:190-300; layout attention_receipts.hpp:16-29).

Cases: wrapped rings with several rows of ragged lengths (a single position, exact
multiples of the block, one past, longer than the capacity), blocks 32 / 64 / 96 /
128 / 256 / 512, both packet layouts, GQA ratios 1 / 2 / 4 / 8 and odd kv-head counts 3 and 5; histories of identical packets
(every weight but the first reused, one value run); the error paths (too few records,
a slot outside the packet array, arguments the host refuses).

Bar: count, traversal and coverage words bit exact; exp evaluations, value runs and
flags bit exact except on records where an fp32 score lies within 1e-5 of the running
maximum or its neighbour (the oracle marks them; value runs are always exact); m within
1e-5, Z within 1e-4 relative, U within 2e-4 of max(|U|, Z); merged records within the
decode-attention bar of the whole-history attention; device error word 0."""
import ctypes

import numpy as np
import pytest

import oracle as orc
from receipt_check import bounds, compare, merge, rows_heads
from rta import _lib, ops, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def _run(torch, dev, q, packets, fmts, base, ctx, cap, hkv, block):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    max_ctx = int(min(max(ctx), cap))
    raw = ops.attention_receipts(t(q), t(packets), fmts[0], fmts[1], t(np.asarray(base, np.int64)),
                                 t(np.asarray(ctx, np.int32)), cap, max_ctx, hkv, block)
    torch.cuda.synchronize()
    return raw.cpu().numpy().view(np.uint32)


CASES = [  # hq, hkv, capacity, block, ctx lengths
    (8, 2, 300, 128, [1, 127, 128, 129, 300, 420]),
    (16, 2, 512, 32, [33, 64, 5, 512]),
    (4, 4, 96, 32, [96, 97, 31]),
    (32, 8, 1024, 256, [1000, 257, 1, 4096]),
    (8, 1, 600, 512, [513, 600, 1200]),
    (6, 3, 200, 64, [64, 65, 199, 450]),      # odd kv heads: packets with a padded superblock
    (10, 5, 160, 96, [96, 97, 2, 161]),       # block not a power of two
]


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_receipts_match_oracle(torch_dev, fmts, case):
    torch, dev = torch_dev
    hq, hkv, cap, block, ctx = CASES[case]
    hd = 128
    print(f"receipts: case {case} fmts {fmts} hq {hq} hkv {hkv} cap {cap} block {block} ctx {ctx}", flush=True)
    rng = np.random.default_rng(700 + case)
    base = [i * cap for i in range(len(ctx))]
    packets = synth.random_packets(rng, cap * len(ctx), hkv * hd, *fmts)
    q = rng.standard_normal((len(ctx), hq, hd)).astype(np.float32)
    ops.device_error(clear=True)
    raw = _run(torch, dev, q, packets, fmts, base, ctx, cap, hkv, block)
    assert ops.device_error() == 0
    vals, words, tie = orc.attention_receipts(q, packets, fmts[0], fmts[1], np.asarray(base, np.int64),
                                              np.asarray(ctx, np.int32), cap, hkv, block)
    compare(raw, vals, words, tie, block, hd, f"case {case}")
    index = rows_heads(ctx, cap, block, hq)
    bounds(raw, index, block)
    f = raw.view(np.float32)
    out, M, Z = merge(f[:, 0], f[:, 1], f[:, 8 + block // 32:], index, len(ctx), hq)
    ref, m, z = orc.decode_attention(q, packets, fmts[0], fmts[1], base, ctx, cap, hkv)
    err = np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert err <= 1e-3, err


def test_receipts_identical_history(torch_dev):
    torch, dev = torch_dev
    hq, hkv, hd, cap, block = 8, 2, 128, 256, 128
    rng = np.random.default_rng(710)
    one = synth.random_packets(rng, 1, hkv * hd, orc.Q4_K, orc.Q6_K)
    packets = np.repeat(one, cap, 0)
    ctx = [1, 2, 129, 256]
    q = rng.standard_normal((len(ctx), hq, hd)).astype(np.float32)
    ops.device_error(clear=True)
    raw = _run(torch, dev, q, packets, (orc.Q4_K, orc.Q6_K), [0] * len(ctx), ctx, cap, hkv, block)
    assert ops.device_error() == 0
    vals, words, tie = orc.attention_receipts(q, packets, orc.Q4_K, orc.Q6_K, np.zeros(len(ctx), np.int64),
                                              np.asarray(ctx, np.int32), cap, hkv, block)
    assert not tie.any()
    compare(raw, vals, words, tie, block, hd, "identical")
    assert (raw[:, 3] == 1).all() and (raw[:, 4] == 1).all()        # one exp, one run per group
    count = raw[:, 2]
    assert ((raw[:, 7] & 4) != 0).tolist() == (count > 1).tolist()


def test_receipts_error_paths(torch_dev):
    torch, dev = torch_dev
    hq, hkv, hd, cap, block = 4, 1, 128, 64, 32
    rng = np.random.default_rng(720)
    packets = synth.random_packets(rng, cap, hkv * hd, orc.Q4_K, orc.Q6_K)
    q = rng.standard_normal((2, hq, hd)).astype(np.float32)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    ctx = t(np.array([40, 64], np.int32))
    need = ops.attention_receipt_records([40, 64], hq, cap, block)
    assert need == 4 * hq
    # too few records: the records past the end are not written, the error bit is set
    ops.device_error(clear=True)
    raw = ops.attention_receipts(t(q), t(packets), orc.Q4_K, orc.Q6_K, t(np.zeros(2, np.int64)), ctx, cap, 64,
                                 hkv, block, n_records=need - hq)
    torch.cuda.synchronize()
    assert ops.device_error() & 8
    full = ops.attention_receipts(t(q), t(packets), orc.Q4_K, orc.Q6_K, t(np.zeros(2, np.int64)), ctx, cap, 64,
                                  hkv, block)
    torch.cuda.synchronize()
    assert ops.device_error() == 0
    assert torch.equal(raw, full[:need - hq])
    # a slot outside the packet array: not read, error bit set
    ops.device_error(clear=True)
    ops.attention_receipts(t(q), t(packets), orc.Q4_K, orc.Q6_K, t(np.array([0, 10], np.int64)), ctx, cap, 64,
                           hkv, block)
    torch.cuda.synchronize()
    assert ops.device_error() & 8
    # max_ctx below a row's length: that row's records are refused, the error bit set
    ops.device_error(clear=True)
    ops.attention_receipts(t(q), t(packets), orc.Q4_K, orc.Q6_K, t(np.zeros(2, np.int64)), ctx, cap, 32, hkv,
                           block, n_records=need)
    torch.cuda.synchronize()
    assert ops.device_error() & 8
    # host refusals: nothing launched
    lib = _lib.load()
    buf = torch.zeros(need * (hd + 8 + block // 32), dtype=torch.int32, device=dev)
    qd, pd, bd = t(q), t(packets), t(np.zeros(2, np.int64))
    p = lambda x: ctypes.c_void_p(x.data_ptr())
    call = lambda **k: lib.rta_attention_receipts(
        p(qd), 2, hq, hkv, k.get("hd", hd), p(pd), orc.Q4_K, k.get("fv", orc.Q6_K), p(bd), p(ctx), cap, cap, 64,
        k.get("block", block), p(buf), need, None)
    assert call(block=48) == 7 and call(block=2048) == 7 and call(hd=64) == 7
    assert call(fv=orc.F32) == 3
    assert lib.rta_attention_receipts(None, 2, hq, hkv, hd, p(pd), orc.Q4_K, orc.Q6_K, p(bd), p(ctx), cap, cap,
                                      64, block, p(buf), need, None) == 1
    assert ops.attention_receipt_records([0, 0], hq, cap, block) == 0
