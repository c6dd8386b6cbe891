"""rta_decode_attention_noalloc (the variant that allocates nothing and works in the
library's own device scratch) through the C ABI: on two calls in a row, the second
with a smaller input, its outputs equal rta_decode_attention's on the same inputs
(bit for bit: the same kernels) and meet the oracle's bar; a call that needs more
than RTA_NOALLOC_SCRATCH_BYTES is refused before anything is launched."""
import numpy as np
import pytest

import oracle as orc
from conftest import tolerance_ok
from rta import _lib, ops, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def _case(torch, dev, seed, ctx, hq, hkv, fmts, gate):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    base = np.concatenate([[0], np.cumsum(ctx)[:-1]]).astype(np.int64)
    packets = synth.random_packets(rng, int(ctx.sum()), hkv * 128, *fmts)
    q = rng.standard_normal((len(ctx), hq, 128)).astype(np.float32)
    g = rng.normal(0, 2.0, q.shape).astype(np.float32) if gate else None
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    args = (t(q), t(packets), fmts[0], fmts[1], t(base), t(ctx), 1 << 20, int(ctx.max()), hkv)
    return args, t(g), (q, packets, fmts, base, ctx, g, hkv)


@pytest.mark.parametrize("fmts", [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)])
def test_noalloc_matches_workspace_entry_point(torch_dev, fmts):
    torch, dev = torch_dev
    big = synth.log_uniform_lengths(np.random.default_rng(81), 16, 512, 32768)
    big[0] = 32768
    cases = [(82, big, 16, 4, False), (83, [700, 3, 1500], 32, 8, True)]   # the second call is smaller
    assert ops.decode_attention_workspace_bytes(16, 16, 4, 128, 32768) <= _lib.NOALLOC_SCRATCH_BYTES
    for seed, ctx, hq, hkv, gate in cases:
        args, g, host = _case(torch, dev, seed, ctx, hq, hkv, fmts, gate)
        print(f"no-alloc: fmts {fmts} seed {seed} sequences {len(ctx)} heads {hq}/{hkv}", flush=True)
        out_n, m_n, z_n = ops.decode_attention_noalloc(*args, gate=g)
        out_w, m_w, z_w = ops.decode_attention(*args, gate=g)
        assert ops.device_error() == 0
        for a, b in ((out_n, out_w), (m_n, m_w), (z_n, z_w)):
            assert torch.equal(a, b)
        q, packets, f, base, c, gh, kv = host
        rout, rm, rz = orc.decode_attention(q, packets, f[0], f[1], base, c, 1 << 20, kv, gate=gh)
        for got, ref in ((out_n, rout), (m_n, rm), (z_n, rz)):
            ok, frac = tolerance_ok(got.cpu().numpy(), ref)
            assert ok, frac


def test_noalloc_refuses_oversized_calls(torch_dev):
    torch, dev = torch_dev
    nseq, hq, hkv, max_ctx = 64, 32, 8, 32768
    assert ops.decode_attention_workspace_bytes(nseq, hq, hkv, 128, max_ctx) > _lib.NOALLOC_SCRATCH_BYTES
    q = torch.zeros(nseq, hq, 128, device=dev)
    packets = torch.zeros(64 * ops.history_bytes(hkv * 128), dtype=torch.uint8, device=dev)
    base = torch.zeros(nseq, dtype=torch.int64, device=dev)
    ctx = torch.ones(nseq, dtype=torch.int32, device=dev)
    out = torch.full_like(q, 7.0)
    with pytest.raises(_lib.RtaError) as e:
        ops.decode_attention_noalloc(q, packets, orc.Q4_K, orc.Q6_K, base, ctx, 1 << 20, max_ctx, hkv, out=out)
    assert e.value.status == _lib.ERR_SCRATCH
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())                       # nothing was launched
