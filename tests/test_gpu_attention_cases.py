"""GPU parity of decode attention on the reference verifier's edge cases and at the
sizes the decode step runs.

Edge cases: every case of verification/verify_attention_receipts.py:206-281 (cases)
and :286-331 (compact_cases) that the C ABI can express.  As the reference's op 14
does (resident_attention_runtime.inl:646-754), the fp32 K / V rows are packed into
history packets on the device (rta_pack_history, checked byte for byte against the
oracle's packer), and query row r, at position query_start + r, attends causally to
the positions from history_start on (slot = position - history_start, the worker's
origin); the oracle is the dense fp64 attention over the decoded packets
(verify_attention_receipts.py:84-114).  Both kernels run: K Q4_K / V Q6_K (the
reference layout, matrix cores) and K Q6_K / V Q4_K.

Sizes: tile lists of >= 2 tiles per workgroup with runs crossing sequences, the decode
step's own attention workload (32 sequences, 32 / 8 heads, contexts U[256, 8192]), the
full log-uniform [512, 32768] range of the GQA workload in both layouts, odd kv-head
counts and a wrapped ring on the matrix-core kernel.

Bar: max|gpu - ref| <= 1e-5 + 1e-3 max|ref| per output tensor; device error word 0."""
import numpy as np
import pytest

import oracle as orc
from conftest import assert_close
from rta import ops, synth

pytestmark = pytest.mark.gpu
REL, ABS = 1e-3, 1e-5
BLOCK = 256
LAYOUTS = [(orc.Q4_K, orc.Q6_K), (orc.Q6_K, orc.Q4_K)]


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    return torch, torch.device("cuda:0")


def to_dev(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


# ----------------------------------------------------- the verifier's cases ----
def verifier_cases(heads, kv, dim=128, block=BLOCK):
    """The inputs of verify_attention_receipts.py cases() and compact_cases(), same
    distributions and shapes (the seeds are this file's)."""
    rng = np.random.default_rng(20261110)
    f4 = np.float32

    def sample(name, count, rows=1, history_start=0):
        return {"name": name, "query": rng.normal(0, .25, (rows, heads, dim)).astype(f4),
                "keys": rng.normal(0, .25, (count, kv, dim)).astype(f4),
                "values": rng.normal(0, .5, (count, kv, dim)).astype(f4),
                "gate": rng.normal(0, .5, (rows, heads, dim)).astype(f4),
                "history_start": history_start, "query_start": history_start + count - rows}

    for count in sorted({1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 127, 128, 129, block - 1, block, block + 1,
                         2 * block + 1}):
        yield sample(f"boundary_{count}", count, min(count, 7))
    c = sample("zero_q_uniform", 33, 8)
    c["query"].fill(0)
    yield c
    c = sample("subnormal_and_signed_zero_q", 33)
    c["query"].fill(np.nextafter(f4(0), f4(1)))
    c["query"][:, :, 1::4] = f4(-0.)
    c["query"][:, :, 2::4] = f4(0.)
    c["query"][:, :, 3::4] *= f4(-1.)
    yield c
    c = sample("tiny_q_with_nontrivial_scores", 65, 17)
    c["query"].fill(0)
    c["query"][:, :, 0] = f4(1e-6)
    c["query"][:, :, 1] = f4(.25)
    c["keys"].fill(0)
    c["keys"][:, :, 0] = np.linspace(-1e6, 1e6, len(c["keys"]), dtype=f4)[:, None]
    c["values"][:, :, 0] = np.linspace(-1., 1., len(c["values"]), dtype=f4)[:, None]
    yield c
    c = sample("identical_q_distinct_keys", block + 1, 7)
    c["query"].fill(f4(.01))
    yield c
    c = sample("identical_scores_distinct_values", 2 * block + 1)
    c["query"].fill(0)
    c["query"][:, :, 0] = .25
    c["keys"].fill(0)
    c["keys"][:, :, 0] = 4.
    yield c
    c = sample("identical_values_distinct_scores", block + 17, 8)
    c["values"][:] = c["values"][0]
    yield c
    c = sample("value_runs_cross_16_and_block", 2 * block + 17)
    runs = rng.normal(0, .5, ((len(c["values"]) + 16) // 17, kv, dim)).astype(f4)
    c["values"][:] = runs[np.arange(len(c["values"])) // 17]
    yield c
    c = sample("large_signed_value_cancellation", block + 1)
    c["query"].fill(0)
    c["values"][:] = np.where(np.arange(len(c["values"]))[:, None, None] % 2, -1024., 1024.)
    c["values"][-1] = .25
    yield c
    c = sample("extreme_scores_and_gates", 129, 8)
    c["query"].fill(0)
    c["query"][:, :, 0] = 4096.
    c["keys"].fill(0)
    c["keys"][:, :, 0] = np.linspace(-16., 16., len(c["keys"]), dtype=f4)[:, None]
    c["gate"][:] = np.where(np.arange(dim) % 2, -80., 80.)
    yield c
    c = sample("gqa_head_identity", 33, 32)
    for head in range(kv):
        c["keys"][:, head] += f4(head / 4.)
        c["values"][:, head] += f4(head * 2.)
    yield c
    yield sample("nonzero_start_and_ring_slots", 2 * block + 1, 32,
                 history_start=3 * (1 << (2 * block).bit_length()) + 13)
    c = sample("early_queries_exclude_future", block + 33, 17, history_start=19)
    c["query_start"] = c["history_start"] + 7
    c["values"][32:] += f4(1e4)
    yield c
    count, rows = 2 * block + 17, 8
    line = np.linspace(-1., 1., count, dtype=f4)[:, None, None]
    for name in ("identical_packets", "one_value_column", "two_value_columns", "one_key_column",
                 "equivalence_splits_at_block", "uniform_complete_contributions", "nonconsecutive_packets",
                 "cancelled_key_group"):
        c = sample("compact_" + name, count, rows)
        if name == "identical_packets":
            c["keys"][:] = c["keys"][0]
            c["values"][:] = c["values"][0]
        elif name in ("one_value_column", "two_value_columns", "equivalence_splits_at_block"):
            c["values"][:] = line
            if name == "two_value_columns":
                c["values"][:] *= np.where(np.arange(dim) % 2, -1., 1.).astype(f4)
            elif name == "equivalence_splits_at_block":
                c["values"][:block, :, 1] *= -1
        elif name == "one_key_column":
            c["keys"][:] = line * .5
        elif name == "nonconsecutive_packets":
            ident = (np.arange(count) * 7) % 5
            c["keys"][:] = c["keys"][:5].copy()[ident]
            c["values"][:] = c["values"][:5].copy()[ident]
        elif name == "cancelled_key_group":
            c["keys"][:] = line * .5
            c["query"][:] = np.where(np.arange(dim) % 2, -.25, .25).astype(f4)
            c["query"][:, :, 0] += f4(1e-6)
        else:
            c["query"].fill(0)
            c["keys"].fill(0)
            c["values"].fill(.5)
        yield c
    q = np.zeros((1, heads, dim), f4)
    k = np.zeros((block, kv, dim), f4)
    v = np.full_like(k, .5)
    v[block // 4, :, min(120, dim - 1)] = -.5
    yield {"name": "compact_sampled_hash_collision", "query": q, "keys": k, "values": v, "gate": q,
           "query_start": block - 1, "history_start": 0}


def run_case(torch, dev, c, fmts, capacity):
    q, keys, values, gate = c["query"], c["keys"], c["values"], c["gate"]
    rows, heads, hd = q.shape
    count, kv = keys.shape[:2]
    kvw = kv * hd
    # pack every K / V row into slot (position - history_start), as op 14 does
    packets = torch.zeros(capacity * ops.history_bytes(kvw), dtype=torch.uint8, device=dev)
    slots = np.arange(count, dtype=np.int64)
    ops.pack_history(to_dev(torch, keys.reshape(count, kvw), dev), to_dev(torch, values.reshape(count, kvw), dev),
                     to_dev(torch, slots, dev), packets, *fmts)
    pk = packets.cpu().numpy().reshape(capacity, -1)
    for i in (0, count // 2, count - 1):
        assert np.array_equal(pk[i], orc.pack_history(keys[i].ravel(), values[i].ravel(), *fmts)), (c["name"], i)
    ctx = (c["query_start"] - c["history_start"] + np.arange(rows) + 1).astype(np.int32)
    base = np.zeros(rows, np.int64)
    out, m, z = ops.decode_attention(to_dev(torch, q, dev), packets, fmts[0], fmts[1], to_dev(torch, base, dev),
                                     to_dev(torch, ctx, dev), capacity, int(min(ctx.max(), capacity)), kv,
                                     gate=to_dev(torch, gate, dev))
    err = ops.device_error()
    rout, rm, rz = orc.decode_attention(q, pk[:count], fmts[0], fmts[1], base, ctx, capacity, kv, gate=gate)
    assert err == 0, (c["name"], err)
    out, m, z = out.cpu().numpy(), m.cpu().numpy(), z.cpu().numpy()
    assert_close(out, rout, f"{c['name']} output")
    assert_close(m, rm, f"{c['name']} maximum")
    assert_close(z, rz, f"{c['name']} normaliser")
    return out, m, z, ctx


@pytest.mark.parametrize("fmts", LAYOUTS)
@pytest.mark.parametrize("heads,kv", [(16, 4), (32, 8)])
def test_verifier_cases(torch_dev, fmts, heads, kv):
    torch, dev = torch_dev
    suite = list(verifier_cases(heads, kv))
    largest = max(len(c["keys"]) for c in suite)
    capacity = max(32, 1 << (largest - 1).bit_length())   # verify_attention_receipts.py:389
    for c in suite:
        out, m, z, ctx = run_case(torch, dev, c, fmts, capacity)
        if c["name"] in ("zero_q_uniform", "compact_sampled_hash_collision", "compact_uniform_complete_contributions"):
            # every score is exactly 0: m = 0 and Z = the visible count, exactly
            assert not m.any(), c["name"]
            assert np.array_equal(z, np.repeat(np.minimum(ctx, capacity)[:, None], heads, 1).astype(np.float32))
        if c["name"] == "subnormal_and_signed_zero_q":
            # scores vanish in fp32: uniform weights over the visible positions
            assert np.allclose(z, np.minimum(ctx, capacity)[:, None], rtol=1e-6)


@pytest.mark.parametrize("fmts", LAYOUTS)
def test_tiny_and_huge_queries(torch_dev, fmts):
    """Queries whose largest value is an fp32 subnormal, or near 1e30 (all scores of one
    sign beyond 1e29): outputs stay finite and match the oracle, the error word stays 0."""
    torch, dev = torch_dev
    rng = np.random.default_rng(41)
    heads, kv, count = 16, 4, 300
    keys = rng.normal(0, .25, (count, kv, 128)).astype(np.float32)
    values = rng.normal(0, .5, (count, kv, 128)).astype(np.float32)
    for name, scale in (("subnormal", 1e-40), ("tiny", 1e-30), ("large", 1e-3)):
        q = (rng.standard_normal((3, heads, 128)) * scale).astype(np.float32)
        c = {"name": name, "query": q, "keys": keys, "values": values, "gate": np.zeros_like(q),
             "query_start": count - 3, "history_start": 0}
        run_case(torch, dev, c, fmts, 512)


# ------------------------------------------------------------------ sizes ----
def _sized_case(torch, dev, seed, ctx, hq, hkv, fmts, capacity=None, gate=False):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    nseq = len(ctx)
    cap = int(capacity or (1 << 20))
    held = np.minimum(ctx, cap)
    base = np.concatenate([[0], np.cumsum(held)[:-1]]).astype(np.int64)
    packets = synth.random_packets(rng, int(held.sum()), hkv * 128, *fmts)
    q = rng.standard_normal((nseq, hq, 128)).astype(np.float32)
    g = rng.normal(0, 2.0, (nseq, hq, 128)).astype(np.float32) if gate else None
    out, m, z = ops.decode_attention(to_dev(torch, q, dev), to_dev(torch, packets, dev), fmts[0], fmts[1],
                                     to_dev(torch, base, dev), to_dev(torch, ctx, dev), cap, int(held.max()), hkv,
                                     gate=None if g is None else to_dev(torch, g, dev))
    err = ops.device_error()
    rout, rm, rz = orc.decode_attention(q, packets, fmts[0], fmts[1], base, ctx, cap, hkv, gate=g)
    assert err == 0
    assert_close(out.cpu().numpy(), rout, "attention output")
    assert_close(m.cpu().numpy(), rm, "attention max")
    assert_close(z.cpu().numpy(), rz, "attention Z")


@pytest.mark.parametrize("fmts", LAYOUTS)
def test_tile_split_16_sequences_32_8_heads(torch_dev, fmts):
    """16 sequences with contexts U[2048, 8192] at 32 / 8 heads: about 1,300 tiles of 64
    positions over 512 workgroups, so workgroups take several tiles and runs cross
    sequence boundaries (online max / Z rescale across tiles, several records per
    sequence in the merge)."""
    torch, dev = torch_dev
    ctx = np.random.default_rng(51).integers(2048, 8193, 16)
    _sized_case(torch, dev, 52, ctx, 32, 8, fmts, gate=True)


def test_tile_split_64_sequences_8_2_heads(torch_dev):
    torch, dev = torch_dev
    ctx = np.random.default_rng(53).integers(900, 1100, 64)
    ctx[:3] = [1, 64, 65]
    _sized_case(torch, dev, 54, ctx, 8, 2, (orc.Q4_K, orc.Q6_K))


@pytest.mark.parametrize("ctx", [[8192, 8192], [8192, 1], [8192, 8100, 64]])
def test_one_workgroup_per_cu_switch(torch_dev, ctx):
    """32 / 8 heads, K Q4_K / V Q6_K.  A tile list that cannot exceed one tile per compute
    unit (nseq x ceil(max_ctx / 64) <= 256 on MI355X) runs one 8-wave workgroup per CU, one
    kv head per wave: [8192, 8192] gives each of the 256 workgroups exactly one tile,
    [8192, 1] a ragged list of 129.  [8192, 8100, 64] (384 > 256) runs two 4-wave
    workgroups per CU again."""
    torch, dev = torch_dev
    _sized_case(torch, dev, 57, ctx, 32, 8, (orc.Q4_K, orc.Q6_K), gate=True)


def test_decode_step_attention_workload(torch_dev):
    """The attention call of one full layer of the 9B decode step at batch 32: 32 / 8 heads,
    contexts U[256, 8192] (2,200+ tiles, four or five per workgroup)."""
    torch, dev = torch_dev
    ctx = np.random.default_rng(20261115).integers(256, 8193, 32)
    _sized_case(torch, dev, 55, ctx, 32, 8, (orc.Q4_K, orc.Q6_K))


@pytest.mark.parametrize("fmts", LAYOUTS)
def test_gqa_workload_full_context_range(torch_dev, fmts):
    """16 sequences, 16 / 4 heads, contexts log-uniform over the whole [512, 32768]."""
    torch, dev = torch_dev
    ctx = synth.log_uniform_lengths(np.random.default_rng(20261112), 16, 512, 32768)
    ctx[:2] = [32768, 512]
    _sized_case(torch, dev, 8, ctx, 16, 4, fmts)


@pytest.mark.parametrize("hq,hkv", [(20, 5), (28, 7), (32, 16), (40, 5)])
def test_odd_and_wide_kv_head_counts(torch_dev, hq, hkv):
    """hkv 5 / 7 (a paired wave holding one kv head) and 16 (hkv > 8)."""
    torch, dev = torch_dev
    _sized_case(torch, dev, 56, [700, 3, 1500, 2100], hq, hkv, (orc.Q4_K, orc.Q6_K), gate=True)


def test_ring_wrap_matrix_core_layout(torch_dev):
    """A ring of 300 slots below contexts of 600 / 1000 on the K Q4_K / V Q6_K kernel."""
    torch, dev = torch_dev
    _sized_case(torch, dev, 57, [600, 1000, 90, 4000], 16, 4, (orc.Q4_K, orc.Q6_K), capacity=300)


@pytest.mark.parametrize("fmts", LAYOUTS)
@pytest.mark.parametrize("nseq", [65, 200])
def test_more_than_64_sequences(torch_dev, fmts, nseq):
    """Above 64 sequences the matrix-core kernels read their tile list from the plan a
    separate pass writes (Q6_K keys: attn_plan_kernel; Q4_K keys: the multi-wave scan of
    attn_plan_wave) instead of the one each wave builds in registers.  Mixed contexts,
    including 1, 64, 65 and several chunks."""
    torch, dev = torch_dev
    ctx = np.random.default_rng(60 + nseq).integers(1, 2500, nseq)
    ctx[:5] = [1, 64, 65, 4097, 2]
    ctx[-3:] = [1, 64, 65]
    _sized_case(torch, dev, 61 + nseq, ctx, 16, 4, fmts, gate=True)


def test_more_than_64_sequences_decode_step_heads(torch_dev):
    """300 sequences at the decode step's 32 / 8 heads (K Q4_K / V Q6_K)."""
    torch, dev = torch_dev
    ctx = np.random.default_rng(62).integers(1, 900, 300)
    ctx[:3] = [1, 64, 65]
    _sized_case(torch, dev, 63, ctx, 32, 8, (orc.Q4_K, orc.Q6_K))
