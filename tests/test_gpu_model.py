"""End-to-end parity of rta_hybrid_decode_step (a small hybrid decoder: delta-net
recurrent layers and full-attention layers) against an fp64 step composed from the
oracle's restatements of every op (step_reference.check_steps), over two steps."""
import pytest

from step_reference import check_steps

pytestmark = pytest.mark.gpu


# hidden 256 puts every packed in-projection in one K slab (written straight to the
# projection rows); hidden 512 leaves two slabs for the fused consumers to add
@pytest.mark.parametrize("packed,hidden", [(False, 512), (True, 512), (True, 256)])
def test_hybrid_decode_steps(packed, hidden):
    from rta import model
    from rta._lib import Q4_K, Q6_K, TILED
    shape = model.HybridShape(hidden=hidden, layers=4, full_every=2, q_heads=4, kv_heads=2, head_dim=128, rec_heads=2,
                              ff=512, vocab=3001, capacity=64, fmt_embed=Q4_K,
                              fmt_proj=Q4_K | (TILED if packed else 0), fmt_lm=Q6_K | (TILED if packed else 0),
                              fmt_k=Q4_K, fmt_v=Q6_K, rope_rotary=128, eps=1e-6, margin=1e-4, rope_theta=1e6)
    ctx = [5, 17, 70]                                      # 70 > capacity: the ring has wrapped
    m = model.DecodeModel(shape, 3, ctx, seed=7, keep_gguf=True)
    check_steps(m, 2)


# Batch 1: the GGUF-row readouts take the RMSNorm in front of them themselves (x is the
# residual row), the packed ones run the matrix-core paths with one real row.
@pytest.mark.parametrize("packed", [False, True])
def test_hybrid_decode_steps_batch1(packed):
    from rta import model
    from rta._lib import Q4_K, Q6_K, TILED
    shape = model.HybridShape(hidden=512, layers=4, full_every=2, q_heads=4, kv_heads=2, head_dim=128, rec_heads=2,
                              ff=768, vocab=3001, capacity=64, fmt_embed=Q4_K,
                              fmt_proj=Q4_K | (TILED if packed else 0), fmt_lm=Q6_K | (TILED if packed else 0),
                              fmt_k=Q4_K, fmt_v=Q6_K, rope_rotary=128, eps=1e-6, margin=1e-4, rope_theta=1e6)
    m = model.DecodeModel(shape, 1, [70], seed=9, keep_gguf=True)
    check_steps(m, 3)


# What the exporter emits beyond the plain layout (compiler/export.py:96-113): the
# attention output gate, fewer delta-net key heads than heads (repeated), the a / b rows
# as matrices of their own (F32, as ssm_alpha / ssm_beta), and a format per matrix --
# packed, GGUF rows and float mixed within and across layers.  Batch 3 and 20 run the
# fused paths (one batch tile of 16 and 32 rows), 40 the plain ones.
def _exporter_fmts(l, full):
    from rta._lib import BF16, F16, Q4_K, Q6_K, TILED
    if full:
        return {"in": Q4_K | TILED, "o": Q6_K, "gate_up": Q4_K | TILED, "down": Q6_K | TILED}
    if l % 2:
        return {"in": Q6_K | TILED, "o": Q4_K | TILED, "gate_up": Q4_K, "down": BF16, "ab": 0}
    return {"in": Q4_K, "o": F16, "gate_up": Q6_K | TILED, "down": Q4_K | TILED, "ab": 0}


def _part_fmts(l, full):
    from rta._lib import F32, Q4_K, Q6_K, TILED
    return [Q4_K, Q6_K] if full else [Q4_K, Q6_K | TILED, F32]


@pytest.mark.parametrize("batch", [1, 5, 32])
def test_hybrid_decode_steps_in_projection_parts(batch):
    """In-projections as matrices of their own formats (the exporter's attn_q / attn_k /
    attn_v / attn_qkv / attn_gate), and the attention output in the exporter's column
    order in front of w_o (o_axis_remap)."""
    from rta import model
    from rta._lib import Q4_K, Q6_K, TILED
    shape = model.HybridShape(hidden=512, layers=4, full_every=2, q_heads=4, kv_heads=2, head_dim=128, rec_heads=4,
                              ff=512, vocab=3001, capacity=64, fmt_embed=Q4_K, fmt_proj=Q4_K,
                              fmt_lm=Q6_K, fmt_k=Q4_K, fmt_v=Q6_K, rope_rotary=64, eps=1e-6, margin=1e-4,
                              rope_theta=1e6, attn_gate=1, rec_key_heads=2, layer_formats=1, o_axis_remap=1)
    ctx = [(7 + 11 * b) % 90 for b in range(batch)]
    fmts = lambda l, full: {"in": Q4_K, "o": Q4_K, "gate_up": Q4_K, "down": Q6_K | (TILED if batch > 1 else 0),  # noqa
                            "ab": 0}
    m = model.DecodeModel(shape, batch, ctx, seed=31 + batch, keep_gguf=True, layer_fmts=fmts, separate_ab=True,
                          in_parts=_part_fmts)
    check_steps(m, 2)


@pytest.mark.parametrize("batch", [1, 3, 20, 40])
def test_hybrid_decode_steps_exported_layout(batch):
    from rta import model
    from rta._lib import Q4_K, Q6_K, TILED
    shape = model.HybridShape(hidden=512, layers=4, full_every=2, q_heads=4, kv_heads=2, head_dim=128, rec_heads=4,
                              ff=512, vocab=3001, capacity=64, fmt_embed=Q4_K, fmt_proj=Q4_K | TILED,
                              fmt_lm=Q6_K | TILED, fmt_k=Q4_K, fmt_v=Q6_K, rope_rotary=64, eps=1e-6, margin=1e-4,
                              rope_theta=1e6, attn_gate=1, rec_key_heads=2, layer_formats=1)
    ctx = [(5 + 13 * b) % 90 for b in range(batch)]
    m = model.DecodeModel(shape, batch, ctx, seed=11 + batch, keep_gguf=True, layer_fmts=_exporter_fmts,
                          separate_ab=True)
    check_steps(m, 2)


# Both history field orders (the reference's K Q4_K / V Q6_K and the swapped K Q6_K / V
# Q4_K) and an odd kv-head count (3 heads: the second superblock of each field half
# zeros): every step's packets byte for byte against the oracle's packer of the rows the
# step quantised (step_reference.check_steps).
@pytest.mark.parametrize("fmt_k,hq,hkv", [("Q6_K", 4, 2), ("Q4_K", 6, 3), ("Q6_K", 6, 3)])
def test_hybrid_decode_steps_history_layouts(fmt_k, hq, hkv):
    from rta import model
    from rta._lib import Q4_K, Q6_K, TILED
    fk = Q4_K if fmt_k == "Q4_K" else Q6_K
    fv = Q6_K if fk == Q4_K else Q4_K
    shape = model.HybridShape(hidden=512, layers=4, full_every=2, q_heads=hq, kv_heads=hkv, head_dim=128,
                              rec_heads=2, ff=512, vocab=3001, capacity=64, fmt_embed=Q4_K, fmt_proj=Q4_K | TILED,
                              fmt_lm=Q6_K | TILED, fmt_k=fk, fmt_v=fv, rope_rotary=128, eps=1e-6, margin=1e-4,
                              rope_theta=1e6)
    m = model.DecodeModel(shape, 5, [3, 40, 64, 65, 100], seed=41 + hkv, keep_gguf=True)
    check_steps(m, 2)
