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
