"""The fp32 CPU decode step (oracle/rta_cpu_step.c, the timed CPU baseline of the
decode benchmark) against the fp64 composition of the oracle's ops
(step_reference.reference_step) on a small hybrid decoder, on the CPU."""
from types import SimpleNamespace

import numpy as np

import oracle as orc
from conftest import tolerance_ok
from rta import synth
from step_reference import reference_step


def small_model(rng, hidden=512, layers=4, full_every=2, hq=4, hkv=2, H=2, ff=512, vocab=3001, capacity=64):
    shape = SimpleNamespace(hidden=hidden, layers=layers, full_every=full_every, q_heads=hq, kv_heads=hkv,
                            head_dim=128, rec_heads=H, ff=ff, vocab=vocab, capacity=capacity, fmt_embed=orc.Q4_K,
                            fmt_proj=orc.Q4_K, fmt_lm=orc.Q6_K, fmt_k=orc.Q4_K, fmt_v=orc.Q6_K, rope_rotary=128,
                            eps=1e-6, margin=1e-4, rope_theta=1e6, attn_gate=0, rec_key_heads=0, layer_formats=0)
    S = H * 128
    near1 = lambda n: (1.0 + 0.05 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    g = {"embed": synth.random_matrix(rng, orc.Q4_K, vocab, hidden), "norm_final": near1(hidden),
         "lm_head": synth.random_matrix(rng, orc.Q6_K, vocab, hidden)}
    for l in range(layers):
        g[f"{l}.norm_in"], g[f"{l}.norm_post"] = near1(hidden), near1(hidden)
        if l % full_every == full_every - 1:
            g[f"{l}.w_in"] = synth.random_matrix(rng, orc.Q4_K, (hq + 2 * hkv) * 128, hidden)
            g[f"{l}.w_o"] = synth.random_matrix(rng, orc.Q4_K, hidden, hq * 128)
            g[f"{l}.q_norm"], g[f"{l}.k_norm"] = near1(hq * 128), near1(hkv * 128)
        else:
            w = synth.random_matrix(rng, orc.Q4_K, 4 * S + 2 * H, hidden).reshape(4 * S + 2 * H, -1, 144)
            w[4 * S:, :, 0:2] = (np.abs(rng.standard_normal((2 * H, w.shape[1]))) * 1e-6).astype(np.float16)[
                ..., None].view(np.uint8)                     # a / b rows: tiny, decay near its target
            w[4 * S:, :, 2:4] = 0
            g[f"{l}.w_in"] = w.reshape(4 * S + 2 * H, -1)
            g[f"{l}.w_o"] = synth.random_matrix(rng, orc.Q4_K, hidden, S)
            g[f"{l}.conv_w"] = (0.5 * rng.standard_normal((3 * S, 4))).astype(np.float32)
            target = 0.9 + 0.099 * rng.random(H)
            dt = 2.0 * rng.random(H) - 1.0
            g[f"{l}.a_log"] = np.log(-np.log(target) / np.log1p(np.exp(dt))).astype(np.float32)
            g[f"{l}.dt_bias"] = dt.astype(np.float32)
            g[f"{l}.out_norm"] = near1(S)
        g[f"{l}.w_gate"] = synth.random_matrix(rng, orc.Q4_K, ff, hidden)
        g[f"{l}.w_up"] = synth.random_matrix(rng, orc.Q4_K, ff, hidden)
        g[f"{l}.w_down"] = synth.random_matrix(rng, orc.Q4_K, hidden, ff)
    return shape, g


def test_cpu_step_matches_fp64_composition():
    rng = np.random.default_rng(71)
    shape, g = small_model(rng)
    B, cap, H = 3, shape.capacity, shape.rec_heads
    nfull = shape.layers // shape.full_every
    nrec = shape.layers - nfull
    rec = (0.1 * rng.standard_normal((nrec, B, H, 128, 128))).astype(np.float32)
    conv = rng.standard_normal((nrec, B, 3 * H * 128, 3)).astype(np.float32)
    pb = orc.history_bytes(shape.kv_heads * 128)
    packets = np.stack([synth.random_packets(rng, B * cap, shape.kv_heads * 128, orc.Q4_K, orc.Q6_K)
                        for _ in range(nfull)]).reshape(nfull, B, cap, pb)
    ctx = np.array([5, 17, 70], np.int32)                 # 70 > capacity: the ring has wrapped
    tokens = rng.integers(0, shape.vocab, B).astype(np.uint32)
    cpu = orc.CpuStep(shape, g)
    fmts = {k: (orc.Q6_K if k == "lm_head" else orc.Q4_K) for k in g}
    m = SimpleNamespace(shape=shape, gguf=g, batch=B, fmts=fmts)
    for step in range(2):
        rec0, conv0, ctx0, tok0 = rec.copy(), conv.copy(), ctx.copy(), tokens.copy()
        logits = np.empty((B, shape.vocab), np.float32)
        cpu.step(B, rec, conv, packets, ctx, tokens, logits, threads=4)
        ref_logits, ref_rec, ref_conv, _, _ = reference_step(m, tok0, ctx0, rec0, conv0, packets)
        assert np.array_equal(ctx, ctx0 + 1)
        for b in range(B):
            ok, frac = tolerance_ok(logits[b], ref_logits[b])
            assert ok, (step, b, frac)
            assert int(tokens[b]) == orc.argmax_margin_f32(logits[b], 1e-4)
        assert np.array_equal(conv[..., :2], ref_conv[..., :2])
        assert tolerance_ok(conv[..., 2], ref_conv[..., 2])[0]
        assert tolerance_ok(rec, ref_rec)[0], tolerance_ok(rec, ref_rec)[1]
