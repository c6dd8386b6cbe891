"""The fp64 reference of one rta_hybrid_decode_step, composed from the oracle's
restatements of every op, and the comparison of a model's steps with it.  Each step's
reference starts from the GPU's state before that step, so float drift does not
compound across steps.  The step runs with its capture on: the embedding rows are
checked bit exactly and the residual stream after every layer to the float bar; the
key and value rows each full layer quantised are checked against the reference's to
the float bar, and the new history packets byte for byte against the oracle's packer
(orc_pack_history, resident_history_quant.glsl:9-41) of those same rows.  The shifted
conv windows are checked bit exactly; the recurrent state, the new window entries,
logits and next tokens to the float bar / the margin rule."""
import numpy as np

import oracle as orc
from conftest import assert_close

REL, ABS = 1e-3, 1e-5
f32 = np.float32
Q4_K, Q6_K = orc.Q4_K, orc.Q6_K


def reference_step(m, tokens, ctx, rec, conv, packets_after):
    s, g = m.shape, m.gguf
    hq, hkv, hd, H, D, B, cap = s.q_heads, s.kv_heads, s.head_dim, s.rec_heads, s.hidden, m.batch, s.capacity
    S = H * hd
    KH = s.rec_key_heads or H
    fmt = lambda name: m.fmts[name] & 0xff   # the GGUF format a (possibly packed) matrix came from
    gemv = lambda name, rows, cols, x: orc.gemv_f64(fmt(name), g[name], rows, cols, x.astype(f32))
    parts = getattr(m, "parts", {})

    def in_projection(l, rows, x):   # w_in, or its parts side by side
        if l not in parts:
            return gemv(f"{l}.w_in", rows, D, x)
        assert sum(r for r, _ in parts[l]) == rows
        return np.concatenate([gemv(f"{l}.w_in.{i}", r, D, x) for i, (r, _) in enumerate(parts[l])], axis=1)
    x = orc.embed(s.fmt_embed, g["embed"], s.vocab, D, tokens).astype(np.float64)
    xs = [x.copy()]   # the residual stream: embedding rows, then after each layer
    new_rec, new_conv = rec.astype(np.float64).copy(), conv.copy()
    kv_new = []
    lf = lr = 0
    for l in range(s.layers):
        n = orc.rmsnorm(x.astype(f32), g[f"{l}.norm_in"], s.eps)
        if l % s.full_every == s.full_every - 1:
            rows = (hq * (2 if s.attn_gate else 1) + 2 * hkv) * hd
            p = in_projection(l, rows, n)
            q = orc.head_norm(p[:, :hq * hd].astype(f32), hq, hd, w=g[f"{l}.q_norm"], eps=s.eps)
            k = orc.head_norm(p[:, hq * hd:(hq + hkv) * hd].astype(f32), hkv, hd, w=g[f"{l}.k_norm"], eps=s.eps)
            q = np.stack([orc.rope(q[b].reshape(hq, hd).astype(f32), ctx[b], s.rope_rotary, s.rope_theta)
                          for b in range(B)])
            k = np.stack([orc.rope(k[b].reshape(hkv, hd).astype(f32), ctx[b], s.rope_rotary, s.rope_theta)
                          for b in range(B)]).reshape(B, -1)
            kv_new.append((k, p[:, (hq + hkv) * hd:(hq + 2 * hkv) * hd]))
            # the output gate (resident_ray.comp:75-76): rows after q | k | v
            gate = p[:, (hq + 2 * hkv) * hd:].reshape(B, hq, hd).astype(f32) if s.attn_gate else None
            flat = packets_after[lf].reshape(B * cap, -1)
            attn, _, _ = orc.decode_attention(q.astype(f32), flat, s.fmt_k, s.fmt_v, [b * cap for b in range(B)],
                                              [c + 1 for c in ctx], cap, hkv, gate=gate)
            if getattr(s, "o_axis_remap", 0):   # dim d of a head back to the exporter's column rot(d)
                to = [orc.remap_row(3, hd, s.rope_rotary, 0, r) for r in range(hq * hd)]
                out = np.empty_like(attn.reshape(B, -1))
                out[:, to] = attn.reshape(B, -1)
                attn = out
            x = x + gemv(f"{l}.w_o", D, hq * hd, attn.reshape(B, -1))
            lf += 1
        else:
            sep = f"{l}.w_a" in g
            rows = 2 * KH * hd + 2 * S + (0 if sep else 2 * H)
            p = in_projection(l, rows, n)
            # q and k of delta-net head h are rows of key head h % KH: the key repeat of
            # resident_quant.glsl:26 (mode 5) over the logical rows
            rep = np.array([orc.remap_row(5, 0, 0, KH * hd, r) for r in range(S)])
            qkv = np.concatenate((p[:, rep], p[:, KH * hd + rep], p[:, 2 * KH * hd:2 * KH * hd + S]), axis=1)
            z = p[:, 2 * KH * hd + S:2 * KH * hd + 2 * S]
            if sep:
                a_in, b_in = gemv(f"{l}.w_a", H, D, n), gemv(f"{l}.w_b", H, D, n)
            else:
                a_in, b_in = p[:, 2 * KH * hd + 2 * S:2 * KH * hd + 2 * S + H], p[:, 2 * KH * hd + 2 * S + H:]
            decay, beta = orc.delta_gates(a_in.astype(f32), b_in.astype(f32), g[f"{l}.a_log"], g[f"{l}.dt_bias"])
            y, ns = orc.short_conv(qkv.astype(f32), conv[lr], g[f"{l}.conv_w"], H, hd, s.eps)
            new_conv[lr] = ns
            st, o = orc.delta_rule(rec[lr].astype(np.float64), y[:, :S], y[:, S:2 * S], y[:, 2 * S:], decay, beta)
            new_rec[lr] = st
            o = orc.head_norm(o.astype(f32), H, hd, w=g[f"{l}.out_norm"], gate=z.astype(f32), eps=s.eps)
            x = x + gemv(f"{l}.w_o", D, S, o)
            lr += 1
        n = orc.rmsnorm(x.astype(f32), g[f"{l}.norm_post"], s.eps)
        _, y = orc.mlp_swiglu((fmt(f"{l}.w_gate"), fmt(f"{l}.w_up"), fmt(f"{l}.w_down")), g[f"{l}.w_gate"],
                              g[f"{l}.w_up"], g[f"{l}.w_down"], D, s.ff, n.astype(f32))
        x = x + y
        xs.append(x.copy())
    n = orc.rmsnorm(x.astype(f32), g["norm_final"], s.eps)
    logits = gemv("lm_head", s.vocab, D, n)
    return logits, new_rec, new_conv, kv_new, xs


def check_steps(m, steps=2):
    shape, batch = m.shape, m.batch
    cap = shape.capacity
    kvw = shape.kv_heads * 128
    for step in range(steps):
        tokens = m.tokens.cpu().numpy().view(np.uint32).copy()
        pos = m.state_view("ctx")
        rec, conv = m.state_view("recurrent"), m.state_view("conv")
        m.step(logits=True, capture=True)
        got_tokens = m.tokens.cpu().numpy().view(np.uint32)
        got_logits = m.logits.cpu().numpy()
        packets = m.state_view("packets")
        ref_logits, ref_rec, ref_conv, kv_new, ref_x = reference_step(m, tokens, pos, rec, conv, packets)
        assert np.array_equal(m.state_view("ctx"), pos + 1)
        res = m.residual.cpu().numpy()
        assert np.array_equal(res[0], ref_x[0].astype(f32)), step   # embedding rows: exact
        for l in range(1, shape.layers + 1):
            for b in range(batch):
                assert_close(res[l, b], ref_x[l][b], f"step {step} residual after layer {l - 1} row {b}")
        for b in range(batch):
            assert_close(got_logits[b], ref_logits[b], f"step {step} logits row {b}")
            assert int(got_tokens[b]) == orc.argmax_margin_f32(got_logits[b], 1e-4), (step, b)
        got_conv = m.state_view("conv")
        assert np.array_equal(got_conv[..., :2], ref_conv[..., :2]), step     # shifted window: exact
        assert_close(got_conv[..., 2], ref_conv[..., 2], f"step {step} conv window (new raw value)")
        assert_close(m.state_view("recurrent"), ref_rec, f"step {step} recurrent state")
        # each full layer's new packet: the oracle's packer of the rows the step quantised,
        # byte for byte; those rows: the reference's normed, rotated k and its v
        kv = m.kv.cpu().numpy()
        nb = orc.history_bytes(kvw)
        for lf, (k, v) in enumerate(kv_new):
            for b in range(batch):
                assert_close(kv[lf, b, 0], k[b], f"step {step} full layer {lf} key row {b}")
                assert_close(kv[lf, b, 1], v[b], f"step {step} full layer {lf} value row {b}")
                want = orc.pack_history(kv[lf, b, 0], kv[lf, b, 1], shape.fmt_k, shape.fmt_v)
                got = packets[lf, b, pos[b] % cap, :nb]
                bad = np.flatnonzero(got != want)
                assert bad.size == 0, (f"step {step} full layer {lf} row {b}: packet bytes differ at {bad[:8]} "
                                       f"(got {got[bad[:8]]}, oracle {want[bad[:8]]})")
