"""fp64 forward of one sequence through a model in the exporter's layout, composed from
the oracle's restatements (test infrastructure).

Every projection is read as the reference's quantizedWeight reads its descriptor
(resident_quant.glsl:20-31, orc.gemv_remap_f64): rows and axes through the mode the
exporter gave it (export.py:96-109), not through any re-layout of the worker.  The
layer ops follow the reference worker's order (optical_resident.cpp:455-530): full
layers QK-norm, RoPE on adjacent pairs, history packet, attention with the output
gate, O through its axis mode; recurrent layers the repeated key heads, short conv,
gates, delta rule and gated norm; then RMSNorm and the SwiGLU MLP; the LM head.
"""
import numpy as np

import oracle as orc

f32 = np.float32
HD = 128


class AssetReference:
    def __init__(self, spec, packed, floats):
        self.spec, self.packed, self.floats = spec, packed, floats
        self.d = spec["hidden_size"]
        self.kinds = spec["layer_types"]
        self.history = {l: [] for l, k in enumerate(self.kinds) if k == "full"}   # packets per position
        H = spec["state_heads"]
        self.rec = {l: np.zeros((1, H, HD, HD)) for l, k in enumerate(self.kinds) if k != "full"}
        self.conv = {l: np.zeros((1, 3 * H * HD, 3), f32) for l, k in enumerate(self.kinds) if k != "full"}
        self.pos = 0
        self.residual = []   # the residual stream after each layer of the last forward

    def _proj(self, tensor, rows, x, mode=0, first_row=0, key_rows=0, cols=None):
        fmt, raw = self.packed[tensor]   # uint8 [rows, row bytes]
        cols = cols or self.d
        raw = raw.reshape(raw.shape[0], -1)[first_row:]
        return orc.gemv_remap_f64(fmt, raw, raw.shape[0], rows, cols, mode, HD, self.spec["rotary_dim"], key_rows,
                                  np.atleast_2d(x).astype(f32))

    def forward(self, token):
        """Logits (fp64) after the token at the current position; the position advances."""
        sp, d = self.spec, self.d
        eps, theta, r = sp["norm_epsilon"], sp["rope_theta"], sp["rotary_dim"]
        fe, te = self.packed["token_embd.weight"]
        x = orc.embed(fe, te, sp["vocabulary_size"], d, [token]).astype(np.float64)
        # the exporter's q/k norm order (export.py:100-104): axis i of a head reads rot(i)
        perm = [orc.remap_row(3, HD, r, 0, i) for i in range(HD)]
        self.residual = []
        for l, kind in enumerate(self.kinds):
            p = f"blk.{l}."
            n = orc.rmsnorm(x.astype(f32), self.floats[p + "attn_norm.weight"], eps)
            if kind == "full":
                hq, hkv = sp["attention_heads"], sp["kv_heads"]
                gate_on = sp.get("attention_gate", False)
                q = self._proj(p + "attn_q.weight", hq * HD, n, 1 if gate_on else 3)
                k = self._proj(p + "attn_k.weight", hkv * HD, n, 3)
                v = self._proj(p + "attn_v.weight", hkv * HD, n, 3)
                gate = self._proj(p + "attn_q.weight", hq * HD, n, 2) if gate_on else None
                qn = np.tile(self.floats[p + "attn_q_norm.weight"][perm], hq)
                kn = np.tile(self.floats[p + "attn_k_norm.weight"][perm], hkv)
                q = orc.head_norm(q.astype(f32), hq, HD, w=qn, eps=eps)
                k = orc.head_norm(k.astype(f32), hkv, HD, w=kn, eps=eps)
                q = orc.rope(q.reshape(hq, HD).astype(f32), self.pos, r, theta)
                k = orc.rope(k.reshape(hkv, HD).astype(f32), self.pos, r, theta)
                self.history[l].append(orc.pack_history(k, v.astype(f32)))
                packets = np.stack(self.history[l])
                g = None if gate is None else gate.reshape(1, hq, HD).astype(f32)
                att, _, _ = orc.decode_attention(q.reshape(1, hq, HD), packets, orc.Q4_K, orc.Q6_K, [0],
                                                 [self.pos + 1], len(packets), hkv, gate=g)
                x = x + self._proj(p + "attn_output.weight", d, att.reshape(1, -1), 4, cols=hq * HD)
            else:
                H, KH = sp["state_heads"], sp["state_key_heads"]
                S, key = H * HD, KH * HD
                qkv = p + "attn_qkv.weight"
                q = self._proj(qkv, S, n, 5, 0, key)
                k = self._proj(qkv, S, n, 5, key, key)
                v = self._proj(qkv, S, n, 0, 2 * key)
                z = self._proj(p + "attn_gate.weight", S, n)
                b_in = self._proj(p + "ssm_beta.weight", H, n)
                a_in = self._proj(p + "ssm_alpha.weight", H, n)
                conv_w = self.floats[p + "ssm_conv1d.weight"].reshape(-1, 4)
                rep = H // KH
                conv_w = np.concatenate((np.tile(conv_w[:key], (rep, 1)), np.tile(conv_w[key:2 * key], (rep, 1)),
                                         conv_w[2 * key:]))
                decay, beta = orc.delta_gates(a_in.astype(f32), b_in.astype(f32), self.floats[p + "ssm_a"],
                                              self.floats[p + "ssm_dt.bias"])
                y, self.conv[l] = orc.short_conv(np.concatenate((q, k, v), 1).astype(f32), self.conv[l], conv_w, H,
                                                 HD, eps)
                self.rec[l], o = orc.delta_rule(self.rec[l], y[:, :S], y[:, S:2 * S], y[:, 2 * S:], decay, beta)
                o = orc.head_norm(o.astype(f32), H, HD, w=np.tile(self.floats[p + "ssm_norm.weight"], H),
                                  gate=z.astype(f32), eps=eps)
                x = x + self._proj(p + "ssm_out.weight", d, o, cols=S)
            n = orc.rmsnorm(x.astype(f32), self.floats[p + "post_attention_norm.weight"], eps)
            (fg, wg), (fu, wu), (fd, wd) = (self.packed[p + t + ".weight"] for t in ("ffn_gate", "ffn_up", "ffn_down"))
            _, y = orc.mlp_swiglu((fg, fu, fd), wg, wu, wd, d, sp["middle_size"], n.astype(f32))
            x = x + y
            self.residual.append(x[0].copy())
        n = orc.rmsnorm(x.astype(f32), self.floats["output_norm.weight"], eps)
        fl, wl = self.packed["output.weight"]
        self.pos += 1
        return orc.gemv_f64(fl, wl, sp["vocabulary_size"], d, n.astype(f32))[0]
