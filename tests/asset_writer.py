"""Writes a synthetic model in the exporter's on-disk layout (test infrastructure).

Restates ray_tracing/compiler/export.py:51-149 for given tensors instead of a GGUF /
safetensors source: optical_model.bin (RTRES004 + 9 words + parameter words),
geometry_weights.bin (raw payloads per layer, word padded), vocabulary.bin
(RTBASQ01 + vocab, hidden + payloads) and model.json (the model_spec the worker
reads).  Norm vectors are fp32; packed matrices are raw GGUF rows.
"""
import json
import struct
from pathlib import Path

import numpy as np

STRIDE = 64
ROW = {0: 4.0, 1: 2.0, 30: 2.0, 12: 144 / 256, 14: 210 / 256}


def row_bytes(fmt, cols):
    return int(cols * ROW[fmt])


def write(dest, spec, packed, floats):
    """spec: model_spec dict; packed: name -> (fmt, uint8 [rows, row_bytes]);
    floats: name -> fp32 array (norms, conv, dt bias, a).  Returns the header words."""
    dest = Path(dest)
    dest.mkdir(parents=True, exist_ok=True)
    d, middle, vocab = spec["hidden_size"], spec["middle_size"], spec["vocabulary_size"]
    types = spec["layer_types"]
    depth = len(types)
    hd, heads, kvh = spec["attention_head_dim"], spec["attention_heads"], spec["kv_heads"]
    header = np.zeros(32 + depth * STRIDE, np.uint32)
    header[:4] = [depth, depth, middle, 4]
    header[11:13] = [1, 1]
    parts, count = [], [len(header)]

    def add(value):
        v = np.ascontiguousarray(value, dtype="<f4").ravel().view("<u4")
        start = count[0]
        parts.append(v)
        count[0] += len(v)
        return start

    header[4] = add(floats["output_norm.weight"])
    header[7] = add(np.zeros(8))
    matrix_words = 0
    with open(dest / "geometry_weights.bin", "wb") as stream:
        for layer, kind in enumerate(types):
            base, prefix, start, written = 32 + layer * STRIDE, f"blk.{layer}.", matrix_words, {}

            def put(name):
                nonlocal matrix_words
                if name in written:
                    return written[name]
                fmt, raw = packed[prefix + name]
                raw = np.ascontiguousarray(raw, np.uint8)
                at = matrix_words - start
                stream.write(raw.tobytes())
                pad = (-raw.nbytes) % 4
                stream.write(bytes(pad))
                matrix_words += (raw.nbytes + pad) // 4
                written[name] = (at, fmt)
                return written[name]

            def descriptor(index, name, mode=0, offset_rows=0):
                at, fmt = put(name)
                rb = row_bytes(fmt, d)
                assert offset_rows * rb % 4 == 0
                off = base + 32 if index == 8 else base + 9 + index * 2
                header[off] = at + offset_rows * rb // 4
                header[off + 1] = fmt | (mode << 8)

            header[base] = add(floats[prefix + "attn_norm.weight"])
            header[base + 1] = add(floats[prefix + "post_attention_norm.weight"])
            header[base + 5] = add(np.zeros(8))
            if kind == "full":
                gate = spec.get("attention_gate", False)
                descriptor(0, "attn_q.weight", 1 if gate else 3)
                descriptor(1, "attn_k.weight", 3)
                descriptor(8, "attn_v.weight", 3)
                descriptor(2, "attn_output.weight", 4)
                if gate:
                    descriptor(6, "attn_q.weight", 2)
                r = spec["rotary_dim"]
                perm = np.arange(hd)
                perm[:r] = np.stack((np.arange(r // 2), np.arange(r // 2) + r // 2), -1).ravel()
                header[base + 2] = add(np.zeros(heads * hd // 2))
                for name, field in (("attn_q_norm.weight", 24), ("attn_k_norm.weight", 25)):
                    norm = floats[prefix + name][perm] if spec.get("qk_norm", True) else np.ones(hd)
                    header[base + field] = add(np.tile(norm, heads))
                header[base + 23] = heads
                header[base + 29] = r
            else:
                key, s = spec["state_key_heads"] * 128, spec["state_heads"] * 128
                descriptor(0, "attn_qkv.weight", 5)
                descriptor(1, "attn_qkv.weight", 5, key)
                descriptor(8, "attn_qkv.weight", 0, 2 * key)
                descriptor(2, "ssm_out.weight")
                descriptor(6, "attn_gate.weight")
                header[base + 34] = add(floats[prefix + "ssm_conv1d.weight"])
                header[base + 35], header[base + 39] = put("ssm_beta.weight")
                header[base + 36], header[base + 40] = put("ssm_alpha.weight")
                header[base + 37] = add(floats[prefix + "ssm_dt.bias"])
                header[base + 38] = add(floats[prefix + "ssm_a"])
                header[base + 24] = add(np.ones(s))
                header[base + 25] = add(np.ones(s))
                header[base + 31] = add(np.tile(floats[prefix + "ssm_norm.weight"], spec["state_heads"]))
                header[base + 23] = spec["state_heads"]
            descriptor(3, "ffn_gate.weight")
            descriptor(4, "ffn_down.weight")
            descriptor(5, "ffn_up.weight")
            header[base + 26] = header[base + 30] = 1 if kind == "full" else 2
            header[base + 27] = start
            header[base + 28] = matrix_words - start
    basis_words, seen = 0, {}
    with open(dest / "vocabulary.bin", "wb") as stream:
        stream.write(b"RTBASQ01")
        stream.write(struct.pack("<2I", vocab, d))
        for name, kind, offset in (("token_embd.weight", 13, 14), ("output.weight", 15, 16)):
            fmt, raw = packed[name]
            ident = id(raw)
            header[kind] = fmt
            header[offset] = seen.get(ident, basis_words)
            if ident not in seen:
                seen[ident] = basis_words
                stream.write(np.ascontiguousarray(raw, np.uint8).tobytes())
                pad = (-raw.nbytes) % 4
                stream.write(bytes(pad))
                basis_words += (raw.nbytes + pad) // 4
    params = np.concatenate((header, *parts))
    with open(dest / "optical_model.bin", "wb") as stream:
        stream.write(b"RTRES004")
        stream.write(struct.pack("<9I", d, depth, depth, middle, vocab, 4, len(params), matrix_words, 0))
        stream.write(params.astype("<u4").tobytes())
    meta = {"architecture": "synthetic", "model_spec": spec, "depth": depth, "hidden_size": d, "middle": middle,
            "vocabulary": vocab, "precision": "original coefficient formats"}
    (dest / "model.json").write_text(json.dumps(meta, indent=2))
    return params


def random_model(rng, spec, kquant_matrix):
    """Tensors of a small hybrid model: kquant_matrix(fmt, rows, cols) -> uint8 rows."""
    d, f, v = spec["hidden_size"], spec["middle_size"], spec["vocabulary_size"]
    hd, heads, kvh = spec["attention_head_dim"], spec["attention_heads"], spec["kv_heads"]
    packed, floats = {}, {}
    near1 = lambda n: (1.0 + rng.normal(0, 0.05, n)).astype(np.float32)  # noqa: E731
    floats["output_norm.weight"] = near1(d)
    for layer, kind in enumerate(spec["layer_types"]):
        p = f"blk.{layer}."
        floats[p + "attn_norm.weight"] = near1(d)
        floats[p + "post_attention_norm.weight"] = near1(d)
        packed[p + "ffn_gate.weight"] = (12, kquant_matrix(12, f, d))
        packed[p + "ffn_up.weight"] = (12, kquant_matrix(12, f, d))
        packed[p + "ffn_down.weight"] = (14, kquant_matrix(14, d, f))
        if kind == "full":
            qrows = heads * hd * (2 if spec.get("attention_gate", False) else 1)
            packed[p + "attn_q.weight"] = (12, kquant_matrix(12, qrows, d))
            packed[p + "attn_k.weight"] = (12, kquant_matrix(12, kvh * hd, d))
            packed[p + "attn_v.weight"] = (14, kquant_matrix(14, kvh * hd, d))
            packed[p + "attn_output.weight"] = (12, kquant_matrix(12, d, heads * hd))
            floats[p + "attn_q_norm.weight"] = near1(hd)
            floats[p + "attn_k_norm.weight"] = near1(hd)
        else:
            key, s = spec["state_key_heads"] * 128, spec["state_heads"] * 128
            packed[p + "attn_qkv.weight"] = (12, kquant_matrix(12, 2 * key + s, d))
            packed[p + "attn_gate.weight"] = (12, kquant_matrix(12, s, d))
            packed[p + "ssm_out.weight"] = (12, kquant_matrix(12, d, s))
            packed[p + "ssm_beta.weight"] = (0, rng.standard_normal((spec["state_heads"], d)).astype(np.float32)
                                             .view(np.uint8))
            packed[p + "ssm_alpha.weight"] = (0, rng.standard_normal((spec["state_heads"], d)).astype(np.float32)
                                              .view(np.uint8))
            floats[p + "ssm_conv1d.weight"] = rng.standard_normal((2 * key + s) * 4).astype(np.float32)
            floats[p + "ssm_dt.bias"] = rng.standard_normal(spec["state_heads"]).astype(np.float32)
            floats[p + "ssm_a"] = rng.standard_normal(spec["state_heads"]).astype(np.float32)
            floats[p + "ssm_norm.weight"] = near1(128)
    packed["token_embd.weight"] = (14, kquant_matrix(14, v, d))
    packed["output.weight"] = (14, kquant_matrix(14, v, d))
    return packed, floats


SMALL_SPEC = {"hidden_size": 512, "middle_size": 1024, "vocabulary_size": 1000,
              "layer_types": ["recurrent", "full"], "attention_heads": 8, "kv_heads": 2,
              "attention_head_dim": 128, "rotary_dim": 64, "state_heads": 2, "state_key_heads": 1,
              "attention_gate": False, "qk_norm": True, "rope_theta": 1e7, "norm_epsilon": 1e-6}
