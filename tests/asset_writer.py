"""Writes a synthetic model in the exporter's on-disk layout (test infrastructure).

The files and the meaning of each word are those compiler/export.py:51-149 produces
(optical_model.bin: RTRES004, 9 words, then the parameter words; geometry_weights.bin:
every layer's matrix payloads, word padded; vocabulary.bin: RTBASQ01, vocab, hidden,
then the embedding and LM-head payloads; model.json with the model_spec the worker
reads), written here from the word map below for given tensors instead of a GGUF /
safetensors source.  Norm vectors are fp32; matrices are raw GGUF rows.
"""
import json
import struct
from pathlib import Path

import numpy as np

# ---- the word map of the parameter region (export.py:87-123) ----------------------
STRIDE = 64          # words per layer record, after 32 global words
GLOBAL_WORDS = 32
G_DEPTH, G_BLOCKS, G_MIDDLE, G_FOUR = 0, 1, 2, 3
G_OUTPUT_NORM, G_SPARE_VECTOR = 4, 7
G_FLAGS = (11, 12)                     # both 1
G_EMBED_CODE, G_EMBED_AT, G_LM_CODE, G_LM_AT = 13, 14, 15, 16
L_NORM_IN, L_NORM_POST, L_ROTARY_ZERO, L_SPARE_VECTOR = 0, 1, 2, 5
L_HEADS, L_NORM_A, L_NORM_B, L_KIND_A, L_MATRIX_START, L_MATRIX_WORDS, L_ROTARY, L_KIND_B = 23, 24, 25, 26, 27, 28, 29, 30
L_OUT_NORM, L_CONV, L_DT_BIAS, L_A = 31, 34, 37, 38
L_BETA, L_ALPHA = (35, 39), (36, 40)   # (payload word offset, format code) of a separate matrix


def descriptor_word(index):
    """First of the two words (offset, format | mode << 8) of projection descriptor index."""
    return 32 if index == 8 else 9 + 2 * index


# projections per layer kind: (descriptor index, tensor, mode, first row) -- the modes
# and row offsets export.py:96-108 gives them
def _full_projections(spec):
    gate = spec.get("attention_gate", False)
    rows = [(0, "attn_q.weight", 1 if gate else 3, 0), (1, "attn_k.weight", 3, 0), (8, "attn_v.weight", 3, 0),
            (2, "attn_output.weight", 4, 0)]
    return rows + ([(6, "attn_q.weight", 2, 0)] if gate else [])


def _recurrent_projections(spec):
    key = spec["state_key_heads"] * 128
    return [(0, "attn_qkv.weight", 5, 0), (1, "attn_qkv.weight", 5, key), (8, "attn_qkv.weight", 0, 2 * key),
            (2, "ssm_out.weight", 0, 0), (6, "attn_gate.weight", 0, 0)]


_MLP = [(3, "ffn_gate.weight", 0, 0), (4, "ffn_down.weight", 0, 0), (5, "ffn_up.weight", 0, 0)]
ROW = {0: 4.0, 1: 2.0, 30: 2.0, 12: 144 / 256, 14: 210 / 256}


def row_bytes(fmt, cols):
    return int(cols * ROW[fmt])


class _Words:
    """An append-only run of little-endian 32-bit words; add() returns where a block starts."""

    def __init__(self, first=0):
        self.blocks, self.size = [], first

    def add(self, words):
        at = self.size
        self.blocks.append(words)
        self.size += len(words)
        return at

    def add_floats(self, values):
        return self.add(np.ascontiguousarray(values, dtype="<f4").ravel().view("<u4"))

    def add_bytes(self, raw):
        raw = np.ascontiguousarray(raw, np.uint8).ravel()
        return self.add(np.concatenate((raw, np.zeros((-raw.size) % 4, np.uint8))).view("<u4"))

    def array(self):
        return np.concatenate(self.blocks) if self.blocks else np.zeros(0, "<u4")


def _rotary_pairs(hd, r):
    """The norm order of the detector's rotary-pair layout: exported index of axis i."""
    order = np.arange(hd)
    order[:r] = np.arange(r).reshape(2, r // 2).T.ravel()
    return order


def write(dest, spec, packed, floats):
    """spec: model_spec dict; packed: name -> (fmt, uint8 [rows, row_bytes]);
    floats: name -> fp32 array (norms, conv, dt bias, a).  Returns the parameter words."""
    dest = Path(dest)
    dest.mkdir(parents=True, exist_ok=True)
    d, middle, vocab, kinds = spec["hidden_size"], spec["middle_size"], spec["vocabulary_size"], spec["layer_types"]
    hd, heads = spec["attention_head_dim"], spec["attention_heads"]
    depth = len(kinds)
    head = np.zeros(GLOBAL_WORDS + depth * STRIDE, "<u4")
    vectors = _Words(first=len(head))          # parameter words after the header
    matrices = _Words()                         # geometry_weights.bin
    head[[G_DEPTH, G_BLOCKS, G_MIDDLE, G_FOUR]] = [depth, depth, middle, 4]
    head[list(G_FLAGS)] = 1
    head[G_OUTPUT_NORM] = vectors.add_floats(floats["output_norm.weight"])
    head[G_SPARE_VECTOR] = vectors.add_floats(np.zeros(8))
    for layer, kind in enumerate(kinds):
        rec = head[GLOBAL_WORDS + layer * STRIDE:GLOBAL_WORDS + (layer + 1) * STRIDE]   # a view
        name = lambda t: f"blk.{layer}.{t}"   # noqa: E731
        first_word, placed = matrices.size, {}

        def place(tensor):   # a payload once per layer, at its word offset inside the layer
            if tensor not in placed:
                fmt, raw = packed[name(tensor)]
                placed[tensor] = (matrices.add_bytes(raw) - first_word, fmt)
            return placed[tensor]

        rec[L_NORM_IN] = vectors.add_floats(floats[name("attn_norm.weight")])
        rec[L_NORM_POST] = vectors.add_floats(floats[name("post_attention_norm.weight")])
        rec[L_SPARE_VECTOR] = vectors.add_floats(np.zeros(8))
        full = kind == "full"

        def describe(projections):
            for index, tensor, mode, row0 in projections:
                at, fmt = place(tensor)
                skip = row0 * row_bytes(fmt, d)
                assert skip % 4 == 0, "a row offset must be whole words"
                w = descriptor_word(index)
                rec[w], rec[w + 1] = at + skip // 4, fmt | (mode << 8)

        describe(_full_projections(spec) if full else _recurrent_projections(spec))
        if full:
            r = spec["rotary_dim"]
            order = _rotary_pairs(hd, r)
            rec[L_ROTARY_ZERO] = vectors.add_floats(np.zeros(heads * hd // 2))
            for field, tensor in ((L_NORM_A, "attn_q_norm.weight"), (L_NORM_B, "attn_k_norm.weight")):
                norm = floats[name(tensor)][order] if spec.get("qk_norm", True) else np.ones(hd)
                rec[field] = vectors.add_floats(np.tile(norm, heads))
            rec[L_HEADS], rec[L_ROTARY] = heads, r
        else:
            sh, key = spec["state_heads"], spec["state_key_heads"] * 128
            # the q and k channels' conv taps repeated over the key repeat, like their rows
            conv = floats[name("ssm_conv1d.weight")].reshape(-1, 4)
            rep = sh // spec["state_key_heads"]
            rec[L_CONV] = vectors.add_floats(np.concatenate((np.tile(conv[:key], (rep, 1)),
                                                             np.tile(conv[key:2 * key], (rep, 1)), conv[2 * key:])))
            for (w_at, w_code), tensor in ((L_BETA, "ssm_beta.weight"), (L_ALPHA, "ssm_alpha.weight")):
                rec[w_at], rec[w_code] = place(tensor)
            rec[L_DT_BIAS] = vectors.add_floats(floats[name("ssm_dt.bias")])
            rec[L_A] = vectors.add_floats(floats[name("ssm_a")])
            rec[L_NORM_A] = vectors.add_floats(np.ones(sh * 128))
            rec[L_NORM_B] = vectors.add_floats(np.ones(sh * 128))
            rec[L_OUT_NORM] = vectors.add_floats(np.tile(floats[name("ssm_norm.weight")], sh))
            rec[L_HEADS] = sh
        describe(_MLP)   # (after the delta-net's beta / alpha payloads, in the exporter's order)
        rec[L_KIND_A] = rec[L_KIND_B] = 1 if full else 2
        rec[L_MATRIX_START], rec[L_MATRIX_WORDS] = first_word, matrices.size - first_word
    (dest / "geometry_weights.bin").write_bytes(matrices.array().tobytes())
    basis, where = _Words(), {}
    for tensor, code_word, at_word in (("token_embd.weight", G_EMBED_CODE, G_EMBED_AT),
                                       ("output.weight", G_LM_CODE, G_LM_AT)):
        fmt, raw = packed[tensor]
        if id(raw) not in where:   # a tied LM head shares the embedding's payload
            where[id(raw)] = basis.add_bytes(raw)
        head[code_word], head[at_word] = fmt, where[id(raw)]
    (dest / "vocabulary.bin").write_bytes(b"RTBASQ01" + struct.pack("<2I", vocab, d) + basis.array().tobytes())
    params = np.concatenate((head, vectors.array()))
    (dest / "optical_model.bin").write_bytes(
        b"RTRES004" + struct.pack("<9I", d, depth, depth, middle, vocab, 4, len(params), matrices.size, 0) +
        params.astype("<u4").tobytes())
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
