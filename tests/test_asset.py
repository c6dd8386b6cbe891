"""The asset reader (rta_asset_*, host only) against models written in the exporter's
layout (export.py:51-149, restated in asset_writer.py): every descriptor, vector,
header word and basis payload comes back byte for byte, and damaged files fail with
the reference loader's messages (optical_resident.cpp:139-152)."""
import copy
import struct

import numpy as np
import pytest

import asset_writer as aw
from rta import asset as ra
from rta import synth


def _model(tmp_path, spec=None, seed=3):
    spec = copy.deepcopy(spec or aw.SMALL_SPEC)
    rng = np.random.default_rng(seed)
    packed, floats = aw.random_model(rng, spec, lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    params = aw.write(tmp_path, spec, packed, floats)
    return spec, packed, floats, params


def test_reader_returns_every_tensor(tmp_path):
    spec, packed, floats, params = _model(tmp_path)
    d, f = spec["hidden_size"], spec["middle_size"]
    hd, heads = spec["attention_head_dim"], spec["attention_heads"]
    with ra.open_dir(tmp_path) as a:
        i = a.info
        assert (i.hidden, i.depth, i.blocks, i.middle, i.vocab, i.quantization, i.step) == \
            (d, 2, 2, f, spec["vocabulary_size"], 4, 0)
        assert i.param_words == len(params)
        np.testing.assert_array_equal(a.params(), params)
        np.testing.assert_array_equal(a.vector(-1, 4, d), floats["output_norm.weight"])
        for layer, kind in enumerate(spec["layer_types"]):
            p = f"blk.{layer}."
            np.testing.assert_array_equal(a.vector(layer, 0, d), floats[p + "attn_norm.weight"])
            np.testing.assert_array_equal(a.vector(layer, 1, d), floats[p + "post_attention_norm.weight"])
            assert a.word(layer, 26) == (1 if kind == "full" else 2)
            for idx, name in ((ra.FFN_GATE, "ffn_gate"), (ra.FFN_UP, "ffn_up"), (ra.FFN_DOWN, "ffn_down")):
                fmt, raw = packed[p + name + ".weight"]
                got_fmt, mode, got = a.matrix(layer, idx, raw.nbytes)
                assert (got_fmt, mode) == (fmt, 0)
                np.testing.assert_array_equal(got, raw.ravel())
            if kind == "full":
                assert a.word(layer, 23) == heads and a.word(layer, 29) == spec["rotary_dim"]
                for idx, name, mode in ((ra.Q, "attn_q", 3), (ra.K, "attn_k", 3), (ra.V, "attn_v", 3),
                                        (ra.OUT, "attn_output", 4)):
                    fmt, raw = packed[p + name + ".weight"]
                    got_fmt, got_mode, got = a.matrix(layer, idx, raw.nbytes)
                    assert (got_fmt, got_mode) == (fmt, mode), name
                    np.testing.assert_array_equal(got, raw.ravel())
                # q/k norms: the rotary half-split permutation, tiled over the heads
                r = spec["rotary_dim"]
                perm = np.concatenate([np.stack((np.arange(r // 2), np.arange(r // 2) + r // 2), -1).ravel(),
                                       np.arange(r, hd)])
                np.testing.assert_array_equal(a.vector(layer, 24, heads * hd),
                                              np.tile(floats[p + "attn_q_norm.weight"][perm], heads))
            else:
                fmt, raw = packed[p + "attn_qkv.weight"]
                rb = aw.row_bytes(fmt, d)
                key = spec["state_key_heads"] * 128
                for idx, r0, mode in ((ra.Q, 0, 5), (ra.K, key, 5), (ra.V, 2 * key, 0)):
                    got_fmt, got_mode, got = a.matrix(layer, idx, rb * 16)
                    assert (got_fmt, got_mode) == (fmt, mode)
                    np.testing.assert_array_equal(got, raw[r0:r0 + 16].ravel())
                np.testing.assert_array_equal(a.vector(layer, 37, spec["state_heads"]), floats[p + "ssm_dt.bias"])
                # conv taps of the q / k channels tiled over the key repeat (export.py:115-116)
                s_w, rep = spec["state_heads"] * 128, spec["state_heads"] // spec["state_key_heads"]
                conv = floats[p + "ssm_conv1d.weight"].reshape(-1, 4)
                got = a.vector(layer, 34, 3 * s_w * 4).reshape(3 * s_w, 4)
                for c in (0, key - 1, key, s_w - 1, s_w, s_w + key, 2 * s_w, 3 * s_w - 1):
                    src = c % key if c < s_w else key + (c - s_w) % key if c < 2 * s_w else 2 * key + c - 2 * s_w
                    np.testing.assert_array_equal(got[c], conv[src])
                for idx, name in ((ra.BETA, "ssm_beta"), (ra.ALPHA, "ssm_alpha")):
                    fmt, raw = packed[p + name + ".weight"]
                    got_fmt, got_mode, got = a.matrix(layer, idx, raw.nbytes)
                    assert (got_fmt, got_mode) == (fmt, 0), name
                    np.testing.assert_array_equal(got, raw.ravel())
        for which, name in ((0, "token_embd.weight"), (1, "output.weight")):
            fmt, raw = packed[name]
            got_fmt, got = a.basis(which, raw.nbytes)
            assert got_fmt == fmt
            np.testing.assert_array_equal(got, raw.ravel())


def test_shared_basis_is_written_once(tmp_path):
    spec = copy.deepcopy(aw.SMALL_SPEC)
    rng = np.random.default_rng(4)
    packed, floats = aw.random_model(rng, spec, lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    packed["output.weight"] = packed["token_embd.weight"]   # tied embeddings (export.py:131-134)
    aw.write(tmp_path, spec, packed, floats)
    with ra.open_dir(tmp_path) as a:
        assert a.info.embed_offset_words == a.info.lm_offset_words == 0
        fmt, raw = packed["output.weight"]
        np.testing.assert_array_equal(a.basis(1, raw.nbytes)[1], raw.ravel())


def test_out_of_range_requests(tmp_path):
    _model(tmp_path)
    with ra.open_dir(tmp_path) as a:
        with pytest.raises(Exception):
            a.matrix(2, 0, 16)
        with pytest.raises(Exception):
            a.matrix(0, 11, 16)
        with pytest.raises(Exception):
            a.vector(0, 0, a.info.param_words + 1)
        for count in (2 ** 64 - 1, 2 ** 64 - 8, 2 ** 63):     # off + count would wrap past the check
            with pytest.raises(Exception, match="rta_asset_vector"):
                a.vector(0, 0, count)
        with pytest.raises(ValueError, match="Truncated geometric weights"):
            a.matrix(0, ra.FFN_GATE, 1 << 30)


def _patch(path, offset, data):
    b = bytearray(path.read_bytes())
    b[offset:offset + len(data)] = data
    path.write_bytes(bytes(b))


@pytest.mark.parametrize("case,message", [
    ("magic", "Invalid resident optical student"),
    ("quantization", "Invalid resident optical student"),
    ("blocks", "Invalid resident optical student"),
    ("middle", "Invalid resident optical student"),
    ("params", "Truncated resident parameters"),
    ("translation", "Complete equivalent optical translation required"),
    ("matrices", "Truncated geometric weights"),
    ("basis_magic", "Complete model vocabulary basis required"),
    ("basis_shape", "Complete model vocabulary basis required"),
])
def test_damaged_assets_fail_with_the_loaders_messages(tmp_path, case, message):
    _model(tmp_path)
    model, geo, voc = tmp_path / "optical_model.bin", tmp_path / "geometry_weights.bin", tmp_path / "vocabulary.bin"
    if case == "magic":
        _patch(model, 0, b"RTRES003")
    elif case == "quantization":
        _patch(model, 8 + 20, struct.pack("<I", 3))
    elif case == "blocks":
        _patch(model, 8 + 8, struct.pack("<I", 3))
    elif case == "middle":
        _patch(model, 8 + 12, struct.pack("<I", 1000))
    elif case == "params":
        model.write_bytes(model.read_bytes()[:-4])
    elif case == "translation":
        _patch(model, 8 + 36 + 11 * 4, struct.pack("<I", 0))
    elif case == "matrices":
        geo.write_bytes(geo.read_bytes()[:-4])
    elif case == "basis_magic":
        _patch(voc, 0, b"RTBAS001")
    elif case == "basis_shape":
        _patch(voc, 8, struct.pack("<I", 999))
    with pytest.raises(ValueError, match=message):
        ra.open_dir(tmp_path)


def test_header_sizes_beyond_memory_are_reported(tmp_path):
    """A parameter-word count no allocation can hold fails with the loader's message
    instead of an exception escaping the C ABI."""
    _model(tmp_path)
    model = tmp_path / "optical_model.bin"
    _patch(model, 8 + 28, struct.pack("<I", 0xFFFFFFFF))   # parameter words
    _patch(model, 8 + 32, struct.pack("<I", 0xFFFFFFFF))   # matrix words
    with pytest.raises(ValueError, match="Invalid resident optical student|Truncated"):
        ra.open_dir(tmp_path)
