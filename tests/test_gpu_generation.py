"""Generation through the resident worker (lib/rt_optical_resident): a model written in
the exporter's layout (row modes 1/2/3 on the attention projections, mode 4 on O, the
key repeat of mode 5 on the delta-net, an attention output gate, separate F32
beta / alpha, mixed formats inside the attention in-projection) is prefilled (op 1)
and decoded through op 9 (stream), op 2 (generate) and op 10 (history growth), and
every emitted id is checked against an fp64 composition of the oracle that reads each
descriptor through its mode (asset_reference.py), fed the same ids.

Bar (the margin rule): an emitted id's reference logit is within
1e-5 + 1e-3 max|logits| of the reference's maximum."""
import copy
import os
from pathlib import Path

import numpy as np
import pytest

import asset_writer as aw
from asset_reference import AssetReference
from conftest import assert_close
from resident_client import Worker
from rta import synth

pytestmark = pytest.mark.gpu
EXE = Path(__file__).resolve().parent.parent / "ray-tracing-attention_amd" / "lib" / "rt_optical_resident"
NO_STOP = 0xFFFFFFFF

SPEC = dict(copy.deepcopy(aw.SMALL_SPEC), layer_types=["recurrent", "full", "recurrent", "full"],
            attention_gate=True, state_heads=4, state_key_heads=2, rotary_dim=64, vocabulary_size=3000)


@pytest.fixture(scope="module")
def model(tmp_path_factory):
    if not EXE.is_file():
        raise FileNotFoundError(f"{EXE} not built; run __graft_entry__.build()")
    d = tmp_path_factory.mktemp("gen_asset")
    rng = np.random.default_rng(21)
    packed, floats = aw.random_model(rng, copy.deepcopy(SPEC), lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, SPEC, packed, floats)
    return d, packed, floats


def _worker(d, capacity):
    return Worker(EXE, d, capacity, env=dict(os.environ))


def _check(ref, ids, what):
    """Each id against the reference's logits at its position; the reference then reads it."""
    exact = 0
    for i, tok in enumerate(ids):
        logits = ref.last
        bar = 1e-5 + 1e-3 * np.abs(logits).max()
        assert logits[tok] >= logits.max() - bar, (what, i, int(tok), int(np.argmax(logits)))
        exact += int(tok == int(np.argmax(logits)))
        ref.last = ref.forward(int(tok))
    return exact


def _reference(model, prompt):
    _, packed, floats = model
    ref = AssetReference(SPEC, packed, floats)
    for t in prompt:
        ref.last = ref.forward(int(t))
    return ref


def test_generation_matches_the_oracle(model):
    d, _, _ = model
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, SPEC["vocabulary_size"], 40)
    w = _worker(d, 32)
    try:
        assert w.hello[0] == 0x5254523A   # native token stream
        print("generation: grow 32 -> 64, prefill 40", flush=True)
        np.testing.assert_array_equal(w.grow(64)[:2], [32, 64])
        r = w.prefill(prompt)
        assert r["control"].tolist() == [0, 0, 1, 0, NO_STOP, NO_STOP, 0, 0]
        assert r["footer"].tolist() == [1, 40, 0, 40]
        print("generation: stream 8", flush=True)
        stream = w.stream(8)
        assert len(stream) == 8 and all(len(p["ids"]) == 1 and p["control"][2] == 1 for p in stream)
        ids = [int(p["ids"][0]) for p in stream]
        assert [int(p["timing"][6]) for p in stream] == list(range(41, 49))   # absolute positions
        print("generation: generate 16, grow 64 -> 128, stream 12", flush=True)
        g = w.generate(16)
        assert len(g["ids"]) == 16 and g["control"][1] == 16 and int(g["timing"][6]) == 64
        assert g["hits"][:3].tolist() == [16 * 4 * SPEC["middle_size"]] * 2 + [16 * SPEC["vocabulary_size"]]
        ids += g["ids"].tolist()
        np.testing.assert_array_equal(w.grow(128)[:2], [64, 128])
        ids += [int(p["ids"][0]) for p in w.stream(12)]
        assert w.finish()[0].tolist() == [0, 0, 0]
    finally:
        assert w.close() == 0, w.error_text()
    print(f"generation: {len(ids)} ids, checking against the oracle", flush=True)
    exact = _check(_reference(model, prompt), ids, "generated")
    assert exact >= len(ids) - 2, exact


def test_stop_ids_end_the_stream(model):
    d, _, _ = model
    prompt = np.arange(7, 7 + 23) * 37 % SPEC["vocabulary_size"]
    w = _worker(d, 300)
    try:
        print("generation: stop ids", flush=True)
        w.prefill(prompt)
        first = w.generate(6)["ids"].tolist()
        w.prefill(prompt, stops=(first[3],))          # the same prompt again from position 0
        out = w.stream(8)
        got = [int(p["ids"][0]) for p in out]
        assert got == first[:first.index(first[3]) + 1]   # the stop id is emitted, then nothing
        assert out[-1]["control"][2] == 0 and out[-1]["control"][0] == first[3]
        after = w.generate(4)
        assert len(after["ids"]) == 0 and after["control"][2] == 0
        # checkpoint forms of the prefill (ops 11 / 12) compute the same prefix
        w.prefill(prompt, checkpoint_tokens=10)
        assert w.generate(6)["ids"].tolist() == first
        w.prefill(prompt, boundaries=[(5, 1), (23, 2)])
        assert w.generate(6, debug=2)["ids"].tolist() == first
    finally:
        assert w.close() == 0, w.error_text()
    _check(_reference(model, prompt), first, "before the stop")


def test_generation_errors(model):
    d, _, _ = model
    w = _worker(d, 64)
    with pytest.raises(RuntimeError, match="after prefill"):
        w.generate(1)
    assert w.close() == 1
    w = _worker(d, 64)
    with pytest.raises(RuntimeError, match="Invalid tree growth request"):
        w.grow(64)
    assert w.close() == 1
    w = _worker(d, 64)
    with pytest.raises(RuntimeError, match="Invalid resident prefix"):
        w.prefill(np.zeros(65, np.uint32))
    assert w.close() == 1
    w = _worker(d, 64)
    with pytest.raises(RuntimeError, match="Invalid prefix word IDs"):
        w.prefill([1, SPEC["vocabulary_size"]])
    assert w.close() == 1
    # an attention diagnostic replaces the history (resident_attention_runtime.inl:657)
    w = _worker(d, 64)
    w.prefill([1, 2, 3])
    hq, kv = SPEC["attention_heads"], SPEC["kv_heads"]
    z = np.zeros((4, kv, 128), np.float32)
    w.attention(np.ones((1, hq, 128), np.float32), z, z, None, 1, 3, 0, hq, kv, 128)
    with pytest.raises(RuntimeError, match="prefill again before generation"):
        w.generate(1)
    assert w.close() == 1


def test_layer_capture_matches_the_oracle(model):
    """Layer capture (debug 1): prefill returns every position's residual stream after each
    layer and the state after the last one (optical_resident.cpp:481,686;
    resident_runtime.py:136-139); generation returns the state after its last step
    (optical_resident.cpp:832,870; resident_runtime.py:199).  Each row against the fp64
    composition fed the same ids, to the float bar."""
    d, packed, floats = model
    D, depth = SPEC["hidden_size"], len(SPEC["layer_types"])
    prompt = np.arange(3, 3 + 12) * 53 % SPEC["vocabulary_size"]
    w = _worker(d, 64)
    try:
        print("generation: layer capture", flush=True)
        r = w.prefill(prompt, debug=1, hidden=D, depth=depth)
        assert r["footer"].tolist() == [1, 12, 0, 12]
        g = w.generate(3, debug=1, hidden=D)
    finally:
        assert w.close() == 0, w.error_text()
    ref = AssetReference(SPEC, packed, floats)
    for i, t in enumerate(prompt):
        ref.last = ref.forward(int(t))
        for l in range(depth):
            assert_close(r["layers"][l, i], ref.residual[l], f"position {i} after layer {l}")
        np.testing.assert_array_equal(r["state"][i], r["layers"][depth - 1, i])
    assert len(g["ids"]) == 3
    for t in g["ids"]:   # each emitted id is forwarded; the state is the last forward's
        ref.last = ref.forward(int(t))
    assert_close(g["state"], ref.residual[-1], "generation state")


def test_generation_profile(model):
    """debug 2: the GenerationPacket's stage sums (time[8:18], optical_resident.cpp:849-853;
    resident_runtime.py:195) and detector sums (attention, recurrent; :229-231) from events
    at the decode step's stage marks.  No BVH update, history trace, payload restore or
    vocabulary trace runs here, so those stages are 0; the stages of a step cover its GPU
    time but for the embedding, the final norm and the host's token read between steps."""
    d, _, _ = model
    prompt = np.arange(5, 5 + 20) * 29 % SPEC["vocabulary_size"]
    w = _worker(d, 64)
    try:
        w.prefill(prompt)
        plain = w.generate(6)["ids"].tolist()
        w.prefill(prompt)
        g = w.generate(6, debug=2)
    finally:
        assert w.close() == 0, w.error_text()
    assert g["ids"].tolist() == plain
    p = g["profile"]
    print("generation profile (ms):", {k: round(v, 4) for k, v in p.items()}, "gpu", g["timing"][0],
          "detector", g["detector"].tolist(), flush=True)
    for k in ("projection_geometry", "detector", "output_mlp", "vocabulary", "vocabulary_coefficients",
              "vocabulary_reduce"):
        assert p[k] > 0, k
    for k in ("bvh_update", "lens_history_trace", "coordinate_restore", "vocabulary_rt"):
        assert p[k] == 0, k
    assert g["detector"][0] > 0 and g["detector"][1] > 0
    assert abs(g["detector"].sum() - p["detector"]) <= 1e-6 + 1e-4 * p["detector"]
    parts = p["vocabulary_rt"] + p["vocabulary_coefficients"] + p["vocabulary_reduce"]
    assert abs(parts - p["vocabulary"]) <= 1e-6 + 1e-4 * p["vocabulary"]
    stages = sum(p[k] for k in Worker.PROFILE[:7])
    assert 0.5 * g["timing"][0] <= stages <= g["timing"][0]
