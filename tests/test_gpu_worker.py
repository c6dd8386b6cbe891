"""The resident worker (lib/rt_optical_resident) end to end on the GPU: a model written
in the exporter's layout is served over the reference's stdin/stdout protocol, and the
vocabulary (op 4), MLP (op 6) and attention (op 14) replies are checked against the
oracle on the same weights and inputs.  Bars: ids, packets and payload layouts exact;
floats max|gpu - ref| <= 1e-5 + 1e-3 max|ref| per tensor."""
import copy
import os
from pathlib import Path

import numpy as np
import pytest

import asset_writer as aw
import oracle as orc
from receipt_check import compare as compare_receipts
from conftest import tolerance_ok
from resident_client import Worker
from rta import synth

pytestmark = pytest.mark.gpu
EXE = Path(__file__).resolve().parent.parent / "ray-tracing-attention_amd" / "lib" / "rt_optical_resident"
CAPACITY = 300


def _close(got, ref, what):
    ok, frac = tolerance_ok(got, ref, 1e-3, 1e-5)
    assert ok, f"{what}: max|err|/peak = {frac:.3e}"


@pytest.fixture(scope="module")
def served(tmp_path_factory):
    if not EXE.is_file():
        raise FileNotFoundError(f"{EXE} not built; run __graft_entry__.build()")
    d = tmp_path_factory.mktemp("asset")
    spec = copy.deepcopy(aw.SMALL_SPEC)
    rng = np.random.default_rng(11)
    packed, floats = aw.random_model(rng, spec, lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, spec, packed, floats)
    print(f"worker: asset {d}", flush=True)
    w = Worker(EXE, d, CAPACITY, env=dict(os.environ))
    yield w, spec, packed
    assert w.close() == 0, w.error_text()


def test_hello(served):
    w, spec, _ = served
    magic, depth, blocks, middle, mode = w.hello
    assert magic in (0x52545239, 0x5254523A)
    assert (depth, blocks, middle) == (2, 2, spec["middle_size"])
    assert mode & 4096 and mode & 0xFF == 4   # full-matrix MLP, quantised assets


@pytest.mark.parametrize("layer,rows", [(0, 1), (1, 5), (1, 32)])
def test_mlp_check(served, layer, rows):
    w, spec, packed = served
    d, f = spec["hidden_size"], spec["middle_size"]
    rng = np.random.default_rng(100 + rows)
    x = rng.standard_normal((rows, d)).astype(np.float32)
    print(f"worker: mlp layer {layer} rows {rows}", flush=True)
    r = w.mlp(x, layer, d, f)
    p = f"blk.{layer}."
    (fg, wg), (fu, wu), (fd, wd) = (packed[p + n + ".weight"] for n in ("ffn_gate", "ffn_up", "ffn_down"))
    act, y = orc.mlp_swiglu((fg, fu, fd), wg, wu, wd, d, f, x)
    _close(r["activation"], act, "activation")
    _close(r["output"], y, "output")
    assert (r["feature_hits"] == f).all()
    # (setup, gate_up, down) GPU ms (optical_resident.cpp:946; resident_runtime.py:259-262)
    setup, gate_up, down = r["times"]
    assert np.isfinite(r["times"]).all() and setup >= 0 and gate_up > 0 and down > 0


@pytest.mark.parametrize("seed", [1, 2])
def test_vocabulary_check(served, seed):
    w, spec, packed = served
    d, v = spec["hidden_size"], spec["vocabulary_size"]
    rng = np.random.default_rng(200 + seed)
    q = (rng.standard_normal(d) * 2).astype(np.float32)
    print(f"worker: vocabulary seed {seed}", flush=True)
    r = w.vocabulary(q, d, v)
    fmt, wl = packed["output.weight"]
    logits, _ = orc.lm_head(fmt, wl, v, d, q, margin=0.0)
    logits = logits[0]
    best = int(np.argmax(logits))
    tok = int(r["winner"][0])
    # exact ties go to the lower id; a different id is only a near tie of the fp32 logits
    assert tok == best or logits[tok] >= logits[best] - 1e-5 * abs(logits[best]), (tok, best)
    np.testing.assert_allclose(r["winner"][1:2].view(np.float32)[0], logits[tok] + 20, rtol=1e-5, atol=1e-4)
    assert r["winner"][2:].view(np.float32).tolist() == [1.0, 1.0]
    assert r["hit_count"] == v and (r["ids"] == np.arange(v)).all()
    ref_rows = orc.dequant(fmt, wl[:256], 256 * d).reshape(256, d)
    np.testing.assert_array_equal(r["geometric_words"], ref_rows)
    np.testing.assert_array_equal(r["query_packets"].ravel(), q.view(np.uint32))
    blocks = d // 256
    for b in range(blocks):   # chart of the block's first pair (resident_common.glsl:78)
        blk = q[256 * b:256 * (b + 1)].astype(np.float64)
        val = blk[:2] * 16.0 / max(np.linalg.norm(blk), 1e-20)
        rad = np.linalg.norm(val)
        a = np.log1p(rad)
        np.testing.assert_allclose(r["block_charts"][b, :2], 0.7 * a / (1 + a) * val / rad, rtol=1e-5, atol=1e-6)
    assert r["block_hits"] == v * blocks


@pytest.mark.parametrize("rows,count,hstart,gap", [(3, 40, 0, 0), (4, 100, 7, 2), (1, 300, 0, 0), (32, 257, 1000, 5)])
def test_attention_check(served, rows, count, hstart, gap):
    w, spec, _ = served
    heads, kvh, hd = spec["attention_heads"], spec["kv_heads"], spec["attention_head_dim"]
    rng = np.random.default_rng(300 + count)
    q = rng.standard_normal((rows, heads, hd)).astype(np.float32)
    k = rng.standard_normal((count, kvh, hd)).astype(np.float32)
    v = rng.standard_normal((count, kvh, hd)).astype(np.float32)
    qstart = hstart + count - rows - gap
    print(f"worker: attention rows {rows} count {count} history_start {hstart} query_start {qstart}", flush=True)
    r = w.attention(q, k, v, None, 1, qstart, hstart, heads, kvh, hd)
    pb = orc.history_bytes(kvh * hd)
    assert (r["magic"], r["rows"], r["count"], r["heads"], r["kv_heads"], r["dim"], r["packet_bytes"]) == \
        (0x41545231, rows, count, heads, kvh, hd, pb)
    assert r["error"] == 0
    block = r["block"]
    assert block == 128 and r["stride"] == hd + 8 + block // 32
    assert r["records"] == heads * sum((min(qstart - hstart + i + 1, CAPACITY) + block - 1) // block
                                       for i in range(rows))
    assert r["legacy"] == int(hstart == 0)
    # (producer, merge, legacy, wall) ms (resident_attention_runtime.inl:707-726,752): the history
    # pack and records, then the output; the legacy output is the same computation
    fused, merge, legacy, wall = r["timing"]
    assert fused > 0 and merge > 0 and legacy == 0 and wall >= fused + merge
    packets = np.stack([orc.pack_history(k[i], v[i]) for i in range(count)])
    np.testing.assert_array_equal(r["history_packets"], packets)
    ctx = np.array([qstart - hstart + i + 1 for i in range(rows)], np.int32)
    out, m, z = orc.decode_attention(q, packets, orc.Q4_K, orc.Q6_K, np.zeros(rows, np.int64), ctx, CAPACITY, kvh)
    _close(r["output"], out, "attention output")
    _close(r["physical"][..., 0], m + 20, "intensity m + 20")
    _close(r["physical"][..., 1], z, "Z")
    if r["legacy"]:
        np.testing.assert_array_equal(r["legacy_output"], r["output"])
    else:
        assert not r["legacy_output"].any()
    # dense receipts (attention_receipts.hpp:16-29) against the oracle's records
    vals, words, tie = orc.attention_receipts(q, packets, orc.Q4_K, orc.Q6_K, np.zeros(rows, np.int64), ctx,
                                              CAPACITY, kvh, block)
    compare_receipts(r["receipts"], vals, words, tie, block, hd, "worker receipts")


@pytest.mark.parametrize("block", [256, 512])
def test_attention_check_receipt_blocks(served, tmp_path, block):
    """The dense receipts at the worker's other attention blocks (RT_ATTENTION_BLOCK)."""
    _, spec, _ = served
    d = tmp_path / "asset"
    d.mkdir()
    rng = np.random.default_rng(12)
    sp = copy.deepcopy(aw.SMALL_SPEC)
    packed, floats = aw.random_model(rng, sp, lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, sp, packed, floats)
    w = Worker(EXE, d, CAPACITY, env=dict(os.environ, RT_ATTENTION_BLOCK=str(block)))
    heads, kvh, hd = sp["attention_heads"], sp["kv_heads"], sp["attention_head_dim"]
    rows, count, hstart = 5, 290, 3
    qstart = hstart + count - rows
    q = rng.standard_normal((rows, heads, hd)).astype(np.float32)
    k = rng.standard_normal((count, kvh, hd)).astype(np.float32)
    v = rng.standard_normal((count, kvh, hd)).astype(np.float32)
    print(f"worker: attention receipts block {block} rows {rows} count {count}", flush=True)
    r = w.attention(q, k, v, None, sp["layer_types"].index("full"), qstart, hstart, heads, kvh, hd)
    assert w.close() == 0, w.error_text()
    assert r["error"] == 0 and r["block"] == block and r["stride"] == hd + 8 + block // 32
    packets = np.stack([orc.pack_history(k[i], v[i]) for i in range(count)])
    ctx = np.array([qstart - hstart + i + 1 for i in range(rows)], np.int32)
    vals, words, tie = orc.attention_receipts(q, packets, orc.Q4_K, orc.Q6_K, np.zeros(rows, np.int64), ctx,
                                              CAPACITY, kvh, block)
    compare_receipts(r["receipts"], vals, words, tie, block, hd, f"worker receipts block {block}")


def test_resources(served):
    w, _, _ = served
    v = w.resources()
    assert len(v) >= 61 and v[0] > 0 and v[38] == 128


def test_invalid_requests_end_the_worker(tmp_path_factory, served):
    _, spec, _ = served
    d = tmp_path_factory.mktemp("asset_err")
    rng = np.random.default_rng(12)
    packed, floats = aw.random_model(rng, copy.deepcopy(spec), lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, spec, packed, floats)
    w = Worker(EXE, d, CAPACITY, env=dict(os.environ))
    with pytest.raises(RuntimeError, match="Invalid optical MLP input"):
        w.mlp(np.zeros((1, spec["hidden_size"]), np.float32), 2, spec["hidden_size"], spec["middle_size"])
    assert w.close() == 1
    w = Worker(EXE, d, CAPACITY, env=dict(os.environ))
    with pytest.raises(RuntimeError, match="Unknown resident operation"):
        w.request(7, 1, 0)   # aperture update: not served
    assert w.close() == 1
    # non-finite MLP input is refused (verify_rt_mlp.py:103-109; optical_resident.cpp:925)
    for bad in (np.nan, np.inf):
        w = Worker(EXE, d, CAPACITY, env=dict(os.environ))
        with pytest.raises(RuntimeError, match="Optical MLP input must be finite"):
            w.mlp(np.full((1, spec["hidden_size"]), bad, np.float32), 0, spec["hidden_size"], spec["middle_size"])
        assert w.close() == 1
    # and so is a non-finite attention query
    hd, heads, kv = spec["attention_head_dim"], spec["attention_heads"], spec["kv_heads"]
    w = Worker(EXE, d, CAPACITY, env=dict(os.environ))
    q = np.zeros((1, heads, hd), np.float32)
    q[0, 0, 0] = np.inf
    k = np.zeros((4, kv, hd), np.float32)
    with pytest.raises(RuntimeError, match="Attention diagnostic values must be finite"):
        w.attention(q, k, k, None, spec["layer_types"].index("full"), 3, 0, heads, kv, hd)
    assert w.close() == 1


def test_unsupported_backend_is_refused(served, tmp_path_factory):
    _, spec, _ = served
    d = tmp_path_factory.mktemp("asset_env")
    rng = np.random.default_rng(13)
    packed, floats = aw.random_model(rng, copy.deepcopy(spec), lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, spec, packed, floats)
    with pytest.raises(RuntimeError, match="standard attention backend only"):
        Worker(EXE, d, CAPACITY, env=dict(os.environ, RT_ATTENTION_BACKEND="grouped_rt"))
