"""The resident worker's start-up checks, which run before any HIP call, on the CPU:
arguments, environment and damaged assets end it with exit status 1 and the reference
worker's messages on stderr (optical_resident.cpp:139-152,968)."""
import copy
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

import asset_writer as aw
from rta import synth

EXE = Path(__file__).resolve().parent.parent / "ray-tracing-attention_amd" / "lib" / "rt_optical_resident"


def _run(args, env=None):
    if not EXE.is_file():
        raise FileNotFoundError(f"{EXE} not built; run __graft_entry__.build()")
    p = subprocess.run([str(EXE), *map(str, args)], input=b"", capture_output=True, timeout=60,
                       env=dict(os.environ, **(env or {})))
    return p.returncode, p.stderr.decode(errors="replace")


@pytest.fixture(scope="module")
def asset(tmp_path_factory):
    d = tmp_path_factory.mktemp("asset")
    spec = copy.deepcopy(aw.SMALL_SPEC)
    rng = np.random.default_rng(21)
    packed, floats = aw.random_model(rng, spec, lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, spec, packed, floats)
    return d


def test_usage():
    rc, err = _run([])
    assert rc == 1 and "Usage: rt_optical_resident" in err


@pytest.mark.parametrize("extra,env,message", [
    (["0"], None, "Invalid initial tree capacity"),
    (["300", "1", "sparse"], None, "Sparse routing"),
    (["300", "1", "rt_full", "0.08", "32", "8", "1", "4", "100"], None, "Prefill batch requires a power of two"),
    ([], {"RT_ATTENTION_BACKEND": "grouped_rt"}, "standard attention backend only"),
    ([], {"RT_MLP_BACKEND": "rt_transmission"}, "standard MLP backend only"),
    ([], {"RT_ATTENTION_BLOCK": "64"}, "Invalid attention history block"),
])
def test_arguments_and_environment(asset, extra, env, message):
    rc, err = _run([asset / "optical_model.bin", asset / "vocabulary.bin", *extra], env)
    assert rc == 1 and message in err, err


def test_damaged_asset(asset, tmp_path):
    bad = tmp_path / "optical_model.bin"
    bad.write_bytes(b"RTRES003" + (asset / "optical_model.bin").read_bytes()[8:])
    rc, err = _run([bad, asset / "vocabulary.bin"])
    assert rc == 1 and "Invalid resident optical student" in err, err


def test_missing_model_json(asset, tmp_path):
    for name in ("optical_model.bin", "geometry_weights.bin", "vocabulary.bin"):
        (tmp_path / name).write_bytes((asset / name).read_bytes())
    rc, err = _run([tmp_path / "optical_model.bin", tmp_path / "vocabulary.bin"])
    assert rc == 1 and "model.json lacks model_spec.kv_heads" in err, err
