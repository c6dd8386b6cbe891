"""CPU sanitizer builds of the host code that parses or computes on the host.

- The exported-model reader (csrc/rta_asset.cpp, host only) is built with
  AddressSanitizer and UndefinedBehaviorSanitizer into tests/sanitize/asset_probe.cpp,
  which asks for every word, vector, matrix and basis of a model (in range, at the edges
  and past them) and reads every byte it gets back; the probe runs on a valid model and
  on damaged ones (the loader's refusal cases, truncations, patched header words).
- The oracle (oracle/rta_oracle.c, rta_cpu_step.c) is built the same way
  (`make -C oracle asan`) and its own tests run against that build, in a Python
  process that preloads the gcc sanitizer runtimes.

Either run fails on any sanitizer report."""
import copy
import os
import shutil
import struct
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import asset_writer as aw
from rta import synth

ROOT = Path(__file__).resolve().parent.parent
SAN = ["-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
REPORTS = ("ERROR: AddressSanitizer", "runtime error:", "ERROR: LeakSanitizer")


def _runtime(name):
    p = subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True).stdout.strip()
    return p if p and os.path.isabs(p) and os.path.isfile(p) else None


@pytest.fixture(scope="module")
def probe(tmp_path_factory):
    if shutil.which("g++") is None or _runtime("libasan.so") is None:
        pytest.skip("g++ with the AddressSanitizer runtime is not installed")
    exe = tmp_path_factory.mktemp("san") / "asset_probe"
    cmd = ["g++", "-std=c++17", *SAN, "-o", str(exe), str(ROOT / "tests" / "sanitize" / "asset_probe.cpp"),
           str(ROOT / "ray-tracing-attention_amd" / "csrc" / "rta_asset.cpp")]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return exe


def _run_probe(exe, d, vocab=True):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="halt_on_error=1")
    r = subprocess.run([str(exe), str(d / "optical_model.bin"), str(d / "vocabulary.bin") if vocab else "-"],
                       capture_output=True, text=True, env=env, timeout=120)
    text = r.stdout + r.stderr
    assert r.returncode == 0 and not any(m in text for m in REPORTS), text[-3000:]
    return r.stdout


def _model(d, seed=3):
    spec = copy.deepcopy(aw.SMALL_SPEC)
    rng = np.random.default_rng(seed)
    packed, floats = aw.random_model(rng, spec, lambda fmt, r, c: synth.random_matrix(rng, fmt, r, c))
    aw.write(d, spec, packed, floats)


def _patch(path, offset, data):
    b = bytearray(path.read_bytes())
    b[offset:offset + len(data)] = data
    path.write_bytes(bytes(b))


def test_asset_reader_valid_model(probe, tmp_path):
    _model(tmp_path)
    out = _run_probe(probe, tmp_path)
    assert out.startswith("info 0") and "calls ok" in out, out
    assert "calls ok" in _run_probe(probe, tmp_path, vocab=False)


DAMAGE = [
    ("magic", "model", 0, b"RTRES003"),
    ("quantization", "model", 8 + 20, struct.pack("<I", 3)),
    ("blocks", "model", 8 + 8, struct.pack("<I", 3)),
    ("middle", "model", 8 + 12, struct.pack("<I", 1000)),
    ("depth", "model", 8 + 4, struct.pack("<I", 0xFFFF)),
    ("param_words", "model", 8 + 28, struct.pack("<I", 0xFFFFFFFF)),
    ("matrix_words", "model", 8 + 32, struct.pack("<I", 0xFFFFFFFF)),
    ("translation", "model", 8 + 36 + 11 * 4, struct.pack("<I", 0)),
    ("layer_offset", "model", 8 + 36 + 64 * 4 + 2 * 4, struct.pack("<I", 0xFFFFFFF0)),
    ("embed_offset", "model", 8 + 36 + 14 * 4, struct.pack("<I", 0xFFFFFFFF)),
    ("basis_magic", "vocab", 0, b"RTBAS001"),
    ("basis_shape", "vocab", 8, struct.pack("<I", 999)),
    ("basis_huge", "vocab", 8, struct.pack("<2I", 0xFFFFFFFF, 0xFFFFFFFF)),
]


@pytest.mark.parametrize("case,which,offset,data", DAMAGE, ids=[c[0] for c in DAMAGE])
def test_asset_reader_damaged_model(probe, tmp_path, case, which, offset, data):
    _model(tmp_path)
    path = tmp_path / ("optical_model.bin" if which == "model" else "vocabulary.bin")
    _patch(path, offset, data)
    _run_probe(probe, tmp_path)


@pytest.mark.parametrize("name", ["optical_model.bin", "geometry_weights.bin", "vocabulary.bin"])
def test_asset_reader_truncated_files(probe, tmp_path, name):
    _model(tmp_path)
    path = tmp_path / name
    full = path.read_bytes()
    for n in sorted({0, 4, 8, 12, 40, len(full) // 2, len(full) - 4, len(full) - 1}):
        path.write_bytes(full[:n])
        _run_probe(probe, tmp_path)
    path.write_bytes(full)


def test_asset_reader_random_header_words(probe, tmp_path):
    """Random values in the model header and the first layer header, one word at a time."""
    _model(tmp_path)
    model = tmp_path / "optical_model.bin"
    full = model.read_bytes()
    rng = np.random.default_rng(11)
    for word in list(range(0, 9 + 64)) + list(range(9 + 64, 9 + 64 + 64, 5)):
        value = int(rng.integers(0, 2 ** 32, dtype=np.uint64))
        b = bytearray(full)
        b[8 + 4 * word:12 + 4 * word] = struct.pack("<I", value)
        model.write_bytes(bytes(b))
        _run_probe(probe, tmp_path)
    model.write_bytes(full)


def test_oracle_tests_under_sanitizers():
    asan, ubsan = _runtime("libasan.so"), _runtime("libubsan.so")
    if shutil.which("gcc") is None or asan is None or ubsan is None:
        pytest.skip("gcc with the AddressSanitizer / UndefinedBehaviorSanitizer runtimes is not installed")
    r = subprocess.run(["make", "-s", "-C", str(ROOT / "oracle"), "asan"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    env = dict(os.environ, LD_PRELOAD=f"{asan}:{ubsan}", ASAN_OPTIONS="detect_leaks=0",
               UBSAN_OPTIONS="halt_on_error=1", RTA_ORACLE_LIB=str(ROOT / "oracle" / "lib" / "librta_oracle_asan.so"))
    r = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider",
                        str(ROOT / "tests" / "test_oracle.py"), str(ROOT / "tests" / "test_remap.py")],
                       capture_output=True, text=True, env=env, cwd=str(ROOT), timeout=900)
    text = r.stdout + r.stderr
    assert r.returncode == 0 and not any(m in text for m in REPORTS), text[-3000:]
    assert " passed" in text
