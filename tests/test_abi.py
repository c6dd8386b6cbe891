"""CPU checks of the C ABI: the library loads, exports every symbol the header
declares, answers the host-only queries, and rejects bad arguments on the host
(no kernel is launched by any call in this file)."""
import ctypes
import re
from pathlib import Path

import pytest

from rta import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "rta.h"
FAKE = ctypes.c_void_p(0x100000)      # never dereferenced: every call below fails validation first
FAKE_ODD = ctypes.c_void_p(0x100002)


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def declared():
    text = HEADER.read_text()
    body = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rta_[a-z0-9_]+)\s*\(", body)))


def test_every_declared_symbol_is_exported_and_bound(lib):
    names = declared()
    assert len(names) >= 13
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, n


def test_host_queries(lib):
    assert lib.rta_version() >= 1
    assert lib.rta_status_string(0) == b"ok"
    assert lib.rta_row_bytes(_lib.Q4_K, 4096) == 16 * 144
    assert lib.rta_row_bytes(_lib.Q6_K, 2048) == 8 * 210
    assert lib.rta_row_bytes(_lib.Q4_K, 100) == -1
    assert lib.rta_row_bytes(_lib.F16, 10) == 20
    assert lib.rta_history_bytes(512) == 712          # resident_dimensions.hpp:10
    assert lib.rta_history_bytes(1024) == 1416
    # the LM head's task maxima; from batch 2 its 151936 x 2048 readout runs on the matrix cores
    # (more than 2^27 weights), which add their scratch
    assert lib.rta_lm_head_workspace_bytes(_lib.Q6_K, 151936, 2048, 1) == 151936 * 4
    assert lib.rta_lm_head_workspace_bytes(_lib.Q6_K, 151936, 2048, 2) > 151936 * 2 * 4
    # the 4096 x 4096 readout stays on the vector ALUs up to batch 4, the 12288 x 4096 one to 2
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 4096, 4096, 4) == 0
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 4096, 4096, 5) > 0
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 12288, 4096, 2) == 0
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 12288, 4096, 3) > 0
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 4096, 4096, 1) == 0
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 4096, 4096, 32) > 0
    assert lib.rta_mlp_workspace_bytes(_lib.Q4_K, _lib.Q6_K, 2048, 6144, 4) == 0
    # room for one (U[128], m, Z, 2 pad) record per (sequence, 64-position tile, q head);
    # then 6 x 64 16-byte q-operand words per (sequence, kv head); then the tile-list
    # plan, nseq + 1 + 2048 int32 rounded up to 16 bytes
    q = lambda nseq, hkv: nseq * hkv * 6 * 64 * 16
    plan = lambda nseq: ((nseq + 1 + 2048) * 4 + 15) // 16 * 16
    assert lib.rta_decode_attention_workspace_bytes(16, 16, 4, 128, 32768) == \
        16 * 512 * 16 * 132 * 4 + q(16, 4) + plan(16)
    assert lib.rta_decode_attention_workspace_bytes(32, 32, 8, 128, 8448) == \
        32 * 132 * 32 * 132 * 4 + q(32, 8) + plan(32)
    assert lib.rta_decode_attention_workspace_bytes(64, 32, 8, 128, 16384) == \
        64 * 256 * 32 * 132 * 4 + q(64, 8) + plan(64)
    assert lib.rta_decode_attention_workspace_bytes(16, 16, 4, 64, 32768) == 0
    # packed (tiled) matrices: ceil(rows/16) * (cols/256) tiles of 16 blocks
    assert lib.rta_pack_bytes(_lib.Q4_K, 4096, 4096) == 256 * 16 * 2304
    assert lib.rta_pack_bytes(_lib.Q6_K, 37, 512) == 3 * 2 * 3360
    assert lib.rta_pack_bytes(_lib.Q4_K, 8, 100) == -1
    assert lib.rta_pack_bytes(_lib.F16, 8, 256) == -1
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K | _lib.TILED, 4096, 4096, 1) > 0   # matrix cores at any batch
    # size queries answer 0 for shapes the K-quant formats cannot hold (no division by zero)
    T = _lib.TILED
    assert lib.rta_mlp_workspace_bytes(_lib.Q4_K | T, _lib.Q4_K | T, 512, 37, 32) == 0
    assert lib.rta_mlp_workspace_bytes(_lib.Q4_K | T, _lib.Q4_K | T, 300, 512, 32) == 0
    assert lib.rta_lm_head_workspace_bytes(_lib.Q6_K | T, 1000, 300, 1) == 0
    assert lib.rta_lm_head_workspace_bytes(_lib.Q6_K, 1000, 100, 1) == 0
    assert lib.rta_gemv_workspace_bytes(_lib.Q6_K | T, 300, 100, 32) == 0


def test_argument_errors_are_reported_before_launch(lib):
    E = {"null": 1, "shape": 2, "format": 3, "align": 4, "ws": 5, "range": 7}
    G = lambda *a: lib.rta_gemv(*a, None, 0, None)
    assert G(99, FAKE, 8, 256, FAKE, 1, FAKE, 0) == E["format"]
    assert G(_lib.Q4_K, None, 8, 256, FAKE, 1, FAKE, 0) == E["null"]
    assert G(_lib.Q4_K, FAKE, 8, 255, FAKE, 1, FAKE, 0) == E["shape"]
    assert G(_lib.Q4_K, FAKE, 0, 256, FAKE, 1, FAKE, 0) == E["shape"]
    assert G(_lib.Q4_K, FAKE, 8, 256, FAKE, 0, FAKE, 0) == E["shape"]
    assert G(_lib.Q4_K, FAKE_ODD, 8, 256, FAKE, 1, FAKE, 0) == E["align"]
    assert G(_lib.Q4_K, FAKE, 8, 256, FAKE_ODD, 1, FAKE, 0) == E["align"]
    assert G(_lib.Q4_K, FAKE, 8, 256, FAKE, 1, FAKE, 7) == E["range"]
    assert lib.rta_mlp_swiglu(_lib.Q4_K, FAKE, _lib.Q6_K, FAKE, _lib.Q6_K, FAKE, 256, 512, FAKE, 1, FAKE, FAKE, 0,
                              None, 0, None) == E["format"]
    assert G(_lib.Q4_K, FAKE, 8, 256, FAKE, 8, FAKE, 0) == E["ws"]             # matrix-core tile needs scratch
    assert lib.rta_lm_head(_lib.Q6_K, FAKE, 300, 256, FAKE, 1, ctypes.c_float(1e-4), FAKE, FAKE, None, 0,
                           None) == E["ws"]
    assert lib.rta_lm_head(_lib.Q6_K, FAKE, 300, 256, FAKE, 1, ctypes.c_float(-1.0), FAKE, FAKE, FAKE, 1 << 20,
                           None) == E["range"]
    assert lib.rta_dequant(_lib.Q6_K, FAKE, 100, FAKE, None) == E["shape"]
    assert lib.rta_pack(_lib.F32, FAKE, 8, 256, FAKE, None) == E["format"]
    assert lib.rta_pack(_lib.Q4_K, FAKE, 8, 256, FAKE_ODD, None) == E["align"]
    assert lib.rta_pack(_lib.Q4_K, FAKE, 8, 200, FAKE, None) == E["shape"]
    assert G(_lib.Q4_K | _lib.TILED, FAKE_ODD, 8, 256, FAKE, 1, FAKE, 0) == E["align"]
    assert G(_lib.Q4_K | _lib.TILED, FAKE, 8, 256, FAKE, 1, FAKE, 0) == E["ws"]     # tiled always needs scratch
    assert lib.rta_rope(FAKE, 1, 1, 7, 7, FAKE, ctypes.c_double(1e6), None) == E["shape"]
    assert lib.rta_rope(FAKE, 1, 1, 8, 8, FAKE, ctypes.c_double(-1.0), None) == E["range"]
    args = [FAKE, 1, 16, 4, 64, FAKE, _lib.Q4_K, _lib.Q6_K, FAKE, FAKE, 1024, 4096, 1024, None, FAKE, FAKE, FAKE,
            FAKE, 1 << 30, None]
    assert lib.rta_decode_attention(*args) == E["range"]          # hd != 128
    args[4] = 128
    args[7] = 13
    assert lib.rta_decode_attention(*args) == E["format"]
    args[6] = args[7] = _lib.Q6_K                                 # two Q6_K fields overrun a packet
    assert lib.rta_decode_attention(*args) == E["format"]
    args[6] = _lib.Q4_K
    args[7] = _lib.Q6_K
    args[18] = 16
    assert lib.rta_decode_attention(*args) == E["ws"]
    args[18] = 1 << 30
    args[11] = 0
    assert lib.rta_decode_attention(*args) == E["shape"]           # n_slots <= 0
    # dense receipts: host refusals, and the record count of ragged rows
    R = lambda **k: lib.rta_attention_receipts(
        k.get("q", FAKE), 2, k.get("hq", 8), 2, k.get("hd", 128), FAKE, _lib.Q4_K, k.get("fv", _lib.Q6_K), FAKE,
        FAKE, 300, 600, 300, k.get("block", 128), k.get("rec", FAKE), k.get("n", 64), None)
    assert R(q=None) == E["null"] and R(hq=7) == E["shape"] and R(n=0) == E["shape"]
    assert R(fv=_lib.F32) == E["format"] and R(hd=64) == E["range"]
    assert R(block=96 + 1) == E["range"] and R(block=2048) == E["range"] and R(block=16) == E["range"]
    assert R(rec=FAKE_ODD) == E["align"]
    lens = (ctypes.c_int32 * 5)(1, 128, 129, 400, 0)
    assert lib.rta_attention_receipt_records(lens, 5, 8, 300, 128) == 8 * (1 + 1 + 2 + 3 + 0)
    assert lib.rta_attention_receipt_records(lens, 5, 8, 300, 0) == -1


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(FileNotFoundError):
        _lib.load(tmp_path / "librta.so")


def test_read_ceiling_probe_loads_and_checks_arguments():
    """The benchmark's HBM read-ceiling probe (lib/librta_ceiling.so, not part of the C ABI)
    exports its one entry point and refuses bad arguments before any launch."""
    path = Path(_lib.__file__).resolve().parent.parent / "lib" / "librta_ceiling.so"
    assert path.is_file(), "build() compiles lib/librta_ceiling.so"
    probe = ctypes.CDLL(str(path))
    f = probe.rta_ceiling_stream_read
    f.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    f.restype = ctypes.c_int
    assert f(None, 1024, FAKE, 16, 0, None) == 2        # no buffer
    assert f(FAKE, 1000, FAKE, 16, 0, None) == 2        # not a multiple of 16 bytes
    assert f(FAKE_ODD, 1024, FAKE, 16, 0, None) == 2    # misaligned
    assert f(FAKE, 1024, FAKE, 0, 0, None) == 2         # no blocks
    assert f(FAKE, 1024, FAKE, 16, 4, None) == 2        # unknown variant


def test_hybrid_shape_refuses_attention_the_kernels_do_not_serve(lib):
    """The decode step checks its full layers' attention shape on the host, before it
    advances any state: 16 query heads per kv head, a kv-head count whose thread split
    exceeds a workgroup, and two Q6_K history fields (a packet holds one) are refused by
    the size queries (0) and by the step itself with rta_decode_attention's codes."""
    from rta import model
    E = {"format": 3, "range": 7}
    hybrid = model._lib_h()
    cases = [({"kv_heads": 2}, E["range"]),                                   # G = 16
             ({"q_heads": 64, "kv_heads": 64, "rec_heads": 64}, E["range"]),   # 64 x 8 threads > 256
             ({"fmt_k": _lib.Q6_K, "fmt_v": _lib.Q6_K}, E["format"])]
    for change, code in cases:
        s = model.shape_9b(1024)
        for k, v in change.items():
            setattr(s, k, v)
        assert hybrid.rta_hybrid_state_bytes(ctypes.byref(s), 4) == 0, change
        assert hybrid.rta_hybrid_workspace_bytes(ctypes.byref(s), 4) == 0, change
        w = model.HybridWeights(embed=FAKE.value, layers=ctypes.cast(FAKE.value, ctypes.POINTER(model.HybridLayer)),
                                norm_final=FAKE.value, lm_head=FAKE.value)
        assert hybrid.rta_hybrid_decode_step(ctypes.byref(s), ctypes.byref(w), 4, FAKE, FAKE, None, FAKE, 1 << 40,
                                             None) == code, change
    ok = model.shape_9b(1024)
    assert hybrid.rta_hybrid_state_bytes(ctypes.byref(ok), 4) > 0
    # a misaligned capture buffer is refused before any launch
    cap = model.HybridCapture(residual=FAKE_ODD.value, residual_from=0, kv=None, marks=None)
    need = hybrid.rta_hybrid_workspace_bytes(ctypes.byref(ok), 4)
    w = model.HybridWeights(embed=FAKE.value, layers=ctypes.cast(FAKE.value, ctypes.POINTER(model.HybridLayer)),
                            norm_final=FAKE.value, lm_head=FAKE.value)
    assert hybrid.rta_hybrid_decode_step_capture(ctypes.byref(ok), ctypes.byref(w), 4, FAKE, FAKE, None,
                                                 ctypes.byref(cap), FAKE, need, None) == 4
    # the first captured residual block lies in 0 .. layers
    cap = model.HybridCapture(residual=FAKE.value, residual_from=33, kv=None, marks=None)
    assert hybrid.rta_hybrid_decode_step_capture(ctypes.byref(ok), ctypes.byref(w), 4, FAKE, FAKE, None,
                                                 ctypes.byref(cap), FAKE, need, None) == 7


def test_part_readout_workspace_is_not_monotonic_in_rows(lib):
    """Why the decode step sizes its projection workspace over every in-projection part row
    count: at 4096 columns and batch 32 a 7168-row Q4_K readout needs more workspace than
    the whole 10240-row in-projection (fewer row tiles take more K slabs).  The step with
    such parts runs in tests/test_gpu_sizes.py."""
    assert lib.rta_gemv_workspace_bytes(_lib.Q4_K, 7168, 4096, 32) > lib.rta_gemv_workspace_bytes(_lib.Q4_K, 10240,
                                                                                                    4096, 32)


def test_image_readout_refusals(lib):
    """rta_image_readout: the RMSNorm chunk sums cover at most 4096 columns; img and the
    workspace must be 16-byte aligned, y 4-byte aligned (checked before any launch)."""
    P = _lib.Q4_K | _lib.TILED
    ns = ctypes.c_int(0)
    R = lambda **k: lib.rta_image_readout(  # noqa: E731
        P, 0, FAKE, None, 256, k.get("cols", 4096), k.get("img", FAKE), 4, k.get("ss", None), ctypes.c_float(1e-6),
        k.get("y", FAKE), 1, k.get("ws", FAKE), 1 << 30, ctypes.byref(ns), None)
    assert R(cols=8192, ss=FAKE) == 2          # shape: ss holds four 1024-column chunk sums
    assert R(img=ctypes.c_void_p(FAKE.value + 8)) == 4
    assert R(ws=ctypes.c_void_p(FAKE.value + 8)) == 4
    assert R(y=FAKE_ODD) == 4
    assert R(ss=ctypes.c_void_p(FAKE.value + 4)) == 4
