"""Reader of the exported assets (optical_model.bin, geometry_weights.bin, vocabulary.bin)
through librta's rta_asset_* entry points (host memory only; no GPU needed).

Mirrors the reference worker's loader (ray_tracing/native/src/optical_resident.cpp:139-152)
and the exporter's layout (ray_tracing/compiler/export.py:51-138): a failed open raises
ValueError with the loader's message.
"""
import ctypes
from pathlib import Path

import numpy as np

from . import _lib

_u32, _u64 = ctypes.c_uint32, ctypes.c_uint64


class AssetInfo(ctypes.Structure):
    _fields_ = [(n, _u32) for n in ("hidden", "depth", "blocks", "middle", "vocab", "quantization", "step")] + \
               [(n, _u64) for n in ("param_words", "matrix_words", "basis_words")] + \
               [("fmt_embed", _u32), ("fmt_lm", _u32), ("embed_offset_words", _u64), ("lm_offset_words", _u64)]


class AssetMatrix(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("offset_words", _u64), ("avail_bytes", _u64), ("fmt", _u32),
                ("mode", _u32)]


# descriptor indices (export.py:96-98, 108-109, 121); the delta-net's separate ssm_beta /
# ssm_alpha payloads (export.py:113)
Q, K, OUT, FFN_GATE, FFN_DOWN, FFN_UP, GATE, V = 0, 1, 2, 3, 4, 5, 6, 8
BETA, ALPHA = 9, 10


class Asset:
    def __init__(self, model_path, vocabulary_path=None):
        self._h = None
        self._lib = _lib.load()
        handle = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        vp = None if vocabulary_path is None else str(vocabulary_path).encode()
        rc = self._lib.rta_asset_open(str(model_path).encode(), vp, ctypes.byref(handle), err, 256)
        if rc != 0:
            raise ValueError(err.value.decode() or f"rta_asset_open status {rc}")
        self._h = handle
        self.info = AssetInfo()
        _lib.check(self._lib.rta_asset_get_info(self._h, ctypes.byref(self.info)), "rta_asset_get_info")

    def close(self):
        if getattr(self, "_h", None):
            self._lib.rta_asset_close(self._h)
            self._h = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def params(self):
        n = ctypes.c_uint64()
        p = self._lib.rta_asset_params(self._h, ctypes.byref(n))
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy()

    def word(self, layer, field):
        v = ctypes.c_uint32()
        _lib.check(self._lib.rta_asset_word(self._h, layer, field, ctypes.byref(v)), "rta_asset_word")
        return v.value

    def vector(self, layer, field, count):
        p = ctypes.POINTER(ctypes.c_float)()
        _lib.check(self._lib.rta_asset_vector(self._h, layer, field, count, ctypes.byref(p)), "rta_asset_vector")
        return np.ctypeslib.as_array(p, shape=(count,)).copy()

    def _bytes(self, m, nbytes):
        if nbytes > m.avail_bytes:
            raise ValueError("Truncated geometric weights")
        return np.frombuffer(ctypes.string_at(m.data, nbytes), dtype=np.uint8)

    def matrix(self, layer, index, nbytes):
        """(fmt, mode, raw bytes) of a layer's projection descriptor."""
        m = AssetMatrix()
        _lib.check(self._lib.rta_asset_layer_matrix(self._h, layer, index, ctypes.byref(m)), "rta_asset_layer_matrix")
        return m.fmt, m.mode, self._bytes(m, nbytes)

    def basis(self, which, nbytes):
        """(fmt, raw bytes) of token_embd (0) or output (1)."""
        m = AssetMatrix()
        _lib.check(self._lib.rta_asset_basis(self._h, which, ctypes.byref(m)), "rta_asset_basis")
        return m.fmt, self._bytes(m, nbytes)


def open_dir(directory):
    d = Path(directory)
    return Asset(d / "optical_model.bin", d / "vocabulary.bin")
