"""ctypes binding of librta.so (the C ABI declared in include/rta.h).

The library is loaded from the package's own lib/ directory.  There is no
fallback: if the shared object is missing or lacks a symbol, loading fails with an
error naming the path, so no caller can silently run anything but the HIP path.
"""
import ctypes
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_ROOT / "lib" / "librta.so"

# GGUF type codes (resident_quant.glsl:6-20)
F32, F16, Q4_K, Q6_K, BF16 = 0, 1, 12, 14, 30
TILED = 0x100   # fmt | TILED: a K-quant matrix packed by rta_pack
EPI_STORE, EPI_ACCUMULATE = 0, 1
DEVERR_HITS, DEVERR_VOCAB, DEVERR_DETECTOR = 8, 2048, 65536
NOALLOC_SCRATCH_BYTES = 96 << 20   # RTA_NOALLOC_SCRATCH_BYTES
ERR_SCRATCH = 9                    # RTA_ERR_SCRATCH

_i, _i64, _sz, _f, _d, _p, _u32p = (ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float,
                                    ctypes.c_double, ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint32))

# row/axis remap modes (resident_quant.glsl:21-31): rta_remap.mode
REMAP_NONE, REMAP_QUERY, REMAP_GATE, REMAP_ROTARY, REMAP_AXES, REMAP_KEY_REPEAT = 0, 1, 2, 3, 4, 5


class Remap(ctypes.Structure):
    """struct rta_remap {mode, head_dim, rotary_dim, key_rows}."""
    _fields_ = [("mode", ctypes.c_int), ("head_dim", ctypes.c_int), ("rotary_dim", ctypes.c_int),
                ("key_rows", ctypes.c_int)]


_remap_p = ctypes.POINTER(Remap)

# name -> (restype, argtypes); must match include/rta.h
SIGNATURES = {
    "rta_version": (_i, []),
    "rta_status_string": (ctypes.c_char_p, [_i]),
    "rta_device_error": (_i, [_u32p, _i]),
    "rta_row_bytes": (_i64, [_i, _i64]),
    "rta_dequant": (_i, [_i, _p, _i64, _p, _p]),
    "rta_embed": (_i, [_i, _p, _i, _i, _p, _i, _p, _p]),
    "rta_rmsnorm": (_i, [_p, _p, _i, _i, _f, _p, _p]),
    "rta_head_norm": (_i, [_p, _i, _p, _p, _i, _i, _i, _i, _i, _f, _p]),
    "rta_delta_gates": (_i, [_p, _p, _i, _p, _p, _i, _i, _p, _p, _p]),
    "rta_short_conv": (_i, [_p, _i, _p, _p, _i, _i, _i, _f, _p, _p]),
    "rta_delta_rule": (_i, [_p, _p, _i, _p, _p, _i, _i, _i, _p, _p, _i, _f, _p, _i, _p]),
    "rta_pack_history": (_i, [_p, _i, _p, _i, _i, _i, _i, _i, _p, _i64, _p, _p]),
    "rta_pack_bytes": (_i64, [_i, _i, _i]),
    # struct-pointer arguments as void*; rta.model rebinds them with typed pointers
    "rta_hybrid_state_bytes": (_sz, [_p, _i]),
    "rta_hybrid_workspace_bytes": (_sz, [_p, _i]),
    "rta_hybrid_layout": (_i, [_p, _i, _p, _p]),
    "rta_hybrid_init": (_i, [_p, _i, _p, _p, _p]),
    "rta_hybrid_decode_step": (_i, [_p, _p, _i, _p, _p, _p, _p, _sz, _p]),
    "rta_hybrid_decode_step_capture": (_i, [_p, _p, _i, _p, _p, _p, _p, _p, _sz, _p]),
    "rta_pack": (_i, [_i, _p, _i, _i, _p, _p]),
    "rta_gemv_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "rta_gemv": (_i, [_i, _p, _i, _i, _p, _i, _p, _i, _p, _sz, _p]),
    "rta_gemv_remap_workspace_bytes": (_sz, [_i, _remap_p, _i, _i, _i]),
    "rta_gemv_remap": (_i, [_i, _p, _i, _i, _i, _remap_p, _p, _i, _p, _i, _p, _sz, _p]),
    "rta_pack_remap": (_i, [_i, _p, _i, _i, _remap_p, _i, _p, _p]),
    "rta_mlp_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "rta_mlp_swiglu": (_i, [_i, _p, _i, _p, _i, _p, _i, _i, _p, _i, _p, _p, _i, _p, _sz, _p]),
    "rta_swiglu": (_i, [_i, _p, _p, _i, _i, _p, _i, _p, _p, _sz, _p]),
    "rta_lm_head_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "rta_lm_head": (_i, [_i, _p, _i, _i, _p, _i, _f, _p, _p, _p, _sz, _p]),
    "rta_rope": (_i, [_p, _i, _i, _i, _i, _p, _d, _p]),
    "rta_history_bytes": (_i64, [_i]),
    "rta_decode_attention_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "rta_decode_attention": (_i, [_p, _i, _i, _i, _i, _p, _i, _i, _p, _p, _i64, _i64, _i, _p, _p, _p, _p, _p, _sz,
                                  _p]),
    "rta_decode_attention_noalloc": (_i, [_p, _i, _i, _i, _i, _p, _i, _i, _p, _p, _i64, _i64, _i, _p, _p, _p, _p,
                                          _p]),
    "rta_image_bytes": (_sz, [_i, _i]),
    "rta_image_readout_workspace_bytes": (_sz, [_i, _i, _i]),
    "rta_image_from_swiglu": (_i, [_i, _p, _i, _i, _i, _p, _p]),
    "rta_image_from_rows": (_i, [_i, _p, _p, _i, _i, _p, _p, _p]),
    "rta_image_readout": (_i, [_i, _i, _p, _p, _i, _i, _p, _i, _p, _f, _p, _i, _p, _sz, ctypes.POINTER(_i), _p]),
    "rta_attention_receipt_records": (_i64, [_p, _i, _i, _i64, _i]),
    "rta_attention_receipts": (_i, [_p, _i, _i, _i, _i, _p, _i, _i, _p, _p, _i64, _i64, _i, _i, _p, _i64, _p]),
    # host-only asset reader (rta.asset binds the structs)
    "rta_asset_open": (_i, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_p), ctypes.c_char_p, _sz]),
    "rta_asset_close": (None, [_p]),
    "rta_asset_get_info": (_i, [_p, _p]),
    "rta_asset_params": (_u32p, [_p, ctypes.POINTER(ctypes.c_uint64)]),
    "rta_asset_layer_matrix": (_i, [_p, _i, _i, _p]),
    "rta_asset_vector": (_i, [_p, _i, _i, ctypes.c_uint64, ctypes.POINTER(ctypes.POINTER(_f))]),
    "rta_asset_word": (_i, [_p, _i, _i, _u32p]),
    "rta_asset_basis": (_i, [_p, _i, _p]),
}


class RtaError(RuntimeError):
    def __init__(self, status, what=""):
        self.status = status
        text = _LIB.rta_status_string(status).decode() if _LIB is not None else str(status)
        super().__init__(f"{what}: rta status {status} ({text})" if what else f"rta status {status} ({text})")


_LIB = None


def load(path=None):
    """Loads librta.so once and binds every declared entry point."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path else LIB_PATH
    if not p.is_file():
        raise FileNotFoundError(f"librta.so not built at {p}; run __graft_entry__.build()")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)  # AttributeError if the symbol is missing
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def check(status, what=""):
    if status != 0:
        raise RtaError(status, what)
