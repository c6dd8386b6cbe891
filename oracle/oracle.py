"""ctypes wrapper of the CPU oracle (oracle/lib/librta_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker (or the timed CPU baseline),
never as the product path.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# RTA_ORACLE_LIB: another build of the same sources (the sanitizer build of the tests)
LIB_PATH = Path(os.environ["RTA_ORACLE_LIB"]) if os.environ.get("RTA_ORACLE_LIB") else HERE / "lib" / "librta_oracle.so"

F32, F16, Q4_K, Q6_K, BF16 = 0, 1, 12, 14, 30

_i, _i64, _f, _d, _p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double, ctypes.c_void_p
_SIG = {
    "orc_half_to_float": (_f, [ctypes.c_uint16]),
    "orc_float_to_half": (ctypes.c_uint16, [_f]),
    "orc_row_bytes": (_i64, [_i, _i64]),
    "orc_dequant": (_i, [_i, _p, _i64, _p]),
    "orc_gemv_f64": (_i, [_i, _p, _i, _i, _p, _i, _p]),
    "orc_gemv_f32": (_i, [_i, _p, _i, _i, _p, _i, _p, _i]),
    "orc_rotary_source": (_i64, [_i64, _i]),
    "orc_remap_row": (_i64, [_i, _i, _i, _i, _i64]),
    "orc_remap_axis": (_i64, [_i, _i, _i, _i64]),
    "orc_gemv_remap_f64": (_i, [_i, _p, _i, _i, _i, _i, _i, _i, _i, _p, _i, _p]),
    "orc_sigmoid": (_d, [_d]),
    "orc_mlp_swiglu": (_i, [_i, _p, _i, _p, _i, _p, _i, _i, _p, _i, _p, _p, _p]),
    "orc_argmax_margin_f32": (ctypes.c_uint32, [_p, _i64, _f]),
    "orc_argmax_margin_f64": (ctypes.c_uint32, [_p, _i64, _d]),
    "orc_lm_head": (_i, [_i, _p, _i, _i, _p, _i, _d, _p, _p]),
    "orc_rope": (None, [_p, _i, _i, _i, _i64, _d]),
    "orc_history_bytes": (_i64, [_i]),
    "orc_pack_history": (_i, [_p, _p, _i, _i, _i, _p]),
    "orc_packet_value": (_f, [_p, _i, _i, _i, _i, _i]),
    "orc_decode_attention": (_i, [_p, _i, _i, _i, _i, _p, _i, _i, _p, _p, _i64, _p, _p, _p, _p]),
    "orc_attention_receipts": (_i64, [_p, _i, _i, _i, _i, _p, _i, _i, _p, _p, _i64, _i, _i64, _p, _p, _p]),
    "orc_embed": (_i, [_i, _p, _i, _i, _p, _i, _p]),
    "orc_rmsnorm": (None, [_p, _p, _i, _i, _d, _p]),
    "orc_head_norm": (None, [_p, _i, _p, _p, _i, _i, _i, _i, _i, _d, _p]),
    "orc_delta_gates": (None, [_p, _p, _i, _p, _p, _i, _i, _p, _p]),
    "orc_short_conv": (None, [_p, _i, _p, _p, _i, _i, _i, _d, _p, _p]),
    "orc_delta_rule": (None, [_p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _p]),
}

_LIB = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.is_file():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIG.items():
            f = getattr(l, name)
            f.restype, f.argtypes = res, args
        _LIB = l
    return _LIB


def _p_(a):
    return None if a is None else a.ctypes.data_as(_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def dequant(fmt, raw, n):
    raw = _c(raw, np.uint8)
    out = np.empty(n, dtype=np.float32)
    rc = lib().orc_dequant(fmt, _p_(raw), n, _p_(out))
    assert rc == 0, rc
    return out


def gemv_f64(fmt, w, rows, cols, x):
    w, x = _c(w, np.uint8), _c(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), dtype=np.float64)
    assert lib().orc_gemv_f64(fmt, _p_(w), rows, cols, _p_(x), x.shape[0], _p_(y)) == 0
    return y


def gemv_remap_f64(fmt, w, src_rows, rows, cols, mode, hd, rotary, key_rows, x):
    w, x = _c(w, np.uint8), _c(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), dtype=np.float64)
    rc = lib().orc_gemv_remap_f64(fmt, _p_(w), src_rows, rows, cols, mode, hd, rotary, key_rows, _p_(x),
                                  x.shape[0], _p_(y))
    assert rc == 0, rc
    return y


def remap_row(mode, hd, rotary, key_rows, row):
    return int(lib().orc_remap_row(mode, hd, rotary, key_rows, row))


def remap_axis(mode, hd, rotary, axis):
    return int(lib().orc_remap_axis(mode, hd, rotary, axis))


def gemv_f32(fmt, w, rows, cols, x, threads=0):
    w, x = _c(w, np.uint8), _c(x, np.float32).reshape(-1, cols)
    y = np.empty((x.shape[0], rows), dtype=np.float32)
    assert lib().orc_gemv_f32(fmt, _p_(w), rows, cols, _p_(x), x.shape[0], _p_(y), threads) == 0
    return y


def mlp_swiglu(fmts, wg, wu, wd, hidden, inter, x, y_in=None):
    x = _c(x, np.float32).reshape(-1, hidden)
    b = x.shape[0]
    act = np.empty((b, inter), dtype=np.float64)
    y = np.empty((b, hidden), dtype=np.float64)
    yi = None if y_in is None else _c(y_in, np.float32)
    rc = lib().orc_mlp_swiglu(fmts[0], _p_(_c(wg, np.uint8)), fmts[1], _p_(_c(wu, np.uint8)), fmts[2],
                              _p_(_c(wd, np.uint8)), hidden, inter, _p_(x), b, _p_(yi), _p_(act), _p_(y))
    assert rc == 0, rc
    return act, y


def argmax_margin_f32(logits, margin):
    logits = _c(logits, np.float32)
    return int(lib().orc_argmax_margin_f32(_p_(logits), logits.size, margin))


def argmax_margin_f64(logits, margin):
    logits = _c(logits, np.float64)
    return int(lib().orc_argmax_margin_f64(_p_(logits), logits.size, margin))


def lm_head(fmt, w, vocab, hidden, h, margin=1e-4):
    h = _c(h, np.float32).reshape(-1, hidden)
    b = h.shape[0]
    logits = np.empty((b, vocab), dtype=np.float64)
    ids = np.empty(b, dtype=np.uint32)
    assert lib().orc_lm_head(fmt, _p_(_c(w, np.uint8)), vocab, hidden, _p_(h), b, margin, _p_(logits), _p_(ids)) == 0
    return logits, ids


def rope(v, t, rotary=None, theta=1e6):
    v = _c(v, np.float32).copy()
    heads, hd = v.shape[-2], v.shape[-1]
    lib().orc_rope(_p_(v), heads, hd, hd if rotary is None else rotary, int(t), theta)
    return v


def history_bytes(kvw):
    return int(lib().orc_history_bytes(kvw))


def pack_history(k, v, fmt_k=Q4_K, fmt_v=Q6_K):
    k, v = _c(k, np.float32).ravel(), _c(v, np.float32).ravel()
    kvw = k.size
    out = np.zeros(history_bytes(kvw), dtype=np.uint8)
    assert lib().orc_pack_history(_p_(k), _p_(v), kvw, fmt_k, fmt_v, _p_(out)) == 0
    return out


def decode_attention(q, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity, hkv, gate=None):
    q = _c(q, np.float32)
    nseq, hq, hd = q.shape
    out = np.empty((nseq, hq, hd), dtype=np.float64)
    m = np.empty((nseq, hq), dtype=np.float64)
    z = np.empty((nseq, hq), dtype=np.float64)
    g = None if gate is None else _c(gate, np.float32)
    rc = lib().orc_decode_attention(_p_(q), nseq, hq, hkv, hd, _p_(_c(packets, np.uint8)), fmt_k, fmt_v,
                                    _p_(_c(slot_base, np.int64)), _p_(_c(ctx_len, np.int32)), int(capacity), _p_(g),
                                    _p_(out), _p_(m), _p_(z))
    assert rc == 0, rc
    return out, m, z


def attention_receipts(q, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity, hkv, block):
    """Expected dense receipts: (vals [n, 3 + hd] fp64 = m, Z, count, U; words [n, 8 + block//32]
    uint32 with words 0 and 1 zero; tie [n] bool, records whose events may differ with the
    fp32 summation order)."""
    q = _c(q, np.float32)
    rows, hq, hd = q.shape
    ctx = _c(ctx_len, np.int32)
    act = np.minimum(np.maximum(ctx.astype(np.int64), 0), capacity)
    n = int(((act + block - 1) // block).sum()) * hq
    vals = np.zeros((max(n, 1), 3 + hd), dtype=np.float64)
    words = np.zeros((max(n, 1), 8 + block // 32), dtype=np.uint32)
    tie = np.zeros(max(n, 1), dtype=np.uint8)
    got = lib().orc_attention_receipts(_p_(q), rows, hq, hkv, hd, _p_(_c(packets, np.uint8)), fmt_k, fmt_v,
                                       _p_(_c(slot_base, np.int64)), _p_(ctx), int(capacity), block, max(n, 1),
                                       _p_(vals), _p_(words), _p_(tie))
    assert got == n, (got, n)
    return vals[:n], words[:n], tie[:n].astype(bool)


# ---- the rest of a decoder step ----
def embed(fmt, table, vocab, hidden, ids):
    ids = _c(ids, np.uint32)
    out = np.empty((ids.size, hidden), dtype=np.float32)
    rc = lib().orc_embed(fmt, _p_(_c(table, np.uint8)), vocab, hidden, _p_(ids), ids.size, _p_(out))
    assert rc == 0, rc
    return out


def rmsnorm(x, w, eps=1e-6):
    x = _c(x, np.float32)
    rows, width = x.reshape(-1, x.shape[-1]).shape
    out = np.empty((rows, width), dtype=np.float64)
    lib().orc_rmsnorm(_p_(x), _p_(_c(w, np.float32)), rows, width, eps, _p_(out))
    return out.reshape(x.shape)


def head_norm(x, heads, hd, w=None, gate=None, mean=True, eps=1e-6):
    """x [rows, >= heads*hd] (row stride = x.shape[1]); gate likewise or None."""
    x = _c(x, np.float32)
    rows = x.shape[0]
    g = None if gate is None else _c(gate, np.float32)
    out = np.empty((rows, heads * hd), dtype=np.float64)
    lib().orc_head_norm(_p_(x), x.shape[1], _p_(None if w is None else _c(w, np.float32)), _p_(g),
                        0 if g is None else g.shape[1], rows, heads, hd, int(bool(mean)), eps, _p_(out))
    return out


def delta_gates(a, b, a_log, dt_bias):
    a, b = _c(a, np.float32), _c(b, np.float32)
    batch, heads = a.shape
    decay = np.empty((batch, heads), dtype=np.float64)
    beta = np.empty((batch, heads), dtype=np.float64)
    bb = np.ascontiguousarray(b)
    assert bb.shape == a.shape
    # a and b are passed as separate [batch, heads] arrays with the same row stride
    lib().orc_delta_gates(_p_(a), _p_(bb), heads, _p_(_c(a_log, np.float32)), _p_(_c(dt_bias, np.float32)), batch,
                          heads, _p_(decay), _p_(beta))
    return decay, beta


def short_conv(raw, state, w, heads, hd, eps=1e-6):
    """raw [batch, >= 3*heads*hd]; state [batch, 3*heads*hd, 3]; w [3*heads*hd, 4]."""
    raw = _c(raw, np.float32)
    batch = raw.shape[0]
    W3 = 3 * heads * hd
    out = np.empty((batch, W3), dtype=np.float64)
    new_state = np.empty((batch, W3, 3), dtype=np.float32)
    lib().orc_short_conv(_p_(raw), raw.shape[1], _p_(_c(state, np.float32)), _p_(_c(w, np.float32)), batch, heads,
                         hd, eps, _p_(out), _p_(new_state))
    return out, new_state


def delta_rule(state, q, k, v, decay, beta):
    """state [batch, heads, hd, hd] fp64 (updated copy returned); q, k, v [batch, heads*hd]."""
    state = np.array(state, dtype=np.float64, order="C", copy=True)
    batch, heads, hd, _ = state.shape
    q, k, v = (_c(a, np.float64) for a in (q, k, v))
    out = np.empty((batch, heads * hd), dtype=np.float64)
    lib().orc_delta_rule(_p_(state), _p_(q), _p_(k), _p_(v), q.shape[1], _p_(_c(decay, np.float64)),
                         _p_(_c(beta, np.float64)), batch, heads, hd, _p_(out))
    return state, out


# ---- one whole decode step on the CPU (fp32, OpenMP; rta_cpu_step.c) ----
class StepLayer(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("norm_in", "norm_post", "w_in", "w_o", "w_gate", "w_up", "w_down", "q_norm",
                                  "k_norm", "conv_w", "a_log", "dt_bias", "out_norm")]


class StepModel(ctypes.Structure):
    _fields_ = [(n, _i) for n in ("hidden", "layers", "full_every", "q_heads", "kv_heads", "head_dim", "rec_heads",
                                  "ff", "vocab", "capacity", "fmt_embed", "fmt_proj", "fmt_lm", "fmt_k", "fmt_v",
                                  "rope_rotary")] + \
        [("eps", _f), ("margin", _f), ("rope_theta", _d), ("embed", _p), ("layers_ptr", ctypes.POINTER(StepLayer)),
         ("norm_final", _p), ("lm_head", _p)]


class CpuStep:
    """The hybrid decoder's weights as GGUF rows in host memory (names as in the product's
    test models: "embed", "norm_final", "lm_head", "{l}.norm_in", "{l}.w_in", ...), and
    the fp32 CPU step over a state laid out as the product's."""

    def __init__(self, shape, gguf):
        self.shape = shape
        self._keep = []

        def ptr(name):
            a = gguf.get(name)
            if a is None:
                return None
            a = np.ascontiguousarray(a)
            self._keep.append(a)
            return a.ctypes.data

        s = shape
        self.layers = (StepLayer * s.layers)()
        for l in range(s.layers):
            L = self.layers[l]
            for n, _ in StepLayer._fields_:
                setattr(L, n, ptr(f"{l}.{n}"))
        self.model = StepModel(hidden=s.hidden, layers=s.layers, full_every=s.full_every, q_heads=s.q_heads,
                               kv_heads=s.kv_heads, head_dim=s.head_dim, rec_heads=s.rec_heads, ff=s.ff,
                               vocab=s.vocab, capacity=s.capacity, fmt_embed=s.fmt_embed & 0xff,
                               fmt_proj=s.fmt_proj & 0xff, fmt_lm=s.fmt_lm & 0xff, fmt_k=s.fmt_k, fmt_v=s.fmt_v,
                               rope_rotary=s.rope_rotary, eps=s.eps, margin=s.margin, rope_theta=s.rope_theta,
                               embed=ptr("embed"), layers_ptr=self.layers, norm_final=ptr("norm_final"),
                               lm_head=ptr("lm_head"))
        f = lib().orc_step_f32
        f.restype = _i
        f.argtypes = [ctypes.POINTER(StepModel), _i, _p, _p, _p, _p, _p, _p, _i]

    def step(self, batch, rec, conv, packets, ctx, tokens, logits=None, threads=0):
        """Updates rec [nrec,B,H,128,128] f32, conv [nrec,B,3S,3] f32, packets [nfull,B,cap,pb] u8,
        ctx [B] i32 and tokens [B] u32 in place; logits [B, vocab] f32 or None."""
        for a, dt in ((rec, np.float32), (conv, np.float32), (packets, np.uint8), (ctx, np.int32),
                      (tokens, np.uint32)):
            assert a.dtype == dt and a.flags.c_contiguous
        assert logits is None or (logits.dtype == np.float32 and logits.flags.c_contiguous)
        rc = lib().orc_step_f32(ctypes.byref(self.model), batch, _p_(rec), _p_(conv), _p_(packets), _p_(ctx),
                                _p_(tokens), _p_(logits), threads)
        assert rc == 0, rc
