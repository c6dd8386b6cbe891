"""Torch-tensor front of the C ABI: device buffers in, device buffers out.

PyTorch only provides device memory and the current stream; every computation is
one of librta.so's HIP kernels.  Shapes follow the reference's operator layouts
(resident_math.comp op 2 / 16, resident_ray.comp op 3).
"""
import ctypes

import torch

from . import _lib
from ._lib import BF16, F16, F32, Q4_K, Q6_K, TILED, EPI_ACCUMULATE, EPI_STORE, check

KQUANT_BYTES = {Q4_K: 144, Q6_K: 210}


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t, name):
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA (HIP) tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def row_bytes(fmt, cols):
    return int(_lib.load().rta_row_bytes(fmt, cols))


def history_bytes(kvw):
    return int(_lib.load().rta_history_bytes(kvw))


def dequant(fmt, blocks, n):
    """fp32 values of n quantised coordinates (bit exact, resident_quant.glsl:6-20)."""
    lib = _lib.load()
    _dev(blocks, "blocks")
    out = torch.empty(n, dtype=torch.float32, device=blocks.device)
    check(lib.rta_dequant(fmt, _ptr(blocks), n, _ptr(out), _stream()), "rta_dequant")
    return out


def pack_bytes(fmt, rows, cols):
    return int(_lib.load().rta_pack_bytes(fmt, rows, cols))


def pack(fmt, w, rows, cols):
    """Packed (tiled) copy of a device GGUF Q4_K / Q6_K matrix, for use with fmt | TILED."""
    lib = _lib.load()
    _dev(w, "w")
    n = pack_bytes(fmt, rows, cols)
    if n < 0:
        raise ValueError(f"cannot pack format {fmt} of shape {rows}x{cols}")
    out = torch.empty(n, dtype=torch.uint8, device=w.device)
    check(lib.rta_pack(fmt, _ptr(w), rows, cols, _ptr(out), _stream()), "rta_pack")
    return out


def _workspace(nbytes, dev, given):
    if given is not None:
        return given
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def gemv_workspace_bytes(fmt, rows, cols, batch):
    return int(_lib.load().rta_gemv_workspace_bytes(fmt, rows, cols, batch))


def gemv(fmt, w, rows, cols, x, y=None, accumulate=False, workspace=None):
    """y[b] = W x[b] (or y += W x); x [batch, cols] fp32 -> y [batch, rows]."""
    lib = _lib.load()
    _dev(w, "w"), _dev(x, "x")
    x2 = x.reshape(-1, cols)
    batch = x2.shape[0]
    if y is None:
        if accumulate:
            raise ValueError("accumulate needs y")
        y = torch.empty(batch, rows, dtype=torch.float32, device=x.device)
    _dev(y, "y")
    ws = _workspace(gemv_workspace_bytes(fmt, rows, cols, batch), x.device, workspace)
    check(lib.rta_gemv(fmt, _ptr(w), rows, cols, _ptr(x2), batch, _ptr(y),
                       EPI_ACCUMULATE if accumulate else EPI_STORE, _ptr(ws), ws.numel(), _stream()), "rta_gemv")
    return y


def mlp_workspace_bytes(fmt_g, fmt_d, hidden, inter, batch):
    return int(_lib.load().rta_mlp_workspace_bytes(fmt_g, fmt_d, hidden, inter, batch))


def mlp_swiglu(fmts, wg, wu, wd, hidden, inter, x, y=None, accumulate=False, act=None, workspace=None):
    """act = sign(g)sign(u)|g||u|sigmoid(g); y (=|+=) Wd act.  Returns (act, y)."""
    lib = _lib.load()
    fg, fu, fd = fmts
    for t, n in ((wg, "wg"), (wu, "wu"), (wd, "wd"), (x, "x")):
        _dev(t, n)
    x2 = x.reshape(-1, hidden)
    batch = x2.shape[0]
    if act is None:
        act = torch.empty(batch, inter, dtype=torch.float32, device=x.device)
    if y is None:
        y = torch.empty(batch, hidden, dtype=torch.float32, device=x.device)
    ws = _workspace(mlp_workspace_bytes(fg, fd, hidden, inter, batch), x.device, workspace)
    check(lib.rta_mlp_swiglu(fg, _ptr(wg), fu, _ptr(wu), fd, _ptr(wd), hidden, inter, _ptr(x2), batch,
                             _ptr(act), _ptr(y), EPI_ACCUMULATE if accumulate else EPI_STORE, _ptr(ws), ws.numel(),
                             _stream()), "rta_mlp_swiglu")
    return act, y


def lm_head_workspace_bytes(fmt, vocab, hidden, batch):
    return int(_lib.load().rta_lm_head_workspace_bytes(fmt, vocab, hidden, batch))


def lm_head(fmt, w, vocab, hidden, h, margin=1e-4, workspace=None, logits=None, ids=None):
    """fp32 logits [batch, vocab] and margin-argmax ids [batch] (uint32 as int32)."""
    lib = _lib.load()
    _dev(w, "w"), _dev(h, "h")
    h2 = h.reshape(-1, hidden)
    batch = h2.shape[0]
    dev = h.device
    if logits is None:
        logits = torch.empty(batch, vocab, dtype=torch.float32, device=dev)
    if ids is None:
        ids = torch.empty(batch, dtype=torch.int32, device=dev)
    ws = _workspace(lm_head_workspace_bytes(fmt, vocab, hidden, batch), dev, workspace)
    check(lib.rta_lm_head(fmt, _ptr(w), vocab, hidden, _ptr(h2), batch, ctypes.c_float(margin), _ptr(logits),
                          _ptr(ids), _ptr(ws), ws.numel(), _stream()), "rta_lm_head")
    return logits, ids


def rope(v, positions, rotary=None, theta=1e6):
    """In-place rotary embedding of v [rows, heads, hd] at positions [rows] (int64)."""
    lib = _lib.load()
    _dev(v, "v"), _dev(positions, "positions")
    rows, heads, hd = v.shape
    check(lib.rta_rope(_ptr(v), rows, heads, hd, hd if rotary is None else rotary, _ptr(positions),
                       ctypes.c_double(theta), _stream()), "rta_rope")
    return v


def decode_attention_workspace_bytes(nseq, hq, hkv, hd, max_ctx):
    return int(_lib.load().rta_decode_attention_workspace_bytes(nseq, hq, hkv, hd, max_ctx))


def decode_attention(q, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity, max_ctx, hkv, gate=None,
                     workspace=None, out=None):
    """Split-K decode attention; returns (out [nseq,hq,hd], m [nseq,hq], z [nseq,hq])."""
    lib = _lib.load()
    for t, n in ((q, "q"), (packets, "packets"), (slot_base, "slot_base"), (ctx_len, "ctx_len")):
        _dev(t, n)
    nseq, hq, hd = q.shape
    dev = q.device
    if out is None:
        out = torch.empty_like(q)
    m = torch.empty(nseq, hq, dtype=torch.float32, device=dev)
    z = torch.empty(nseq, hq, dtype=torch.float32, device=dev)
    need = decode_attention_workspace_bytes(nseq, hq, hkv, hd, max_ctx)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
    n_slots = packets.numel() // history_bytes(hkv * hd)
    check(lib.rta_decode_attention(_ptr(q), nseq, hq, hkv, hd, _ptr(packets), fmt_k, fmt_v, _ptr(slot_base),
                                   _ptr(ctx_len), capacity, n_slots, max_ctx, _ptr(gate), _ptr(out), _ptr(m), _ptr(z),
                                   _ptr(workspace), workspace.numel(), _stream()), "rta_decode_attention")
    return out, m, z


def device_error(clear=True):
    """Sticky device error bits (RTA_DEVERR_*); synchronises the device."""
    bits = ctypes.c_uint32(0)
    check(_lib.load().rta_device_error(ctypes.byref(bits), 1 if clear else 0), "rta_device_error")
    return bits.value
