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


def remap(mode, head_dim=0, rotary_dim=0, key_rows=0):
    """An rta_remap: the reference's descriptor mode with the geometry it reads."""
    return _lib.Remap(mode, head_dim, rotary_dim, key_rows)


def pack_remap(fmt, w, src_rows, cols, rm, rows, out=None):
    """Packed copy of the row-remapped matrix (logical row r = GGUF row src(r)).

    out: optional uint8 view to pack into (e.g. a part of a larger packed matrix)."""
    lib = _lib.load()
    _dev(w, "w")
    n = pack_bytes(fmt, rows, cols)
    if n < 0:
        raise ValueError(f"cannot pack format {fmt} of shape {rows}x{cols}")
    if out is None:
        out = torch.empty(n, dtype=torch.uint8, device=w.device)
    elif out.numel() < n:
        raise ValueError("out is smaller than the packed matrix")
    check(lib.rta_pack_remap(fmt, _ptr(w), src_rows, cols, ctypes.byref(rm), rows, _ptr(out), _stream()),
          "rta_pack_remap")
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


def gemv_remap_workspace_bytes(fmt, rm, rows, cols, batch):
    return int(_lib.load().rta_gemv_remap_workspace_bytes(fmt, ctypes.byref(rm), rows, cols, batch))


def gemv_remap(fmt, w, src_rows, rows, cols, rm, x, y=None, accumulate=False, workspace=None):
    """y[b, r] (=|+=) sum_a W[src(r), src(a)] x[b, a] for the remap rm."""
    lib = _lib.load()
    _dev(w, "w"), _dev(x, "x")
    x2 = x.reshape(-1, cols)
    batch = x2.shape[0]
    if y is None:
        if accumulate:
            raise ValueError("accumulate needs y")
        y = torch.empty(batch, rows, dtype=torch.float32, device=x.device)
    _dev(y, "y")
    ws = _workspace(gemv_remap_workspace_bytes(fmt, rm, rows, cols, batch), x.device, workspace)
    check(lib.rta_gemv_remap(fmt, _ptr(w), src_rows, rows, cols, ctypes.byref(rm), _ptr(x2), batch, _ptr(y),
                             EPI_ACCUMULATE if accumulate else EPI_STORE, _ptr(ws), ws.numel(), _stream()),
          "rta_gemv_remap")
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


def swiglu(fmt, wg, wu, hidden, inter, x, act=None, workspace=None):
    """The fused gate/up stage alone (op 2 index 3): act = swiglu(Wg x, Wu x) [batch, inter]."""
    lib = _lib.load()
    for t, n in ((wg, "wg"), (wu, "wu"), (x, "x")):
        _dev(t, n)
    batch = x.shape[0]
    if act is None:
        act = torch.empty(batch, inter, dtype=torch.float32, device=x.device)
    need = mlp_workspace_bytes(fmt, fmt, hidden, inter, batch)
    ws = _workspace(need, x.device, workspace)
    check(lib.rta_swiglu(fmt, _ptr(wg), _ptr(wu), hidden, inter, _ptr(x), batch, _ptr(act), _ptr(ws), ws.numel(),
                         _stream()), "rta_swiglu")
    return act


IMAGE_SWIGLU = 2


def image_readout_workspace_bytes(rows, cols, dual):
    return int(_lib.load().rta_image_readout_workspace_bytes(rows, cols, 1 if dual else 0))


def image_from_rows(fmt, x, w=None):
    """(img, ss): the matrix-core image of x * w [batch <= 32, cols] for packed format fmt
    and the rows' chunk sums of x^2 (rta_image_from_rows); w defaults to ones."""
    lib = _lib.load()
    _dev(x, "x")
    batch, cols = x.shape
    if w is None:
        w = torch.ones(cols, dtype=torch.float32, device=x.device)
    n = int(lib.rta_image_bytes(cols, batch))
    if n == 0:
        raise ValueError("rta_image_bytes: unsupported shape")
    img = torch.empty(n, dtype=torch.uint8, device=x.device)
    ss = torch.empty(4 * batch, dtype=torch.float32, device=x.device)
    check(lib.rta_image_from_rows(fmt, _ptr(x), _ptr(w), batch, cols, _ptr(ss), _ptr(img), _stream()),
          "rta_image_from_rows")
    return img, ss


def image_from_swiglu(fmt, part, nslab, width, batch):
    """The down projection's x image from a SwiGLU image readout's K slabs (part: that
    readout's workspace) (rta_image_from_swiglu)."""
    lib = _lib.load()
    n = int(lib.rta_image_bytes(width, batch))
    if n == 0:
        raise ValueError("rta_image_bytes: unsupported shape")
    img = torch.empty(n, dtype=torch.uint8, device=part.device)
    check(lib.rta_image_from_swiglu(fmt, _ptr(part), nslab, width, batch, _ptr(img), _stream()),
          "rta_image_from_swiglu")
    return img


def image_readout(fmt, mode, w, w2, rows, cols, img, batch, y, ss=None, eps=1e-6, reduce=True, workspace=None):
    """rta_image_readout into y [batch, rows]; returns the K-slab count left in the
    workspace (1 when the slabs were added into y)."""
    lib = _lib.load()
    need = image_readout_workspace_bytes(rows, cols, mode == IMAGE_SWIGLU)
    ws = _workspace(need, img.device, workspace)
    ns = ctypes.c_int(0)
    check(lib.rta_image_readout(fmt, mode, _ptr(w), _ptr(w2), rows, cols, _ptr(img), batch, _ptr(ss), eps, _ptr(y),
                                1 if reduce else 0, _ptr(ws), ws.numel(), ctypes.byref(ns), _stream()),
          "rta_image_readout")
    return ns.value


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


def decode_attention_noalloc(q, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity, max_ctx, hkv, gate=None,
                             out=None):
    """decode_attention on the library's own scratch (rta_decode_attention_noalloc): no
    workspace; raises RtaError (status RTA_ERR_SCRATCH) when the call would need more
    than RTA_NOALLOC_SCRATCH_BYTES."""
    lib = _lib.load()
    for t, n in ((q, "q"), (packets, "packets"), (slot_base, "slot_base"), (ctx_len, "ctx_len")):
        _dev(t, n)
    nseq, hq, hd = q.shape
    if out is None:
        out = torch.empty_like(q)
    m = torch.empty(nseq, hq, dtype=torch.float32, device=q.device)
    z = torch.empty(nseq, hq, dtype=torch.float32, device=q.device)
    n_slots = packets.numel() // history_bytes(hkv * hd)
    check(lib.rta_decode_attention_noalloc(_ptr(q), nseq, hq, hkv, hd, _ptr(packets), fmt_k, fmt_v, _ptr(slot_base),
                                           _ptr(ctx_len), capacity, n_slots, max_ctx, _ptr(gate), _ptr(out), _ptr(m),
                                           _ptr(z), _stream()), "rta_decode_attention_noalloc")
    return out, m, z


def attention_receipt_records(ctx_len, hq, capacity, block):
    """Number of dense receipt records for host context lengths ctx_len (a sequence)."""
    lens = (ctypes.c_int32 * len(ctx_len))(*[int(x) for x in ctx_len])
    n = int(_lib.load().rta_attention_receipt_records(lens, len(ctx_len), hq, capacity, block))
    if n < 0:
        raise ValueError("rta_attention_receipt_records: bad arguments")
    return n


def attention_receipts(q, packets, fmt_k, fmt_v, slot_base, ctx_len, capacity, max_ctx, hkv, block, n_records=None):
    """Dense per-group attention receipts (rta_attention_receipts): uint32 tensor
    [n_records, hd + 8 + block // 32] on q's device.  n_records defaults to the count
    for ctx_len's values (read back to the host)."""
    lib = _lib.load()
    for t, n in ((q, "q"), (packets, "packets"), (slot_base, "slot_base"), (ctx_len, "ctx_len")):
        _dev(t, n)
    rows, hq, hd = q.shape
    if n_records is None:
        n_records = attention_receipt_records(ctx_len.cpu().tolist(), hq, capacity, block)
    out = torch.zeros(max(n_records, 1), hd + 8 + block // 32, dtype=torch.int32, device=q.device)
    n_slots = packets.numel() // history_bytes(hkv * hd)
    check(lib.rta_attention_receipts(_ptr(q), rows, hq, hkv, hd, _ptr(packets), fmt_k, fmt_v, _ptr(slot_base),
                                     _ptr(ctx_len), capacity, n_slots, max_ctx, block, _ptr(out), max(n_records, 1),
                                     _stream()), "rta_attention_receipts")
    return out[:n_records]


def device_error(clear=True):
    """Sticky device error bits (RTA_DEVERR_*); synchronises the device."""
    bits = ctypes.c_uint32(0)
    check(_lib.load().rta_device_error(ctypes.byref(bits), 1 if clear else 0), "rta_device_error")
    return bits.value


# ---------------------------------------------------- the rest of a decoder step ----
def _rows(t, name):
    """A 2-D float32 CUDA tensor whose rows may be strided views (unit column stride)."""
    if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D CUDA tensor with unit column stride")
    return t


def _rs(t):
    """Row stride in elements as the C ABI takes it: a tensor of one row may carry any
    stride for its single row (torch gives 0 or 1), which stands for the row width."""
    return t.stride(0) if t.shape[0] > 1 else max(t.stride(0), t.shape[1])


def embed(fmt, table, vocab, hidden, ids, out=None):
    """op 0: decoded embedding rows of `ids` (uint32/int32 device tensor)."""
    lib = _lib.load()
    _dev(table, "table")
    _dev(ids, "ids")
    batch = ids.numel()
    if out is None:
        out = torch.empty(batch, hidden, dtype=torch.float32, device=table.device)
    check(lib.rta_embed(fmt, _ptr(table), vocab, hidden, _ptr(ids), batch, _ptr(out), _stream()), "rta_embed")
    return out


def rmsnorm(x, w, eps=1e-6, out=None):
    """op 1: x * w / sqrt(mean(x^2) + eps) per row (out may be x)."""
    lib = _lib.load()
    _dev(x, "x")
    if out is None:
        out = torch.empty_like(x)
    rows, width = x.reshape(-1, x.shape[-1]).shape
    check(lib.rta_rmsnorm(_ptr(x), _ptr(w), rows, width, ctypes.c_float(eps), _ptr(out), _stream()), "rta_rmsnorm")
    return out


def head_norm(x, heads, hd, w=None, gate=None, mean=True, eps=1e-6):
    """ops 14 / 15 / 20, in place on x [rows, >= heads*hd] (rows may be strided)."""
    lib = _lib.load()
    _rows(x, "x")
    gs = 0
    if gate is not None:
        _rows(gate, "gate")
        gs = _rs(gate)
    check(lib.rta_head_norm(_ptr(x), _rs(x), _ptr(w), _ptr(gate), gs, x.shape[0], heads, hd, int(bool(mean)),
                            ctypes.c_float(eps), _stream()), "rta_head_norm")
    return x


def delta_gates(a, b, a_log, dt_bias, decay=None, beta=None):
    """op 18 after its projections: a, b [batch, heads] views with one row stride."""
    lib = _lib.load()
    _rows(a, "a")
    _rows(b, "b")
    if _rs(a) != _rs(b):
        raise ValueError("a and b must share a row stride")
    batch, heads = a.shape
    decay = torch.empty(batch, heads, dtype=torch.float32, device=a.device) if decay is None else decay
    beta = torch.empty(batch, heads, dtype=torch.float32, device=a.device) if beta is None else beta
    check(lib.rta_delta_gates(_ptr(a), _ptr(b), _rs(a), _ptr(a_log), _ptr(dt_bias), batch, heads, _ptr(decay),
                              _ptr(beta), _stream()), "rta_delta_gates")
    return decay, beta


def short_conv(raw, state, w, heads, hd=128, eps=1e-6, out=None):
    """ops 19 + 20 for one token: raw [batch, >= 3*heads*hd] (strided rows), state
    [batch, 3*heads*hd, 3] shifted in place, w [3*heads*hd, 4]; returns out [batch, 3*heads*hd]."""
    lib = _lib.load()
    _rows(raw, "raw")
    _dev(state, "state")
    batch = raw.shape[0]
    if out is None:
        out = torch.empty(batch, 3 * heads * hd, dtype=torch.float32, device=raw.device)
    check(lib.rta_short_conv(_ptr(raw), _rs(raw), _ptr(state), _ptr(w), batch, heads, hd, ctypes.c_float(eps),
                             _ptr(out), _stream()), "rta_short_conv")
    return out


def delta_rule(state, qkv, decay, beta, heads, hd=128, norm_w=None, gate=None, eps=1e-6, out=None):
    """op 21 (+ op 15 when norm_w is given): state [batch, heads, hd, hd] updated in place."""
    lib = _lib.load()
    _dev(state, "state")
    _rows(qkv, "qkv")
    batch = qkv.shape[0]
    if out is None:
        out = torch.empty(batch, heads * hd, dtype=torch.float32, device=qkv.device)
    gs = 0
    if gate is not None:
        _rows(gate, "gate")
        gs = _rs(gate)
    check(lib.rta_delta_rule(_ptr(state), _ptr(qkv), _rs(qkv), _ptr(decay), _ptr(beta), batch, heads, hd,
                             _ptr(norm_w), _ptr(gate), gs, ctypes.c_float(eps), _ptr(out), _rs(out), _stream()),
          "rta_delta_rule")
    return out


def pack_history(k, v, slot, packets, fmt_k=Q4_K, fmt_v=Q6_K):
    """op 34: quantise k[b], v[b] ([batch, kvw] strided rows) into packet slot[b] of packets."""
    lib = _lib.load()
    _rows(k, "k")
    _rows(v, "v")
    _dev(slot, "slot")
    _dev(packets, "packets")
    batch, kvw = k.shape
    n_slots = packets.numel() // history_bytes(kvw)
    check(lib.rta_pack_history(_ptr(k), _rs(k), _ptr(v), _rs(v), batch, kvw, fmt_k, fmt_v, _ptr(slot),
                               n_slots, _ptr(packets), _stream()), "rta_pack_history")
    return packets
