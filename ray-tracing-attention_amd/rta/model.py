"""Hybrid decoder (gated delta-net recurrent layers + full attention) over
librta.so's rta_hybrid_* entry points: ctypes mirrors of the C structs, synthetic
random-init weights and states of a given shape, and one greedy decode step.

The C driver (rta_hybrid_decode_step) sequences the layers the way the reference's
worker does (optical_resident.cpp:455-530); this module only owns device memory.
"""
import ctypes
import math

import torch

from . import _lib
from ._lib import Q4_K, Q6_K, TILED, check
from . import ops

_i, _f, _d, _p, _i64 = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_void_p, ctypes.c_int64


class HybridShape(ctypes.Structure):
    _fields_ = [("hidden", _i), ("layers", _i), ("full_every", _i), ("q_heads", _i), ("kv_heads", _i),
                ("head_dim", _i), ("rec_heads", _i), ("ff", _i), ("vocab", _i), ("capacity", _i),
                ("fmt_embed", _i), ("fmt_proj", _i), ("fmt_lm", _i), ("fmt_k", _i), ("fmt_v", _i),
                ("rope_rotary", _i), ("eps", _f), ("margin", _f), ("rope_theta", _d),
                ("attn_gate", _i), ("rec_key_heads", _i), ("layer_formats", _i), ("o_axis_remap", _i)]


class HybridLayer(ctypes.Structure):
    _fields_ = [(n, _p) for n in ("norm_in", "norm_post", "w_in", "w_o", "w_gate", "w_up", "w_down", "q_norm",
                                  "k_norm", "conv_w", "a_log", "dt_bias", "out_norm")] + \
               [("fmt_in", _i), ("fmt_o", _i), ("fmt_gate_up", _i), ("fmt_down", _i), ("w_a", _p), ("w_b", _p),
                ("fmt_ab", _i), ("in_parts", _i), ("in_w", _p * 4), ("in_rows", _i * 4), ("in_fmt", _i * 4)]


class HybridWeights(ctypes.Structure):
    _fields_ = [("embed", _p), ("layers", ctypes.POINTER(HybridLayer)), ("norm_final", _p), ("lm_head", _p)]


class HybridViews(ctypes.Structure):
    _fields_ = [("recurrent", _p), ("conv", _p), ("packets", _p), ("slot_base", _p), ("ctx", _p),
                ("recurrent_per_layer", _i64), ("conv_per_layer", _i64), ("packet_bytes", _i64),
                ("slots_per_layer", _i64)]


class HybridCapture(ctypes.Structure):
    _fields_ = [("residual", _p), ("residual_from", _i), ("kv", _p), ("marks", ctypes.POINTER(_p))]


_SIGS = {
    "rta_hybrid_state_bytes": (ctypes.c_size_t, [ctypes.POINTER(HybridShape), _i]),
    "rta_hybrid_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(HybridShape), _i]),
    "rta_hybrid_layout": (_i, [ctypes.POINTER(HybridShape), _i, _p, ctypes.POINTER(HybridViews)]),
    "rta_hybrid_init": (_i, [ctypes.POINTER(HybridShape), _i, _p, _p, _p]),
    "rta_hybrid_decode_step": (_i, [ctypes.POINTER(HybridShape), ctypes.POINTER(HybridWeights), _i, _p, _p, _p, _p,
                                    ctypes.c_size_t, _p]),
    "rta_hybrid_decode_step_capture": (_i, [ctypes.POINTER(HybridShape), ctypes.POINTER(HybridWeights), _i, _p, _p,
                                            _p, ctypes.POINTER(HybridCapture), _p, ctypes.c_size_t, _p]),
}


def _lib_h():
    lib = _lib.load()
    for name, (res, args) in _SIGS.items():
        f = getattr(lib, name)
        f.restype, f.argtypes = res, args
    return lib


def shape_9b(capacity, packed=True):
    """The 9B-like shape: 32 layers (3 recurrent : 1 full), hidden 4096, 32/8 heads x 128,
    32 delta-net heads, FF 12288, vocab 151936, Q4_K projections, Q6_K LM head."""
    return HybridShape(hidden=4096, layers=32, full_every=4, q_heads=32, kv_heads=8, head_dim=128, rec_heads=32,
                       ff=12288, vocab=151936, capacity=capacity, fmt_embed=Q4_K,
                       fmt_proj=Q4_K | (TILED if packed else 0), fmt_lm=Q6_K | (TILED if packed else 0),
                       fmt_k=Q4_K, fmt_v=Q6_K, rope_rotary=128, eps=1e-6, margin=1e-4, rope_theta=1e6)


# ------------------------------------------------------------- synthetic data ----
def random_kquant(fmt, rows, cols, gen, dev, d_scale=0.01):
    """A [rows x cols] GGUF matrix with the fields of the benchmark configs: Q4_K 6-bit
    scale / min codes and 4-bit quants uniform, d and dmin = |N(0,1)| * d_scale;
    Q6_K int8 scales uniform in [-32, 31], 6-bit quants uniform, d = |N(0,1)| * d_scale."""
    nsb = cols // 256
    blk = 144 if fmt == Q4_K else 210
    w = torch.randint(0, 256, (rows * nsb, blk), dtype=torch.uint8, device=dev, generator=gen)
    n = rows * nsb
    half = lambda: (torch.randn(n, device=dev, generator=gen).abs() * d_scale).to(torch.float16).view(torch.uint8)
    if fmt == Q4_K:
        w[:, 0:2] = half().view(n, 2)
        w[:, 2:4] = half().view(n, 2)
    else:
        w[:, 192:208] = torch.randint(-32, 32, (n, 16), dtype=torch.int8, device=dev, generator=gen).view(torch.uint8)
        w[:, 208:210] = half().view(n, 2)
    return w.view(rows, nsb * blk)


def _near_one(n, gen, dev, spread=0.05):
    return (1.0 + spread * torch.randn(n, device=dev, generator=gen)).float()


def random_float_matrix(fmt, rows, cols, gen, dev, scale=0.02):
    """A [rows x cols] F32 / F16 / BF16 matrix (as row bytes) of N(0, scale^2) values."""
    v = torch.randn(rows, cols, device=dev, generator=gen) * scale
    if fmt == _lib.F32:
        return v.contiguous().view(torch.uint8).view(rows, -1)
    if fmt == _lib.F16:
        return v.half().contiguous().view(torch.uint8).view(rows, -1)
    return (v.contiguous().view(torch.int32) >> 16).to(torch.int16).view(torch.uint8).view(rows, -1)


class DecodeModel:
    """Device weights + state of a hybrid decoder and its graph-replayable decode step.

    With shape.layer_formats, layer_fmts(l, full) gives each layer's formats as a dict
    {"in", "o", "gate_up", "down", "ab"}; separate_ab keeps the delta-net a / b rows as
    matrices of their own (w_a, w_b); in_parts(l, full), when it returns a list of
    formats, splits the in-projection into that many parts of equal row counts
    (matrices "<l>.w_in.<i>", each in its format), or, given (rows, format) pairs, into parts of
    those row counts.  self.fmts names each matrix's format."""

    def __init__(self, shape, batch, ctx, seed=20261115, dev="cuda:0", keep_gguf=False, layer_fmts=None,
                 separate_ab=False, in_parts=None):
        self.lib = _lib_h()
        self.shape = shape
        self.batch = batch
        self.dev = torch.device(dev)
        gen = torch.Generator(device=self.dev)
        gen.manual_seed(seed)
        s = shape
        self._keep = []
        self.gguf = {} if keep_gguf else None   # name -> GGUF matrix (tests feed these to the oracle)
        self.mats = {}                            # name -> device matrix as the step reads it
        self.fmts = {}                            # name -> its format code
        base_fmt = lambda f: f & 0xff

        def mat(fmt, rows, cols, d_scale=0.01, small_rows=0, name=None):
            if name:
                self.fmts[name] = fmt
            if base_fmt(fmt) not in (Q4_K, Q6_K):
                w = random_float_matrix(fmt, rows, cols, gen, self.dev, 1e-4 if small_rows else 0.02)
                if self.gguf is not None and name:
                    self.gguf[name] = w.cpu().numpy()
                self._keep.append(w)
                if name:
                    self.mats[name] = w
                return w
            w = random_kquant(base_fmt(fmt), rows, cols, gen, self.dev, d_scale)
            if small_rows:   # the delta-net a / b rows: tiny, so decay stays near its target
                nsb = cols // 256
                tail = w.view(rows, nsb, -1)[rows - small_rows:]
                hv = (torch.randn(small_rows * nsb, device=self.dev, generator=gen).abs() * 1e-6).to(torch.float16)
                hv = hv.view(torch.uint8).view(small_rows, nsb, 2)
                if base_fmt(fmt) == Q4_K:
                    tail[:, :, 0:2] = hv
                    tail[:, :, 2:4] = 0
                else:
                    tail[:, :, 208:210] = hv
            if self.gguf is not None and name:
                self.gguf[name] = w.cpu().numpy()
            if fmt & TILED:
                w = ops.pack(base_fmt(fmt), w, rows, cols)
            self._keep.append(w)
            if name:
                self.mats[name] = w
            return w

        def vec(t, name=None):
            self._keep.append(t)
            if self.gguf is not None and name:
                self.gguf[name] = t.cpu().numpy()
            return t.data_ptr()

        hd, S, H = s.head_dim, s.rec_heads * s.head_dim, s.rec_heads
        KH = s.rec_key_heads or H
        self.separate_ab = separate_ab
        self.layers = (HybridLayer * s.layers)()
        for l in range(s.layers):
            L = self.layers[l]
            L.norm_in = vec(_near_one(s.hidden, gen, self.dev), f"{l}.norm_in")
            L.norm_post = vec(_near_one(s.hidden, gen, self.dev), f"{l}.norm_post")
            full = s.full_every > 0 and l % s.full_every == s.full_every - 1
            lf = layer_fmts(l, full) if (s.layer_formats and layer_fmts) else {}
            f_in, f_o = lf.get("in", s.fmt_proj), lf.get("o", s.fmt_proj)
            f_gu, f_d, f_ab = lf.get("gate_up", s.fmt_proj), lf.get("down", s.fmt_proj), lf.get("ab", s.fmt_proj)
            L.fmt_in, L.fmt_o, L.fmt_gate_up, L.fmt_down, L.fmt_ab = f_in, f_o, f_gu, f_d, f_ab
            split = in_parts(l, full) if in_parts else None
            if full:
                rows = (s.q_heads * (2 if s.attn_gate else 1) + 2 * s.kv_heads) * hd
                if split:
                    self._parts(L, l, split, rows, mat)
                else:
                    L.w_in = mat(f_in, rows, s.hidden, name=f"{l}.w_in").data_ptr()
                L.w_o = mat(f_o, s.hidden, s.q_heads * hd, name=f"{l}.w_o").data_ptr()
                L.q_norm = vec(_near_one(s.q_heads * hd, gen, self.dev), f"{l}.q_norm")
                L.k_norm = vec(_near_one(s.kv_heads * hd, gen, self.dev), f"{l}.k_norm")
            else:
                rows = 2 * KH * hd + 2 * S + (0 if separate_ab else 2 * H)
                if split:
                    assert separate_ab, "in-projection parts hold no a / b rows"
                    self._parts(L, l, split, rows, mat)
                else:
                    L.w_in = mat(f_in, rows, s.hidden, small_rows=0 if separate_ab else 2 * H,
                                 name=f"{l}.w_in").data_ptr()
                if separate_ab:
                    L.w_a = mat(f_ab, H, s.hidden, small_rows=H, name=f"{l}.w_a").data_ptr()
                    L.w_b = mat(f_ab, H, s.hidden, small_rows=H, name=f"{l}.w_b").data_ptr()
                L.w_o = mat(f_o, s.hidden, S, name=f"{l}.w_o").data_ptr()
                L.conv_w = vec((0.5 * torch.randn(3 * S, 4, device=self.dev, generator=gen)).float(), f"{l}.conv_w")
                # decay ~ U(0.9, 0.999) at a = 0: exp(a_log) softplus(dt_bias) = -ln(decay)
                target = 0.9 + 0.099 * torch.rand(H, device=self.dev, generator=gen)
                dt = 2.0 * torch.rand(H, device=self.dev, generator=gen) - 1.0
                sp = torch.nn.functional.softplus(dt)
                L.a_log = vec(torch.log(-torch.log(target) / sp).float(), f"{l}.a_log")
                L.dt_bias = vec(dt.float(), f"{l}.dt_bias")
                L.out_norm = vec(_near_one(S, gen, self.dev), f"{l}.out_norm")
            L.w_gate = mat(f_gu, s.ff, s.hidden, name=f"{l}.w_gate").data_ptr()
            L.w_up = mat(f_gu, s.ff, s.hidden, name=f"{l}.w_up").data_ptr()
            L.w_down = mat(f_d, s.hidden, s.ff, name=f"{l}.w_down").data_ptr()
        self.embed = random_kquant(s.fmt_embed, s.vocab, s.hidden, gen, self.dev)
        self.norm_final = _near_one(s.hidden, gen, self.dev)
        if self.gguf is not None:
            self.gguf["embed"] = self.embed.cpu().numpy()
            self.gguf["norm_final"] = self.norm_final.cpu().numpy()
        self.lm_head = mat(s.fmt_lm, s.vocab, s.hidden, name="lm_head")
        self.weights = HybridWeights(embed=self.embed.data_ptr(), layers=self.layers,
                                     norm_final=self.norm_final.data_ptr(), lm_head=self.lm_head.data_ptr())
        # state: recurrent N(0, 0.1), conv window N(0, 1), history packets random with
        # sane block scales, positions = ctx
        nbytes = self.lib.rta_hybrid_state_bytes(ctypes.byref(s), batch)
        assert nbytes > 0, "invalid hybrid shape"
        self.state = torch.empty(nbytes, dtype=torch.uint8, device=self.dev)
        v = HybridViews()
        check(self.lib.rta_hybrid_layout(ctypes.byref(s), batch, self.state.data_ptr(), ctypes.byref(v)),
              "rta_hybrid_layout")
        self.views = v
        nrec = s.layers - (s.layers // s.full_every if s.full_every else 0)
        nfull = s.layers - nrec
        off = lambda p: p - self.state.data_ptr()
        st = self.state
        if nrec:
            rec = st[off(v.recurrent):off(v.recurrent) + 4 * nrec * v.recurrent_per_layer].view(torch.float32)
            rec.normal_(0.0, 0.1, generator=gen)
            conv = st[off(v.conv):off(v.conv) + 4 * nrec * v.conv_per_layer].view(torch.float32)
            conv.normal_(0.0, 1.0, generator=gen)
        if nfull:
            pk = st[off(v.packets):off(v.packets) + nfull * v.slots_per_layer * v.packet_bytes]
            self._random_packets(pk.view(-1, v.packet_bytes), gen)
        self.ctx = torch.as_tensor(ctx, dtype=torch.int32, device=self.dev)
        check(self.lib.rta_hybrid_init(ctypes.byref(s), batch, self.state.data_ptr(), self.ctx.data_ptr(),
                                       ops._stream()), "rta_hybrid_init")
        self.ws_bytes = self.lib.rta_hybrid_workspace_bytes(ctypes.byref(s), batch)
        self.workspace = torch.empty(self.ws_bytes, dtype=torch.uint8, device=self.dev)
        self.tokens = torch.randint(0, s.vocab, (batch,), dtype=torch.int32, device=self.dev, generator=gen)
        self.logits = None

    def _parts(self, L, l, fmts, rows, mat):
        """fmts: a format per part (equal row counts) or (rows, format) pairs."""
        n = len(fmts)
        if all(isinstance(f, tuple) for f in fmts):
            parts = list(fmts)
        else:
            assert rows % (16 * n) == 0, (rows, n)
            parts = [(rows // n, f) for f in fmts]
        assert 0 < n <= 4 and sum(r for r, _ in parts) == rows, (rows, parts)
        L.in_parts = n
        self.parts = getattr(self, "parts", {})
        self.parts[l] = parts
        for i, (r, f) in enumerate(parts):
            L.in_w[i] = mat(f, r, self.shape.hidden, name=f"{l}.w_in.{i}").data_ptr()
            L.in_rows[i], L.in_fmt[i] = r, f

    def _random_packets(self, pk, gen):
        """K (Q4_K) / V (Q6_K) history fields with random quants and sane block scales."""
        s = self.shape
        kvw = s.kv_heads * s.head_dim
        nb = (kvw + 255) // 256
        pk.random_(0, 256, generator=gen)
        n = pk.shape[0]
        half = lambda: (torch.rand(n, device=self.dev, generator=gen) * 0.01 + 1e-3).to(torch.float16).view(
            torch.uint8).view(n, 2)
        koff, kb = 0, (144 if s.fmt_k == Q4_K else 210)
        voff, vb = nb * kb, (144 if s.fmt_v == Q4_K else 210)
        for fld_off, bb, fmt in ((koff, kb, s.fmt_k), (voff, vb, s.fmt_v)):
            for b in range(nb):
                o = fld_off + b * bb
                if fmt == Q4_K:
                    pk[:, o:o + 2] = half()
                    pk[:, o + 2:o + 4] = half()
                else:
                    pk[:, o + 192:o + 208] = torch.randint(-32, 32, (n, 16), dtype=torch.int8, device=self.dev,
                                                           generator=gen).view(torch.uint8)
                    pk[:, o + 208:o + 210] = half()
        pk[:, nb * (kb + vb):] = 0   # the packet's padding to 8 bytes

    def step(self, logits=False, capture=False):
        """One greedy decode step for every sequence (tokens and positions advance on the device).
        capture: also fill self.residual [layers + 1, B, hidden] (the embedding rows, then the
        residual stream after each layer) and self.kv [full layers, B, 2, kv_heads * 128] (the
        key and value rows each full layer packed into its history)."""
        if logits and self.logits is None:
            self.logits = torch.empty(self.batch, self.shape.vocab, dtype=torch.float32, device=self.dev)
        lg = self.logits.data_ptr() if logits else None
        if not capture:
            check(self.lib.rta_hybrid_decode_step(ctypes.byref(self.shape), ctypes.byref(self.weights), self.batch,
                                                  self.state.data_ptr(), self.tokens.data_ptr(), lg,
                                                  self.workspace.data_ptr(), self.ws_bytes, ops._stream()),
                  "rta_hybrid_decode_step")
            return self.tokens
        s = self.shape
        nfull = s.layers // s.full_every if s.full_every else 0
        self.residual = torch.full((s.layers + 1, self.batch, s.hidden), float("nan"), device=self.dev)
        self.kv = torch.full((max(nfull, 1), self.batch, 2, s.kv_heads * s.head_dim), float("nan"), device=self.dev)
        cap = HybridCapture(residual=self.residual.data_ptr(), residual_from=0,
                            kv=self.kv.data_ptr() if nfull else None, marks=None)
        check(self.lib.rta_hybrid_decode_step_capture(ctypes.byref(self.shape), ctypes.byref(self.weights),
                                                      self.batch, self.state.data_ptr(), self.tokens.data_ptr(), lg,
                                                      ctypes.byref(cap), self.workspace.data_ptr(), self.ws_bytes,
                                                      ops._stream()),
              "rta_hybrid_decode_step_capture")
        return self.tokens

    def weight_bytes(self):
        """HBM bytes of the weights one step streams (embedding rows excluded)."""
        return sum(t.numel() * t.element_size() for t in self._keep)

    def state_view(self, kind):
        """numpy copy of one part of the state: 'recurrent' [nrec, B, H, hd, hd], 'conv'
        [nrec, B, 3S, 3], 'packets' [nfull, B, capacity, packet_bytes], 'ctx' [B]."""
        import numpy as np
        s, v = self.shape, self.views
        nfull = s.layers // s.full_every if s.full_every else 0
        nrec = s.layers - nfull
        B, hd, S = self.batch, s.head_dim, s.rec_heads * s.head_dim

        def part(ptr, n):   # copies only the bytes of that part to the host
            at = ptr - self.state.data_ptr()
            return self.state[at:at + n].cpu().numpy()

        if kind == "recurrent":
            raw = part(v.recurrent, nrec * v.recurrent_per_layer * 4)
            return raw.view(np.float32).reshape(nrec, B, s.rec_heads, hd, hd)
        if kind == "conv":
            raw = part(v.conv, nrec * v.conv_per_layer * 4)
            return raw.view(np.float32).reshape(nrec, B, 3 * S, 3)
        if kind == "packets":
            raw = part(v.packets, nfull * v.slots_per_layer * v.packet_bytes)
            return raw.reshape(nfull, B, s.capacity, v.packet_bytes)
        if kind == "ctx":
            return part(v.ctx, 4 * B).view(np.int32).copy()
        raise ValueError(kind)
