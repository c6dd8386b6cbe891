"""The published GGML dequantisation loops (dequantize_row_q4_K / _q6_K), the
algorithm of the reference oracle's `gguf` dependency (pyproject.toml:12,
gguf>=0.17; not installed here), written in numpy in GGML's own loop structure.
Independent of the C oracle: it pins it, and produces the golden fixtures.
"""
import numpy as np


def ggml_q4k(raw):
    """dequantize_row_q4_K as GGML publishes it: 64-value steps, scale pairs."""
    raw = np.asarray(raw, dtype=np.uint8).reshape(-1, 144)
    out = np.empty((raw.shape[0], 256), dtype=np.float32)
    for b, blk in enumerate(raw):
        d = blk[0:2].view(np.float16)[0].astype(np.float32)
        mn = blk[2:4].view(np.float16)[0].astype(np.float32)
        scales = blk[4:16]
        q = blk[16:144]

        def get_scale_min_k4(j):
            if j < 4:
                return scales[j] & 63, scales[j + 4] & 63
            return ((scales[j + 4] & 0xF) | ((scales[j - 4] >> 6) << 4),
                    (scales[j + 4] >> 4) | ((scales[j] >> 6) << 4))
        y = []
        for j, is_ in zip(range(0, 256, 64), range(0, 8, 2)):
            sc, m = get_scale_min_k4(is_)
            d1, m1 = d * np.float32(sc), mn * np.float32(m)
            sc, m = get_scale_min_k4(is_ + 1)
            d2, m2 = d * np.float32(sc), mn * np.float32(m)
            qq = q[j // 2: j // 2 + 32]
            y += [d1 * np.float32(v & 0xF) - m1 for v in qq]
            y += [d2 * np.float32(v >> 4) - m2 for v in qq]
        out[b] = np.array(y, dtype=np.float32)
    return out.ravel()


def ggml_q6k(raw):
    """dequantize_row_q6_K as GGML publishes it: 128-value halves, four lanes."""
    raw = np.asarray(raw, dtype=np.uint8).reshape(-1, 210)
    out = np.empty((raw.shape[0], 256), dtype=np.float32)
    for b, blk in enumerate(raw):
        ql, qh = blk[0:128], blk[128:192]
        sc = blk[192:208].view(np.int8)
        d = blk[208:210].view(np.float16)[0].astype(np.float32)
        y = np.empty(256, dtype=np.float32)
        for n in range(2):
            qln, qhn, scn = ql[64 * n:], qh[32 * n:], sc[8 * n:]
            for l in range(32):
                is_ = l // 16
                q1 = int((qln[l] & 0xF) | (((qhn[l] >> 0) & 3) << 4)) - 32
                q2 = int((qln[l + 32] & 0xF) | (((qhn[l] >> 2) & 3) << 4)) - 32
                q3 = int((qln[l] >> 4) | (((qhn[l] >> 4) & 3) << 4)) - 32
                q4 = int((qln[l + 32] >> 4) | (((qhn[l] >> 6) & 3) << 4)) - 32
                y[128 * n + l + 0] = d * np.float32(scn[is_ + 0]) * np.float32(q1)
                y[128 * n + l + 32] = d * np.float32(scn[is_ + 2]) * np.float32(q2)
                y[128 * n + l + 64] = d * np.float32(scn[is_ + 4]) * np.float32(q3)
                y[128 * n + l + 96] = d * np.float32(scn[is_ + 6]) * np.float32(q4)
        out[b] = y
    return out.ravel()
