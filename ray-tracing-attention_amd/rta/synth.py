"""Seeded synthetic inputs in GGUF superblock layout.

Field distributions are those of the measured workloads:
  Q4_K: d, dmin = fp16(|N(0,1)| * 0.01); 6-bit scale and min codes ~ U{0..63};
        4-bit quants ~ U{0..15}                                   (144 B / 256 values)
  Q6_K: d = fp16(|N(0,1)| * 0.01); int8 scales ~ U{-32..31}; 6-bit quants ~ U{0..63}
                                                                 (210 B / 256 values)
Byte packing is the inverse of the reference decoder (resident_quant.glsl:10-19;
the scale-byte packing is the one resident_history_quant.glsl:31-32 writes).
"""
import numpy as np

SEED_BASE = 20261110  # the reference verifier's seed (verify_rt_mlp.py:63)


def rng_for(config_index, salt=0):
    return np.random.default_rng([SEED_BASE + config_index, salt])


def pack_q4k(d, dmin, sc, mn, q):
    """d, dmin [n] float; sc, mn [n, 8] codes 0..63; q [n, 256] codes 0..15 -> [n, 144] uint8."""
    n = d.shape[0]
    out = np.zeros((n, 144), dtype=np.uint8)
    out[:, 0:2] = np.asarray(d, dtype=np.float16).reshape(n, 1).view(np.uint8)
    out[:, 2:4] = np.asarray(dmin, dtype=np.float16).reshape(n, 1).view(np.uint8)
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out[:, 4:8] = (sc[:, 0:4] & 63) | ((sc[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (mn[:, 0:4] & 63) | ((mn[:, 4:8] >> 4) << 6)
    out[:, 12:16] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    q = q.astype(np.uint8).reshape(n, 4, 2, 32)       # [chunk j][low/high 32][i]
    out[:, 16:144] = (q[:, :, 0, :] | (q[:, :, 1, :] << 4)).reshape(n, 128)
    return out


def pack_q6k(d, sc, q):
    """d [n]; sc [n, 16] int8; q [n, 256] codes 0..63 -> [n, 210] uint8."""
    n = d.shape[0]
    out = np.zeros((n, 210), dtype=np.uint8)
    q = q.astype(np.uint8).reshape(n, 2, 4, 32)       # [half h][l/32][l%32]
    ql = np.zeros((n, 2, 64), dtype=np.uint8)
    ql[:, :, 0:32] = (q[:, :, 0] & 15) | ((q[:, :, 2] & 15) << 4)
    ql[:, :, 32:64] = (q[:, :, 1] & 15) | ((q[:, :, 3] & 15) << 4)
    qh = (q[:, :, 0] >> 4) | ((q[:, :, 1] >> 4) << 2) | ((q[:, :, 2] >> 4) << 4) | ((q[:, :, 3] >> 4) << 6)
    out[:, 0:128] = ql.reshape(n, 128)
    out[:, 128:192] = qh.reshape(n, 64)
    out[:, 192:208] = np.asarray(sc, dtype=np.int8).view(np.uint8)
    out[:, 208:210] = np.asarray(d, dtype=np.float16).reshape(n, 1).view(np.uint8)
    return out


def random_q4k(rng, nblocks):
    d = (np.abs(rng.standard_normal(nblocks, dtype=np.float32)) * 0.01).astype(np.float16)
    dmin = (np.abs(rng.standard_normal(nblocks, dtype=np.float32)) * 0.01).astype(np.float16)
    sc = rng.integers(0, 64, (nblocks, 8), dtype=np.uint8)
    mn = rng.integers(0, 64, (nblocks, 8), dtype=np.uint8)
    q = rng.integers(0, 16, (nblocks, 256), dtype=np.uint8)
    return pack_q4k(d, dmin, sc, mn, q)


def random_q6k(rng, nblocks):
    d = (np.abs(rng.standard_normal(nblocks, dtype=np.float32)) * 0.01).astype(np.float16)
    sc = rng.integers(-32, 32, (nblocks, 16), dtype=np.int8)
    q = rng.integers(0, 64, (nblocks, 256), dtype=np.uint8)
    return pack_q6k(d, sc, q)


def random_matrix(rng, fmt, rows, cols, chunk_rows=8192):
    """[rows, row_bytes] uint8 matrix with random superblocks (generated in row chunks)."""
    nb = cols // 256
    bb = 144 if fmt == 12 else 210
    out = np.empty((rows, nb * bb), dtype=np.uint8)
    for r0 in range(0, rows, chunk_rows):
        r1 = min(rows, r0 + chunk_rows)
        blocks = random_q4k(rng, (r1 - r0) * nb) if fmt == 12 else random_q6k(rng, (r1 - r0) * nb)
        out[r0:r1] = blocks.reshape(r1 - r0, nb * bb)
    return out


def history_bytes(kvw):
    return ((kvw + 255) // 256 * (144 + 210) + 7) // 8 * 8


def random_packets(rng, count, kvw, fmt_k, fmt_v):
    """count history packets: field K (fmt_k) then field V (fmt_v), random fields."""
    nb = (kvw + 255) // 256
    stride = history_bytes(kvw)
    out = np.zeros((count, stride), dtype=np.uint8)
    at = 0
    for fmt in (fmt_k, fmt_v):
        bb = 144 if fmt == 12 else 210
        blocks = random_q4k(rng, count * nb) if fmt == 12 else random_q6k(rng, count * nb)
        out[:, at:at + nb * bb] = blocks.reshape(count, nb * bb)
        at += nb * bb
    return out


def log_uniform_lengths(rng, n, lo, hi):
    """floor(exp(U(ln lo, ln hi))) -- ragged context lengths."""
    return np.floor(np.exp(rng.uniform(np.log(lo), np.log(hi), n))).astype(np.int64).clip(lo, hi)
