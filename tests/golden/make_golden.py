"""Writes dequant_golden.npz: adversarial Q4_K / Q6_K superblocks and their fp32
values, computed with the published GGML dequantisation loops (the algorithm of
the reference oracle's `gguf` dependency), independently of the C oracle.

Blocks cover: random fields; every 6-bit scale/min code; fp16 subnormal, tiny,
maximal (65504) and negative-zero d/dmin; all-15 / all-0 nibbles; Q6_K codes 0
and 63 with int8 scales -128 and 127.
Run: python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent / "ray-tracing-attention_amd"))
sys.path.insert(0, str(HERE.parent))
from rta import synth  # noqa: E402
from ggml_ref import ggml_q4k, ggml_q6k  # noqa: E402


def main():
    rng = np.random.default_rng(20261110)
    q4 = [synth.random_q4k(rng, 4)]
    codes = np.arange(64, dtype=np.uint8)
    sc = np.stack([np.roll(codes, k)[:8] for k in range(8)])
    mn = np.stack([np.roll(codes[::-1], k)[:8] for k in range(8)])
    d = np.array([1.0, 6e-8, 6.1e-5, 65504.0, -0.0, 0.5, 1e-3, 2.0], np.float16)
    dm = np.array([0.25, 65504.0, 6e-8, -0.0, 1.0, 6.1e-5, 0.0, 3.0], np.float16)
    qq = np.stack([np.full(256, 15), np.zeros(256), np.arange(256) % 16, (np.arange(256) * 5) % 16,
                   np.full(256, 8), np.arange(256)[::-1] % 16, np.full(256, 1), np.arange(256) % 7]).astype(np.uint8)
    q4.append(synth.pack_q4k(d, dm, sc, mn, qq))
    for c0 in range(0, 64, 8):   # every code in every group slot
        s = np.stack([(codes[c0:c0 + 8] + g) % 64 for g in range(8)])
        q4.append(synth.pack_q4k(np.ones(8, np.float16), np.full(8, 0.5, np.float16), s, s[::-1], qq))
    q4 = np.concatenate(q4)
    q6 = [synth.random_q6k(rng, 4)]
    sc6 = np.stack([np.full(16, -128), np.full(16, 127), np.arange(-8, 8), np.zeros(16)]).astype(np.int8)
    q6c = np.stack([np.zeros(256), np.full(256, 63), np.arange(256) % 64, (np.arange(256) * 11) % 64]).astype(np.uint8)
    q6.append(synth.pack_q6k(np.array([1.0, 6e-8, 65504.0, -0.0], np.float16), sc6, q6c))
    q6 = np.concatenate(q6)
    np.savez_compressed(HERE / "dequant_golden.npz", q4k_raw=q4, q4k_values=ggml_q4k(q4),
                        q6k_raw=q6, q6k_values=ggml_q6k(q6))
    print("wrote", HERE / "dequant_golden.npz", q4.shape, q6.shape)


if __name__ == "__main__":
    main()
