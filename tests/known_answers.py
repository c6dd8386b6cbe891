"""Hand-built known-answer inputs shared by the CPU oracle tests and the GPU tests.

The expected bytes come from codes chosen by hand (through the GGUF block writers in
rta.synth, which the dequantisation tests pin), never from the oracle."""
import numpy as np

from rta import synth


def known_answer_fields():
    """One K row (Q4_K) and one V row (Q6_K) of 256 values built from hand-chosen codes so
    that every quantity of resident_history_quant.glsl:14-38 is exact in fp32, with the
    packet bytes the reference writes for them (GGUF blocks from the same codes):
      Q4_K: group g spans [lo_g, lo_g + 15 c_g 2^-6] with lo_g = -m_g 2^-5; the largest
            group scale is 63 * 2^-6 and the largest minimum 63 * 2^-5, so d = maxD / 63 =
            2^-6 and dmin = maxMin / 63 = 2^-5; value x = lo_g + q c_g 2^-6 has code q.
      Q6_K: group g has max|x| = 31 c_g 2^-8 and the largest code is 127, so d = maxD / 127 =
            2^-8; value x = k c_g 2^-8 has code k + 32.
    Values at exact .5 code steps resolve to the even code (the native round-to-nearest-even
    of both GPU vendors, AMD v_rndne_f32 / NVIDIA cvt.rni, which GLSL round() compiles to);
    values at +.25 / +.75 steps pin rounding to nearest against truncation."""
    rng = np.random.default_rng(2026)
    sc = np.array([63, 40, 17, 1, 50, 33, 8, 0])
    mn = np.array([63, 10, 0, 5, 20, 1, 2, 0])
    q4 = rng.integers(0, 16, (8, 32))
    q4[:7, 0], q4[:7, 1] = 0, 15                 # every live group reaches its lo and hi
    q4[7] = 0                                   # an all-zero group: codes 0
    frac = np.zeros((8, 32))
    # group 1 (c = 40): ties and quarter steps; expected codes below
    ties = [(0.5, 0), (1.5, 2), (2.5, 2), (5.5, 6), (13.5, 14), (14.5, 14), (3.25, 3), (3.75, 4), (0.25, 0)]
    for j, (t, code) in enumerate(ties):
        q4[1, 2 + j], frac[1, 2 + j] = code, t
    k = np.empty(256, np.float32)
    for g in range(8):
        lo = -float(mn[g]) * 2.0 ** -5
        for i in range(32):
            steps = frac[g, i] if frac[g, i] else q4[g, i]
            k[32 * g + i] = lo + steps * sc[g] * 2.0 ** -6
    kblk = synth.pack_q4k(np.array([2.0 ** -6]), np.array([2.0 ** -5]), sc[None], mn[None], q4.reshape(1, 256))
    sc6 = np.array([127, 64, 100, 31, 1, 0, 5, 90, 127, 2, 77, 33, 50, 12, 3, 8])
    kq = rng.integers(-31, 32, (16, 16))
    kq[:, 0] = np.where(np.arange(16) % 2, 31, -31)   # the group's max |x| (either sign)
    kq[5] = 0
    vfrac = np.zeros((16, 16))
    vties = [(2.5, 2), (-2.5, -2), (3.5, 4), (-0.5, 0), (0.5, 0), (-30.5, -30), (7.25, 7), (-7.75, -8)]
    for j, (t, code) in enumerate(vties):
        kq[2, 1 + j], vfrac[2, 1 + j] = code, t
    v = np.empty(256, np.float32)
    for g in range(16):
        for i in range(16):
            steps = vfrac[g, i] if vfrac[g, i] else kq[g, i]
            v[16 * g + i] = steps * sc6[g] * 2.0 ** -8
    vblk = synth.pack_q6k(np.array([2.0 ** -8]), sc6[None], (kq + 32).reshape(1, 256))
    expected = np.zeros(360, np.uint8)                 # roundup8(144 + 210)
    expected[:144] = kblk[0]
    expected[144:354] = vblk[0]
    return k, v, expected
