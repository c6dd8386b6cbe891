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


def one_signed_fields():
    """Known answers whose Q4_K groups lie on one side of zero.  The reference starts each
    group's lo and hi at 0 (resident_history_quant.glsl:14-15), so an all-positive group
    spans [0, max] with minimum 0, and an all-negative one [min, 0] with minimum -min;
    taking the true group min / max instead changes the scale and minimum codes.
    Q4_K: d = 2^-6 (group scale c_g 2^-6, the largest c = 63) and dmin = 10 2^-6 (the
    largest minimum 630 2^-6 = 15 * 42 2^-6, / 63); an all-negative group with scale code c
    has minimum 15 c 2^-6 and code 1.5 c (c even), its values lo + q c 2^-6 with q <= 14
    (all below zero); an all-positive group has minimum code 0 and values q c 2^-6 with
    q >= 1.  Q6_K: groups of one sign alternating, d = 2^-8, codes k + 32.  Every quantity is
    exact in fp32; .5 steps resolve to the even code."""
    rng = np.random.default_rng(2027)
    #           neg  pos  neg  pos  neg  mixed pos  neg
    sc = np.array([42, 63, 10, 17, 2, 20, 1, 6])
    mn = np.array([63, 0, 15, 0, 3, 5, 0, 9])
    sign = np.array([-1, 1, -1, 1, -1, 0, 1, -1])
    q4 = np.empty((8, 32), np.int64)
    frac = np.zeros((8, 32))
    for g in range(8):
        if sign[g] < 0:
            q4[g] = rng.integers(0, 15, 32)
            q4[g, 0] = 0                  # lo reached; hi stays 0 (never reached)
        elif sign[g] > 0:
            q4[g] = rng.integers(1, 16, 32)
            q4[g, 0] = 15                 # hi reached; lo stays 0 (never reached)
        else:
            q4[g] = rng.integers(0, 16, 32)
            q4[g, 0], q4[g, 1] = 0, 15
    # .5 / .25 steps in a positive group (c = 17) and a negative one (c = 2)
    for g, ties in ((3, [(2.5, 2), (3.5, 4), (1.25, 1), (14.5, 14)]), (4, [(0.5, 0), (1.5, 2), (13.5, 14)])):
        for j, (t, code) in enumerate(ties):
            q4[g, 2 + j], frac[g, 2 + j] = code, t
    k = np.empty(256, np.float32)
    for g in range(8):
        lo = -float(mn[g]) * 10 * 2.0 ** -6
        for i in range(32):
            steps = frac[g, i] if frac[g, i] else q4[g, i]
            k[32 * g + i] = lo + steps * sc[g] * 2.0 ** -6
    kb = k.reshape(8, 32)
    assert (kb[sign < 0] < 0).all() and (kb[sign > 0] > 0).all()
    kblk = synth.pack_q4k(np.array([2.0 ** -6]), np.array([10 * 2.0 ** -6]), sc[None], mn[None], q4.reshape(1, 256))
    sc6 = np.array([127, 64, 100, 31, 1, 0, 5, 90, 127, 2, 77, 33, 50, 12, 3, 8])
    kq = np.empty((16, 16), np.int64)
    for g in range(16):
        if g % 2:
            kq[g] = rng.integers(-31, 0, 16)
            kq[g, 0] = -31
        else:
            kq[g] = rng.integers(1, 32, 16)
            kq[g, 0] = 31
    kq[5] = 0
    v = (kq * sc6[:, None] * 2.0 ** -8).astype(np.float32).reshape(256)
    vblk = synth.pack_q6k(np.array([2.0 ** -8]), sc6[None], (kq + 32).reshape(1, 256))
    expected = np.zeros(360, np.uint8)
    expected[:144] = kblk[0]
    expected[144:354] = vblk[0]
    return k, v, expected
