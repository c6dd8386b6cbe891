/*
 * rta_oracle.c -- CPU restatement of the Ray Tracing Attention detector path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Only tests/, __graft_entry__.smoke()
 * and bench.py's cpu_baseline leg load this library; the product library never
 * does.  Compiled with -ffp-contract=off: every dequantised value is formed with
 * the reference's fp32 op order, (d*sc)*q - (dmin*m), with no fused multiply-add.
 *
 * Citations are relative to the reference repository root.
 */
#include "rta_oracle.h"
#include <math.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- binary16 ----------------------------------------------------------- */
float orc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u, exp = (h >> 10) & 31u, man = h & 1023u;
    float mag;
    if (exp == 0) mag = ldexpf((float)man, -24);                 /* zero / subnormal */
    else if (exp == 31) mag = man ? NAN : INFINITY;
    else mag = ldexpf((float)(man | 1024u), (int)exp - 25);
    return sign ? -mag : mag;
}

uint16_t orc_float_to_half(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    float a; memcpy(&a, &ax, 4);
    if (a >= 65520.0f) return (uint16_t)(sign | 0x7c00u);        /* rounds to inf */
    if (a < ldexpf(1.0f, -14)) {                                  /* subnormal range */
        float s = a * 16777216.0f;                                /* exact: power of two */
        uint32_t q = (uint32_t)rintf(s);                          /* RNE */
        return (uint16_t)(sign | q);
    }
    int e; float m = frexpf(a, &e);                               /* a = m * 2^e, m in [0.5,1) */
    float scaled = ldexpf(m, 11);                                 /* [1024, 2048) */
    uint32_t q = (uint32_t)rintf(scaled);                         /* RNE on 11 bits */
    int he = e - 1 + 15;
    if (q == 2048u) { q = 1024u; he += 1; }
    if (he >= 31) return (uint16_t)(sign | 0x7c00u);
    return (uint16_t)(sign | ((uint32_t)he << 10) | (q & 1023u));
}

static float bf16_to_float(uint16_t b) { uint32_t x = (uint32_t)b << 16; float f; memcpy(&f, &x, 4); return f; }

int64_t orc_row_bytes(int fmt, int64_t cols) {
    switch (fmt) {
    case ORC_F32: return cols * 4;
    case ORC_F16: case ORC_BF16: return cols * 2;
    case ORC_Q4_K: return (cols / 256) * 144;
    case ORC_Q6_K: return (cols / 256) * 210;
    default: return -1;
    }
}

/* ---- Q4_K: resident_quant.glsl:10-15 (ggufValue type 12) ----------------- */
static void q4k_scale_min(const uint8_t* s, int g, unsigned* sc, unsigned* m) {
    /* s = bytes 4..15 of the superblock; resident_quant.glsl:11-12, q4ScaleMin :39-43 */
    if (g < 4) { *sc = s[g] & 63u; *m = s[g + 4] & 63u; }
    else {
        int p = g - 4; unsigned mixed = s[8 + p];
        *sc = (mixed & 15u) | ((unsigned)(s[p] >> 6) << 4);
        *m  = (mixed >> 4)  | ((unsigned)(s[4 + p] >> 6) << 4);
    }
}

static void dequant_q4k_block(const uint8_t* b, float* out) {
    float d    = orc_half_to_float((uint16_t)(b[0] | (b[1] << 8)));
    float dmin = orc_half_to_float((uint16_t)(b[2] | (b[3] << 8)));
    for (int i = 0; i < 256; ++i) {
        unsigned sc, m; q4k_scale_min(b + 4, i / 32, &sc, &m);
        unsigned q = (b[16 + (i / 64) * 32 + i % 32] >> (((i % 64) / 32) * 4)) & 15u;
        float ds = d * (float)sc;          /* (coefficientHalf(at)*float(sc)) */
        float dq = ds * (float)q;          /*  ... *float(q) */
        float dm = dmin * (float)m;        /* coefficientHalf(at+2)*float(minval) */
        out[i] = dq - dm;
    }
}

/* ---- Q6_K: resident_quant.glsl:16-19 (ggufValue type 14) ----------------- */
static void dequant_q6k_block(const uint8_t* b, float* out) {
    float d = orc_half_to_float((uint16_t)(b[208] | (b[209] << 8)));
    for (int i = 0; i < 256; ++i) {
        int h = i / 128, l = i % 128;
        unsigned ql = (b[h * 64 + l % 64] >> ((l / 64) * 4)) & 15u;
        unsigned qh = (b[128 + h * 32 + l % 32] >> ((l / 32) * 2)) & 3u;
        int sc = (int8_t)b[192 + i / 16];
        float ds = d * (float)sc;
        out[i] = ds * (float)((int)(ql | (qh << 4)) - 32);
    }
}

int orc_dequant(int fmt, const void* src, int64_t n, float* out) {
    const uint8_t* p = (const uint8_t*)src;
    if (!src || !out || n < 0) return 1;
    switch (fmt) {
    case ORC_F32: memcpy(out, src, (size_t)n * 4); return 0;
    case ORC_F16: for (int64_t i = 0; i < n; ++i) out[i] = orc_half_to_float((uint16_t)(p[2*i] | (p[2*i+1] << 8))); return 0;
    case ORC_BF16: for (int64_t i = 0; i < n; ++i) out[i] = bf16_to_float((uint16_t)(p[2*i] | (p[2*i+1] << 8))); return 0;
    case ORC_Q4_K: if (n % 256) return 2; for (int64_t b = 0; b < n / 256; ++b) dequant_q4k_block(p + b * 144, out + b * 256); return 0;
    case ORC_Q6_K: if (n % 256) return 2; for (int64_t b = 0; b < n / 256; ++b) dequant_q6k_block(p + b * 210, out + b * 256); return 0;
    default: return 3;
    }
}

static int valid_shape(int fmt, int rows, int cols) {
    if (rows <= 0 || cols <= 0) return 0;
    if ((fmt == ORC_Q4_K || fmt == ORC_Q6_K) && cols % 256) return 0;
    return orc_row_bytes(fmt, cols) > 0;
}

/* ---- GEMV (resident_math.comp:39-75 op 2; fp64 closed form verify_rt_mlp.py:84-89) */
int orc_gemv_f64(int fmt, const void* W, int rows, int cols, const float* x, int batch, double* y) {
    if (!W || !x || !y || batch <= 0 || !valid_shape(fmt, rows, cols)) return 1;
    int64_t rb = orc_row_bytes(fmt, cols);
    #pragma omp parallel
    {
        float* w = (float*)malloc((size_t)cols * sizeof(float));
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            orc_dequant(fmt, (const uint8_t*)W + (int64_t)r * rb, cols, w);
            for (int b = 0; b < batch; ++b) {
                double acc = 0.0; const float* xb = x + (int64_t)b * cols;
                for (int c = 0; c < cols; ++c) acc += (double)w[c] * (double)xb[c];
                y[(int64_t)b * rows + r] = acc;
            }
        }
        free(w);
    }
    return 0;
}

/* ---- row / axis remap (resident_quant.glsl:20-31 quantizedWeight; the mode is the
 * descriptor's metadata >> 8, assigned by compiler/export.py:96-98,108) ---------- */
/* originalRotaryAxis, resident_quant.glsl:20 */
int64_t orc_rotary_source(int64_t axis, int rotary) {
    return axis < rotary ? (axis % 2) * (rotary / 2) + axis / 2 : axis;
}

/* resident_quant.glsl:23-26: the row a detector row reads (modes 1, 2, 3, 5) */
int64_t orc_remap_row(int mode, int hd, int rotary, int key_rows, int64_t row) {
    if (mode == 1 || mode == 2)
        return (row / hd) * (2 * (int64_t)hd) + (mode == 2 ? hd : 0) + orc_rotary_source(row % hd, rotary);
    if (mode == 3) return (row / hd) * hd + orc_rotary_source(row % hd, rotary);
    if (mode == 5) return row % key_rows;
    return row;
}

/* resident_quant.glsl:25: the column a detector axis reads (mode 4) */
int64_t orc_remap_axis(int mode, int hd, int rotary, int64_t axis) {
    return mode == 4 ? (axis / hd) * hd + orc_rotary_source(axis % hd, rotary) : axis;
}

/* y[b, r] = sum_a quantizedWeight(row r, axis a) x[b, a] in fp64, each weight taken
 * from the remapped (row, axis) of W (src_rows rows) as resident_quant.glsl:27-30 does. */
int orc_gemv_remap_f64(int fmt, const void* W, int src_rows, int rows, int cols, int mode, int hd, int rotary,
                       int key_rows, const float* x, int batch, double* y) {
    if (!W || !x || !y || batch <= 0 || !valid_shape(fmt, src_rows, cols) || rows <= 0) return 1;
    if (mode < 0 || mode > 5 || (mode >= 1 && mode <= 4 && (hd <= 0 || rotary < 0 || rotary > hd)) ||
        (mode == 5 && key_rows <= 0) || (mode == 4 && cols % hd))
        return 2;
    for (int r = 0; r < rows; ++r) {
        int64_t sr = orc_remap_row(mode, hd, rotary, key_rows, r);
        if (sr < 0 || sr >= src_rows) return 3;
    }
    int64_t rb = orc_row_bytes(fmt, cols);
    float* w = (float*)malloc((size_t)cols * sizeof(float));
    for (int r = 0; r < rows; ++r) {
        orc_dequant(fmt, (const uint8_t*)W + orc_remap_row(mode, hd, rotary, key_rows, r) * rb, cols, w);
        for (int b = 0; b < batch; ++b) {
            double acc = 0.0; const float* xb = x + (int64_t)b * cols;
            for (int a = 0; a < cols; ++a) acc += (double)w[orc_remap_axis(mode, hd, rotary, a)] * (double)xb[a];
            y[(int64_t)b * rows + r] = acc;
        }
    }
    free(w);
    return 0;
}

int orc_gemv_f32(int fmt, const void* W, int rows, int cols, const float* x, int batch, float* y, int threads) {
    if (!W || !x || !y || batch <= 0 || !valid_shape(fmt, rows, cols)) return 1;
    int64_t rb = orc_row_bytes(fmt, cols);
#ifdef _OPENMP
    if (threads > 0) omp_set_num_threads(threads);
#else
    (void)threads;
#endif
    #pragma omp parallel
    {
        float* w = (float*)malloc((size_t)cols * sizeof(float));
        #pragma omp for schedule(static)
        for (int r = 0; r < rows; ++r) {
            orc_dequant(fmt, (const uint8_t*)W + (int64_t)r * rb, cols, w);
            for (int b = 0; b < batch; ++b) {
                float acc = 0.0f; const float* xb = x + (int64_t)b * cols;
                for (int c = 0; c < cols; ++c) acc += w[c] * xb[c];
                y[(int64_t)b * rows + r] = acc;
            }
        }
        free(w);
    }
    return 0;
}

/* ---- SwiGLU (resident_math.comp:71; resident_common.glsl:138) ------------- */
double orc_sigmoid(double v) {
    if (v >= 0) return 1.0 / (1.0 + exp(-v));
    double light = exp(v);
    return light / (1.0 + light);
}

static double sgn(double v) { return v > 0 ? 1.0 : (v < 0 ? -1.0 : 0.0); }

int orc_mlp_swiglu(int fmt_g, const void* Wg, int fmt_u, const void* Wu, int fmt_d, const void* Wd,
                   int hidden, int inter, const float* x, int batch, const float* y_in,
                   double* act, double* y) {
    if (!act || !y || batch <= 0) return 1;
    double* g = (double*)malloc(sizeof(double) * (size_t)batch * inter);
    double* u = (double*)malloc(sizeof(double) * (size_t)batch * inter);
    float* a32 = (float*)malloc(sizeof(float) * (size_t)batch * inter);
    double* d = (double*)malloc(sizeof(double) * (size_t)batch * hidden);
    int rc = orc_gemv_f64(fmt_g, Wg, inter, hidden, x, batch, g);
    if (!rc) rc = orc_gemv_f64(fmt_u, Wu, inter, hidden, x, batch, u);
    if (!rc) {
        for (int64_t i = 0; i < (int64_t)batch * inter; ++i) {
            double gv = g[i], uv = u[i];
            act[i] = sgn(gv) * sgn(uv) * (fabs(gv) * fabs(uv) * orc_sigmoid(gv));
            a32[i] = (float)act[i];
        }
        /* The detector stores the activation as fp32 (feedForward buffer) before the
         * down projection reads it (resident_math.comp:71 then :56). */
        rc = orc_gemv_f64(fmt_d, Wd, hidden, inter, a32, batch, d);
    }
    if (!rc) for (int64_t i = 0; i < (int64_t)batch * hidden; ++i) y[i] = (y_in ? (double)y_in[i] : 0.0) + d[i];
    free(g); free(u); free(a32); free(d);
    return rc;
}

/* ---- argmax with margin (resident_math.comp:125-130 generalised) ---------- */
uint32_t orc_argmax_margin_f32(const float* logits, int64_t n, float margin) {
    float M = -INFINITY; int any = 0;
    for (int64_t i = 0; i < n; ++i) if (logits[i] > M) { M = logits[i]; any = 1; }
    if (!any) return 0xffffffffu;
    float mag = fabsf(M);
    float slack = margin * mag;            /* two separate roundings: no fma */
    float T = M - slack;
    for (int64_t i = 0; i < n; ++i) if (logits[i] >= T) return (uint32_t)i;
    return 0xffffffffu;
}

uint32_t orc_argmax_margin_f64(const double* logits, int64_t n, double margin) {
    double M = -INFINITY; int any = 0;
    for (int64_t i = 0; i < n; ++i) if (logits[i] > M) { M = logits[i]; any = 1; }
    if (!any) return 0xffffffffu;
    double T = M - margin * fabs(M);
    for (int64_t i = 0; i < n; ++i) if (logits[i] >= T) return (uint32_t)i;
    return 0xffffffffu;
}

int orc_lm_head(int fmt, const void* W, int vocab, int hidden, const float* h, int batch, double margin,
                double* logits, uint32_t* ids) {
    int rc = orc_gemv_f64(fmt, W, vocab, hidden, h, batch, logits);
    if (rc) return rc;
    for (int b = 0; b < batch; ++b) ids[b] = orc_argmax_margin_f64(logits + (int64_t)b * vocab, vocab, margin);
    return 0;
}

/* ---- RoPE (resident_math.comp:76-77; resident_common.glsl:117,79) --------- */
void orc_rope(float* v, int heads, int hd, int rotary, int64_t t, double theta) {
    int active = rotary / 2;
    for (int h = 0; h < heads; ++h)
        for (int p = 0; p < hd / 2; ++p) {
            if (p >= active) continue;                    /* phase 0: unchanged */
            double phase = (double)t * pow(theta, -(double)p / (double)active);
            double c = cos(phase), s = sin(phase);
            float* e = v + (int64_t)h * hd + 2 * p;
            double x = e[0], y = e[1];
            e[0] = (float)(x * c - y * s);
            e[1] = (float)(x * s + y * c);
        }
}

/* ---- history packets (resident_dimensions.hpp:10; resident_quant.glsl:123-124) */
int64_t orc_history_bytes(int kvw) {
    int64_t blocks = (kvw + 255) / 256;
    return (blocks * (144 + 210) + 7) / 8 * 8;
}

static int64_t field_offset(int kvw, int fmt_k, int content) {
    int64_t blocks = (kvw + 255) / 256;
    return content ? blocks * (fmt_k == ORC_Q4_K ? 144 : 210) : 0;
}

static void decode_field(const uint8_t* packet, int kvw, int fmt_k, int fmt_v, int content, float* out) {
    int fmt = content ? fmt_v : fmt_k;
    int bb = fmt == ORC_Q4_K ? 144 : 210;
    int64_t blocks = (kvw + 255) / 256;
    const uint8_t* base = packet + field_offset(kvw, fmt_k, content);
    for (int64_t b = 0; b < blocks; ++b) {
        if (fmt == ORC_Q4_K) dequant_q4k_block(base + b * bb, out + b * 256);
        else dequant_q6k_block(base + b * bb, out + b * 256);
    }
}

float orc_packet_value(const uint8_t* packet, int kvw, int fmt_k, int fmt_v, int content, int c) {
    int fmt = content ? fmt_v : fmt_k;
    int bb = fmt == ORC_Q4_K ? 144 : 210;
    const uint8_t* blk = packet + field_offset(kvw, fmt_k, content) + (int64_t)(c / 256) * bb;
    float vals[256];
    if (fmt == ORC_Q4_K) dequant_q4k_block(blk, vals); else dequant_q6k_block(blk, vals);
    return vals[c % 256];
}

static float halfround(float v) { return orc_half_to_float(orc_float_to_half(v)); }

/* Codes are rintf() (round to nearest, ties to even) then clamped.  GLSL round() leaves
 * the direction of exact .5 ties to the implementation; both vendors' native rounding
 * instruction (AMD v_rndne_f32, NVIDIA cvt.rni) resolves them to even, and the known-answer
 * packets of tests/test_oracle.py pin that choice. */
static float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* GLSL min / max (returns x unless y is strictly smaller / larger): decides the sign of
 * zero where the packer compares +0 with -0 (a group minimum -min(0, x) of an all-zero
 * group is -0). */
static float glsl_min(float x, float y) { return y < x ? y : x; }
static float glsl_max(float x, float y) { return x < y ? y : x; }

/* Q4_K field of 256 coordinates, min/max groups of 32 (resident_history_quant.glsl:14-16,
 * 21-23, 27-29, 31-33, 36). */
static void pack_q4k_field(const float* x, uint8_t* blk) {
    float gscale[8], gmin[8]; unsigned sc[8], mn[8];
    memset(blk, 0, 144);
    for (int g = 0; g < 8; ++g) {
        float lo = 0.0f, hi = 0.0f;
        for (int i = 0; i < 32; ++i) { float v = x[g * 32 + i]; lo = glsl_min(lo, v); hi = glsl_max(hi, v); }
        float span = hi - lo;
        gscale[g] = span / 15.0f; gmin[g] = -lo;
    }
    float maxD = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 8; ++g) { maxD = glsl_max(maxD, gscale[g]); maxMin = glsl_max(maxMin, gmin[g]); }
    float d = halfround(maxD / 63.0f), dm = halfround(maxMin / 63.0f);
    uint16_t hd = orc_float_to_half(d), hm = orc_float_to_half(dm);
    blk[0] = hd & 255; blk[1] = hd >> 8; blk[2] = hm & 255; blk[3] = hm >> 8;
    for (int g = 0; g < 8; ++g) {
        sc[g] = (unsigned)clampf(rintf(gscale[g] / fmaxf(d, 1e-30f)), 0.0f, 63.0f);
        mn[g] = (unsigned)clampf(rintf(gmin[g] / fmaxf(dm, 1e-30f)), 0.0f, 63.0f);
    }
    for (int g = 0; g < 4; ++g) {
        blk[4 + g]  = (uint8_t)(sc[g] | ((sc[g + 4] >> 4) << 6));
        blk[8 + g]  = (uint8_t)(mn[g] | ((mn[g + 4] >> 4) << 6));
        blk[12 + g] = (uint8_t)((sc[g + 4] & 15u) | ((mn[g + 4] & 15u) << 4));
    }
    for (int i = 0; i < 256; ++i) {
        int g = i / 32;
        float num = x[i] + dm * (float)mn[g];
        float den = fmaxf(d * (float)sc[g], 1e-30f);
        unsigned q = (unsigned)clampf(rintf(num / den), 0.0f, 15.0f);
        blk[16 + (i / 64) * 32 + i % 32] |= (uint8_t)(q << (((i % 64) / 32) * 4));
    }
}

/* Q6_K field of 256 coordinates, abs-max groups of 16 (resident_history_quant.glsl:15-16,
 * 21-22, 27-28, 37-38). */
static void pack_q6k_field(const float* x, uint8_t* blk) {
    float gscale[16]; unsigned sc[16];
    memset(blk, 0, 210);
    for (int g = 0; g < 16; ++g) {
        float hi = 0.0f;
        for (int i = 0; i < 16; ++i) hi = glsl_max(hi, fabsf(x[g * 16 + i]));
        gscale[g] = hi / 31.0f;
    }
    float maxD = 0.0f;
    for (int g = 0; g < 16; ++g) maxD = glsl_max(maxD, gscale[g]);
    float d = halfround(maxD / 127.0f);
    uint16_t hd = orc_float_to_half(d);
    blk[208] = hd & 255; blk[209] = hd >> 8;
    for (int g = 0; g < 16; ++g) {
        sc[g] = (unsigned)clampf(rintf(gscale[g] / fmaxf(d, 1e-30f)), 0.0f, 127.0f);
        blk[192 + g] = (uint8_t)sc[g];
    }
    for (int i = 0; i < 256; ++i) {
        float den = fmaxf(d * (float)sc[i / 16], 1e-30f);
        unsigned q = (unsigned)((int)clampf(rintf(x[i] / den), -32.0f, 31.0f) + 32);
        int part = i / 128, within = i % 128;
        blk[part * 64 + within % 64] |= (uint8_t)((q & 15u) << ((within / 64) * 4));
        blk[128 + part * 32 + within % 32] |= (uint8_t)((q >> 4) << ((within / 32) * 2));
    }
}

int orc_pack_history(const float* k, const float* v, int kvw, int fmt_k, int fmt_v, uint8_t* packet) {
    if (!k || !v || !packet || kvw <= 0) return 1;
    if ((fmt_k != ORC_Q4_K && fmt_k != ORC_Q6_K) || (fmt_v != ORC_Q4_K && fmt_v != ORC_Q6_K)) return 3;
    int64_t blocks = (kvw + 255) / 256, bytes = orc_history_bytes(kvw);
    memset(packet, 0, (size_t)bytes);
    float tmp[256];
    for (int content = 0; content < 2; ++content) {
        const float* src = content ? v : k;
        int fmt = content ? fmt_v : fmt_k;
        int bb = fmt == ORC_Q4_K ? 144 : 210;
        uint8_t* base = packet + field_offset(kvw, fmt_k, content);
        for (int64_t b = 0; b < blocks; ++b) {
            for (int i = 0; i < 256; ++i) { int64_t c = b * 256 + i; tmp[i] = c < kvw ? src[c] : 0.0f; }
            if (fmt == ORC_Q4_K) pack_q4k_field(tmp, base + b * bb); else pack_q6k_field(tmp, base + b * bb);
        }
    }
    return 0;
}

/* ---- decode attention (resident_ray.comp:30-53,56-76; verify_attention_receipts.py:84-114) */
int orc_decode_attention(const float* q, int nseq, int hq, int hkv, int hd,
                         const uint8_t* packets, int fmt_k, int fmt_v,
                         const int64_t* slot_base, const int32_t* ctx_len,
                         int64_t capacity, const float* gate,
                         double* out, double* m, double* z) {
    if (!q || !packets || !slot_base || !ctx_len || !out || !m || !z) return 1;
    if (nseq <= 0 || hq <= 0 || hkv <= 0 || hd <= 0 || hq % hkv || capacity <= 0) return 2;
    int kvw = hkv * hd, group = hq / hkv;
    int64_t stride = orc_history_bytes(kvw);
    double inv = 1.0 / sqrt((double)hd);
    #pragma omp parallel for collapse(2) schedule(dynamic)
    for (int s = 0; s < nseq; ++s)
        for (int h = 0; h < hq; ++h) {
            int64_t t = (int64_t)ctx_len[s] - 1;
            int64_t visible = t + 1 < capacity ? t + 1 : capacity;
            int kvh = h / group;                              /* resident_common.glsl:109 */
            const float* qh = q + ((int64_t)s * hq + h) * hd;
            double* o = out + ((int64_t)s * hq + h) * hd;
            double* scores = (double*)malloc(sizeof(double) * (size_t)(visible > 0 ? visible : 1));
            int64_t padded = (kvw + 255) / 256 * 256;
            float* field = (float*)malloc(sizeof(float) * (size_t)padded);
            double mx = -INFINITY;
            for (int64_t r = 0; r < visible; ++r) {
                int64_t p = t - r;
                const uint8_t* pk = packets + (slot_base[s] + p % capacity) * stride;
                decode_field(pk, kvw, fmt_k, fmt_v, 0, field);
                double acc = 0.0;
                for (int c = 0; c < hd; ++c) acc += (double)qh[c] * (double)field[kvh * hd + c];
                scores[r] = acc * inv;
                if (scores[r] > mx) mx = scores[r];
            }
            double zz = 0.0;
            for (int c = 0; c < hd; ++c) o[c] = 0.0;
            for (int64_t r = 0; r < visible; ++r) {
                int64_t p = t - r;
                const uint8_t* pk = packets + (slot_base[s] + p % capacity) * stride;
                double w = exp(scores[r] - mx);
                zz += w;
                decode_field(pk, kvw, fmt_k, fmt_v, 1, field);
                for (int c = 0; c < hd; ++c) o[c] += w * (double)field[kvh * hd + c];
            }
            for (int c = 0; c < hd; ++c) {
                double g = gate ? orc_sigmoid((double)gate[((int64_t)s * hq + h) * hd + c]) : 1.0;
                o[c] = o[c] / (zz > 1e-30 ? zz : 1e-30) * g;
            }
            m[(int64_t)s * hq + h] = mx;
            z[(int64_t)s * hq + h] = zz;
            free(scores); free(field);
        }
    return 0;
}

/* ---- dense attention receipts --------------------------------------------
 * Events (words 3, 4, 7) follow fusedAttention's online pass (resident_attention_dense.comp:
 * 206-292): fp32 scores q.k / sqrt(hd), tiles of 4 positions raise the running maximum
 * (one exp for the rescale when it moves and Z > 0), a weight is reused when the score
 * and maximum repeat bit for bit, bit-equal consecutive value vectors form one run.
 * Word 6 is traceGroup's count (resident_attention_dense.comp:108-126): two lens faces
 * and one history ray per 16 positions, on head 0.  m, Z, U are the fp64 two-pass sums of
 * verify_attention_receipts.py:117-139 over fp64 scores. */
int64_t orc_attention_receipts(const float* q, int rows, int hq, int hkv, int hd, const uint8_t* packets, int fmt_k,
                               int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                               int block, int64_t n_records, double* vals, uint32_t* words, uint8_t* tie) {
    if (!q || !packets || !slot_base || !ctx_len || !vals || !words || !tie) return -1;
    if (rows <= 0 || hq <= 0 || hkv <= 0 || hd <= 0 || hq % hkv || capacity <= 0 || block <= 0 || block % 32)
        return -1;
    const int kvw = hkv * hd, group = hq / hkv, cov = block / 32, nw = 8 + cov;
    const int64_t stride = orc_history_bytes(kvw), padded = (kvw + 255) / 256 * 256;
    float* kf = (float*)malloc(sizeof(float) * (size_t)padded * (size_t)block);
    float* vf = (float*)malloc(sizeof(float) * (size_t)padded * (size_t)block);
    float* sc = (float*)malloc(sizeof(float) * (size_t)block);
    double* sd = (double*)malloc(sizeof(double) * (size_t)block);
    if (!kf || !vf || !sc || !sd) { free(kf); free(vf); free(sc); free(sd); return -1; }
    int64_t rec = 0;
    for (int r = 0; r < rows; ++r) {
        const int64_t L = ctx_len[r], active = L <= 0 ? 0 : (L < capacity ? L : capacity);
        for (int64_t g = 0; g * block < active; ++g) {
            const int count = (int)(active - g * block < block ? active - g * block : block);
            for (int j = 0; j < count; ++j) {
                const int64_t p = L - 1 - (g * block + j);
                const uint8_t* pk = packets + (slot_base[r] + p % capacity) * stride;
                decode_field(pk, kvw, fmt_k, fmt_v, 0, kf + (size_t)j * padded);
                decode_field(pk, kvw, fmt_k, fmt_v, 1, vf + (size_t)j * padded);
            }
            for (int h = 0; h < hq; ++h, ++rec) {
                if (rec >= n_records) { free(kf); free(vf); free(sc); free(sd); return -1; }
                const int kvh = h / group;
                const float* qh = q + ((int64_t)r * hq + h) * hd;
                for (int j = 0; j < count; ++j) {
                    float total = 0.0f;
                    double exact = 0.0;
                    for (int c = 0; c < hd; ++c) {
                        float prod = qh[c] * kf[(size_t)j * padded + kvh * hd + c];
                        total += prod;
                        exact += (double)qh[c] * (double)kf[(size_t)j * padded + kvh * hd + c];
                    }
                    sc[j] = total / sqrtf((float)hd);
                    sd[j] = exact / sqrt((double)hd);
                }
                /* the online events */
                float maximum = -INFINITY, reference = 0.0f, prev_w = 0.0f;
                uint32_t prev_score = 0, prev_max = 0, exps = 0, runs = 0;
                int have_prev = 0, reused = 0, pending = 0, near = 0, prev_run = -1;
                for (int t0 = 0; t0 < count; t0 += 4) {
                    const int n = count - t0 < 4 ? count - t0 : 4;
                    float local = -INFINITY;
                    for (int j = 0; j < n; ++j) local = fmaxf(local, sc[t0 + j]);
                    const float next = fmaxf(maximum, local);
                    float scale = 0.0f;
                    if (isfinite(maximum) && next != maximum && fabsf(next - maximum) <= 1e-5f * fmaxf(1.0f, fabsf(next))) near = 1;
                    if (isfinite(maximum) && local < maximum && maximum - local <= 1e-5f * fmaxf(1.0f, fabsf(maximum))) near = 1;
                    uint32_t nb, mb; memcpy(&nb, &next, 4); memcpy(&mb, &maximum, 4);
                    if (reference > 0.0f) {
                        if (nb == mb) scale = 1.0f;
                        else { scale = expf(maximum - next); ++exps; }
                    }
                    reference *= scale;
                    maximum = next;
                    for (int j = 0; j < n; ++j) {
                        const float s = sc[t0 + j];
                        uint32_t sb; memcpy(&sb, &s, 4); memcpy(&mb, &maximum, 4);
                        float w;
                        if (have_prev && sb == prev_score && mb == prev_max) { w = prev_w; reused = 1; }
                        else {
                            float ps; memcpy(&ps, &prev_score, 4);
                            if (have_prev && sb != prev_score && fabsf(s - ps) <= 1e-5f * fmaxf(1.0f, fabsf(s))) near = 1;
                            w = expf(s - maximum); ++exps;
                        }
                        prev_score = sb; prev_max = mb; prev_w = w; have_prev = 1;
                        reference += w;
                        const float* v = vf + (size_t)(t0 + j) * padded + kvh * hd;
                        int same = pending;
                        if (same) {
                            const float* pv = vf + (size_t)prev_run * padded + kvh * hd;
                            same = memcmp(v, pv, sizeof(float) * (size_t)hd) == 0;
                        }
                        if (!same) {
                            if (pending) ++runs;
                            prev_run = t0 + j;
                            pending = 1;
                        }
                    }
                }
                if (pending) ++runs;
                /* the expected sums (two-pass, fp64) */
                double* o = vals + rec * (3 + hd);
                double mx = -INFINITY, z = 0.0;
                for (int j = 0; j < count; ++j) if (sd[j] > mx) mx = sd[j];
                for (int c = 0; c < hd; ++c) o[3 + c] = 0.0;
                for (int j = 0; j < count; ++j) {
                    const double w = exp(sd[j] - mx);
                    z += w;
                    for (int c = 0; c < hd; ++c) o[3 + c] += w * (double)vf[(size_t)j * padded + kvh * hd + c];
                }
                o[0] = mx; o[1] = z; o[2] = count;
                uint32_t* wd = words + rec * nw;
                wd[0] = wd[1] = 0u;
                wd[2] = (uint32_t)count; wd[3] = exps; wd[4] = runs; wd[5] = (uint32_t)count;
                wd[6] = h == 0 ? 2u + (uint32_t)(count + 15) / 16u : 0u;
                wd[7] = 3u | (reused ? 4u : 0u) | (runs < (uint32_t)count ? 8u : 0u);
                for (int k = 0; k < cov; ++k) {
                    const int n = k * 32 < count ? (count - k * 32 < 32 ? count - k * 32 : 32) : 0;
                    wd[8 + k] = n == 32 ? 0xFFFFFFFFu : n == 0 ? 0u : (1u << n) - 1u;
                }
                tie[rec] = (uint8_t)near;
            }
        }
    }
    free(kf); free(vf); free(sc); free(sd);
    return rec;
}

/* ---- the rest of a decoder step ---- */

/* resident_math.comp:30-32 (op 0): the embedding row, decoded like every weight. */
int orc_embed(int fmt, const void* table, int vocab, int hidden, const uint32_t* ids, int batch, float* out) {
    int64_t rb = orc_row_bytes(fmt, hidden);
    if (rb <= 0 || !table || !ids || !out) return 2;
    for (int b = 0; b < batch; ++b) {
        if (ids[b] >= (uint32_t)vocab) return 7;
        int rc = orc_dequant(fmt, (const uint8_t*)table + (int64_t)ids[b] * rb, hidden, out + (int64_t)b * hidden);
        if (rc) return rc;
    }
    return 0;
}

/* resident_math.comp:33-38 (op 1). */
void orc_rmsnorm(const float* x, const float* w, int rows, int width, double eps, double* out) {
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (int64_t)r * width;
        double ss = 0.0;
        for (int c = 0; c < width; ++c) ss += (double)xr[c] * xr[c];
        double inv = 1.0 / sqrt(ss / width + eps);
        for (int c = 0; c < width; ++c) out[(int64_t)r * width + c] = xr[c] * inv * (double)w[c];
    }
}

/* resident_math.comp:113-115 (ops 14, 15) and :139-140 (op 20). */
void orc_head_norm(const float* x, int x_stride, const float* w, const float* gate, int gate_stride, int rows,
                   int heads, int hd, int mean, double eps, double* out) {
    for (int r = 0; r < rows; ++r)
        for (int h = 0; h < heads; ++h) {
            const float* xh = x + (int64_t)r * x_stride + (int64_t)h * hd;
            double ss = 0.0;
            for (int c = 0; c < hd; ++c) ss += (double)xh[c] * xh[c];
            double inv = 1.0 / sqrt(ss / (mean ? hd : 1) + eps);
            for (int c = 0; c < hd; ++c) {
                double v = xh[c] * inv * (w ? (double)w[h * hd + c] : 1.0);
                if (gate) {
                    double g = gate[(int64_t)r * gate_stride + (int64_t)h * hd + c];
                    v *= g * orc_sigmoid(g);
                }
                out[((int64_t)r * heads + h) * hd + c] = v;
            }
        }
}

static double softplus_d(double v) { return (v > 0 ? v : 0.0) + log1p(exp(-fabs(v))); }

/* resident_math.comp:131-133 (op 18); softplus as resident_common.glsl:80. */
void orc_delta_gates(const float* a, const float* b, int stride, const float* a_log, const float* dt_bias,
                     int batch, int heads, double* decay, double* beta) {
    for (int r = 0; r < batch; ++r)
        for (int h = 0; h < heads; ++h) {
            double av = a[(int64_t)r * stride + h], bv = b[(int64_t)r * stride + h];
            decay[(int64_t)r * heads + h] = exp(-exp((double)a_log[h]) * softplus_d(av + dt_bias[h]));
            beta[(int64_t)r * heads + h] = orc_sigmoid(bv);
        }
}

/* resident_math.comp:134-140 (ops 19, 20) for one new token. */
void orc_short_conv(const float* raw, int raw_stride, const float* state, const float* w, int batch, int heads,
                    int hd, double eps, double* out, float* new_state) {
    int W = heads * hd, W3 = 3 * W;
    for (int b = 0; b < batch; ++b) {
        double* o = out + (int64_t)b * W3;
        for (int c = 0; c < W3; ++c) {
            const float* st = state + ((int64_t)b * W3 + c) * 3;
            double s = 0.0;
            for (int j = 0; j < 3; ++j) s += (double)w[c * 4 + j] * st[j];
            s += (double)w[c * 4 + 3] * raw[(int64_t)b * raw_stride + c];
            o[c] = s * orc_sigmoid(s);
            float* ns = new_state + ((int64_t)b * W3 + c) * 3;
            ns[0] = st[1]; ns[1] = st[2]; ns[2] = raw[(int64_t)b * raw_stride + c];
        }
        for (int part = 0; part < 2; ++part)
            for (int h = 0; h < heads; ++h) {
                double* y = o + part * W + h * hd;
                double ss = 0.0;
                for (int c = 0; c < hd; ++c) ss += y[c] * y[c];
                double inv = 1.0 / sqrt(ss + eps);
                for (int c = 0; c < hd; ++c) y[c] *= inv;
            }
    }
}

/* resident_math.comp:141-147 (op 21) and resident_state.comp:16-33. */
void orc_delta_rule(double* state, const double* q, const double* k, const double* v, int stride,
                    const double* decay, const double* beta, int batch, int heads, int hd, double* out) {
    double scale = 1.0 / sqrt((double)hd);
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < heads; ++h) {
            double* S = state + ((int64_t)b * heads + h) * hd * hd;
            const double* qh = q + (int64_t)b * stride + (int64_t)h * hd;
            const double* kh = k + (int64_t)b * stride + (int64_t)h * hd;
            const double* vh = v + (int64_t)b * stride + (int64_t)h * hd;
            double dc = decay[(int64_t)b * heads + h], bt = beta[(int64_t)b * heads + h];
            for (int row = 0; row < hd; ++row) {
                double* s = S + (int64_t)row * hd;
                double u = 0.0;
                for (int c = 0; c < hd; ++c) { s[c] *= dc; u += s[c] * kh[c]; }
                double delta = bt * (vh[row] - u), o = 0.0;
                for (int c = 0; c < hd; ++c) { s[c] += delta * kh[c]; o += s[c] * qh[c]; }
                out[((int64_t)b * heads + h) * hd + row] = o * scale;
            }
        }
}
