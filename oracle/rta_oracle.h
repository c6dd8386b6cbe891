/*
 * rta_oracle.h -- CPU restatement of the Ray Tracing Attention detector path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (librta.so) never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the reference repository root).  Built with -ffp-contract=off so that the
 * dequantisation op order is exactly the reference's fp32 order.
 */
#ifndef RTA_ORACLE_H
#define RTA_ORACLE_H
#include <stdint.h>
#include <stddef.h>
#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type codes used by the reference (resident_quant.glsl:6-20). */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q4_K = 12, ORC_Q6_K = 14, ORC_BF16 = 30 };

/* IEEE binary16 <-> binary32 (unpackHalf2x16 / packHalf2x16 semantics). */
float    orc_half_to_float(uint16_t h);
uint16_t orc_float_to_half(float f);           /* round to nearest even */

/* Bytes per row of a [rows x cols] matrix in format fmt (cols % 256 == 0 for K-quants). */
int64_t  orc_row_bytes(int fmt, int64_t cols);

/* Dequantise n values (n % 256 == 0 for K-quants) -- bit exact fp32.
 * ray_tracing/native/shaders/resident_quant.glsl:6-20 (ggufValue). */
int orc_dequant(int fmt, const void* src, int64_t n, float* out);

/* y[b*rows + r] = sum_c W[r,c] * x[b*cols + c]; W dequantised bit-exactly to fp32,
 * products and sums in fp64 (verification/verify_rt_mlp.py:84-89 closed form). */
int orc_gemv_f64(int fmt, const void* W, int rows, int cols,
                 const float* x, int batch, double* y);

/* Same contraction, fp32 accumulation, OpenMP over rows: the timed CPU baseline
 * (dequant + dot as resident_math.comp:39-75 does per output channel). */
/* row / axis remap of a projection (resident_quant.glsl:20-31) */
int64_t orc_rotary_source(int64_t axis, int rotary);
int64_t orc_remap_row(int mode, int hd, int rotary, int key_rows, int64_t row);
int64_t orc_remap_axis(int mode, int hd, int rotary, int64_t axis);
int orc_gemv_remap_f64(int fmt, const void* W, int src_rows, int rows, int cols, int mode, int hd, int rotary,
                       int key_rows, const float* x, int batch, double* y);
int orc_gemv_f32(int fmt, const void* W, int rows, int cols,
                 const float* x, int batch, float* y, int threads);

/* Stable sigmoid, resident_common.glsl:138 (detectorSigmoid), in fp64. */
double orc_sigmoid(double v);

/* SwiGLU MLP, resident_math.comp:54-58,70-71 + optical_resident.cpp:484-491:
 *   a = sign(g) sign(u) |g| |u| sigmoid(g)   (g = Wg x, u = Wu x)
 *   y = y_in + Wd a                         (y_in may be NULL: mlpCheck zeroes state)
 * act: [batch, inter], y: [batch, hidden]; fp64 throughout. */
int orc_mlp_swiglu(int fmt_g, const void* Wg, int fmt_u, const void* Wu,
                   int fmt_d, const void* Wd, int hidden, int inter,
                   const float* x, int batch, const float* y_in,
                   double* act, double* y);

/* Argmax with the relative-margin tie rule: M = max finite logit,
 * T = M - margin*|M|, id = lowest v with logit[v] >= T.  margin = 0 is the
 * reference's exact rule (resident_math.comp:125-130: strict > , equal -> lower id).
 * The f32 variant evaluates T in fp32 with two roundings (no fma). */
uint32_t orc_argmax_margin_f32(const float* logits, int64_t n, float margin);
uint32_t orc_argmax_margin_f64(const double* logits, int64_t n, double margin);

/* LM head readout (resident_math.comp:117-130, ops 16/17/23): fp64 logits
 * [batch, vocab] and ids [batch] under the margin rule. */
int orc_lm_head(int fmt, const void* W, int vocab, int hidden,
                const float* h, int batch, double margin,
                double* logits, uint32_t* ids);

/* RoPE on adjacent pairs (resident_math.comp:76-77, resident_common.glsl:117):
 * pair p of each head, local = p < rotary/2 ? p : none;
 * phase = t * theta^(-local/(rotary/2)); (x,y) -> (x cos - y sin, x sin + y cos).
 * Phase, sin and cos in fp64; result rounded to fp32.  v: [heads, hd] in place. */
void orc_rope(float* v, int heads, int hd, int rotary, int64_t t, double theta);

/* History packet geometry (resident_dimensions.hpp:10, spec.py:45):
 * bytes = roundup8(ceil(kvw/256) * (144 + 210)).  K blocks first, then V blocks. */
int64_t orc_history_bytes(int kvw);

/* Pack one token's compact K and V rows (kvw floats each) into a packet,
 * restating resident_history_quant.glsl:9-41 (reference format: K Q4_K, V Q6_K).
 * fmt_k/fmt_v choose the per-field format (Q4_K or Q6_K); for Q4_K the
 * min/max group scheme and for Q6_K the abs-max scheme of that file apply. */
int orc_pack_history(const float* k, const float* v, int kvw, int fmt_k, int fmt_v,
                     uint8_t* packet);

/* Decode coordinate c (0..kvw) of field K (content=0) or V (content=1) of a
 * packet (resident_quant.glsl:123-124, quantizedPath). */
float orc_packet_value(const uint8_t* packet, int kvw, int fmt_k, int fmt_v,
                       int content, int c);

/* Decode attention over quantised history for one query token per sequence
 * (resident_ray.comp:56-76 detector; verify_attention_receipts.py:84-114 dense oracle).
 *   q        [nseq, hq, hd] (already rotated)
 *   packets  base of the packet array, stride orc_history_bytes(hkv*hd)
 *   slot_base[s], ctx_len[s]: sequence s holds absolute positions 0..ctx_len-1 in
 *            ring slots slot_base + p % capacity; the query sits at t = ctx_len-1 and
 *            sees positions t-r, r < min(t+1, capacity) (resident_ray.comp:30-53).
 *   gate     [nseq, hq, hd] or NULL; out *= sigmoid(gate) (resident_ray.comp:75-76)
 * Outputs fp64: out [nseq, hq, hd], m [nseq, hq] (running max), z [nseq, hq]. */
int orc_decode_attention(const float* q, int nseq, int hq, int hkv, int hd,
                         const uint8_t* packets, int fmt_k, int fmt_v,
                         const int64_t* slot_base, const int32_t* ctx_len,
                         int64_t capacity, const float* gate,
                         double* out, double* m, double* z);

/* Dense attention receipts (resident_attention_dense.comp:190-300): for each record
 * (row, group, head) in the order (groups of rows < r + g) * hq + h, vals[rec] =
 * {m, Z, count, U[0..hd)} in fp64 from the two-pass sums over fp64 scores that verify_attention_receipts.py:
 * 117-139 expects, words[rec] = the integer words 2..7 and the coverage bits (words 0
 * and 1 left 0), tie[rec] = 1 where an fp32 score lies within 1e-5 of the running
 * maximum or of its neighbour without being bit-equal (events 3, 4, 7 may then differ
 * with the summation order).  Returns the record count, or -1 on a bad argument or when
 * more than n_records are needed. */
int64_t orc_attention_receipts(const float* q, int rows, int hq, int hkv, int hd, const uint8_t* packets, int fmt_k,
                               int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                               int block, int64_t n_records, double* vals, uint32_t* words, uint8_t* tie);

/* ---- the rest of a decoder step (resident_math.comp ops 0, 1, 14, 15, 18-21) ----
 * Test infrastructure: restatements in fp64 (fp32 inputs, fp32 embedding values). */

/* op 0 (resident_math.comp:30-32): out[b, c] = dequant(table row ids[b])[c], bit exact. */
int orc_embed(int fmt, const void* table, int vocab, int hidden, const uint32_t* ids, int batch, float* out);

/* op 1 (resident_math.comp:33-38): out = x * w / sqrt(sum(x^2)/width + eps) per row. */
void orc_rmsnorm(const float* x, const float* w, int rows, int width, double eps, double* out);

/* ops 14 / 15 / 20 (resident_math.comp:113-115,139-140): per head of hd values,
 *   out = x * w[h*hd + c] / sqrt(sum(x^2)/(mean ? hd : 1) + eps) * (gate ? g*sigmoid(g) : 1)
 * w may be NULL (1).  x, gate: [rows, heads*hd] with row strides x_stride, gate_stride. */
void orc_head_norm(const float* x, int x_stride, const float* w, const float* gate, int gate_stride, int rows,
                   int heads, int hd, int mean, double eps, double* out);

/* op 18 (resident_math.comp:131-133): decay = exp(-exp(a_log[h]) * softplus(a + dt_bias[h])),
 * beta = sigmoid(b); a, b: [batch, heads] with row stride `stride`. */
void orc_delta_gates(const float* a, const float* b, int stride, const float* a_log, const float* dt_bias,
                     int batch, int heads, double* decay, double* beta);

/* ops 19 + 20 for one new token per sequence (resident_math.comp:134-140):
 *   raw [batch, 3W] (q | k | v projections, W = heads*hd, row stride raw_stride),
 *   state [batch, 3W, 3] the three previous raw values (oldest first), w [3W, 4]:
 *   s = sum_j<3 w[c][j] state[c][j] + w[c][3] raw[c];  y = s * sigmoid(s);
 *   q and k parts then L2-normalised per head: y / sqrt(sum(y^2) + eps).
 * out [batch, 3W]; new_state receives the shifted window (state[1], state[2], raw). */
void orc_short_conv(const float* raw, int raw_stride, const float* state, const float* w, int batch, int heads,
                    int hd, double eps, double* out, float* new_state);

/* op 21 / resident_state.comp, one token per sequence (the gated delta rule): per
 * sequence b and head h with S = state[b][h] ([value][key], hd x hd):
 *   S = decay S;  u = S k;  S += beta (v - u) k^T;  o = S q / sqrt(hd)
 * q, k, v: [batch, heads*hd] with row stride `stride`; state fp64 in/out; out [batch, heads*hd]. */
void orc_delta_rule(double* state, const double* q, const double* k, const double* v, int stride,
                    const double* decay, const double* beta, int batch, int heads, int hd, double* out);


/* ---- one whole decode step on the CPU (rta_cpu_step.c) ----
 * fp32, OpenMP: the timed CPU baseline of the decode-step benchmark and a second
 * composition of the step for the tests.  Shapes and state layout as the product's
 * hybrid decode step: per recurrent layer the state [batch][rec_heads][128][128]
 * ([value][key]) and the conv window [batch][3 S][3] (S = rec_heads * 128); per full
 * layer the packet ring [batch][capacity] (sequence b owns slots b*capacity ..);
 * ctx[b] = tokens already in the history = the new token's position.  The step reads
 * tokens[b], writes the greedy next tokens and logits [batch][vocab] (may be NULL),
 * and advances ctx. */
typedef struct orc_step_layer {
    const float *norm_in, *norm_post;               /* [hidden] */
    const void *w_in, *w_o, *w_gate, *w_up, *w_down; /* GGUF rows of fmt_proj */
    const float *q_norm, *k_norm;                   /* full layers */
    const float *conv_w, *a_log, *dt_bias, *out_norm; /* recurrent layers */
} orc_step_layer;

typedef struct orc_step_model {
    int hidden, layers, full_every, q_heads, kv_heads, head_dim, rec_heads, ff, vocab, capacity;
    int fmt_embed, fmt_proj, fmt_lm, fmt_k, fmt_v, rope_rotary;
    float eps, margin;
    double rope_theta;
    const void* embed;
    const orc_step_layer* layers_ptr;
    const float* norm_final;
    const void* lm_head;
} orc_step_model;

int orc_step_f32(const orc_step_model* m, int batch, float* rec, float* conv, uint8_t* packets, int32_t* ctx,
                 uint32_t* tokens, float* logits, int threads);

#ifdef __cplusplus
}
#endif
#endif
