/*
 * rta.h -- C ABI of the MI355X (gfx950) detector path of Ray Tracing Attention.
 *
 * Conventions
 *   - Every pointer named w/x/y/q/out/... is a DEVICE pointer owned by the caller.
 *     The library never allocates device memory in these entry points; kernels
 *     that need scratch take a caller-provided workspace (size from the matching
 *     *_workspace_bytes query).
 *   - All calls are stream ordered on `stream` (a hipStream_t; NULL = default
 *     stream) and return immediately after launching.  Argument errors are
 *     detected on the host before anything is launched.
 *   - Return value: RTA_OK (0) or one of the RTA_ERR_* codes below.
 *   - Quantised matrices are GGUF superblocks, byte for byte, row-major: row r of
 *     a [rows x cols] matrix occupies cols/256 consecutive superblocks
 *     (ray_tracing/native/shaders/resident_quant.glsl:28-30,59).
 *
 * Each entry point names the reference interface it replaces (paths relative to
 * the reference repository root).
 */
#ifndef RTA_H
#define RTA_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

typedef void* rta_stream_t; /* hipStream_t */
typedef void* rta_event_t;  /* hipEvent_t */

enum rta_status {
    RTA_OK = 0,
    RTA_ERR_NULL = 1,      /* a required pointer is NULL                         */
    RTA_ERR_SHAPE = 2,     /* a dimension is <= 0 or not a multiple it must be    */
    RTA_ERR_FORMAT = 3,    /* unsupported format code                             */
    RTA_ERR_ALIGN = 4,     /* a device pointer is not aligned as required         */
    RTA_ERR_WORKSPACE = 5, /* workspace missing or smaller than required          */
    RTA_ERR_LAUNCH = 6,    /* the HIP runtime reported an error at launch         */
    RTA_ERR_RANGE = 7,     /* an argument is outside the supported range          */
    RTA_ERR_DEVICE = 8,    /* the device error word is non-zero (rta_device_error) */
    RTA_ERR_SCRATCH = 9    /* the call needs more than RTA_NOALLOC_SCRATCH_BYTES of scratch */
};

/* GGUF type codes, as the reference uses them (resident_quant.glsl:6-20).
 * RTA_TILED marks a K-quant matrix repacked by rta_pack (no counterpart in the
 * reference, which streams GGUF rows as uploaded); every projection entry point
 * accepts RTA_Q4_K | RTA_TILED and RTA_Q6_K | RTA_TILED and then runs on the matrix
 * cores at every batch size. */
enum rta_format { RTA_F32 = 0, RTA_F16 = 1, RTA_Q4_K = 12, RTA_Q6_K = 14, RTA_BF16 = 30, RTA_TILED = 0x100 };

/* Epilogue of a projection: y = W x, or y += W x (the residual add of the O and
 * down projections, resident_math.comp:70). */
enum rta_epilogue { RTA_EPI_STORE = 0, RTA_EPI_ACCUMULATE = 1 };

/* Device error bits; same meanings as the reference's control[3] word
 * (resident_ray.comp:80, resident_math.comp:152, resident_detector_ordered_scores.comp:20). */
#define RTA_DEVERR_HITS 8u          /* visible history count mismatch          */
#define RTA_DEVERR_VOCAB 2048u      /* vocabulary coverage != V                */
#define RTA_DEVERR_DETECTOR 65536u  /* non-finite query / key / score          */
#define RTA_DEVERR_TOKEN 4096u      /* token id >= vocabulary (rta_embed); no reference bit */

int rta_version(void);
const char* rta_status_string(int status);

/* Reads (and optionally clears) the device error word of the current device.
 * Synchronises the device.  Replaces the host readback of control[3]
 * (optical_resident.cpp:837-838, :945). */
int rta_device_error(uint32_t* bits, int clear);

/* Bytes per row of a [rows x cols] matrix of format fmt, -1 if invalid. */
int64_t rta_row_bytes(int fmt, int64_t cols);

/* Dequantise n values (n % 256 == 0 for K-quants) to fp32, bit exact with the
 * reference decoder.  Replaces ggufValue (resident_quant.glsl:6-20).
 * Alignment: src 4 bytes (F32, Q4_K) or 2 bytes (F16, BF16, Q6_K); out 4 bytes. */
int rta_dequant(int fmt, const void* src, int64_t n, float* out, rta_stream_t stream);

/* Bytes of the packed (tiled) form of a [rows x cols] Q4_K or Q6_K matrix, -1 if
 * invalid: ceil(rows/16) * (cols/256) tiles of 16 GGUF blocks (2304 / 3360 bytes).
 * No reference counterpart: the packed layout is this library's own. */
int64_t rta_pack_bytes(int fmt, int rows, int cols);

/* Repacks a device-resident GGUF Q4_K / Q6_K matrix (rows of cols/256 blocks, as
 * the reference uploads it, optical_resident.cpp:213-252) into tiles of 16 rows x 1
 * superblock whose bytes are ordered the way the matrix-core readout loads them
 * (each load instruction reads whole cache lines).  One-time, at load; the result
 * is used with fmt | RTA_TILED.  dst: rta_pack_bytes() bytes, 16-byte aligned; src
 * aligned as for rta_gemv.  No reference counterpart. */
int rta_pack(int fmt, const void* src, int rows, int cols, void* dst, rta_stream_t stream);

/* y[b, r] (=|+=) sum_c W[r, c] x[b, c],  b < batch, r < rows.
 *   x: [batch, cols] fp32 row-major, y: [batch, rows] fp32.
 *   K-quants need cols % 256 == 0; W 16-byte aligned (Q4_K) / 2-byte (Q6_K).
 *   K-quant batches of 5 or more rows (3 or more when rows x cols >= 2^25, 2 or more
 *   when >= 2^27; a SwiGLU pair counts both matrices), and packed matrices
 *   (fmt | RTA_TILED) at every batch, run on the matrix cores and need a workspace of
 *   rta_gemv_workspace_bytes() (256-byte aligned); 0 bytes otherwise.
 * Replaces the projection detector, resident_math.comp:39-75 (op 2, indices
 * 0/1/2/4/6/8) dispatched by Resident::launch, optical_resident.cpp:304-347, and its
 * batched pipelines (optical_resident.cpp:168,343; resident_batch2.comp). */
size_t rta_gemv_workspace_bytes(int fmt, int rows, int cols, int batch);
int rta_gemv(int fmt, const void* w, int rows, int cols, const float* x, int batch,
             float* y, int epilogue, void* workspace, size_t workspace_bytes,
             rta_stream_t stream);

/* Row/axis remap of a projection matrix: the descriptor mode (metadata >> 8) of
 * quantizedWeight / quantizedOctet, resident_quant.glsl:20-31,53-58, as
 * compiler/export.py:96-98,108 assigns it.  Logical row r reads GGUF row src(r),
 * logical axis a reads GGUF column src(a), with rot(i) = i < R ? (i % 2)(R / 2) + i / 2
 * : i (originalRotaryAxis, resident_quant.glsl:20), hd = head_dim, R = rotary_dim:
 *   RTA_REMAP_QUERY      1  src(r) = (r / hd) 2 hd + rot(r % hd)       (Q of Q|gate rows)
 *   RTA_REMAP_GATE       2  src(r) = (r / hd) 2 hd + hd + rot(r % hd)  (its gate)
 *   RTA_REMAP_ROTARY     3  src(r) = (r / hd) hd + rot(r % hd)         (Q / K / V rows)
 *   RTA_REMAP_AXES       4  src(a) = (a / hd) hd + rot(a % hd)         (O columns)
 *   RTA_REMAP_KEY_REPEAT 5  src(r) = r % key_rows                      (recurrent q / k)
 * head_dim > 0; 0 <= rotary_dim <= head_dim, even; key_rows > 0 for mode 5. */
enum rta_remap_mode {
    RTA_REMAP_NONE = 0, RTA_REMAP_QUERY = 1, RTA_REMAP_GATE = 2, RTA_REMAP_ROTARY = 3,
    RTA_REMAP_AXES = 4, RTA_REMAP_KEY_REPEAT = 5
};
typedef struct rta_remap { int mode, head_dim, rotary_dim, key_rows; } rta_remap;

/* rta_gemv over the remapped matrix: y[b, r] (=|+=) sum_a W[src(r), src(a)] x[b, a],
 * r < rows, a < cols, for a GGUF (or rta_pack-ed, fmt | RTA_TILED) matrix w of
 * src_rows rows.  Modes 1-3 need rows % head_dim == 0 and src_rows >= 2 rows (1, 2)
 * or rows (3); mode 4 cols % head_dim == 0; mode 5 src_rows >= min(rows, key_rows).
 * Row modes read each source row once into the workspace and gather the rows;
 * mode 4 permutes x into the workspace.  Workspace: rta_gemv_remap_workspace_bytes().
 * Replaces op 2 with a descriptor mode != 0 (resident_math.comp:39-75 reading
 * through quantizedOctet, resident_quant.glsl:44-58). */
size_t rta_gemv_remap_workspace_bytes(int fmt, const rta_remap* remap, int rows, int cols, int batch);
int rta_gemv_remap(int fmt, const void* w, int src_rows, int rows, int cols, const rta_remap* remap,
                   const float* x, int batch, float* y, int epilogue, void* workspace,
                   size_t workspace_bytes, rta_stream_t stream);

/* rta_pack of the row-remapped matrix: tile rows are the logical rows r < rows, read
 * from GGUF row src(r) of src (src_rows rows); modes 0, 1, 2, 3, 5 (mode 4 moves
 * columns inside superblocks, which no repacking can express: use rta_gemv_remap
 * on the packed matrix).  dst: rta_pack_bytes(fmt, rows, cols) bytes.  A packed
 * matrix of several parts (Q | gate | K | V) is packed part by part at row offsets
 * that are multiples of 16: part p starts rta_pack_bytes(fmt, offset_p, cols) bytes
 * into dst.  The remap is then free at run time.  No reference counterpart. */
int rta_pack_remap(int fmt, const void* src, int src_rows, int cols, const rta_remap* remap, int rows,
                   void* dst, rta_stream_t stream);

/* SwiGLU MLP: act = sign(g) sign(u) |g| |u| sigmoid(g) with g = Wg x, u = Wu x
 * ([batch, inter]); then y (=|+=) Wd act ([batch, hidden]).
 *   Wg, Wu: [inter, hidden] (one format); Wd: [hidden, inter].
 *   Workspace: rta_mlp_workspace_bytes() (0 for batch < 8).
 * Replaces Resident::executeMLP (optical_resident.cpp:484-491): op 2 index 3
 * (resident_math.comp:54-58,71) then op 2 index 4 with the residual (:70).
 * mlpCheck (optical_resident.cpp:922-949) is epilogue STORE (state zeroed). */
size_t rta_mlp_workspace_bytes(int fmt_g, int fmt_d, int hidden, int inter, int batch);
int rta_mlp_swiglu(int fmt_g, const void* wg, int fmt_u, const void* wu,
                   int fmt_d, const void* wd, int hidden, int inter,
                   const float* x, int batch, float* act, float* y, int epilogue,
                   void* workspace, size_t workspace_bytes, rta_stream_t stream);

/* The fused gate/up stage alone: act = sign(g) sign(u) |g| |u| sigmoid(g), g = Wg x,
 * u = Wu x ([batch, inter]), both matrices streamed in one pass.  Workspace:
 * rta_mlp_workspace_bytes(fmt, fmt, hidden, inter, batch).  Replaces op 2 index 3
 * (resident_math.comp:54-58,71) as Resident::executeMLP launches it
 * (optical_resident.cpp:484-491). */
int rta_swiglu(int fmt, const void* wg, const void* wu, int hidden, int inter, const float* x, int batch,
               float* act, void* workspace, size_t workspace_bytes, rta_stream_t stream);

/* The decode step's readout path for packed matrices at batch <= 32, split in its two
 * stages (rta_hybrid_decode_step runs them inside the step; these expose them alone):
 *  - rta_image_from_rows: img = the matrix-core image of x * w (x [batch, cols] fp32,
 *    w [cols]; cols % 256 == 0, cols <= 4096) for packed format fmt (RTA_Q4_K | RTA_TILED
 *    or RTA_Q6_K | RTA_TILED): per (row, 256-column superblock) a power-of-two scale,
 *    binary16 hi and lo planes and group sums; ss [4 * batch] receives the rows' chunk sums
 *    of x^2.  img holds rta_image_bytes(cols, batch) bytes, 256-byte aligned.
 *  - rta_image_readout: y (=|+=) W x (mode RTA_EPI_STORE / RTA_EPI_ACCUMULATE) or, mode
 *    RTA_IMAGE_SWIGLU, y = act of (W = wg, w2 = wu) as rta_swiglu, from img; with ss the
 *    results take the RMSNorm factor 1 / sqrt(sum(ss of the row) / cols + eps) (x * w then
 *    reads as rmsnorm(x) * w).  reduce != 0 adds the K slabs into y; reduce == 0 leaves
 *    *nslab > 1 slabs in the workspace as [slab][32][rows] (SwiGLU: gate and up interleaved,
 *    2 rows each) and writes y only when *nslab == 1.  Workspace:
 *    rta_image_readout_workspace_bytes(rows, cols, dual = mode is SwiGLU).
 * Replace op 1 + op 2 (resident_math.comp:33-38,39-75) as Resident::layer runs them for
 * a batch of rows (optical_resident.cpp:455-491). */
#define RTA_IMAGE_SWIGLU 2
size_t rta_image_bytes(int cols, int batch);
/* The image of act = swiglu(g, u) from the nslab K slabs a RTA_IMAGE_SWIGLU readout left
 * with reduce == 0 (part = its workspace; width = its rows), slabs added in slab order:
 * the x image of the down projection, as the decode step builds it. */
int rta_image_from_swiglu(int fmt, const float* part, int nslab, int width, int batch, void* img,
                          rta_stream_t stream);
size_t rta_image_readout_workspace_bytes(int rows, int cols, int dual);
int rta_image_from_rows(int fmt, const float* x, const float* w, int batch, int cols, float* ss, void* img,
                        rta_stream_t stream);
int rta_image_readout(int fmt, int mode, const void* w, const void* w2, int rows, int cols, const void* img,
                      int batch, const float* ss, float eps, float* y, int reduce, void* workspace,
                      size_t workspace_bytes, int* nslab, rta_stream_t stream);

/* LM-head vocabulary readout with fused argmax.
 *   logits[b, v] = sum_k W[v, k] h[b, k]   (fp32, all v < vocab)
 *   ids[b] = lowest v with logits[b, v] >= M - margin*|M|, M = max_v logits[b, v]
 *   (fp32, no fma; margin 0 is the reference's exact-tie rule).
 *   Workspace: rta_lm_head_workspace_bytes() (always needed; 256-byte aligned).
 * Replaces Resident::word (optical_resident.cpp:523-530): ops 11, 24, 16, 17, 23
 * (resident_math.comp:99-105,117-130,152-153) and the vocabulary ray query
 * (resident_ray.comp:91-116), which always returned every word. */
size_t rta_lm_head_workspace_bytes(int fmt, int vocab, int hidden, int batch);
int rta_lm_head(int fmt, const void* w, int vocab, int hidden, const float* h, int batch,
                float margin, float* logits, uint32_t* ids,
                void* workspace, size_t workspace_bytes, rta_stream_t stream);

/* Rotary embedding on adjacent pairs, in place: v [rows, heads, hd];
 * row r is at absolute position positions[r] (device int64).  Pairs p < rotary/2
 * of each head turn by positions[r] * theta^(-p/(rotary/2)) (phase, sin, cos in
 * fp64).  Replaces op 3's rotation (resident_math.comp:76-77,
 * resident_common.glsl:117). */
int rta_rope(float* v, int rows, int heads, int hd, int rotary, const int64_t* positions,
             double theta, rta_stream_t stream);

/* History packet size for a compact K/V width kvw = kv_heads * head_dim:
 * roundup8(ceil(kvw/256) * (144 + 210)) (resident_dimensions.hpp:10). */
int64_t rta_history_bytes(int kvw);

/* Decode attention over quantised K/V history, one query token per sequence.
 *   q         [nseq, hq, hd] fp32, already rotated
 *   packets   history packets (stride rta_history_bytes(hkv*hd), 4-byte aligned);
 *             field K first (format fmt_k), then field V (fmt_v); Q4_K or Q6_K each,
 *             not both Q6_K (two Q6_K fields do not fit the packet size).
 *             The reference layout is fmt_k = Q4_K, fmt_v = Q6_K
 *             (resident_quant.glsl:123-124).
 *   slot_base [nseq] int64, ctx_len [nseq] int32 (device): sequence s holds
 *             positions 0..ctx_len[s]-1 in slots slot_base[s] + p % capacity; its
 *             query is at t = ctx_len[s]-1 and sees positions t-r, r < min(t+1, capacity).
 *   n_slots   number of packets in the array; a slot outside [0, n_slots) is not read
 *             and sets RTA_DEVERR_HITS.
 *   max_ctx   host upper bound of min(ctx_len[s], capacity) over s (grid sizing).
 *   gate      [nseq, hq, hd] or NULL: out *= sigmoid(gate).
 *   out [nseq, hq, hd]; m_out, z_out [nseq, hq] (each may be NULL): m = max score,
 *   z = sum exp(s - m) (the reference reports physical = (m + 20, z)).
 *   workspace: rta_decode_attention_workspace_bytes() bytes, 16-byte aligned.
 * hd must be 128, hq/hkv in {1, 2, 4, 8} and hkv * 128 / (16 if hq/hkv < 8, else 8) <= 256.
 * Replaces Resident::detectHistory (optical_resident.cpp:429-449): history ray
 * trace op 0 + check op 8 (resident_ray.comp:30-53,80) and the detector op 3
 * (resident_ray.comp:56-76) / ordered three-pass detector
 * (resident_detector_ordered_{scores,normalize,value}.comp). */
size_t rta_decode_attention_workspace_bytes(int nseq, int hq, int hkv, int hd, int max_ctx);
int rta_decode_attention(const float* q, int nseq, int hq, int hkv, int hd,
                         const void* packets, int fmt_k, int fmt_v,
                         const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                         int64_t n_slots, int max_ctx, const float* gate, float* out, float* m_out, float* z_out,
                         void* workspace, size_t workspace_bytes, rta_stream_t stream);

/* The same decode attention for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc): no workspace
 * argument; the library's own scratch, a device array of RTA_NOALLOC_SCRATCH_BYTES per
 * GPU held until the process ends, stands in for it.  The call allocates nothing (no
 * hipMalloc / hipFree, no allocating library routine).  A call whose
 * rta_decode_attention_workspace_bytes() exceeds RTA_NOALLOC_SCRATCH_BYTES returns
 * RTA_ERR_SCRATCH and launches nothing.  Every call on one GPU shares that GPU's
 * scratch: calls that overlap on one GPU (concurrent streams, threads) race.
 * No counterpart in the reference, whose worker owns every buffer itself
 * (vulkan_engine.hpp:41); it exists for the callers above.
 * 96 MiB holds the decode step's attention at batch 32 (32 / 8 heads, contexts up to
 * 8192) and the GQA workload (16 sequences, 16 / 4 heads, contexts up to 32768). */
#define RTA_NOALLOC_SCRATCH_BYTES ((size_t)96 << 20)
int rta_decode_attention_noalloc(const float* q, int nseq, int hq, int hkv, int hd,
                                 const void* packets, int fmt_k, int fmt_v,
                                 const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                                 int64_t n_slots, int max_ctx, const float* gate, float* out, float* m_out,
                                 float* z_out, rta_stream_t stream);

/* Dense attention receipts, the per-group records the standard backend's attention
 * writes for the diagnostic (resident_attention_dense.comp:190-300, layout
 * attention_receipts.hpp:16-29 with compact false; the worker's op 14 returns them,
 * rt_optical_resident.cpp attention_check).  Same q, packets, slot_base, ctx_len,
 * capacity, n_slots and max_ctx as rta_decode_attention (rows = nseq).  Row r's
 * min(ctx_len[r], capacity) newest positions form groups of block positions, newest
 * first; record (groups of rows < r + g) * hq + h holds hd + 8 + block/32 uint32 words:
 * m, Z = sum exp(s - m) (fp32 bits), count, exp evaluations, value runs, count, the
 * traversal count (2 + ceil(count/16) on head 0, else 0), flags 3|4|8, the coverage
 * bits, then U = sum exp(s - m) v (hd fp32 bits), in the reference's online order.
 * block: a multiple of 32 in [32, 1024].  receipts holds n_records records
 * (rta_attention_receipt_records); a record index past it sets RTA_DEVERR_HITS and is
 * not written; a row with min(ctx_len, capacity) above max_ctx sets it too (that row's
 * records are incomplete); a non-finite value sets RTA_DEVERR_DETECTOR. */
int64_t rta_attention_receipt_records(const int32_t* ctx_len_host, int rows, int hq, int64_t capacity, int block);
int rta_attention_receipts(const float* q, int rows, int hq, int hkv, int hd, const void* packets, int fmt_k,
                           int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                           int64_t n_slots, int max_ctx, int block, uint32_t* receipts, int64_t n_records,
                           rta_stream_t stream);

/* ---------------- the rest of a decoder step (resident_math.comp ops 0, 1, 14, 15,
 * 18-21, 34); every call is stream ordered, allocates nothing, validates on the host. */

/* op 0, token embedding (resident_math.comp:30-32; optical_resident.cpp generation
 * feeds control[0]): out[b, :] = decoded row ids[b] of table [vocab x hidden] in fmt
 * (bit exact with rta_dequant).  Ids >= vocab give zeros and set RTA_DEVERR_TOKEN. */
int rta_embed(int fmt, const void* table, int vocab, int hidden, const uint32_t* ids, int batch, float* out,
              rta_stream_t stream);

/* op 1, RMSNorm (resident_math.comp:33-38; Resident::layer, optical_resident.cpp:456,481):
 * out[r, :] = x[r, :] * w / sqrt(mean(x[r, :]^2) + eps).  width % 4 == 0; x, w, out
 * 16-byte aligned; out may equal x (op 1 index 2 normalises in place). */
int rta_rmsnorm(const float* x, const float* w, int rows, int width, float eps, float* out, rta_stream_t stream);

/* ops 14 (QK-norm), 15 (gated norm) and the L2 norm of op 20
 * (resident_math.comp:113-115,139-140), in place over heads of hd (64/128/256) values:
 *   x = x * w[h*hd + c] / sqrt(sum(x^2) / (mean ? hd : 1) + eps) * (gate ? g*sigmoid(g) : 1)
 * w may be NULL (no weight); gate NULL for ops 14 and 20.  Row strides in floats. */
int rta_head_norm(float* x, int x_stride, const float* w, const float* gate, int gate_stride, int rows, int heads,
                  int hd, int mean, float eps, rta_stream_t stream);

/* op 18 after its two projections (resident_math.comp:131-133):
 *   decay[b, h] = exp(-exp(a_log[h]) * softplus(a[b, h] + dt_bias[h])),  beta = sigmoid(b[b, h]);
 * a, b: [batch, >= heads] with row stride `stride`. */
int rta_delta_gates(const float* a, const float* b, int stride, const float* a_log, const float* dt_bias, int batch,
                    int heads, float* decay, float* beta, rta_stream_t stream);

/* ops 19 + 20 for one new token per sequence (resident_math.comp:134-140): causal
 * depthwise convolution of 4 taps + SiLU over the q | k | v projections (3 W values,
 * W = heads * hd, hd = 128), then per-head L2 normalisation of q and k.
 *   raw [batch, >= 3W] (stride raw_stride); state [batch, 3W, 3] the three previous raw
 *   values, oldest first, shifted in place; w [3W, 4] (16-byte aligned); out [batch, 3W]. */
int rta_short_conv(const float* raw, int raw_stride, float* state, const float* w, int batch, int heads, int hd,
                   float eps, float* out, rta_stream_t stream);

/* op 21 / resident_state.comp, one token per sequence: the gated delta rule on the
 * fp32 state [batch, heads, hd, hd] ([value][key], updated in place), hd = 128:
 *   S = decay S;  u = S k;  S += beta (v - u) k^T;  o = S q / sqrt(hd)
 * qkv: [batch, >= 3 heads hd] (q | k | v as rta_short_conv writes them).  With norm_w,
 * op 15 is fused: o = rmsnorm_hd(o) * norm_w[h hd + c] * g sigmoid(g), g = gate[b, h hd + c].
 * out [batch, >= heads hd] with row stride out_stride. */
int rta_delta_rule(float* state, const float* qkv, int qkv_stride, const float* decay, const float* beta, int batch,
                   int heads, int hd, const float* norm_w, const float* gate, int gate_stride, float eps, float* out,
                   int out_stride, rta_stream_t stream);

/* op 34, history packer (resident_history_quant.glsl:9-41; Resident::layer,
 * optical_resident.cpp:461): the new key and value rows of each sequence, k[b, :kvw]
 * and v[b, :kvw], quantised into one packet (one Q4_K and one Q6_K field, fmt_k !=
 * fmt_v, rta_history_bytes(kvw) bytes) written to packet slot[b] of `packets`
 * (n_slots slots; a slot outside sets RTA_DEVERR_HITS).  Bit exact with the
 * reference's fp32 op order; exact .5 ties of the code rounding resolve to even. */
int rta_pack_history(const float* k, int k_stride, const float* v, int v_stride, int batch, int kvw, int fmt_k,
                     int fmt_v, const int64_t* slot, int64_t n_slots, void* packets, rta_stream_t stream);

/* ---------------- one greedy decode step of a hybrid decoder (gated delta-net
 * recurrent layers and full-attention layers, 128-wide heads), for a batch of
 * independent sequences.  The host sequencing of Resident::forward / layer / word
 * (optical_resident.cpp:455-530): per layer RMSNorm, the fused in-projection, then
 *   full layers:      QK-norm + RoPE (ops 14, 3), history pack (op 34), attention,
 *   recurrent layers: gates (op 18), short conv + L2 norm (ops 19, 20), delta rule
 *                     with the gated norm (ops 21, 15),
 * the O projection with the residual add, RMSNorm and the SwiGLU MLP (executeMLP),
 * and finally RMSNorm, the LM head and the margin argmax.  Tokens, positions and
 * ring slots stay on the device and are advanced there, so one step can be
 * captured in a HIP graph and replayed. */
typedef struct rta_hybrid_shape {
    int hidden, layers;
    int full_every;                   /* layer l is full attention when l % full_every == full_every - 1 */
    int q_heads, kv_heads, head_dim;  /* head_dim must be 128 */
    int rec_heads;                    /* delta-net heads, each with a head_dim x head_dim fp32 state */
    int ff, vocab;
    int capacity;                     /* history ring slots per sequence and full layer */
    int fmt_embed, fmt_proj, fmt_lm;  /* GGUF codes; fmt_proj / fmt_lm may carry RTA_TILED */
    int fmt_k, fmt_v;                 /* history packet fields (the reference: K Q4_K, V Q6_K) */
    int rope_rotary;                  /* rotated dimensions per head (even, <= head_dim) */
    float eps;                        /* RMSNorm epsilon */
    float margin;                     /* argmax tie margin (relative), as rta_lm_head */
    double rope_theta;
    /* What compiler/export.py emits beyond the plain layout (zero: not used): */
    int attn_gate;      /* 1: full layers' w_in holds q_heads * 128 gate rows after [q | k | v], and the
                           attention output is times sigmoid(gate) (export.py:98,103;
                           resident_ray.comp:75-76) */
    int rec_key_heads;  /* q and k heads of the recurrent in-projection, 0 < rec_key_heads <= rec_heads
                           (0: rec_heads); delta-net head h reads q / k head h % rec_key_heads, the
                           key repeat of export.py:107-112 / resident_quant.glsl:26 */
    int layer_formats;  /* 1: each layer's fmt_* fields give its matrices' formats (else fmt_proj) */
    int o_axis_remap;   /* 1: q, k, v and gate rows of full layers are in the rotary-pair order of
                           modes 1-3 and w_o's columns in the exporter's order (descriptor 2 mode
                           4, export.py:97): the attention output goes back to the exporter's
                           order before w_o, so w_o is used as exported */
} rta_hybrid_shape;

typedef struct rta_hybrid_layer {   /* device pointers; fmt_proj matrices [rows x cols] */
    const float* norm_in;            /* [hidden] */
    const float* norm_post;          /* [hidden] */
    const void* w_in;                /* full: (q_heads + 2 kv_heads) * 128 rows [q | k | v] (+ q_heads *
                                        128 gate rows with attn_gate);
                                        recurrent: [q | k | v | z | a | b], q and k KH * 128 rows each
                                        (KH = rec_key_heads), v and z S rows, a and b rec_heads rows
                                        (not with w_a), S = rec_heads * 128; cols = hidden */
    const void* w_o;                 /* [hidden x (q_heads * 128 or S)] */
    const void* w_gate;              /* [ff x hidden] */
    const void* w_up;                /* [ff x hidden] */
    const void* w_down;              /* [hidden x ff] */
    const float* q_norm;             /* full: [q_heads * 128] or NULL (no QK-norm) */
    const float* k_norm;             /* full: [kv_heads * 128] or NULL */
    const float* conv_w;             /* recurrent: [3 S][4] */
    const float* a_log;              /* recurrent: [rec_heads] */
    const float* dt_bias;            /* recurrent: [rec_heads] */
    const float* out_norm;           /* recurrent: [S] gated-norm weight */
    int fmt_in, fmt_o, fmt_gate_up, fmt_down;   /* with shape->layer_formats: GGUF codes, | RTA_TILED */
    const void* w_a;                 /* recurrent: the a (decay) and b (beta) rows [rec_heads x hidden]
                                        as matrices of their own (format fmt_ab), as export.py:113 keeps
                                        ssm_alpha / ssm_beta; NULL: the last 2 rec_heads rows of w_in */
    const void* w_b;
    int fmt_ab;
    /* The in-projection as up to 4 matrices of their own formats (compiler/export.py keeps
       attn_q, attn_k, attn_v / attn_qkv and attn_gate as tensors of their own GGUF types,
       export.py:96-109): with in_parts > 0 the rows of w_in are those of in_w[0] (in_rows[0]
       rows, format in_fmt[0]), then of in_w[1], ..., and w_in / fmt_in are not read.  The
       row counts must add up to w_in's; parts need shape->layer_formats.  0: w_in holds
       every row. */
    int in_parts;
    const void* in_w[4];
    int in_rows[4];
    int in_fmt[4];
} rta_hybrid_layer;

typedef struct rta_hybrid_weights {
    const void* embed;               /* [vocab x hidden] fmt_embed */
    const rta_hybrid_layer* layers;  /* host array of `layers` entries */
    const float* norm_final;         /* [hidden] */
    const void* lm_head;             /* [vocab x hidden] fmt_lm */
} rta_hybrid_weights;

typedef struct rta_hybrid_views {   /* where the state buffer keeps each part */
    float* recurrent;                /* [recurrent layer][batch][rec_heads][128 value][128 key] */
    float* conv;                     /* [recurrent layer][batch][3 S][3] previous raw q|k|v, oldest first */
    uint8_t* packets;                /* [full layer][batch][capacity] history packets */
    int64_t* slot_base;              /* [full layer][batch] first ring slot of each sequence */
    int32_t* ctx;                    /* [batch] tokens already in the history = next position */
    int64_t recurrent_per_layer, conv_per_layer, packet_bytes, slots_per_layer;
} rta_hybrid_views;

/* Device bytes of the persistent state and of the per-step workspace; 0 if invalid. */
size_t rta_hybrid_state_bytes(const rta_hybrid_shape* shape, int batch);
size_t rta_hybrid_workspace_bytes(const rta_hybrid_shape* shape, int batch);

/* Pointers into a state buffer (256-byte aligned) for filling or reading it. */
int rta_hybrid_layout(const rta_hybrid_shape* shape, int batch, void* state, rta_hybrid_views* views);

/* Sets the ring bases and the starting positions ctx[batch] (device int32) of a state
 * buffer; the recurrent, conv and packet parts are left as the caller filled them. */
int rta_hybrid_init(const rta_hybrid_shape* shape, int batch, void* state, const int32_t* ctx, rta_stream_t stream);

/* One decode step: reads tokens[batch] (device uint32; the embedding of each
 * sequence's newest token), writes the greedy next tokens into the same array, and
 * optionally the logits [batch x vocab] (logits_out may be NULL).  Positions advance
 * by one on the device. */
int rta_hybrid_decode_step(const rta_hybrid_shape* shape, const rta_hybrid_weights* weights, int batch, void* state,
                           uint32_t* tokens, float* logits_out, void* workspace, size_t workspace_bytes,
                           rta_stream_t stream);

/* What a step can copy out or mark besides its tokens and logits (NULL: not captured). */
typedef struct rta_hybrid_capture {
    float* residual;    /* device [layers + 1 - residual_from][batch][hidden]: residual row
                           blocks residual_from .. layers, block 0 being the embedding rows and
                           block l + 1 the residual stream after layer l's MLP -- the
                           reference's layer capture (debug 1: the state snapshot after
                           executeMLP, optical_resident.cpp:481, returned by prefill and
                           generation, resident_runtime.py:136-139,199) */
    int residual_from;  /* 0 .. layers (layers: only the state after the last layer) */
    float* kv;          /* device [full layer][batch][2][kv_heads * 128]: the normed, rotated key
                           row and the value row each full layer quantises into its history
                           packet (op 34's input, resident_history_quant.glsl:5) */
    rta_event_t* marks; /* host array of layers * 7 + 4 events, recorded on the stream at the
                           reference's profile points (debug 2, optical_resident.cpp:450,455-481,
                           522-530): per layer l, marks 7l + 0 .. 6 = layer start | after the
                           in-projection and (full) QK-norm, RoPE and history pack | (1-4 equal:
                           no BVH update, trace or payload here) | after the detector (full:
                           attention; recurrent: gates, conv, delta rule and gated norm, one
                           kernel) | after the O projection and MLP; then 7 layers + 0 .. 3 =
                           LM head start (after the final norm) | (same) | after the readout |
                           after the argmax.  NULL entries are skipped; an event repeated at
                           consecutive marks is recorded once (its stages then read 0 ms) */
} rta_hybrid_capture;

/* rta_hybrid_decode_step that also fills the capture buffers and records the marks
 * (replaces the debug-1 capture and debug-2 profile paths of Resident::layer / word,
 * optical_resident.cpp:450,481,522,609-686,849-853).  capture NULL or with every pointer
 * NULL: exactly rta_hybrid_decode_step. */
int rta_hybrid_decode_step_capture(const rta_hybrid_shape* shape, const rta_hybrid_weights* weights, int batch,
                                   void* state, uint32_t* tokens, float* logits_out,
                                   const rta_hybrid_capture* capture, void* workspace, size_t workspace_bytes,
                                   rta_stream_t stream);

/* ---------------- on-disk assets (host only: no device work, no GPU needed).
 * Reads the exporter's optical_model.bin (RTRES004), geometry_weights.bin and
 * vocabulary.bin (RTBASQ01) into host memory (ray_tracing/compiler/export.py:51-138),
 * with the checks and messages of the reference worker's loader
 * (ray_tracing/native/src/optical_resident.cpp:139-152).  Replaces that loader; the
 * payloads are GGUF rows as the projection entry points take them. */
typedef struct rta_asset rta_asset;

typedef struct rta_asset_info {
    uint32_t hidden, depth, blocks, middle, vocab, quantization, step;
    uint64_t param_words, matrix_words, basis_words;
    uint32_t fmt_embed, fmt_lm;                  /* model header words 13, 15 */
    uint64_t embed_offset_words, lm_offset_words; /* model header words 14, 16 */
} rta_asset_info;

typedef struct rta_asset_matrix {
    const void* data;      /* host pointer to the raw payload */
    uint64_t offset_words; /* from the start of geometry_weights.bin / the basis payload */
    uint64_t avail_bytes;  /* bytes from data to the end of the layer range / file */
    uint32_t fmt, mode;    /* GGUF code; the exporter's mode byte (export.py:91) */
} rta_asset_matrix;

/* Opens model_path (optical_model.bin; geometry_weights.bin is read from the same
 * directory) and vocabulary_path (may be NULL to skip the basis).  On failure returns
 * RTA_ERR_FORMAT and writes the reference's message into err (err_len bytes). */
int rta_asset_open(const char* model_path, const char* vocabulary_path, rta_asset** out, char* err, size_t err_len);
void rta_asset_close(rta_asset* asset);
int rta_asset_get_info(const rta_asset* asset, rta_asset_info* info);
/* The parameter words (model header, 64-word layer headers, fp32 vectors). */
const uint32_t* rta_asset_params(const rta_asset* asset, uint64_t* words);
/* Projection descriptor index 0..8 of a layer (export.py:87-91, 96-98, 108-109, 121):
 * 0 q / qkv, 1 k, 2 output / ssm_out, 3 ffn_gate, 4 ffn_down, 5 ffn_up, 6 gate, 8 v;
 * and the delta-net's separate payloads (export.py:113; offset and code words 35 / 39,
 * 36 / 40, no mode): 9 ssm_beta, 10 ssm_alpha. */
int rta_asset_layer_matrix(const rta_asset* asset, int layer, int index, rta_asset_matrix* out);
/* fp32 vector (count values) that word `field` of a layer header (layer -1: the model
 * header) points at, e.g. 0 attn_norm, 1 post_attention_norm, 24/25 q/k norm; model 4
 * output_norm. */
int rta_asset_vector(const rta_asset* asset, int layer, int field, uint64_t count, const float** out);
/* Word `field` of a layer header (layer -1: the model header). */
int rta_asset_word(const rta_asset* asset, int layer, int field, uint32_t* value);
/* token_embd (which 0) or output (which 1) payload in vocabulary.bin. */
int rta_asset_basis(const rta_asset* asset, int which, rta_asset_matrix* out);

#ifdef __cplusplus
}
#endif
#endif
