// rta_internal.hpp -- library-internal entry points shared between translation units
// (no C ABI): the pieces the decode step fuses across kernel boundaries.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "rta_common.hpp"

namespace rta {

constexpr int kSlabBatch = 32;   // batch rows of one K-slab partial block [slab][32][rows]

// Packed-tile projection y (+)= W x for batch <= 32 rows whose K slabs are left in
// the workspace for the caller to add: partials [slab][32][rows] fp32 at ws.  *nslab = 1
// means the kernel wrote (accumulate: added into) y itself and nothing is pending.
// ws_bytes must cover rta_gemv_workspace_bytes(fmt, rows, cols, batch).
// rn (packed readouts only): a deferred RMSNorm factor per batch row, see RowNorm.
int tiled_partials(int fmt, const void* w, int rows, int cols, const float* x, int batch, float* y, bool accumulate,
                   void* ws, size_t ws_bytes, hipStream_t s, int* nslab, const RowNorm& rn = RowNorm{});

// The RMSNorm taken by a batch-1 readout itself: x is the residual row and the readout
// multiplies it by w / sqrt(mean(x^2) + eps) while staging it (b1_norm_fusable shapes).
struct XNorm {
    const float* w = nullptr;
    float eps = 0.0f;
};
bool b1_norm_fusable(int fmt, int cols, int batch);

// y = W x (rta_gemv with the STORE epilogue) with a deferred RMSNorm factor (rn) or the
// batch-1 readout's own RMSNorm (xn).
int projection_store(int fmt, const void* w, int rows, int cols, const float* x, int batch, float* y, void* ws,
                     size_t ws_bytes, hipStream_t s, const RowNorm& rn, const XNorm& xn = XNorm{});

// rta_lm_head with a deferred RMSNorm factor per batch row; readout_done (optional) is
// recorded after the last batch tile's readout, before its argmax.
int lm_head_rownorm(int fmt, const void* w, int vocab, int hidden, const float* h, int batch, float margin,
                    float* logits, uint32_t* ids, void* workspace, size_t workspace_bytes, hipStream_t s,
                    const RowNorm& rn, const XNorm& xn = XNorm{}, hipEvent_t readout_done = nullptr);

// The fused gate/up projection of the SwiGLU MLP alone: act = swiglu(Wg x, Wu x).
int swiglu_activation(int fmt, const void* wg, const void* wu, int inter, int hidden, const float* x, int batch,
                      float* act, void* ws, size_t ws_bytes, hipStream_t s, const RowNorm& rn = RowNorm{},
                      const XNorm& xn = XNorm{});

// The middle of a recurrent layer (ops 18-21 and 15) for every (head, sequence):
// in-projection row r of sequence b = sum_k proj[k * slab_stride + b * row_stride + r]
// over k < nslab (q | k | v | z | a | b: q and k key_heads heads of 128 rows each, v and
// z heads * 128, a and b heads rows; head h reads q / k head h % key_heads), conv window
// and recurrent state updated in place, gated-norm output to out (row stride
// out_stride).  With ext_a / ext_b ([batch] rows of stride ext_stride) a and b come from
// there, times the row factor rn, and the projection rows end after z.
int recurrent_mix(const float* proj, int64_t slab_stride, int row_stride, int nslab, int key_heads, const float* ext_a,
                  const float* ext_b, int ext_stride, const RowNorm& rn, float* conv_state, const float* conv_w,
                  const float* a_log, const float* dt_bias, float* state, const float* norm_w, int batch, int heads,
                  float eps, float* out, int out_stride, hipStream_t s);

// hidden[b, :] += sum over slabs k < nslab of part[(k * 32 + b) * width + :] (slab order),
// then out[b, :] = hidden[b, :] * w / sqrt(mean(hidden[b, :]^2) + eps).  nslab may be 0.
// width % 4 == 0; pointers 16-byte aligned.
int residual_rmsnorm(float* hidden, const float* part, int nslab, const float* w, int batch, int width, float eps,
                     float* out, hipStream_t s);

// The same residual add, but the normalisation is left to the readouts that take out:
// out[b, :] = hidden[b, :] * w (no row factor) and ss[4 b + c] = sum of hidden^2 over
// column chunk c of 1024 (unused entries zero), for a RowNorm {ss, width, eps}.
// width <= 4096; ss 16-byte aligned, 4 batch floats.
int residual_norm_deferred(float* hidden, const float* part, int nslab, const float* w, int batch, int width,
                           float* out, float* ss, hipStream_t s);

// The head counts and field formats the attention kernels serve (rta_decode_attention's
// own checks): RTA_OK, or the status it would return for them.
int attention_shape_check(int hq, int hkv, int hd, int fmt_k, int fmt_v);

// rta_decode_attention with the gate of sequence s at gate + s gate_stride (head h at
// + h hd), gate_stride >= hq hd: the gate rows of a fused in-projection.  out_rotary R > 0:
// output dim d < R of each head is written to column (d % 2)(R / 2) + d / 2 of the head.
int decode_attention_gate_stride(const float* q, int nseq, int hq, int hkv, int hd, const void* packets, int fmt_k,
                                 int fmt_v, const int64_t* slot_base, const int32_t* ctx_len, int64_t capacity,
                                 int64_t n_slots, int max_ctx, const float* gate, int64_t gate_stride, float* out,
                                 float* m_out, float* z_out, void* workspace, size_t workspace_bytes,
                                 rta_stream_t stream, int out_rotary = 0, bool prepared = false);

// The middle of a full-attention layer in one kernel, between its in-projection and the
// attention: in-projection rows (q | k | v | gate, hq / hkv / hkv / hq heads of 128) of
// sequence b summed over nslab K slabs, proj[k slab_stride + b row_stride + r];
// QK-norm + RoPE of q (to q_out, [batch][hq][128]) and k; k and v quantised into packet
// slots[b] (fmt_k / fmt_v fields, as rta_pack_history), and with kv_out those normed,
// rotated k rows and v rows as well ([batch][2][hkv 128]); gate rows summed into gate_out
// (row b at + b gate_stride; null: no gate).  For the layout whose attention runs on the
// Q4_K-key matrix-core kernel it also writes that kernel's q operands and tile plan into
// attn_ws (the workspace of the decode_attention_gate_stride call that follows with
// prepared = true, same batch, heads, ctx_len, capacity and max_ctx).
int full_layer_middle(const float* proj, int64_t slab_stride, int row_stride, int nslab, int batch, int hq, int hkv,
                      const float* q_norm, const float* k_norm, float eps, const int64_t* positions, int rotary,
                      double theta, float* q_out, float* gate_out, int64_t gate_stride, int fmt_k, int fmt_v,
                      const int64_t* slots, int64_t n_slots, void* packets, const int32_t* ctx_len, int64_t capacity,
                      int max_ctx, void* attn_ws, float* kv_out, hipStream_t s);

// ---- the decode step's readouts of a staged x image (rta_packed.hpp) ----
constexpr int kReadStore = 0, kReadAccumulate = 1, kReadSwiglu = 2;   // image_readout modes
// Bytes of the image of x [batch <= 32, cols] (cols % 256 == 0); 0 for other shapes.
size_t image_bytes(int cols, int batch);
// Workspace of image_readout's K-slab partials, either batch-tile width.
size_t image_readout_ws_bytes(int rows, int cols, bool dual);

// residual_norm_deferred writing x = hidden * w as the readout image of a packed
// format (fmt | RTA_TILED, which fixes the group-sum layout), and in fp32 to out (may
// be null); ss as there, for a RowNorm {ss, width, eps}.  width % 256 == 0, <= 4096;
// batch <= 32.
int residual_norm_image(int fmt, float* hidden, const float* part, int nslab, const float* w, int batch, int width,
                        float* ss, float* out, void* img, hipStream_t s);

// The SwiGLU of a kSwiglu readout's nslab K-slab partials (left by image_readout with
// reduce = false) written as the readout image of x = act [batch <= 32, width] for a
// packed format fmt (the down projection's); width % 256 == 0.
int swiglu_image(int fmt, const float* part, int nslab, int width, int batch, void* img, hipStream_t s);

// y (=|+=) W x (mode kStore / kAccumulate) or act = swiglu(Wg x, Wu x) (kSwiglu, w2 the up
// matrix) from the image of x, each result times the row's RMSNorm factor rn.  reduce:
// K slabs are added into y here; else *nslab > 1 leaves them in ws as [slab][32][rows]
// (kSwiglu: 2 rows, gate and up interleaved) for the caller.
int image_readout(int fmt, int mode, const void* w, const void* w2, int rows, int cols, const void* img, int batch,
                  float* y, bool reduce, void* ws, size_t ws_bytes, hipStream_t s, int* nslab, const RowNorm& rn);

}  // namespace rta
