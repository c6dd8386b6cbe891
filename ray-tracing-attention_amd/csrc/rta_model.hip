// rta_model.hip -- one greedy decode step of a hybrid (gated delta-net + full
// attention) decoder, sequenced on the host over the library's kernels; the role of
// Resident::forward / Resident::layer / Resident::word (optical_resident.cpp:455-530)
// for a batch of independent sequences.
//
// Everything a step reads per sequence (token, position, ring slots) lives in device
// memory and is advanced on the device, so a caller may capture one step in a HIP
// graph and replay it.
#include <math.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <tuple>

#include "rta_common.hpp"
#include "rta_host.hpp"
#include "rta_internal.hpp"

namespace rta {

// Step prologue and the token embedding (op 0) in one launch.  Block (x, b) decodes
// columns 256 x .. 256 x + 255 of the table row tokens[b] into hidden[b]; thread 0 of
// block (0, b) places sequence b's new token: it sits at position pos = ctx[b], is
// written to ring slot base[l][b] + pos % capacity of every full layer l and sees
// min(pos + 1, capacity) history entries (visible = pos + 1, the attention clamps it);
// ctx advances by one.
__global__ void __launch_bounds__(256) step_prologue_kernel(int32_t* __restrict__ ctx, int n_full,
                                                            int64_t capacity, const int64_t* __restrict__ base,
                                                            int64_t* __restrict__ pos64, int32_t* __restrict__ visible,
                                                            int64_t* __restrict__ slots, int fmt,
                                                            const uint8_t* __restrict__ table, int64_t row_bytes,
                                                            int vocab, int hidden, const uint32_t* __restrict__ tokens,
                                                            float* __restrict__ out) {
    const int b = blockIdx.y, batch = gridDim.y;
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        const int32_t pos = ctx[b];
        pos64[b] = pos;
        visible[b] = pos + 1;
        for (int l = 0; l < n_full; ++l) slots[(int64_t)l * batch + b] = base[(int64_t)l * batch + b] + pos % capacity;
        ctx[b] = pos + 1;
    }
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c < hidden) out[(int64_t)b * hidden + c] = embed_value(fmt, table, row_bytes, vocab, tokens[b], c);
}

// Ring bases (sequence b owns slots [b * capacity, (b + 1) * capacity) of every
// full layer's packet array) and the starting positions.
__global__ void __launch_bounds__(256) state_init_kernel(const int32_t* __restrict__ ctx_in, int batch, int n_full,
                                                         int64_t capacity, int64_t* __restrict__ base,
                                                         int32_t* __restrict__ ctx) {
    const int b = blockIdx.x * 256 + threadIdx.x;
    if (b >= batch) return;
    for (int l = 0; l < n_full; ++l) base[(int64_t)l * batch + b] = (int64_t)b * capacity;
    ctx[b] = ctx_in[b];
}

namespace {

struct Carve {
    uint8_t* p;
    size_t off = 0;
    explicit Carve(void* base) : p(static_cast<uint8_t*>(base)) {}
    template <class T>
    T* take(size_t n) {
        off = (off + 255) & ~(size_t)255;
        T* r = p ? reinterpret_cast<T*>(p + off) : nullptr;
        off += n * sizeof(T);
        return r;
    }
};

struct Dims {
    int D, L, nfull, nrec, hq, hkv, hd, H, S, FF, V, cap, B;
    int KH;              // q / k heads of the recurrent in-projection
    int rows_full;       // full in-projection rows: q | k | v (| gate)
    int rows_rec;        // recurrent in-projection rows with a | b (without: rows_rec - 2 H)
    int kvw;
    int64_t stride;
};

Dims dims_of(const rta_hybrid_shape* s, int batch) {
    Dims d{};
    d.D = s->hidden;
    d.L = s->layers;
    d.nfull = s->full_every > 0 ? s->layers / s->full_every : 0;
    d.nrec = d.L - d.nfull;
    d.hq = s->q_heads;
    d.hkv = s->kv_heads;
    d.hd = s->head_dim;
    d.H = s->rec_heads;
    d.S = s->rec_heads * s->head_dim;
    d.FF = s->ff;
    d.V = s->vocab;
    d.cap = s->capacity;
    d.B = batch;
    d.KH = s->rec_key_heads > 0 ? s->rec_key_heads : s->rec_heads;
    d.rows_full = (d.hq + 2 * d.hkv + (s->attn_gate ? d.hq : 0)) * d.hd;
    d.rows_rec = 2 * d.KH * d.hd + 2 * d.S + 2 * d.H;
    d.kvw = d.hkv * d.hd;
    d.stride = host::history_bytes(d.kvw);
    return d;
}

bool is_full(const rta_hybrid_shape* s, int l) { return s->full_every > 0 && l % s->full_every == s->full_every - 1; }

int check_shape(const rta_hybrid_shape* s, int batch) {
    if (!s) return RTA_ERR_NULL;
    if (batch <= 0 || batch > 4096 || s->layers <= 0 || s->full_every < 0 || s->hidden <= 0 ||
        s->hidden % 256 || s->ff <= 0 || s->ff % 256 || s->vocab <= 0 || s->capacity <= 0)
        return RTA_ERR_SHAPE;
    if (s->head_dim != 128 || (s->full_every > 0 && (s->q_heads <= 0 || s->kv_heads <= 0 || s->q_heads % s->kv_heads)) ||
        (s->full_every != 1 && s->rec_heads <= 0) || s->rope_rotary <= 0 || s->rope_rotary > 128 || s->rope_rotary % 2 ||
        !(s->eps >= 0.0f) || !(s->rope_theta > 0.0))
        return RTA_ERR_RANGE;
    if ((s->full_every > 0 && (s->q_heads * 128) % 256) || (s->rec_heads * 128) % 256) return RTA_ERR_SHAPE;
    if (s->attn_gate < 0 || s->attn_gate > 1 || s->layer_formats < 0 || s->layer_formats > 1 ||
        s->o_axis_remap < 0 || s->o_axis_remap > 1 ||
        s->rec_key_heads < 0 || s->rec_key_heads > s->rec_heads)
        return RTA_ERR_RANGE;
    // the full layers' attention: refused here, before the step advances any state
    if (s->full_every > 0 && s->layers >= s->full_every)
        return attention_shape_check(s->q_heads, s->kv_heads, s->head_dim, s->fmt_k, s->fmt_v);
    return RTA_OK;
}

struct State {
    float* rec;        // [nrec][B][H][hd][hd]
    float* conv;       // [nrec][B][3S][3]
    uint8_t* packets;  // [nfull][B][cap][stride]
    int64_t* base;     // [nfull][B]
    int32_t* ctx;      // [B]
};

State carve_state(const Dims& d, void* p, size_t* bytes) {
    Carve c(p);
    State s;
    s.rec = c.take<float>((size_t)d.nrec * d.B * d.H * d.hd * d.hd);
    s.conv = c.take<float>((size_t)d.nrec * d.B * 3 * d.S * 3);
    s.packets = c.take<uint8_t>((size_t)d.nfull * d.B * d.cap * d.stride);
    s.base = c.take<int64_t>((size_t)d.nfull * d.B);
    s.ctx = c.take<int32_t>((size_t)d.B);
    if (bytes) *bytes = (c.off + 255) & ~(size_t)255;
    return s;
}

struct Work {
    float *hidden, *normed, *proj, *part, *q, *ext_a, *ext_b, *mix, *act, *logits, *rms;
    int64_t *pos, *slots;
    int32_t* visible;
    void *attn_ws, *lm_ws, *gemm_ws, *ximg;
    size_t attn_bytes, lm_bytes, gemm_bytes;
};

// The largest projection workspace of an in-projection part: parts may have any row
// count up to the whole in-projection's, and a readout's workspace does not grow steadily
// with its rows (fewer row tiles get more K slabs).  Within one run of row counts that
// share a plan (the same number of 16- or 32-row tiles) the slab partials grow with the
// rows, so the multiples of 16 bound every count.  Cached per (hidden, batch tile, rows).
size_t parts_ws_bytes(int D, int B, int rows_max) {
    static std::mutex mu;
    static std::map<std::tuple<int, int, int>, size_t> memo;
    const auto key = std::make_tuple(D, std::min(B, 32), rows_max);
    {
        std::lock_guard<std::mutex> g(mu);
        const auto it = memo.find(key);
        if (it != memo.end()) return it->second;
    }
    size_t m = 0;
    for (const int f : {(int)RTA_Q4_K, (int)RTA_Q6_K, RTA_Q4_K | RTA_TILED, RTA_Q6_K | RTA_TILED})
        for (int n = 16; n < rows_max + 16; n += 16) m = std::max(m, rta_gemv_workspace_bytes(f, n, D, B));
    std::lock_guard<std::mutex> g(mu);
    memo[key] = m;
    return m;
}

// The projection workspace: enough for every format a layer may use (the shape alone
// fixes the size), the K-quant and packed ones being the only that need any.
size_t gemm_ws_bytes(const rta_hybrid_shape* s, const Dims& d) {
    size_t m = 0;
    auto up = [&](size_t v) { m = std::max(m, v); };
    const int fmts[5] = {s->fmt_proj, RTA_Q4_K, RTA_Q6_K, RTA_Q4_K | RTA_TILED, RTA_Q6_K | RTA_TILED};
    for (int i = s->layer_formats ? 0 : 4; i < 5; ++i) {
        const int f = s->layer_formats ? fmts[i] : s->fmt_proj;
        if (d.nfull) up(rta_gemv_workspace_bytes(f, d.rows_full, d.D, d.B));
        if (d.nrec) up(rta_gemv_workspace_bytes(f, d.rows_rec, d.D, d.B));
        if (d.nrec) up(rta_gemv_workspace_bytes(f, d.H, d.D, d.B));
        if (d.nfull) up(rta_gemv_workspace_bytes(f, d.D, d.hq * d.hd, d.B));
        if (d.nrec) up(rta_gemv_workspace_bytes(f, d.D, d.S, d.B));
        up(rta_mlp_workspace_bytes(f, f, d.D, d.FF, d.B));
    }
    if (d.nfull) up(image_readout_ws_bytes(d.rows_full, d.D, false));
    if (d.nrec) up(image_readout_ws_bytes(d.rows_rec, d.D, false));
    up(image_readout_ws_bytes(d.FF, d.D, true));
    up(image_readout_ws_bytes(d.D, d.FF, false));
    if (s->layer_formats)   // in-projection parts of any row count (they need layer formats)
        up(parts_ws_bytes(d.D, d.B, std::max(d.nfull ? d.rows_full : 0, d.nrec ? d.rows_rec : 0)));
    if (d.nrec && s->layer_formats) {   // separate a / b readouts behind a layer's pending K slabs
        size_t ab = 0;
        for (int f : {RTA_Q4_K, RTA_Q6_K}) ab = std::max(ab, rta_gemv_workspace_bytes(f, d.H, d.D, d.B));
        const size_t slabs = std::max(image_readout_ws_bytes(d.rows_rec, d.D, false),
                                      rta_gemv_workspace_bytes(RTA_Q6_K | RTA_TILED, d.rows_rec, d.D, d.B));
        up(((slabs + 255) & ~(size_t)255) + ab);
    }
    return m;
}

Work carve_work(const rta_hybrid_shape* s, const Dims& d, void* p, size_t* bytes) {
    Carve c(p);
    Work w{};
    const size_t B = d.B;
    w.hidden = c.take<float>(B * d.D);
    w.normed = c.take<float>(B * d.D);
    w.proj = c.take<float>(B * std::max(d.nfull ? d.rows_full : 0, d.nrec ? d.rows_rec : 0));
    // one in-projection part's rows before they are laid into w.proj (batch > 1)
    w.part = c.take<float>(B > 1 ? B * std::max(d.nfull ? d.rows_full : 0, d.nrec ? d.rows_rec : 0) : 1);
    w.q = c.take<float>(B * std::max(1, d.hq * d.hd));
    w.ext_a = c.take<float>(B * std::max(1, d.H));
    w.ext_b = c.take<float>(B * std::max(1, d.H));
    w.mix = c.take<float>(B * std::max(d.hq * d.hd, d.S));
    w.act = c.take<float>(B * d.FF);
    w.logits = c.take<float>(B * d.V);
    w.rms = c.take<float>(B * 4);   // per-chunk sums of squares of the deferred norms
    w.pos = c.take<int64_t>(B);
    w.slots = c.take<int64_t>(B * std::max(1, d.nfull));
    w.visible = c.take<int32_t>(B);
    w.attn_bytes = d.nfull ? rta_decode_attention_workspace_bytes(d.B, d.hq, d.hkv, d.hd, d.cap) : 0;
    w.attn_ws = c.take<uint8_t>(std::max<size_t>(w.attn_bytes, 1));
    w.lm_bytes = rta_lm_head_workspace_bytes(s->fmt_lm, d.V, d.D, d.B);
    w.lm_ws = c.take<uint8_t>(std::max<size_t>(w.lm_bytes, 1));
    w.gemm_bytes = gemm_ws_bytes(s, d);
    w.gemm_ws = c.take<uint8_t>(std::max<size_t>(w.gemm_bytes, 1));
    // x images: in front of the in-projections and gate/up (D columns) and of the down
    // projection (FF columns), one at a time
    const int bi = std::min(d.B, 32);
    w.ximg = c.take<uint8_t>(std::max<size_t>(std::max(image_bytes(d.D, bi), image_bytes(d.FF, bi)), 1));
    if (bytes) *bytes = (c.off + 255) & ~(size_t)255;
    return w;
}

}  // namespace
}  // namespace rta

using namespace rta;

extern "C" {

size_t rta_hybrid_state_bytes(const rta_hybrid_shape* shape, int batch) {
    if (check_shape(shape, batch)) return 0;
    size_t bytes = 0;
    carve_state(dims_of(shape, batch), nullptr, &bytes);
    return bytes;
}

size_t rta_hybrid_workspace_bytes(const rta_hybrid_shape* shape, int batch) {
    if (check_shape(shape, batch)) return 0;
    size_t bytes = 0;
    carve_work(shape, dims_of(shape, batch), nullptr, &bytes);
    return bytes;
}

int rta_hybrid_layout(const rta_hybrid_shape* shape, int batch, void* state, rta_hybrid_views* views) {
    int rc = check_shape(shape, batch);
    if (rc) return rc;
    if (!state || !views) return RTA_ERR_NULL;
    const Dims d = dims_of(shape, batch);
    const State s = carve_state(d, state, nullptr);
    views->recurrent = s.rec;
    views->conv = s.conv;
    views->packets = s.packets;
    views->slot_base = s.base;
    views->ctx = s.ctx;
    views->recurrent_per_layer = (int64_t)d.B * d.H * d.hd * d.hd;
    views->conv_per_layer = (int64_t)d.B * 3 * d.S * 3;
    views->packet_bytes = d.stride;
    views->slots_per_layer = (int64_t)d.B * d.cap;
    return RTA_OK;
}

int rta_hybrid_init(const rta_hybrid_shape* shape, int batch, void* state, const int32_t* ctx, rta_stream_t stream) {
    int rc = check_shape(shape, batch);
    if (rc) return rc;
    if (!state || !ctx) return RTA_ERR_NULL;
    if (!host::aligned(state, 256)) return RTA_ERR_ALIGN;
    const Dims d = dims_of(shape, batch);
    const State st = carve_state(d, state, nullptr);
    hipLaunchKernelGGL(state_init_kernel, dim3((batch + 255) / 256), dim3(256), 0, (hipStream_t)stream, ctx, batch,
                       d.nfull, (int64_t)d.cap, st.base, st.ctx);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_hybrid_decode_step(const rta_hybrid_shape* shape, const rta_hybrid_weights* weights, int batch, void* state,
                           uint32_t* tokens, float* logits_out, void* workspace, size_t workspace_bytes,
                           rta_stream_t stream) {
    return rta_hybrid_decode_step_capture(shape, weights, batch, state, tokens, logits_out, nullptr, workspace,
                                          workspace_bytes, stream);
}

int rta_hybrid_decode_step_capture(const rta_hybrid_shape* shape, const rta_hybrid_weights* weights, int batch,
                                   void* state, uint32_t* tokens, float* logits_out,
                                   const rta_hybrid_capture* capture, void* workspace, size_t workspace_bytes,
                                   rta_stream_t stream) {
    int rc = check_shape(shape, batch);
    if (rc) return rc;
    if (!weights || !weights->layers || !weights->embed || !weights->lm_head || !weights->norm_final || !state ||
        !tokens || !workspace)
        return RTA_ERR_NULL;
    if (workspace_bytes < rta_hybrid_workspace_bytes(shape, batch)) return RTA_ERR_WORKSPACE;
    if (!host::aligned(state, 256) || !host::aligned(workspace, 256)) return RTA_ERR_ALIGN;
    if (capture && !(host::aligned(capture->residual, 4) && host::aligned(capture->kv, 4))) return RTA_ERR_ALIGN;
    if (capture && capture->residual && (capture->residual_from < 0 || capture->residual_from > shape->layers))
        return RTA_ERR_RANGE;
    const Dims d = dims_of(shape, batch);
    const State st = carve_state(d, state, nullptr);
    Work w = carve_work(shape, d, workspace, nullptr);
    int64_t embed_rb = 0;
    rc = host::embed_args(shape->fmt_embed, weights->embed, d.V, d.D, tokens, d.B, w.hidden, &embed_rb);
    if (rc) return rc;
    hipStream_t s = (hipStream_t)stream;
    const int pf = shape->fmt_proj;
    const float eps = shape->eps;
    const int B = d.B;
#define RTA_TRY(call)            \
    do {                         \
        const int e_ = (call);   \
        if (e_) return e_;       \
    } while (0)

    // prologue: positions, visible counts, ring slots, and the token embedding (op 0)
    hipLaunchKernelGGL(step_prologue_kernel, dim3((d.D + 255) / 256, B), dim3(256), 0, s, st.ctx, d.nfull,
                       (int64_t)d.cap, st.base, w.pos, w.visible, w.slots, shape->fmt_embed,
                       static_cast<const uint8_t*>(weights->embed), embed_rb, d.V, d.D, tokens, w.hidden);
    if (hipGetLastError() != hipSuccess) return RTA_ERR_LAUNCH;

    // Layer capture: the residual stream after layer l is whole once the next norm has
    // added the last projection's pending K slabs, so it is copied right after that norm.
    float* cap_res = capture ? capture->residual : nullptr;
    const int cap_from = capture ? capture->residual_from : 0;
    float* cap_kv = capture ? capture->kv : nullptr;
    int cap_due = -1;   // residual row block still to copy (0: the embedding rows)
    auto capture_residual = [&]() -> int {
        if (!cap_res || cap_due < cap_from) return RTA_OK;
        const size_t n = (size_t)B * d.D;
        const hipError_t e = hipMemcpyAsync(cap_res + (size_t)(cap_due - cap_from) * n, w.hidden, n * sizeof(float),
                                            hipMemcpyDeviceToDevice, s);
        cap_due = -1;
        return e == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
    };
    // the profile marks (events recorded between the stages)
    rta_event_t* marks = capture ? capture->marks : nullptr;
    auto mark = [&](int i) -> int {   // an event repeated at consecutive marks is recorded once
        if (!marks || !marks[i] || (i > 0 && marks[i] == marks[i - 1])) return RTA_OK;
        return hipEventRecord((hipEvent_t)marks[i], s) == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
    };
    cap_due = 0;
    RTA_TRY(capture_residual());

    // Per matrix: packed formats at one batch tile run on the fused paths.  The residual
    // projections (O and down) then leave their K slabs in the GEMM workspace and the
    // next norm adds them into the residual stream; the norm in front of a packed
    // in-projection or gate/up pair writes x as the readout's matrix-core image
    // (w.ximg), the one in front of the packed LM head h * w with the row factor
    // deferred to the readout (rn).
    auto fmt_of = [&](int f) { return shape->layer_formats ? f : pf; };
    auto fused = [&](int f) { return (f & RTA_TILED) != 0 && B <= 32; };
    auto imaged = [&](int f) {
        return fused(f) && d.D <= 4096 && (f == (RTA_Q4_K | RTA_TILED) || f == (RTA_Q6_K | RTA_TILED));
    };
    int pending = 0;   // K slabs of the last residual projection still in gemm_ws
    auto residual_proj = [&](int f, const void* wm, int cols, const float* x) -> int {
        if (!fused(f))
            return rta_gemv(f, wm, d.D, cols, x, B, w.hidden, RTA_EPI_ACCUMULATE, w.gemm_ws, w.gemm_bytes, stream);
        int ns = 1;
        const int rc = tiled_partials(f, wm, d.D, cols, x, B, w.hidden, true, w.gemm_ws, w.gemm_bytes, s, &ns);
        pending = ns > 1 ? ns : 0;
        return rc;
    };
    // The norm in front of a consumer of format f.  keep_fp32: w.normed must hold x in
    // fp32 as well (a separate readout reads it), h * w when rn is set.  At batch 1 a
    // GGUF-row K-quant readout takes the norm itself (xn; its x is then w.hidden).
    RowNorm rn{};
    XNorm xn{};
    auto norm = [&](const float* nw, int f, bool keep_fp32) -> int {
        rn = RowNorm{};
        xn = XNorm{};
        const float* part = static_cast<const float*>(w.gemm_ws);
        int rc;
        if (!keep_fp32 && !pending && b1_norm_fusable(f, d.D, B)) {
            xn = XNorm{nw, eps};
            return capture_residual();
        }
        if (imaged(f)) {
            rc = residual_norm_image(f, w.hidden, part, pending, nw, B, d.D, w.rms, keep_fp32 ? w.normed : nullptr,
                                     w.ximg, s);
            rn = RowNorm{reinterpret_cast<const float4*>(w.rms), (float)d.D, eps};
        } else if (fused(f) && d.D <= 4096) {
            rc = residual_norm_deferred(w.hidden, part, pending, nw, B, d.D, w.normed, w.rms, s);
            rn = RowNorm{reinterpret_cast<const float4*>(w.rms), (float)d.D, eps};
        } else if (pending) {
            rc = residual_rmsnorm(w.hidden, part, pending, nw, B, d.D, eps, w.normed, s);
        } else {
            rc = rta_rmsnorm(w.hidden, nw, B, d.D, eps, w.normed, stream);
        }
        pending = 0;
        return rc ? rc : capture_residual();
    };

    // An in-projection given in parts (formats of their own): each part is read into its
    // rows of w.proj; at batch 1 every K-quant row-layout part takes the norm itself.
    auto in_parts = [&](const rta_hybrid_layer& lw, int rows, bool keep_fp32) -> int {
        if (lw.in_parts > 4) return RTA_ERR_RANGE;
        if (!shape->layer_formats) return RTA_ERR_FORMAT;   // (the workspace covers every format then)
        int sum = 0;
        bool fusable = !keep_fp32;
        for (int i = 0; i < lw.in_parts; ++i) {
            if (!lw.in_w[i]) return RTA_ERR_NULL;
            if (lw.in_rows[i] <= 0) return RTA_ERR_SHAPE;
            sum += lw.in_rows[i];
            fusable = fusable && b1_norm_fusable(lw.in_fmt[i], d.D, B);
        }
        if (sum != rows) return RTA_ERR_SHAPE;
        RTA_TRY(norm(lw.norm_in, fusable ? lw.in_fmt[0] : RTA_F32, keep_fp32));
        int off = 0;
        for (int i = 0; i < lw.in_parts; ++i) {
            const int n = lw.in_rows[i], f = lw.in_fmt[i];
            float* y = B == 1 ? w.proj + off : w.part;
            if (xn.w)
                RTA_TRY(projection_store(f, lw.in_w[i], n, d.D, w.hidden, B, y, w.gemm_ws, w.gemm_bytes, s, RowNorm{},
                                         xn));
            else
                RTA_TRY(rta_gemv(f, lw.in_w[i], n, d.D, w.normed, B, y, RTA_EPI_STORE, w.gemm_ws, w.gemm_bytes,
                                 stream));
            if (B > 1 && hipMemcpy2DAsync(w.proj + off, (size_t)rows * sizeof(float), w.part, (size_t)n * sizeof(float),
                                          (size_t)n * sizeof(float), B, hipMemcpyDeviceToDevice, s) != hipSuccess)
                return RTA_ERR_LAUNCH;
            off += n;
        }
        return RTA_OK;
    };

    int lf = 0, lr = 0;
    for (int l = 0; l < d.L; ++l) {
        const rta_hybrid_layer& lw = weights->layers[l];
        RTA_TRY(mark(7 * l));
        const int fi = fmt_of(lw.fmt_in), fo = fmt_of(lw.fmt_o), fgu = fmt_of(lw.fmt_gate_up),
                  fd = fmt_of(lw.fmt_down);
        if (is_full(shape, l)) {
            // op 2 index 5 (q | k | v | gate); ops 14 + 3 and 34 with the slab sum in one
            // kernel (full_layer_middle); attention; op 2 index 2
            int ns = 1;   // K slabs of the in-projection left in gemm_ws (1: rows final in w.proj)
            if (lw.in_parts > 0) {
                RTA_TRY(in_parts(lw, d.rows_full, false));
            } else {
                RTA_TRY(norm(lw.norm_in, fi, false));
                if (imaged(fi))
                    RTA_TRY(image_readout(fi, kReadStore, lw.w_in, nullptr, d.rows_full, d.D, w.ximg, B, w.proj,
                                          false, w.gemm_ws, w.gemm_bytes, s, &ns, rn));
                else if (rn.part || xn.w)
                    RTA_TRY(projection_store(fi, lw.w_in, d.rows_full, d.D, xn.w ? w.hidden : w.normed, B, w.proj,
                                             w.gemm_ws, w.gemm_bytes, s, rn, xn));
                else
                    RTA_TRY(rta_gemv(fi, lw.w_in, d.rows_full, d.D, w.normed, B, w.proj, RTA_EPI_STORE,
                                     w.gemm_ws, w.gemm_bytes, stream));
            }
            uint8_t* packets = st.packets + (size_t)lf * B * d.cap * d.stride;
            float* gate = shape->attn_gate ? w.proj + (d.hq + 2 * d.hkv) * d.hd : nullptr;
            RTA_TRY(full_layer_middle(ns > 1 ? static_cast<const float*>(w.gemm_ws) : w.proj,
                                      (int64_t)kSlabBatch * d.rows_full, d.rows_full, ns, B, d.hq, d.hkv, lw.q_norm,
                                      lw.k_norm, eps, w.pos, shape->rope_rotary, shape->rope_theta, w.q, gate,
                                      d.rows_full, shape->fmt_k, shape->fmt_v, w.slots + (size_t)lf * B,
                                      (int64_t)B * d.cap, packets, w.visible, d.cap, d.cap, w.attn_ws,
                                      cap_kv ? cap_kv + (size_t)lf * B * 2 * d.kvw : nullptr, s));
            for (int k = 1; k <= 4; ++k) RTA_TRY(mark(7 * l + k));
            RTA_TRY(decode_attention_gate_stride(w.q, B, d.hq, d.hkv, d.hd, packets, shape->fmt_k, shape->fmt_v,
                                                 st.base + (size_t)lf * B, w.visible, d.cap, (int64_t)B * d.cap,
                                                 d.cap, gate, d.rows_full, w.mix, nullptr, nullptr, w.attn_ws,
                                                 w.attn_bytes, stream, shape->o_axis_remap ? shape->rope_rotary : 0,
                                                 true));
            RTA_TRY(mark(7 * l + 5));
            RTA_TRY(residual_proj(fo, lw.w_o, d.hq * d.hd, w.mix));
            ++lf;
        } else {
            // op 2 index 5 (q | k | v | z | a | b), ops 18-21 and 15, op 2 index 2
            const bool ext = lw.w_a != nullptr;
            if (ext && !lw.w_b) return RTA_ERR_NULL;
            const int rows = d.rows_rec - (ext ? 2 * d.H : 0);
            int ns = 1;   // K slabs the middle adds (1: the rows are final in w.proj)
            if (lw.in_parts > 0) {
                RTA_TRY(in_parts(lw, rows, ext));
            } else {
                RTA_TRY(norm(lw.norm_in, fi, ext));
                if (imaged(fi))
                    RTA_TRY(image_readout(fi, kReadStore, lw.w_in, nullptr, rows, d.D, w.ximg, B, w.proj, false,
                                          w.gemm_ws, w.gemm_bytes, s, &ns, rn));
                else if (rn.part)
                    RTA_TRY(tiled_partials(fi, lw.w_in, rows, d.D, w.normed, B, w.proj, false, w.gemm_ws,
                                           w.gemm_bytes, s, &ns, rn));
                else if (xn.w)
                    RTA_TRY(projection_store(fi, lw.w_in, rows, d.D, w.hidden, B, w.proj, w.gemm_ws, w.gemm_bytes,
                                             s, rn, xn));
                else
                    RTA_TRY(rta_gemv(fi, lw.w_in, rows, d.D, w.normed, B, w.proj, RTA_EPI_STORE, w.gemm_ws,
                                     w.gemm_bytes, stream));
            }
            const bool slabs = ns > 1;
            // the a / b readouts into the slabs' place are done before the middle reads them;
            // with slabs pending they use the workspace after them
            if (ext) {
                const int fab = fmt_of(lw.fmt_ab);
                if (fab & RTA_TILED) return RTA_ERR_FORMAT;   // (x is not staged for them)
                uint8_t* ws2 = static_cast<uint8_t*>(w.gemm_ws);
                size_t ws2_bytes = w.gemm_bytes;
                if (slabs) {
                    const size_t used = ((size_t)ns * kSlabBatch * rows * sizeof(float) + 255) & ~(size_t)255;
                    if (used > ws2_bytes) return RTA_ERR_WORKSPACE;
                    ws2 += used;
                    ws2_bytes -= used;
                }
                RTA_TRY(rta_gemv(fab, lw.w_a, d.H, d.D, w.normed, B, w.ext_a, RTA_EPI_STORE, ws2, ws2_bytes, stream));
                RTA_TRY(rta_gemv(fab, lw.w_b, d.H, d.D, w.normed, B, w.ext_b, RTA_EPI_STORE, ws2, ws2_bytes, stream));
            }
            for (int k = 1; k <= 4; ++k) RTA_TRY(mark(7 * l + k));
            RTA_TRY(recurrent_mix(slabs ? static_cast<const float*>(w.gemm_ws) : w.proj, (int64_t)kSlabBatch * rows,
                                  rows, slabs ? ns : 1, d.KH, ext ? w.ext_a : nullptr, ext ? w.ext_b : nullptr, d.H,
                                  rn, st.conv + (size_t)lr * B * 3 * d.S * 3, lw.conv_w, lw.a_log, lw.dt_bias,
                                  st.rec + (size_t)lr * B * d.H * d.hd * d.hd, lw.out_norm, B, d.H, eps, w.mix, d.S,
                                  s));
            RTA_TRY(mark(7 * l + 5));
            RTA_TRY(residual_proj(fo, lw.w_o, d.S, w.mix));
            ++lr;
        }
        // op 1 index 1, then the SwiGLU MLP with the residual add (executeMLP)
        RTA_TRY(norm(lw.norm_post, fgu, false));
        bool down_done = false;
        if (imaged(fgu)) {
            // a packed down projection reads the SwiGLU of the gate/up K slabs as its x
            // image (no fp32 act); it leaves its own K slabs for the next norm
            const bool down_img = imaged(fd);
            int ns = 1;
            RTA_TRY(image_readout(fgu, kReadSwiglu, lw.w_gate, lw.w_up, d.FF, d.D, w.ximg, B, w.act, !down_img,
                                  w.gemm_ws, w.gemm_bytes, s, &ns, rn));
            if (down_img && ns > 1) {
                RTA_TRY(swiglu_image(fd, static_cast<const float*>(w.gemm_ws), ns, d.FF, B, w.ximg, s));
                int nd = 1;
                RTA_TRY(image_readout(fd, kReadAccumulate, lw.w_down, nullptr, d.D, d.FF, w.ximg, B, w.hidden, false,
                                      w.gemm_ws, w.gemm_bytes, s, &nd, RowNorm{}));
                pending = nd > 1 ? nd : 0;
                down_done = true;
            }
        } else {
            RTA_TRY(swiglu_activation(fgu, lw.w_gate, lw.w_up, d.FF, d.D, xn.w ? w.hidden : w.normed, B, w.act,
                                      w.gemm_ws, w.gemm_bytes, s, rn, xn));
        }
        if (!down_done) RTA_TRY(residual_proj(fd, lw.w_down, d.FF, w.act));
        RTA_TRY(mark(7 * l + 6));
        cap_due = l + 1;
    }
    // op 1 index 2, then the readout (Resident::word): logits and the next tokens; the
    // packed LM head takes the row factor itself (never an image: it is read once)
    {
        const int fl = shape->fmt_lm;
        rn = RowNorm{};
        xn = XNorm{};
        const float* part = static_cast<const float*>(w.gemm_ws);
        if (!pending && b1_norm_fusable(fl, d.D, B)) {
            xn = XNorm{weights->norm_final, eps};
        } else if (fused(fl) && d.D <= 4096) {
            RTA_TRY(residual_norm_deferred(w.hidden, part, pending, weights->norm_final, B, d.D, w.normed, w.rms, s));
            rn = RowNorm{reinterpret_cast<const float4*>(w.rms), (float)d.D, eps};
        } else if (pending) {
            RTA_TRY(residual_rmsnorm(w.hidden, part, pending, weights->norm_final, B, d.D, eps, w.normed, s));
        } else {
            RTA_TRY(rta_rmsnorm(w.hidden, weights->norm_final, B, d.D, eps, w.normed, stream));
        }
        pending = 0;
        RTA_TRY(capture_residual());
    }
    RTA_TRY(mark(7 * d.L));
    RTA_TRY(mark(7 * d.L + 1));
    RTA_TRY(lm_head_rownorm(shape->fmt_lm, weights->lm_head, d.V, d.D, xn.w ? w.hidden : w.normed, B, shape->margin,
                            logits_out ? logits_out : w.logits, tokens, w.lm_ws, w.lm_bytes, s, rn, xn,
                            marks && marks[7 * d.L + 2] != marks[7 * d.L + 1] ? (hipEvent_t)marks[7 * d.L + 2]
                                                                               : nullptr));
    RTA_TRY(mark(7 * d.L + 3));
#undef RTA_TRY
    return RTA_OK;
}

}  // extern "C"
