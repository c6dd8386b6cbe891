// rt_optical_resident: a resident worker with the reference worker's command line and
// stdin/stdout protocol (ray_tracing/native/src/optical_resident.cpp:966-969, framing
// ray_tracing/runtime/resident_runtime.py:41-44,101-114) on the gfx950 library:
//   op 1 / 11 / 12  prefill        (prefill,        optical_resident.cpp:609-; resident_runtime.py:116-162)
//   op 2            generate       (generate,       optical_resident.cpp:872-885; resident_runtime.py:171-173)
//   op 9            token stream   (streamGenerate, optical_resident.cpp:886; resident_runtime.py:174-188)
//   op 10           history growth (growTree,       optical_resident.cpp:232-271; resident_runtime.py:91-99)
//   op 13           finish history (finishHistory,  optical_resident.cpp:743-757; resident_runtime.py:164-169)
//   op 4  vocabulary readout  (wordCheck,      optical_resident.cpp:889-905; resident_runtime.py:235-250)
//   op 6  SwiGLU MLP check    (mlpCheck,       optical_resident.cpp:922-949; resident_runtime.py:252-263)
//   op 14 full-attention check (attentionCheck, resident_attention_runtime.inl:646-;
//                               resident_runtime.py:265-345), standard backend, dense receipts
// plus op 8 (resources) and op 0 (end).  Other operations end the worker with "Unknown
// resident operation" on stderr, as the reference does for an operation it does not
// know.  Weights come from the exported assets through rta_asset_*; every computation
// runs in librta's HIP kernels.  Generation runs rta_hybrid_decode_step on one
// sequence: the prompt one token per step, then one step per generated token.  The
// reference's shared-history and reply caches are not kept (every prefill computes
// its whole prompt; replies report no cache hits).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <map>
#include <memory>
#include <sstream>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/rta.h"
#include "../csrc/rta_remap.hpp"

namespace {

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}
void rta_check(int rc, const char* what) {
    if (rc != RTA_OK) throw std::runtime_error(std::string(what) + " failed (status " + std::to_string(rc) + ")");
}

struct Device {
    void* p = nullptr;
    size_t n = 0;
    Device() = default;
    Device(const Device&) = delete;
    Device& operator=(const Device&) = delete;
    ~Device() {
        if (p) (void)hipFree(p);
    }
    void* ensure(size_t bytes) {
        if (bytes > n) {
            if (p) hip_check(hipFree(p), "hipFree");
            p = nullptr;
            n = 0;
            hip_check(hipMalloc(&p, bytes ? bytes : 256), "hipMalloc");
            n = bytes;
        }
        return p;
    }
    template <class T>
    T* as() const { return static_cast<T*>(p); }
};

size_t row_bytes(uint32_t fmt, uint64_t cols) {
    switch (fmt) {
        case RTA_F32: return cols * 4;
        case RTA_F16:
        case RTA_BF16: return cols * 2;
        case RTA_Q4_K: return cols / 256 * 144;
        case RTA_Q6_K: return cols / 256 * 210;
    }
    throw std::runtime_error("Coefficient decoder required for this quantization");
}

// A number or boolean value of "key" inside the "model_spec" object of model.json.
double spec_value(const std::string& json, const char* key, double fallback, bool required) {
    size_t at = json.find("\"model_spec\"");
    if (at == std::string::npos) at = 0;
    const std::string k = std::string("\"") + key + "\"";
    at = json.find(k, at);
    if (at == std::string::npos) {
        if (required) throw std::runtime_error(std::string("model.json lacks model_spec.") + key);
        return fallback;
    }
    at = json.find(':', at + k.size());
    if (at == std::string::npos) throw std::runtime_error("Malformed model.json");
    ++at;
    while (at < json.size() && std::isspace((unsigned char)json[at])) ++at;
    if (json.compare(at, 4, "true") == 0) return 1.0;
    if (json.compare(at, 5, "false") == 0) return 0.0;
    return std::strtod(json.c_str() + at, nullptr);
}

template <class T>
void input(std::vector<T>& v, size_t count) {
    v.resize(count);
    std::cin.read(reinterpret_cast<char*>(v.data()), (std::streamsize)(count * sizeof(T)));
    if (!std::cin) throw std::runtime_error("Incomplete resident request body");
}

template <class T>
void append(std::vector<char>& out, const T* p, size_t count) {
    const char* b = reinterpret_cast<const char*>(p);
    out.insert(out.end(), b, b + count * sizeof(T));
}
template <class T>
void append(std::vector<char>& out, const std::vector<T>& v) { append(out, v.data(), v.size()); }

void reply(const std::vector<char>& bytes) {
    const uint32_t header[2] = {0u, (uint32_t)bytes.size()};
    std::cout.write(reinterpret_cast<const char*>(header), 8);
    std::cout.write(bytes.data(), (std::streamsize)bytes.size());
    std::cout.flush();
}

bool all_finite(const std::vector<float>& v) {
    for (float x : v)
        if (!std::isfinite(x)) return false;
    return true;
}

struct Timer {
    hipEvent_t a{}, b{};
    Timer() {
        hip_check(hipEventCreate(&a), "hipEventCreate");
        hip_check(hipEventCreate(&b), "hipEventCreate");
    }
    ~Timer() {
        (void)hipEventDestroy(a);
        (void)hipEventDestroy(b);
    }
    void start(hipStream_t s) { hip_check(hipEventRecord(a, s), "hipEventRecord"); }
    double stop(hipStream_t s) {
        hip_check(hipEventRecord(b, s), "hipEventRecord");
        hip_check(hipEventSynchronize(b), "hipEventSynchronize");
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, a, b), "hipEventElapsedTime");
        return ms;
    }
};

// The debug-2 profile of generation: events at the decode step's stage marks
// (rta_hybrid_capture.marks: 7 per layer, then 4 around the LM head), read back after
// each step into the reference's ten stage sums and two detector sums
// (optical_resident.cpp:849-853; names at resident_runtime.py:195,229-231).
struct Profile {
    std::vector<hipEvent_t> ev;
    std::vector<rta_event_t> marks;
    double parts[10] = {};
    double detector[2] = {};   // (attention, recurrent)
    Profile() = default;
    Profile(const Profile&) = delete;
    Profile& operator=(const Profile&) = delete;
    ~Profile() {
        for (hipEvent_t e : ev) (void)hipEventDestroy(e);
    }
    // one event per distinct point: marks 1-4 of a layer and the LM head's first two
    // coincide here (no BVH update, history trace, payload or vocabulary trace), and an
    // event repeated at consecutive marks is recorded once, so those stages read 0
    void start(int layers) {
        if (ev.empty()) {
            ev.resize((size_t)layers * 7 + 4);
            for (hipEvent_t& e : ev) hip_check(hipEventCreate(&e), "hipEventCreate");
            marks.assign(ev.begin(), ev.end());
            for (int l = 0; l < layers; ++l)
                for (int k = 2; k <= 4; ++k) marks[7 * l + k] = ev[7 * l + 1];
            marks[7 * layers + 1] = ev[7 * layers];
        }
        std::fill(parts, parts + 10, 0.0);
        detector[0] = detector[1] = 0.0;
    }
    double span(int a, int b) const {
        if (marks[a] == marks[b]) return 0.0;
        float ms = 0.0f;
        hip_check(hipEventElapsedTime(&ms, (hipEvent_t)marks[a], (hipEvent_t)marks[b]), "hipEventElapsedTime");
        return ms;
    }
    // one completed step: projection geometry, BVH update, history trace, coordinate
    // restore, detector, output MLP per layer; the vocabulary and its three parts
    void add(int layers, int full_every) {
        for (int l = 0; l < layers; ++l) {
            const int b = 7 * l;
            for (int j = 0; j < 6; ++j) parts[j] += span(b + j, b + j + 1);
            const bool full = full_every > 0 && l % full_every == full_every - 1;
            detector[full ? 0 : 1] += span(b + 4, b + 5);
        }
        const int w = 7 * layers;
        parts[6] += span(w, w + 3);
        for (int j = 0; j < 3; ++j) parts[7 + j] += span(w + j, w + j + 1);
    }
};

double wall_ms(std::chrono::steady_clock::time_point t0) {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
}

template <class T>
void input_value(T& v) {
    std::cin.read(reinterpret_cast<char*>(&v), sizeof(T));
}

// The asset laid out as rta_hybrid_decode_step reads it, for one sequence in GGUF row
// layout: each projection's rows gathered on the host with the exporter's row mode
// (resident_quant.glsl:20-31) applied, the in-projection sections [q | k | v | gate] /
// [q | k | v | z] of equal formats joined into one matrix, and the O projection's axis
// mode 4 kept as the step's o_axis_remap.
struct Decoder {
    rta_hybrid_shape shape{};
    std::vector<rta_hybrid_layer> layers;
    rta_hybrid_weights weights{};
    std::vector<std::unique_ptr<Device>> mem;
    std::unique_ptr<Device> state;
    Device ws, tokens, prompt, zero_ctx;
    Device last;   // the residual stream after the last layer of the latest step
    size_t ws_bytes = 0;

    const void* put(const void* host, size_t bytes) {
        mem.push_back(std::make_unique<Device>());
        Device& d = *mem.back();
        d.ensure(bytes);
        hip_check(hipMemcpy(d.p, host, bytes, hipMemcpyHostToDevice), "upload");
        return d.p;
    }

    struct Section {
        std::vector<uint8_t> rows;   // gathered GGUF rows
        uint32_t fmt;
        int count;
    };

    // `rows` logical rows of descriptor (layer, index), source row r of the payload for
    // logical row r given by the remap (src_rows rows in the payload)
    static Section gather(rta_asset* a, int layer, int index, int rows, int cols, int src_rows, const rta::Remap& m,
                          const char* what) {
        rta_asset_matrix mx{};
        rta_check(rta_asset_layer_matrix(a, layer, index, &mx), "asset matrix");
        const size_t rb = row_bytes(mx.fmt, (uint64_t)cols);
        if ((uint64_t)src_rows * rb > mx.avail_bytes) throw std::runtime_error("Truncated geometric weights");
        Section out{std::vector<uint8_t>((size_t)rows * rb), mx.fmt, rows};
        const uint8_t* src = static_cast<const uint8_t*>(mx.data);
        for (int r = 0; r < rows; ++r) {
            const int64_t sr = m.source_row(r);
            if (sr < 0 || sr >= src_rows) throw std::runtime_error(std::string("Invalid row mode of ") + what);
            std::memcpy(out.rows.data() + (size_t)r * rb, src + (size_t)sr * rb, rb);
        }
        return out;
    }

    static uint32_t mode_of(rta_asset* a, int layer, int index) {
        rta_asset_matrix mx{};
        rta_check(rta_asset_layer_matrix(a, layer, index, &mx), "asset matrix");
        return mx.mode;
    }

    // a mode-0 matrix as it lies in the payload: (device pointer, format)
    std::pair<const void*, int> plain(rta_asset* a, int layer, int index, int rows, int cols, const char* what) {
        rta_asset_matrix mx{};
        rta_check(rta_asset_layer_matrix(a, layer, index, &mx), "asset matrix");
        if (mx.mode != 0) throw std::runtime_error(std::string("Unsupported projection mode of ") + what);
        const size_t bytes = (size_t)rows * row_bytes(mx.fmt, (uint64_t)cols);
        if (bytes > mx.avail_bytes) throw std::runtime_error("Truncated geometric weights");
        return {put(mx.data, bytes), (int)mx.fmt};
    }

    // joins adjacent sections of one format into one matrix each (at most 4 parts)
    void in_projection(rta_hybrid_layer& L, const std::vector<Section>& sec) {
        std::vector<Section> parts;
        for (const Section& s : sec) {
            if (!parts.empty() && parts.back().fmt == s.fmt) {
                parts.back().rows.insert(parts.back().rows.end(), s.rows.begin(), s.rows.end());
                parts.back().count += s.count;
            } else {
                parts.push_back(s);
            }
        }
        if (parts.size() > 4) throw std::runtime_error("Too many in-projection formats");
        if (parts.size() == 1) {
            L.w_in = put(parts[0].rows.data(), parts[0].rows.size());
            L.fmt_in = (int)parts[0].fmt;
            return;
        }
        L.in_parts = (int)parts.size();
        L.fmt_in = (int)parts[0].fmt;
        for (size_t i = 0; i < parts.size(); ++i) {
            L.in_w[i] = put(parts[i].rows.data(), parts[i].rows.size());
            L.in_rows[i] = parts[i].count;
            L.in_fmt[i] = (int)parts[i].fmt;
        }
    }

    const float* vec(rta_asset* a, int layer, int field, uint64_t count) {
        const float* v = nullptr;
        rta_check(rta_asset_vector(a, layer, field, count, &v), "asset vector");
        return static_cast<const float*>(put(v, count * 4));
    }

    void build(rta_asset* a, const rta_asset_info& info, const std::string& json, uint32_t capacity) {
        const int D = (int)info.hidden, L = (int)info.depth, hd = (int)spec_value(json, "attention_head_dim", 0, true);
        const int kvh = (int)spec_value(json, "kv_heads", 0, true);
        if (hd != 128) throw std::runtime_error("This worker requires 128-wide attention heads");
        std::vector<int> kind(L);
        int first_full = -1, heads = 0, rec_heads = 0, rotary = 0;
        for (int l = 0; l < L; ++l) {
            uint32_t k = 0, h = 0;
            rta_check(rta_asset_word(a, l, 26, &k), "asset word");
            rta_check(rta_asset_word(a, l, 23, &h), "asset word");
            if (k != 1u && k != 2u) throw std::runtime_error("Unknown resident layer kind");
            kind[l] = (int)k;
            if (k == 1u) {
                uint32_t r = 0;
                rta_check(rta_asset_word(a, l, 29, &r), "asset word");
                if (first_full < 0) {
                    first_full = l;
                    heads = (int)h;
                    rotary = (int)r;
                } else if ((int)h != heads || (int)r != rotary) {
                    throw std::runtime_error("Full layers of different shapes");
                }
            } else if (rec_heads && (int)h != rec_heads) {
                throw std::runtime_error("Recurrent layers of different shapes");
            } else {
                rec_heads = (int)h;
            }
        }
        const int every = first_full < 0 ? 0 : first_full + 1;
        for (int l = 0; l < L; ++l)
            if ((kind[l] == 1) != (every > 0 && l % every == every - 1))
                throw std::runtime_error("Full layers must repeat with one period");
        const int key_heads = (int)spec_value(json, "state_key_heads", rec_heads ? rec_heads : 1, false);
        shape.hidden = D;
        shape.layers = L;
        shape.full_every = every;
        shape.q_heads = heads;
        shape.kv_heads = kvh;
        shape.head_dim = hd;
        shape.rec_heads = rec_heads;
        shape.ff = (int)info.middle;
        shape.vocab = (int)info.vocab;
        shape.capacity = (int)capacity;
        shape.fmt_embed = (int)info.fmt_embed;
        shape.fmt_proj = RTA_Q4_K;
        shape.fmt_lm = (int)info.fmt_lm;
        shape.fmt_k = RTA_Q4_K;   // the history quantisation (resident_history_quant.glsl)
        shape.fmt_v = RTA_Q6_K;
        shape.rope_rotary = rotary ? rotary : hd;
        shape.eps = (float)spec_value(json, "norm_epsilon", 1e-6, false);
        shape.margin = 0.0f;      // the plain argmax, ties to the lower id (resident_math.comp:117-130)
        shape.rope_theta = spec_value(json, "rope_theta", 1e7, false);
        shape.rec_key_heads = rec_heads ? key_heads : 0;
        shape.layer_formats = 1;
        const int S = rec_heads * hd, KW = key_heads * hd;
        layers.assign(L, rta_hybrid_layer{});
        int o_remap = -1;
        for (int l = 0; l < L; ++l) {
            rta_hybrid_layer& Lw = layers[l];
            Lw.norm_in = vec(a, l, 0, D);
            Lw.norm_post = vec(a, l, 1, D);
            if (kind[l] == 1) {
                const uint32_t mq = mode_of(a, l, 0), mk = mode_of(a, l, 1), mv = mode_of(a, l, 8),
                               mo = mode_of(a, l, 2), mg = mode_of(a, l, 6);
                const bool gate = mg == RTA_REMAP_GATE;
                if ((mq != 0 && mq != RTA_REMAP_QUERY && mq != RTA_REMAP_ROTARY) || (mk != 0 && mk != RTA_REMAP_ROTARY) ||
                    (mv != 0 && mv != RTA_REMAP_ROTARY) || (mo != 0 && mo != RTA_REMAP_AXES) || (gate && mq != RTA_REMAP_QUERY))
                    throw std::runtime_error("Unsupported attention projection modes");
                if (o_remap >= 0 && o_remap != (mo == RTA_REMAP_AXES)) throw std::runtime_error("Unsupported attention projection modes");
                o_remap = mo == RTA_REMAP_AXES;
                shape.attn_gate = gate;
                auto remap = [&](uint32_t mode) { return rta::Remap{(int)mode, hd, rotary, 0}; };
                const int qw = heads * hd, gw = kvh * hd;
                std::vector<Section> sec;
                sec.push_back(gather(a, l, 0, qw, D, mq == RTA_REMAP_QUERY ? 2 * qw : qw, remap(mq), "attn_q"));
                sec.push_back(gather(a, l, 1, gw, D, gw, remap(mk), "attn_k"));
                sec.push_back(gather(a, l, 8, gw, D, gw, remap(mv), "attn_v"));
                if (gate) sec.push_back(gather(a, l, 6, qw, D, 2 * qw, remap(mg), "attention gate"));
                in_projection(Lw, sec);
                rta_asset_matrix mx{};
                rta_check(rta_asset_layer_matrix(a, l, 2, &mx), "asset matrix");
                const size_t ob = (size_t)D * row_bytes(mx.fmt, (uint64_t)qw);
                if (ob > mx.avail_bytes) throw std::runtime_error("Truncated geometric weights");
                Lw.w_o = put(mx.data, ob);
                Lw.fmt_o = (int)mx.fmt;
                Lw.q_norm = vec(a, l, 24, (uint64_t)qw);
                Lw.k_norm = vec(a, l, 25, (uint64_t)gw);
            } else {
                const uint32_t mq = mode_of(a, l, 0), mk = mode_of(a, l, 1);
                for (uint32_t m : {mq, mk})
                    if (m != RTA_REMAP_KEY_REPEAT && !(m == 0 && key_heads == rec_heads))
                        throw std::runtime_error("Unsupported recurrent projection modes");
                const rta::Remap id{};
                std::vector<Section> sec;
                sec.push_back(gather(a, l, 0, KW, D, KW, id, "attn_qkv"));
                sec.push_back(gather(a, l, 1, KW, D, KW, id, "attn_qkv"));
                for (int idx : {8, 6}) {
                    if (mode_of(a, l, idx) != 0) throw std::runtime_error("Unsupported recurrent projection modes");
                    sec.push_back(gather(a, l, idx, S, D, S, id, idx == 8 ? "attn_qkv" : "attn_gate"));
                }
                in_projection(Lw, sec);
                auto o = plain(a, l, 2, D, S, "ssm_out");
                Lw.w_o = o.first;
                Lw.fmt_o = o.second;
                auto beta = plain(a, l, 9, rec_heads, D, "ssm_beta");
                auto alpha = plain(a, l, 10, rec_heads, D, "ssm_alpha");
                if (beta.second != alpha.second) throw std::runtime_error("ssm_alpha and ssm_beta differ in format");
                Lw.w_a = alpha.first;
                Lw.w_b = beta.first;
                Lw.fmt_ab = alpha.second;
                Lw.conv_w = vec(a, l, 34, (uint64_t)3 * S * 4);
                Lw.dt_bias = vec(a, l, 37, (uint64_t)rec_heads);
                Lw.a_log = vec(a, l, 38, (uint64_t)rec_heads);
                Lw.out_norm = vec(a, l, 31, (uint64_t)S);
            }
            auto g = plain(a, l, 3, (int)info.middle, D, "ffn_gate");
            auto u = plain(a, l, 5, (int)info.middle, D, "ffn_up");
            auto dn = plain(a, l, 4, D, (int)info.middle, "ffn_down");
            if (g.second != u.second) throw std::runtime_error("ffn_gate and ffn_up differ in format");
            Lw.w_gate = g.first;
            Lw.w_up = u.first;
            Lw.fmt_gate_up = g.second;
            Lw.w_down = dn.first;
            Lw.fmt_down = dn.second;
        }
        shape.o_axis_remap = o_remap > 0;
        rta_asset_matrix e{}, h{};
        rta_check(rta_asset_basis(a, 0, &e), "asset basis");
        rta_check(rta_asset_basis(a, 1, &h), "asset basis");
        const size_t eb = (size_t)info.vocab * row_bytes(e.fmt, D), hb = (size_t)info.vocab * row_bytes(h.fmt, D);
        if (eb > e.avail_bytes || hb > h.avail_bytes) throw std::runtime_error("Truncated original word basis");
        weights.embed = put(e.data, eb);
        weights.lm_head = e.offset_words == h.offset_words && e.fmt == h.fmt ? weights.embed : put(h.data, hb);
        weights.norm_final = vec(a, -1, 4, D);
        weights.layers = layers.data();
        tokens.ensure(256);
        last.ensure((size_t)D * 4);
        int32_t zero = 0;
        zero_ctx.ensure(256);
        hip_check(hipMemcpy(zero_ctx.p, &zero, 4, hipMemcpyHostToDevice), "upload");
        allocate(capacity);
    }

    void allocate(uint32_t capacity) {
        shape.capacity = (int)capacity;
        const size_t sb = rta_hybrid_state_bytes(&shape, 1), wb = rta_hybrid_workspace_bytes(&shape, 1);
        if (!sb || !wb) throw std::runtime_error("Unsupported resident model shape");
        state = std::make_unique<Device>();
        state->ensure(sb);
        ws.ensure(wb);
        ws_bytes = wb;
    }

    // a fresh sequence at position 0: zero recurrent and conv states
    void reset(hipStream_t s) {
        hip_check(hipMemsetAsync(state->p, 0, state->n, s), "clear state");
        rta_check(rta_hybrid_init(&shape, 1, state->p, zero_ctx.as<int32_t>(), s), "rta_hybrid_init");
    }

    // one step: tokens[0] in, the greedy next token out.  The residual stream after the
    // last layer goes to `last` (the state a debug-1 generation reply carries); with `all`
    // every layer's as well ([layers + 1][hidden], the embedding first); with `marks` the
    // stage events of a debug-2 profile are recorded.
    void step(hipStream_t s, float* all = nullptr, rta_event_t* marks = nullptr) {
        rta_hybrid_capture cap{};
        cap.residual = all ? all : last.as<float>();
        cap.residual_from = all ? 0 : shape.layers;
        cap.marks = marks;
        rta_check(rta_hybrid_decode_step_capture(&shape, &weights, 1, state->p, tokens.as<uint32_t>(), nullptr, &cap,
                                                 ws.p, ws_bytes, s),
                  "rta_hybrid_decode_step_capture");
        if (all)
            hip_check(hipMemcpyAsync(last.p, all + (size_t)shape.layers * shape.hidden, (size_t)shape.hidden * 4,
                                     hipMemcpyDeviceToDevice, s),
                      "copy state");
    }

    // the history ring grows to `next` slots; recurrent, conv and packet state are kept
    void grow(uint32_t next, hipStream_t s) {
        std::unique_ptr<Device> old = std::move(state);
        const uint32_t previous = (uint32_t)shape.capacity;
        rta_hybrid_views ov{}, nv{};
        rta_check(rta_hybrid_layout(&shape, 1, old->p, &ov), "rta_hybrid_layout");
        allocate(next);
        rta_check(rta_hybrid_layout(&shape, 1, state->p, &nv), "rta_hybrid_layout");
        const int nfull = shape.full_every > 0 ? shape.layers / shape.full_every : 0, nrec = shape.layers - nfull;
        hip_check(hipMemsetAsync(state->p, 0, state->n, s), "clear state");
        if (nrec) {
            hip_check(hipMemcpyAsync(nv.recurrent, ov.recurrent, (size_t)nrec * ov.recurrent_per_layer * 4,
                                     hipMemcpyDeviceToDevice, s), "copy state");
            hip_check(hipMemcpyAsync(nv.conv, ov.conv, (size_t)nrec * ov.conv_per_layer * 4, hipMemcpyDeviceToDevice, s),
                      "copy state");
        }
        for (int l = 0; l < nfull; ++l)
            hip_check(hipMemcpyAsync(nv.packets + (size_t)l * nv.slots_per_layer * nv.packet_bytes,
                                     ov.packets + (size_t)l * ov.slots_per_layer * ov.packet_bytes,
                                     (size_t)previous * ov.packet_bytes, hipMemcpyDeviceToDevice, s),
                      "copy history");
        rta_check(rta_hybrid_init(&shape, 1, state->p, ov.ctx, s), "rta_hybrid_init");
        hip_check(hipStreamSynchronize(s), "sync");
    }
};

struct Worker {
    rta_asset* asset = nullptr;
    rta_asset_info info{};
    uint32_t capacity = 300, work_rows = 512, block = 128;
    uint32_t heads = 0, kv_heads = 0, hd = 0;
    std::vector<int> full;   // full-attention layers
    bool attention_gate = false;
    hipStream_t stream{};
    std::string json;                                 // model.json
    std::unique_ptr<Decoder> dec;                     // built by the first prefill / growth
    bool prefilled = false, diagnostic_dirty = false;
    uint32_t control[8] = {0, 0, 1, 0, 0xffffffffu, 0xffffffffu, 0, 0};   // (resident_math.comp:130)
    uint64_t position = 0;                            // absolute position (emitted tokens count)
    std::map<int, std::unique_ptr<Device>> uploads;   // (layer, index) -> device payload
    Device ws, x, act, y, logits, ids, rows, q, kbuf, vbuf, gate, out, m, z, packets, slots, ctx, rec, layers_cap;
    Profile profile;

    ~Worker() {
        if (asset) rta_asset_close(asset);
    }

    const void* upload(int key, const void* host, size_t bytes) {
        auto& d = uploads[key];
        if (!d) {
            d = std::make_unique<Device>();
            d->ensure(bytes);
            hip_check(hipMemcpy(d->p, host, bytes, hipMemcpyHostToDevice), "upload");
        }
        return d->p;
    }

    rta_asset_matrix matrix(int layer, int index, uint64_t rows, uint64_t cols, const void** dev) {
        rta_asset_matrix mx{};
        rta_check(rta_asset_layer_matrix(asset, layer, index, &mx), "asset matrix");
        const size_t bytes = rows * row_bytes(mx.fmt, cols);
        if (bytes > mx.avail_bytes) throw std::runtime_error("Truncated geometric weights");
        *dev = upload(layer * 16 + index, mx.data, bytes);
        return mx;
    }

    void device_error_check(const char* what) {
        uint32_t bits = 0;
        rta_check(rta_device_error(&bits, 1), "rta_device_error");
        if (bits) throw std::runtime_error(std::string(what) + " error " + std::to_string(bits));
    }

    // op 6: rows already normalised; output = Wd (SiLU(Wg x) * Wu x) with the state
    // zeroed first (optical_resident.cpp:922-949).
    void mlp_check(uint32_t count, uint32_t layer) {
        const uint32_t D = info.hidden, F = info.middle;
        if (!count || count > std::min({capacity, work_rows, 32u}) || layer >= info.depth)
            throw std::runtime_error("Invalid optical MLP input");
        std::vector<float> xs;
        input(xs, (size_t)count * D);
        if (!all_finite(xs)) throw std::runtime_error("Optical MLP input must be finite");
        Timer t;
        t.start(stream);
        const void *wg, *wu, *wd;
        const auto g = matrix((int)layer, 3, F, D, &wg);
        const auto u = matrix((int)layer, 5, F, D, &wu);
        const auto d = matrix((int)layer, 4, D, F, &wd);
        x.ensure(xs.size() * 4);
        hip_check(hipMemcpyAsync(x.p, xs.data(), xs.size() * 4, hipMemcpyHostToDevice, stream), "upload rows");
        const double setup = t.stop(stream);
        act.ensure((size_t)count * F * 4);
        y.ensure((size_t)count * D * 4);
        const size_t wsb = rta_mlp_workspace_bytes((int)g.fmt, (int)d.fmt, (int)D, (int)F, (int)count);
        ws.ensure(wsb);
        if (g.fmt != u.fmt) throw std::runtime_error("ffn_gate and ffn_up differ in format");
        // rta_mlp_swiglu's two passes as separate calls, timed one by one
        t.start(stream);
        rta_check(rta_swiglu((int)g.fmt, wg, wu, (int)D, (int)F, x.as<float>(), (int)count, act.as<float>(), ws.p, wsb,
                             stream),
                  "rta_swiglu");
        const double gate_up = t.stop(stream);
        t.start(stream);
        rta_check(rta_gemv((int)d.fmt, wd, (int)D, (int)F, act.as<float>(), (int)count, y.as<float>(), RTA_EPI_STORE,
                           ws.p, wsb, stream),
                  "rta_gemv");
        const double down = t.stop(stream);
        device_error_check("RT MLP transmission");
        std::vector<float> yo((size_t)count * D), ao((size_t)count * F);
        hip_check(hipMemcpy(yo.data(), y.p, yo.size() * 4, hipMemcpyDeviceToHost), "read output");
        hip_check(hipMemcpy(ao.data(), act.p, ao.size() * 4, hipMemcpyDeviceToHost), "read activation");
        std::vector<char> o;
        append(o, yo);
        append(o, ao);
        const std::vector<uint32_t> hits(count, F);   // the full-matrix MLP reads every feature
        append(o, hits);
        const std::vector<double> times{setup, gate_up, down};
        append(o, times);
        reply(o);
    }

    // op 4: logits of the query over the whole vocabulary, the winner (ties to the lower
    // id), and the readout's coverage fields (optical_resident.cpp:889-905,
    // resident_math.comp:99-105,117-130).
    void word_check() {
        const auto t0 = std::chrono::steady_clock::now();
        const uint32_t D = info.hidden, V = info.vocab;
        std::vector<float> qs;
        input(qs, D);
        rta_asset_matrix b{};
        rta_check(rta_asset_basis(asset, 1, &b), "asset basis");
        const size_t rb = row_bytes(b.fmt, D), bytes = (size_t)V * rb;
        if (bytes > b.avail_bytes) throw std::runtime_error("Truncated original word basis");
        const void* w = upload(-1, b.data, bytes);
        x.ensure((size_t)D * 4);
        hip_check(hipMemcpyAsync(x.p, qs.data(), (size_t)D * 4, hipMemcpyHostToDevice, stream), "upload query");
        logits.ensure((size_t)V * 4);
        ids.ensure(256);
        const size_t wsb = rta_lm_head_workspace_bytes((int)b.fmt, (int)V, (int)D, 1);
        ws.ensure(wsb);
        Timer t;
        t.start(stream);
        rta_check(rta_lm_head((int)b.fmt, w, (int)V, (int)D, x.as<float>(), 1, 0.0f, logits.as<float>(),
                              ids.as<uint32_t>(), ws.p, wsb, stream),
                  "rta_lm_head");
        const double lm_ms = t.stop(stream);
        device_error_check("Resident word optical");
        // decoded rows of the first 256 queued words (every word is queued, in id order)
        const uint32_t nd = std::min<uint32_t>(256u, V);
        rows.ensure((size_t)256 * D * 4);
        hip_check(hipMemsetAsync(rows.p, 0, (size_t)256 * D * 4, stream), "clear rows");
        rta_check(rta_dequant((int)b.fmt, w, (int64_t)nd * D, rows.as<float>(), stream), "rta_dequant");
        uint32_t id = 0;
        float best = 0.0f;
        hip_check(hipMemcpyAsync(&id, ids.p, 4, hipMemcpyDeviceToHost, stream), "read id");
        hip_check(hipStreamSynchronize(stream), "sync");
        if (id >= V) throw std::runtime_error("Resident word optical error 2048");
        hip_check(hipMemcpy(&best, logits.as<float>() + id, 4, hipMemcpyDeviceToHost), "read logit");
        std::vector<float> dec((size_t)256 * D);
        hip_check(hipMemcpy(dec.data(), rows.p, dec.size() * 4, hipMemcpyDeviceToHost), "read rows");
        std::vector<char> o;
        const std::vector<double> times{lm_ms, wall_ms(t0), 0.0, lm_ms, 0.0};
        append(o, times);
        float f20 = best + 20.0f, one = 1.0f;
        uint32_t winner[4] = {id, 0, 0, 0};
        std::memcpy(&winner[1], &f20, 4);
        std::memcpy(&winner[2], &one, 4);
        std::memcpy(&winner[3], &one, 4);
        append(o, winner, 4);
        append(o, &V, 1);
        std::vector<uint32_t> queue(V);
        for (uint32_t i = 0; i < V; ++i) queue[i] = i;
        append(o, queue);
        append(o, dec);
        // the query as the readout stores it: fp32 bits, pairs in order (resident_common.glsl:103)
        append(o, reinterpret_cast<const uint32_t*>(qs.data()), D);
        // per 256-wide block: chart of its first pair scaled by sqrt(256) / |block|
        // (resident_math.comp:99-105, resident_common.glsl:78)
        const uint32_t blocks = D / 256;
        std::vector<float> charts((size_t)blocks * 4, 0.0f);
        for (uint32_t bk = 0; bk < blocks; ++bk) {
            float ss = 0.0f;
            for (uint32_t c = 0; c < 256; ++c) ss += qs[bk * 256 + c] * qs[bk * 256 + c];
            const float inv = 16.0f / std::max(std::sqrt(ss), 1e-20f);
            const float vx = qs[bk * 256] * inv, vy = qs[bk * 256 + 1] * inv;
            const float radius = std::sqrt(vx * vx + vy * vy), a = std::log(1.0f + radius);
            if (radius > 1e-20f) {
                charts[bk * 4] = 0.7f * a / (1.0f + a) * vx / radius;
                charts[bk * 4 + 1] = 0.7f * a / (1.0f + a) * vy / radius;
            }
        }
        append(o, charts);
        const uint32_t block_hits = V * blocks;   // every word meets every block
        append(o, &block_hits, 1);
        reply(o);
    }

    // op 14: pack the supplied K/V rows into history packets, then each query row r
    // attends causally to positions history_start .. query_start + r (all within
    // capacity); standard backend, dense receipts (resident_attention_runtime.inl:646-,
    // attention_receipts.hpp:16-29) written by rta_attention_receipts.
    void attention_check(uint32_t nrows, uint32_t layer) {
        uint32_t hdr[4];
        std::cin.read(reinterpret_cast<char*>(hdr), sizeof(hdr));
        const uint32_t count = hdr[0], qstart = hdr[1], hstart = hdr[2];
        bool full_layer = false;
        for (int l : full)
            if ((uint32_t)l == layer) full_layer = true;
        if (!std::cin || !nrows || nrows > std::min(work_rows, 32u) || !count || count > capacity ||
            layer >= info.depth || !full_layer || qstart < hstart || (uint64_t)qstart + nrows > (uint64_t)hstart + count ||
            (uint64_t)hstart + count > 1048576u || hdr[3])
            throw std::runtime_error("Invalid full-attention diagnostic shape or causal domain");
        const uint32_t Q = heads * hd, G = kv_heads * hd;
        std::vector<float> qs, ks, vs, gs;
        input(qs, (size_t)nrows * Q);
        input(ks, (size_t)count * G);
        input(vs, (size_t)count * G);
        input(gs, (size_t)nrows * Q);
        if (!all_finite(qs) || !all_finite(ks) || !all_finite(vs) || !all_finite(gs))
            throw std::runtime_error("Attention diagnostic values must be finite");
        const auto t0 = std::chrono::steady_clock::now();
        const size_t pb = rta_history_bytes((int)G);
        if (!pb) throw std::runtime_error("Unsupported history width");
        // positions relative to the diagnostic's origin: position history_start + i in slot i
        packets.ensure((size_t)capacity * pb);
        kbuf.ensure(ks.size() * 4);
        vbuf.ensure(vs.size() * 4);
        slots.ensure((size_t)std::max(count, nrows) * 8);
        std::vector<int64_t> sl(count);
        for (uint32_t i = 0; i < count; ++i) sl[i] = i;
        hip_check(hipMemcpyAsync(kbuf.p, ks.data(), ks.size() * 4, hipMemcpyHostToDevice, stream), "upload keys");
        hip_check(hipMemcpyAsync(vbuf.p, vs.data(), vs.size() * 4, hipMemcpyHostToDevice, stream), "upload values");
        hip_check(hipMemcpyAsync(slots.p, sl.data(), (size_t)count * 8, hipMemcpyHostToDevice, stream), "upload slots");
        // one sequence per query row over the shared ring, each with its own length
        std::vector<int32_t> lens(nrows);
        std::vector<int64_t> bases(nrows, 0);
        int max_ctx = 0;
        for (uint32_t r = 0; r < nrows; ++r) {
            lens[r] = (int32_t)(qstart - hstart + r + 1);
            max_ctx = std::max(max_ctx, lens[r]);
        }
        ctx.ensure((size_t)nrows * 4);
        Device base_d;
        base_d.ensure((size_t)nrows * 8);
        q.ensure(qs.size() * 4);
        gate.ensure(gs.size() * 4);
        out.ensure(qs.size() * 4);
        m.ensure((size_t)nrows * heads * 4);
        z.ensure((size_t)nrows * heads * 4);
        hip_check(hipMemcpyAsync(ctx.p, lens.data(), (size_t)nrows * 4, hipMemcpyHostToDevice, stream), "upload lengths");
        hip_check(hipMemcpyAsync(base_d.p, bases.data(), (size_t)nrows * 8, hipMemcpyHostToDevice, stream), "upload bases");
        hip_check(hipMemcpyAsync(q.p, qs.data(), qs.size() * 4, hipMemcpyHostToDevice, stream), "upload queries");
        hip_check(hipMemcpyAsync(gate.p, gs.data(), gs.size() * 4, hipMemcpyHostToDevice, stream), "upload gate");
        const size_t wsb = rta_decode_attention_workspace_bytes((int)nrows, (int)heads, (int)kv_heads, (int)hd, max_ctx);
        ws.ensure(wsb);
        const uint32_t stride = hd + 8 + block / 32;
        const int64_t records = rta_attention_receipt_records(lens.data(), (int)nrows, (int)heads, capacity, (int)block);
        if (records <= 0 || records > 0xFFFFFFFFll) throw std::runtime_error("Attention receipt count out of range");
        rec.ensure((size_t)records * stride * 4);
        // timed as the reference times the diagnostic (resident_attention_runtime.inl:707-726,752):
        // the producer (history pack and the per-group records), then the attention output
        // (the merge's place); the legacy output is the same computation, not run again
        Timer producer, merge;
        producer.start(stream);
        rta_check(rta_pack_history(kbuf.as<float>(), (int)G, vbuf.as<float>(), (int)G, (int)count, (int)G, RTA_Q4_K,
                                   RTA_Q6_K, slots.as<int64_t>(), capacity, packets.p, stream),
                  "rta_pack_history");
        rta_check(rta_attention_receipts(q.as<float>(), (int)nrows, (int)heads, (int)kv_heads, (int)hd, packets.p,
                                         RTA_Q4_K, RTA_Q6_K, base_d.as<int64_t>(), ctx.as<int32_t>(), capacity, capacity,
                                         max_ctx, (int)block, rec.as<uint32_t>(), records, stream),
                  "rta_attention_receipts");
        const double fused = producer.stop(stream);
        merge.start(stream);
        rta_check(rta_decode_attention(q.as<float>(), (int)nrows, (int)heads, (int)kv_heads, (int)hd, packets.p, RTA_Q4_K,
                                       RTA_Q6_K, base_d.as<int64_t>(), ctx.as<int32_t>(), capacity, capacity, max_ctx,
                                       attention_gate ? gate.as<float>() : nullptr, out.as<float>(), m.as<float>(),
                                       z.as<float>(), ws.p, wsb, stream),
                  "rta_decode_attention");
        const double merged = merge.stop(stream);
        uint32_t bits = 0;
        rta_check(rta_device_error(&bits, 1), "rta_device_error");
        std::vector<float> o_h(qs.size()), m_h((size_t)nrows * heads), z_h((size_t)nrows * heads);
        std::vector<uint8_t> pk((size_t)count * pb);
        hip_check(hipMemcpy(o_h.data(), out.p, o_h.size() * 4, hipMemcpyDeviceToHost), "read output");
        hip_check(hipMemcpy(m_h.data(), m.p, m_h.size() * 4, hipMemcpyDeviceToHost), "read m");
        hip_check(hipMemcpy(z_h.data(), z.p, z_h.size() * 4, hipMemcpyDeviceToHost), "read z");
        hip_check(hipMemcpy(pk.data(), packets.p, pk.size(), hipMemcpyDeviceToHost), "read packets");
        std::vector<float> phys((size_t)nrows * heads * 2);
        for (size_t i = 0; i < m_h.size(); ++i) {
            phys[2 * i] = m_h[i] + 20.0f;   // the reported intensity m + 20 (resident_ray.comp:74)
            phys[2 * i + 1] = z_h[i];
        }
        const uint32_t legacy = hstart == 0 ? 1u : 0u;
        std::vector<char> o;
        const uint32_t header[12] = {0x41545231u, nrows, count, heads, kv_heads, hd, (uint32_t)pb,
                                     block, stride, (uint32_t)records, legacy, bits};
        append(o, header, 12);
        const std::vector<double> times{fused, merged, 0.0, wall_ms(t0)};
        append(o, times);
        append(o, o_h);
        append(o, phys);
        // the same computation stands for the legacy detector when the history starts at 0
        if (legacy) {
            append(o, o_h);
            append(o, phys);
        } else {
            const std::vector<float> zeros(o_h.size() + phys.size(), 0.0f);
            append(o, zeros);
        }
        append(o, pk);
        std::vector<uint32_t> receipts((size_t)records * stride);
        hip_check(hipMemcpy(receipts.data(), rec.p, receipts.size() * 4, hipMemcpyDeviceToHost), "read receipts");
        append(o, receipts);
        reply(o);
    }

    Decoder& decoder() {
        if (!dec) {
            dec = std::make_unique<Decoder>();
            dec->build(asset, info, json, capacity);
        }
        return *dec;
    }

    // op 1 / 11 / 12: the prompt (at most capacity ids) from position 0, one decode step
    // per token; the last step leaves the first generated token pending on the device.
    void prefill(uint32_t count, uint32_t debug, uint32_t checkpoint_mode) {
        if (debug > 2u || !count || count > capacity) throw std::runtime_error("Invalid resident prefix");
        std::vector<uint32_t> ids;
        input(ids, count);
        uint32_t stops[2];
        std::cin.read(reinterpret_cast<char*>(stops), 8);
        uint32_t boundary = count;
        if (checkpoint_mode == 1u) input_value(boundary);
        if (checkpoint_mode == 2u) {
            uint32_t n = 0;
            input_value(n);
            if (n > 4096u) throw std::runtime_error("Too many history boundaries");
            uint32_t stable = 0;
            for (uint32_t i = 0; i < n; ++i) {
                uint32_t v[2];
                std::cin.read(reinterpret_cast<char*>(v), 8);
                if (!v[0] || v[0] > count || !(v[1] & 15u) || v[1] > 15u) throw std::runtime_error("Invalid history boundary");
                if (v[1] & 1u) stable = std::max(stable, v[0]);
            }
            if (stable) boundary = stable;
        }
        if (!std::cin || !boundary || boundary > count || *std::max_element(ids.begin(), ids.end()) >= info.vocab)
            throw std::runtime_error("Invalid prefix word IDs or boundary");
        const auto t0 = std::chrono::steady_clock::now();
        Decoder& d = decoder();
        // layer capture (debug 1, optical_resident.cpp:481,614-616,686): every position's
        // residual stream after each layer, [count][depth + 1][hidden] on the device
        const size_t D = info.hidden, depth = info.depth, per = (depth + 1) * D;
        const bool capture = debug == 1u;
        if (capture) {
            if ((uint64_t)count * per * 4 > (1ull << 32))
                throw std::runtime_error("Layer capture exceeds the device storage-buffer range; use a shorter prefix");
            layers_cap.ensure((size_t)count * per * 4);
        }
        d.prompt.ensure((size_t)count * 4);
        hip_check(hipMemcpyAsync(d.prompt.p, ids.data(), (size_t)count * 4, hipMemcpyHostToDevice, stream), "upload prompt");
        Timer t;
        t.start(stream);
        d.reset(stream);
        for (uint32_t i = 0; i < count; ++i) {
            hip_check(hipMemcpyAsync(d.tokens.p, d.prompt.as<uint32_t>() + i, 4, hipMemcpyDeviceToDevice, stream),
                      "prompt token");
            d.step(stream, capture ? layers_cap.as<float>() + (size_t)i * per : nullptr);
        }
        const double gpu = t.stop(stream);
        uint32_t bits = 0;
        rta_check(rta_device_error(&bits, 1), "rta_device_error");
        if (bits) throw std::runtime_error("Resident prefix optical error " + std::to_string(bits));
        const uint32_t initial[8] = {0, 0, 1, 0, stops[0], stops[1], 0, 0};
        std::memcpy(control, initial, sizeof(control));
        prefilled = true;
        diagnostic_dirty = false;
        position = count;
        std::vector<char> o;
        const std::vector<double> times{0.0, gpu, 0.0, wall_ms(t0), 0.0, 0.0};
        append(o, times);
        append(o, control, 8);
        if (capture) {   // the state after the last layer per position, then each layer's rows
            std::vector<float> all((size_t)count * per), rows_out((size_t)count * D * (depth + 1));
            hip_check(hipMemcpy(all.data(), layers_cap.p, all.size() * 4, hipMemcpyDeviceToHost), "read capture");
            for (size_t i = 0; i < count; ++i) {
                std::copy_n(&all[i * per + depth * D], D, &rows_out[i * D]);
                for (size_t l = 0; l < depth; ++l)
                    std::copy_n(&all[i * per + (l + 1) * D], D, &rows_out[((l + 1) * count + i) * D]);
            }
            append(o, rows_out);
        }
        // (tokens per compute batch, batches, tree updates, query positions)
        const std::vector<uint64_t> footer{1u, count, 0u, count};
        append(o, footer);
        reply(o);
    }

    // Up to count tokens (resident_math.comp:130: each readout's id is emitted, and a stop
    // id ends the stream without a forward of it); returns whether the stream goes on.
    bool generate(uint32_t count, uint32_t debug) {
        if (diagnostic_dirty) throw std::runtime_error("Attention diagnostics replace history; prefill again before generation");
        if (!prefilled || !count || count > 64) throw std::runtime_error("Resident generation expects 1..64 tokens after prefill");
        const auto t0 = std::chrono::steady_clock::now();
        Decoder& d = *dec;
        uint32_t ids[64] = {};
        uint32_t emitted = 0, computed = 0;
        const bool profiled = debug == 2u;
        if (profiled) profile.start(d.shape.layers);
        bool marked = false;   // a profiled step whose marks are not read yet
        Timer t;
        t.start(stream);
        while (emitted < count && control[2]) {
            uint32_t id = 0;
            hip_check(hipMemcpyAsync(&id, d.tokens.p, 4, hipMemcpyDeviceToHost, stream), "read token");
            hip_check(hipStreamSynchronize(stream), "sync");
            if (marked) profile.add(d.shape.layers, d.shape.full_every);
            marked = false;
            if (id >= info.vocab) throw std::runtime_error("Resident decode optical error 2048");
            ids[emitted++] = id;
            control[0] = id;
            ++position;
            if (id == control[4] || id == control[5]) {
                control[2] = 0;
                break;
            }
            d.step(stream, nullptr, profiled ? profile.marks.data() : nullptr);   // reads the pending id, leaves the next one
            marked = profiled;
            ++computed;
        }
        const double gpu = t.stop(stream);
        if (marked) profile.add(d.shape.layers, d.shape.full_every);
        uint32_t bits = 0;
        rta_check(rta_device_error(&bits, 1), "rta_device_error");
        if (bits) throw std::runtime_error("Resident decode optical error " + std::to_string(bits));
        control[1] = emitted;
        // GenerationPacket (optical_resident.cpp:57-71): timing, control, ids, hits, then
        // the telemetry / cache / recovery fields, here all zero
        std::vector<double> timing(18, 0.0);
        timing[0] = gpu;
        timing[1] = wall_ms(t0);
        timing[2] = timing[3] = (double)std::max(computed, 1u);
        timing[6] = (double)position;
        if (profiled) std::copy_n(profile.parts, 10, &timing[8]);
        std::vector<char> o;
        append(o, timing);
        append(o, control, 8);
        append(o, ids, 64);
        const uint32_t mlp = computed * info.depth * info.middle;
        const uint32_t hits[5] = {mlp, mlp, emitted * info.vocab, 0u, 0xffffffffu};
        append(o, hits, 5);
        if (debug == 1u) {   // the residual stream after the last layer of the latest step
            std::vector<float> st(info.hidden);
            hip_check(hipMemcpy(st.data(), d.last.p, st.size() * 4, hipMemcpyDeviceToHost), "read state");
            append(o, st);
        }
        append(o, std::vector<double>(4, 0.0));    // RT query time per kind
        append(o, std::vector<uint32_t>(4, 0u));   // cached tokens, cache queries, nodes, capacity
        append(o, std::vector<double>(2 + 3, 0.0));  // cache time; cached-state recovery
        append(o, std::vector<uint32_t>(2, 0u));   // cache candidates, rejected
        append(o, std::vector<uint64_t>(2, 0u));   // MLP route rows
        if (profiled) append(o, std::vector<double>{profile.detector[0], profile.detector[1]});
        reply(o);
        return control[2] != 0;
    }

    void stream_generate(uint32_t count, uint32_t debug) {
        if (!count || count > 64) throw std::runtime_error("Resident stream expects 1..64 tokens");
        for (uint32_t i = 0; i < count; ++i)
            if (!generate(1u, debug)) break;
    }

    // op 10: the history ring grows to `next` slots, the live history kept
    void grow(uint32_t next) {
        if (next <= capacity || next > 1048576u || capacity < 32u) throw std::runtime_error("Invalid tree growth request");
        const auto t0 = std::chrono::steady_clock::now();
        const uint32_t previous = capacity;
        if (dec) {
            if (prefilled) dec->grow(next, stream);
            else dec->allocate(next);
        }
        capacity = next;
        std::vector<char> o;
        append(o, std::vector<double>{(double)previous, (double)next, wall_ms(t0)});
        reply(o);
    }

    // op 13: no shared history cache is kept, so nothing is saved
    void finish_history() {
        std::vector<char> o;
        append(o, std::vector<uint64_t>{0u, 0u, 0u});
        append(o, std::vector<double>{0.0});
        reply(o);
    }

    void resources() {
        size_t free_b = 0, total_b = 0;
        hip_check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
        uint64_t uploaded = 0;
        for (auto& kv : uploads) uploaded += kv.second->n;
        std::vector<uint64_t> v(61, 0);
        v[0] = v[1] = total_b - free_b;      // allocation bytes (device)
        v[9] = uploaded;                      // packed coefficient bytes on the device
        v[11] = total_b - free_b;             // logical device buffer bytes
        v[13] = (uint64_t)full.size() * capacity * rta_history_bytes((int)(kv_heads * hd));
        v[26] = work_rows;
        v[37] = 0;                            // attention backend: standard
        v[38] = block;
        std::vector<char> o;
        append(o, v);
        reply(o);
    }
};

}  // namespace

int main(int argc, char** argv) {
    try {
        if (argc < 3) throw std::runtime_error("Usage: rt_optical_resident student.bin original_head.bin [capacity]");
        Worker w;
        w.capacity = argc > 3 ? (uint32_t)std::stoul(argv[3]) : 300u;
        if (!w.capacity || w.capacity > 1048576u) throw std::runtime_error("Invalid initial tree capacity");
        if (argc > 5 && std::string(argv[5]) == "sparse") throw std::runtime_error("Sparse routing is not provided by this worker");
        w.work_rows = argc > 11 ? (uint32_t)std::stoul(argv[11]) : 512u;
        if (w.work_rows < 32u || w.work_rows > 1024u || (w.work_rows & (w.work_rows - 1u)))
            throw std::runtime_error("Prefill batch requires a power of two in [32,1024]");
        const char* backend = std::getenv("RT_ATTENTION_BACKEND");
        if (backend && std::string(backend) != "standard")
            throw std::runtime_error("This worker provides the standard attention backend only");
        const char* mlp = std::getenv("RT_MLP_BACKEND");
        if (mlp && std::string(mlp) != "standard") throw std::runtime_error("This worker provides the standard MLP backend only");
        if (const char* b = std::getenv("RT_ATTENTION_BLOCK")) w.block = (uint32_t)std::stoul(b);
        if (w.block != 128u && w.block != 256u && w.block != 512u) throw std::runtime_error("Invalid attention history block");

        char err[256] = {};
        if (rta_asset_open(argv[1], argv[2], &w.asset, err, sizeof(err)) != RTA_OK) throw std::runtime_error(err);
        rta_check(rta_asset_get_info(w.asset, &w.info), "asset info");
        if (w.info.hidden % 256u) throw std::runtime_error("Invalid resident optical student");
        std::string dir(argv[1]);
        dir = dir.find('/') == std::string::npos ? std::string(".") : dir.substr(0, dir.find_last_of('/'));
        std::ifstream jf(dir + "/model.json");
        std::stringstream js;
        js << jf.rdbuf();
        w.json = js.str();
        const std::string& json = w.json;
        w.kv_heads = (uint32_t)spec_value(json, "kv_heads", 0, true);
        w.hd = (uint32_t)spec_value(json, "attention_head_dim", 0, true);
        w.heads = (uint32_t)spec_value(json, "attention_heads", 0, true);
        for (int l = 0; l < (int)w.info.depth; ++l) {
            uint32_t kind = 0, gate_desc = 0;
            rta_check(rta_asset_word(w.asset, l, 26, &kind), "asset word");
            if (kind == 1u) {
                w.full.push_back(l);
                rta_check(rta_asset_word(w.asset, l, 9 + 2 * 6 + 1, &gate_desc), "asset word");
                if ((gate_desc >> 8) == 2u) w.attention_gate = true;   // descriptor 6, mode 2 (export.py:98)
            }
        }
        hip_check(hipSetDevice(0), "hipSetDevice");
        hip_check(hipStreamCreate(&w.stream), "hipStreamCreate");
        // 0x5254523a: native token stream (op 9); mode: quantisation 4, full-matrix MLP
        // (4096), exact ordered detector (131072)
        const uint32_t hello[5] = {0x5254523au, w.info.depth, w.info.blocks, w.info.middle, 4u | 4096u | 131072u};
        std::cout.write(reinterpret_cast<const char*>(hello), 20);
        std::cout.flush();
        uint32_t op;
        while (std::cin.read(reinterpret_cast<char*>(&op), 4)) {
            if (!op) break;
            uint32_t count, debug;
            if (!std::cin.read(reinterpret_cast<char*>(&count), 4) || !std::cin.read(reinterpret_cast<char*>(&debug), 4))
                throw std::runtime_error("Incomplete resident request");
            if (op == 1 || op == 11 || op == 12) w.prefill(count, debug, op == 12 ? 2u : op == 11 ? 1u : 0u);
            else if (op == 2) w.generate(count, debug);
            else if (op == 4) w.word_check();
            else if (op == 6) w.mlp_check(count, debug);
            else if (op == 8) w.resources();
            else if (op == 9) w.stream_generate(count, debug);
            else if (op == 10) w.grow(count);
            else if (op == 13) w.finish_history();
            else if (op == 14) {
                w.diagnostic_dirty = true;   // (resident_attention_runtime.inl:657)
                w.attention_check(count, debug);
            } else {
                throw std::runtime_error("Unknown resident operation");
            }
        }
        hip_check(hipStreamDestroy(w.stream), "hipStreamDestroy");
        return 0;
    } catch (const std::exception& e) {
        std::cerr << e.what() << std::endl;
        return 1;
    }
}
