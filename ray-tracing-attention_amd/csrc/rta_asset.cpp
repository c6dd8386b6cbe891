// Reader of the reference's on-disk assets (host code, no device work):
//   optical_model.bin   "RTRES004", 9 header words {hidden, depth, blocks, middle, vocab,
//                       quantization (4), parameter words, matrix words, step}, then the
//                       parameter words: a 32-word model header, 64 words per layer, then
//                       the fp32 vectors those words point at (ray_tracing/compiler/export.py:68-73,
//                       136-138);
//   geometry_weights.bin the raw GGUF payloads of every layer, each padded to a word,
//                       located by the per-layer descriptors (export.py:75-91, 123);
//   vocabulary.bin      "RTBASQ01", {vocab, hidden}, then the raw token_embd / output
//                       payloads (export.py:127-135), located by model header words 13-16.
// Validation follows the reference worker's loader (ray_tracing/native/src/optical_resident.cpp:139-152);
// the compile-time shape checks it makes against its generated constants are left to
// the caller, who compares rta_asset_info with its own model spec.
#include <cstdio>
#include <cstring>
#include <exception>
#include <fstream>
#include <memory>
#include <string>
#include <vector>

#include "../../include/rta.h"

struct rta_asset {
    uint32_t hdr[9] = {};
    std::vector<uint32_t> params;     // parameter words (model header, layer headers, vectors)
    std::vector<uint32_t> matrices;   // geometry_weights.bin
    std::vector<uint32_t> basis;      // vocabulary.bin after its 16-byte header
};

namespace {

constexpr uint32_t kModelWords = 32, kLayerWords = 64;

int fail(char* err, size_t err_len, const char* msg) {
    if (err && err_len) std::snprintf(err, err_len, "%s", msg);
    return RTA_ERR_FORMAT;
}

// Reads `bytes` bytes into dst in pieces of at most 64 MiB; false if the file ends first.
bool read_all(std::ifstream& f, void* dst, size_t bytes) {
    char* p = static_cast<char*>(dst);
    for (size_t off = 0; off < bytes;) {
        const size_t n = std::min<size_t>(size_t(64) << 20, bytes - off);
        f.read(p + off, (std::streamsize)n);
        if (!f) return false;
        off += n;
    }
    return true;
}

uint64_t file_bytes(const char* path) {
    std::ifstream f(path, std::ios::binary | std::ios::ate);
    return f ? (uint64_t)f.tellg() : 0;
}

std::string sibling(const char* path, const char* name) {
    std::string s(path);
    const size_t cut = s.find_last_of('/');
    return (cut == std::string::npos ? std::string() : s.substr(0, cut + 1)) + name;
}

int asset_open(const char* model_path, const char* vocabulary_path, rta_asset** out, char* err, size_t err_len);

}  // namespace

// No exception leaves the C ABI: a header whose sizes cannot be allocated is reported
// like any other damaged file.
extern "C" int rta_asset_open(const char* model_path, const char* vocabulary_path, rta_asset** out, char* err,
                              size_t err_len) {
    if (!model_path || !out) return RTA_ERR_NULL;
    *out = nullptr;
    try {
        return asset_open(model_path, vocabulary_path, out, err, err_len);
    } catch (const std::exception&) {
        return fail(err, err_len, "Invalid resident optical student");
    }
}

namespace {
int asset_open(const char* model_path, const char* vocabulary_path, rta_asset** out, char* err, size_t err_len) {
    std::unique_ptr<rta_asset> a(new rta_asset());
    auto bad = [&](const char* msg) { return fail(err, err_len, msg); };
    std::ifstream in(model_path, std::ios::binary);
    char magic[8];
    in.read(magic, 8);
    in.read(reinterpret_cast<char*>(a->hdr), sizeof(a->hdr));
    const uint32_t* h = a->hdr;
    // optical_resident.cpp:140: magic, quantization 4, depth > 0, 0 < blocks <= depth, middle % 32
    if (!in || std::memcmp(magic, "RTRES004", 8) || h[5] != 4u || !h[1] || !h[2] || h[2] > h[1] || h[3] % 32u ||
        !h[0] || !h[4])
        return bad("Invalid resident optical student");
    if (h[6] < kModelWords + uint64_t(h[1]) * kLayerWords) return bad("Invalid resident optical student");
    // sizes are checked against the files before anything is allocated
    if (file_bytes(model_path) < 44 + uint64_t(h[6]) * 4) return bad("Truncated resident parameters");
    a->params.resize(h[6]);
    if (!read_all(in, a->params.data(), a->params.size() * 4)) return bad("Truncated resident parameters");
    {
        const std::string geo = sibling(model_path, "geometry_weights.bin");
        if (file_bytes(geo.c_str()) < uint64_t(h[7]) * 4) return bad("Truncated geometric weights");
        std::ifstream mf(geo, std::ios::binary);
        a->matrices.resize(h[7]);
        if (!mf || !read_all(mf, a->matrices.data(), a->matrices.size() * 4)) return bad("Truncated geometric weights");
    }
    if (a->params[11] != 1u) return bad("Complete equivalent optical translation required");
    // every layer's matrix range lies in the file (the reference binds it unchecked)
    for (uint32_t l = 0; l < h[1]; ++l) {
        const uint32_t* lh = a->params.data() + kModelWords + l * kLayerWords;
        if (uint64_t(lh[27]) + lh[28] > h[7]) return bad("Truncated geometric weights");
    }
    if (vocabulary_path) {
        std::ifstream vf(vocabulary_path, std::ios::binary | std::ios::ate);
        if (!vf) return bad("Complete model vocabulary basis required");
        const uint64_t size = (uint64_t)vf.tellg();
        vf.seekg(0);
        char bm[8];
        uint32_t shape[2];
        vf.read(bm, 8);
        vf.read(reinterpret_cast<char*>(shape), 8);
        if (!vf || std::memcmp(bm, "RTBASQ01", 8) || shape[0] != h[4] || shape[1] != h[0])
            return bad("Complete model vocabulary basis required");
        a->basis.resize((size - 16) / 4);
        if (!read_all(vf, a->basis.data(), a->basis.size() * 4)) return bad("Truncated original word basis");
    }
    *out = a.release();
    return RTA_OK;
}
}  // namespace

extern "C" void rta_asset_close(rta_asset* a) { delete a; }

extern "C" int rta_asset_get_info(const rta_asset* a, rta_asset_info* info) {
    if (!a || !info) return RTA_ERR_NULL;
    const uint32_t* h = a->hdr;
    info->hidden = h[0];
    info->depth = h[1];
    info->blocks = h[2];
    info->middle = h[3];
    info->vocab = h[4];
    info->quantization = h[5];
    info->step = h[8];
    info->param_words = a->params.size();
    info->matrix_words = a->matrices.size();
    info->basis_words = a->basis.size();
    info->fmt_embed = a->params[13];
    info->fmt_lm = a->params[15];
    info->embed_offset_words = a->params[14];
    info->lm_offset_words = a->params[16];
    return RTA_OK;
}

extern "C" const uint32_t* rta_asset_params(const rta_asset* a, uint64_t* words) {
    if (!a) return nullptr;
    if (words) *words = a->params.size();
    return a->params.data();
}

// Descriptor `index` of a layer: words base+9+2i, base+10+2i (index 8: base+32, base+33),
// the first a word offset into the layer's matrix range, the second code | mode << 8
// (export.py:87-91).  Indices 9 and 10 are the delta-net's ssm_beta / ssm_alpha payloads,
// whose offset and code sit in words 35 / 39 and 36 / 40 (export.py:113), with no mode.
// An index the exporter never set reads code 0 at offset 0.
extern "C" int rta_asset_layer_matrix(const rta_asset* a, int layer, int index, rta_asset_matrix* out) {
    if (!a || !out) return RTA_ERR_NULL;
    if (layer < 0 || (uint32_t)layer >= a->hdr[1] || index < 0 || index > 10) return RTA_ERR_RANGE;
    const uint32_t* lh = a->params.data() + kModelWords + (uint32_t)layer * kLayerWords;
    const bool separate = index >= 9;
    const uint32_t at = separate ? 26u + (uint32_t)index : index == 8 ? 32u : 9u + 2u * (uint32_t)index;
    const uint32_t code = separate ? lh[at + 4] : lh[at + 1];
    const uint64_t start = lh[27], words = lh[28], off = lh[at];
    if (off > words) return RTA_ERR_RANGE;
    out->data = a->matrices.data() + start + off;
    out->offset_words = start + off;
    out->avail_bytes = (words - off) * 4;
    out->fmt = separate ? code : code & 0xFFu;
    out->mode = separate ? 0u : code >> 8;
    return RTA_OK;
}

// fp32 vector of `count` values whose parameter-word offset is at word `field` of the
// layer header (layer -1: the model header), e.g. field 0 attn_norm, 1 post_attention_norm
// (export.py:92), 24/25 the q/k norms (:102-104), 4 of the model header output_norm (:73).
extern "C" int rta_asset_vector(const rta_asset* a, int layer, int field, uint64_t count, const float** out) {
    if (!a || !out) return RTA_ERR_NULL;
    if (layer < -1 || layer >= (int)a->hdr[1] || field < 0 || field >= (int)kLayerWords ||
        (layer < 0 && field >= (int)kModelWords))
        return RTA_ERR_RANGE;
    const uint32_t base = layer < 0 ? 0u : kModelWords + (uint32_t)layer * kLayerWords;
    const uint64_t off = a->params[base + (uint32_t)field];
    const uint64_t words = a->params.size();
    if (off > words || count > words - off) return RTA_ERR_RANGE;   // no wrap for any count
    *out = reinterpret_cast<const float*>(a->params.data() + off);
    return RTA_OK;
}

// Word `field` of a layer header (layer -1: the model header), e.g. 23 the head count,
// 26 the layer kind (1 full, 2 recurrent), 29 the rotary dimension (export.py:105,120,122).
extern "C" int rta_asset_word(const rta_asset* a, int layer, int field, uint32_t* value) {
    if (!a || !value) return RTA_ERR_NULL;
    if (layer < -1 || layer >= (int)a->hdr[1] || field < 0 || field >= (int)kLayerWords ||
        (layer < 0 && field >= (int)kModelWords))
        return RTA_ERR_RANGE;
    *value = a->params[(layer < 0 ? 0u : kModelWords + (uint32_t)layer * kLayerWords) + (uint32_t)field];
    return RTA_OK;
}

// Raw payload of token_embd (which 0) or output (which 1) in vocabulary.bin: model header
// words 13/14 and 15/16 hold the code and the word offset (export.py:129-135).
extern "C" int rta_asset_basis(const rta_asset* a, int which, rta_asset_matrix* out) {
    if (!a || !out) return RTA_ERR_NULL;
    if (which != 0 && which != 1) return RTA_ERR_RANGE;
    const uint64_t off = a->params[which ? 16 : 14];
    if (off > a->basis.size()) return RTA_ERR_RANGE;
    out->data = a->basis.data() + off;
    out->offset_words = off;
    out->avail_bytes = (a->basis.size() - off) * 4;
    out->fmt = a->params[which ? 15 : 13];
    out->mode = 0;
    return RTA_OK;
}
