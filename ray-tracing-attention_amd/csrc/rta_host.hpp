// rta_host.hpp -- host-side argument helpers shared by the C ABI translation units.
#pragma once
#include <stdint.h>

#include "../../include/rta.h"

namespace rta {
namespace host {

inline bool valid_format(int fmt) {
    return fmt == RTA_F32 || fmt == RTA_F16 || fmt == RTA_BF16 || fmt == RTA_Q4_K || fmt == RTA_Q6_K;
}

// Bytes of one row of `cols` values (resident_quant.glsl:28-30: 144 / 210 bytes
// per 256 values for Q4_K / Q6_K).
inline int64_t row_bytes(int fmt, int64_t cols) {
    if (cols < 0) return -1;
    switch (fmt) {
    case RTA_F32: return cols * 4;
    case RTA_F16:
    case RTA_BF16: return cols * 2;
    case RTA_Q4_K: return cols % 256 ? -1 : (cols / 256) * 144;
    case RTA_Q6_K: return cols % 256 ? -1 : (cols / 256) * 210;
    default: return -1;
    }
}

// resident_dimensions.hpp:10 -- roundup8(ceil(kvw/256) * (144 + 210)).
inline int64_t history_bytes(int kvw) {
    if (kvw <= 0) return -1;
    const int64_t blocks = (kvw + 255) / 256;
    return (blocks * (144 + 210) + 7) / 8 * 8;
}

inline bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

// Argument checks of a table lookup (op 0): RTA_OK and the table's row bytes in *rb, or
// the error code.
inline int embed_args(int fmt, const void* table, int vocab, int hidden, const uint32_t* ids, int batch,
                      const float* out, int64_t* rb) {
    if (!valid_format(fmt)) return RTA_ERR_FORMAT;
    if (!table || !ids || !out) return RTA_ERR_NULL;
    *rb = row_bytes(fmt, hidden);
    if (vocab <= 0 || hidden <= 0 || batch <= 0 || *rb <= 0) return RTA_ERR_SHAPE;
    if (!aligned(table, fmt == RTA_F32 || fmt == RTA_Q4_K ? 4 : 2) || !aligned(out, 4) || !aligned(ids, 4))
        return RTA_ERR_ALIGN;
    return RTA_OK;
}

}  // namespace host
}  // namespace rta
