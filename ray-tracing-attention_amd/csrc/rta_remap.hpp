// rta_remap.hpp -- the reference's row/axis remap of a projection matrix
// (resident_quant.glsl:20-31 quantizedWeight, :53-58 quantizedOctet; the mode is the
// descriptor's metadata >> 8, set by compiler/export.py:96-98,108).
//
// Logical row r of the projection reads GGUF row source_row(r); with mode 4 logical
// axis a reads GGUF column source_axis(a).  rot(i) = originalRotaryAxis
// (resident_quant.glsl:20) sends the rotary-pair layout the detector works in
// (pair p = axes 2p, 2p + 1) back to the exporter's half-split layout (p, p + R/2).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rta.h"

namespace rta {

struct Remap {
    int mode = RTA_REMAP_NONE;
    int hd = 0;       // attention head dim (RT_ATTENTION_HEAD_DIM)
    int rotary = 0;   // rotary dim R <= hd (RT_ROTARY_DIM)
    int key_rows = 0; // state key heads x 128 (mode 5)

    __host__ __device__ int rot(int i) const { return i < rotary ? (i & 1) * (rotary >> 1) + (i >> 1) : i; }
    // inverse of rot: the logical axis whose source is column i of a head
    __host__ __device__ int rot_inv(int i) const {
        return i < rotary ? (i < (rotary >> 1) ? 2 * i : 2 * (i - (rotary >> 1)) + 1) : i;
    }
    __host__ __device__ int64_t source_row(int64_t r) const {
        switch (mode) {
        case RTA_REMAP_QUERY:
        case RTA_REMAP_GATE:
            return (r / hd) * (2 * (int64_t)hd) + (mode == RTA_REMAP_GATE ? hd : 0) + rot((int)(r % hd));
        case RTA_REMAP_ROTARY: return (r / hd) * (int64_t)hd + rot((int)(r % hd));
        case RTA_REMAP_KEY_REPEAT: return r % key_rows;
        default: return r;
        }
    }
    // the row mode moves rows (else identity rows)
    __host__ __device__ bool moves_rows() const {
        return mode == RTA_REMAP_QUERY || mode == RTA_REMAP_GATE || mode == RTA_REMAP_ROTARY ||
               mode == RTA_REMAP_KEY_REPEAT;
    }
};

}  // namespace rta
