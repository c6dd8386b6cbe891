// rta_ceiling.hip -- measurement support, not part of the detector path: the
// achievable HBM read rate of this GPU, against which the readouts' rates are set.
//
// stream_read_kernel<U, NT> reads a buffer once with 16-byte loads, U independent loads
// in flight per thread and loop trip (grid-stride), non-temporal when NT, and folds the
// words with xor so that no load can be dropped; each block writes its fold to
// out[blockIdx.x].  Built as its own library (lib/librta_ceiling.so) and called by the
// benchmark only, which takes the best rate over the variants and grid sizes.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

using u32x4 = uint32_t __attribute__((ext_vector_type(4)));

template <int U, bool NT>
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4* __restrict__ p, int64_t n16,
                                                          uint32_t* __restrict__ out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = NT ? __builtin_nontemporal_load(p + i + u * stride) : p[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 a = p[i];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= __shfl_xor(acc, off, 64);
    __shared__ uint32_t red[4];
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] ^ red[1] ^ red[2] ^ red[3];
}

}  // namespace

extern "C" {

// Reads bytes (a multiple of 16, 16-byte aligned) of buf once on the stream with variant
// 0 (4 loads per trip), 1 (8 loads), 2 (4 non-temporal loads) or 3 (8 non-temporal
// loads); out holds blocks words.  0 on success, 2 on a bad argument, 5 on a launch error.
int rta_ceiling_stream_read(const void* buf, int64_t bytes, uint32_t* out, int blocks, int variant, void* stream) {
    if (!buf || !out || bytes <= 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(buf) & 15) || blocks <= 0 ||
        blocks > 65536 || variant < 0 || variant > 3)
        return 2;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const u32x4* p = static_cast<const u32x4*>(buf);
    const int64_t n16 = bytes / 16;
    switch (variant) {
    case 0: hipLaunchKernelGGL((stream_read_kernel<4, false>), dim3(blocks), dim3(256), 0, s, p, n16, out); break;
    case 1: hipLaunchKernelGGL((stream_read_kernel<8, false>), dim3(blocks), dim3(256), 0, s, p, n16, out); break;
    case 2: hipLaunchKernelGGL((stream_read_kernel<4, true>), dim3(blocks), dim3(256), 0, s, p, n16, out); break;
    default: hipLaunchKernelGGL((stream_read_kernel<8, true>), dim3(blocks), dim3(256), 0, s, p, n16, out); break;
    }
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

}  // extern "C"
