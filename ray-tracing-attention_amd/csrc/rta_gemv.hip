// rta_gemv.hip -- C ABI for dequantisation, projections, the SwiGLU MLP and the
// LM-head readout with fused margin argmax (gfx950).
#include <math.h>

#include <climits>
#include "rta_gemm.hpp"
#include "rta_packed.hpp"
#include "rta_remap.hpp"
#include "rta_gemv.hpp"
#include "rta_host.hpp"
#include "rta_internal.hpp"

namespace rta {

__device__ uint32_t g_error_word = 0;

// ---------------------------------------------------------------- dequant ----
// One thread per value, the reference's per-value decoder with its fp32 op order
// (resident_quant.glsl:6-20): contraction is disabled so that (d*sc)*q - dmin*m is
// rounded exactly as the reference rounds it.
__global__ void __launch_bounds__(256) dequant_kernel(int fmt, const uint8_t* __restrict__ src, int64_t n,
                                                      float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    out[i] = dequant_value(fmt, src, i);
}

// ------------------------------------------------------------------ argmax ----
// Phase two of the readout: M = max of the per-task maxima (exact logit values),
// T = M - margin*|M| evaluated in fp32 without contraction, id = lowest v with
// logit >= T.  The first task whose maximum reaches T holds that id, so only its
// rows are scanned (in parallel).  Generalises the
// reference's reduction (resident_math.comp:124-130: strict >, ties -> lower id).
constexpr int kArgmaxThreads = 1024;   // one block per batch row scans the task maxima

// Maxima of groups of 64 task maxima (wave g of the grid: group g of batch row
// blockIdx.y), so that the argmax over many small tasks scans 64 times fewer values.
__global__ void __launch_bounds__(256) group_max_kernel(const float* __restrict__ partial, int ntasks, int ngroups,
                                                        float* __restrict__ gmax) {
    const int g = blockIdx.x * 4 + (threadIdx.x >> 6), b = blockIdx.y, lane = threadIdx.x & 63;
    if (g >= ngroups) return;   // uniform per wave
    const int t = g * kWave + lane;
    float m = t < ntasks ? partial[(int64_t)b * ntasks + t] : -INFINITY;
    m = group_max(m, kWave);
    if (lane == 0) gmax[(int64_t)b * ngroups + g] = m;
}

__global__ void __launch_bounds__(kArgmaxThreads) argmax_margin_kernel(const float* __restrict__ logits, int vocab,
                                                            const float* __restrict__ partial, int ntasks,
                                                            int rows_per_task, float margin,
                                                            uint32_t* __restrict__ ids,
                                                            const float* __restrict__ gmax, int ngroups) {
#pragma clang fp contract(off)
    constexpr int kW = kArgmaxThreads / 64;
    __shared__ float red_f[kW];
    __shared__ int red_i[kW];
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float* pb = partial + (int64_t)b * ntasks;
    const float* lb = logits + (int64_t)b * vocab;
    // with group maxima (gmax), steps 1 and 2 run over the groups and step 2 then picks
    // the first task of the first group reaching T: the same task
    const float* gb = gmax ? gmax + (int64_t)b * ngroups : pb;
    const int nscan = gmax ? ngroups : ntasks;
    // 1. M = max over the task (group) maxima
    float m = -INFINITY;
#pragma unroll 8
    for (int t = tid; t < nscan; t += kArgmaxThreads) m = fmaxf(m, gb[t]);
    m = group_max(m, kWave);
    if (lane == 0) red_f[wave] = m;
    __syncthreads();
    float M = red_f[0];
#pragma unroll
    for (int i = 1; i < kW; ++i) M = fmaxf(M, red_f[i]);
    if (!(M > -INFINITY)) {
        if (tid == 0) ids[b] = 0xffffffffu;
        return;
    }
    const float mag = fabsf(M);
    const float slack = margin * mag;
    const float T = M - slack;
    // 2. the first task whose maximum reaches T holds the lowest index with logit >= T
    int first = INT_MAX;   // branch-free so that the loads of a thread overlap
#pragma unroll 8
    for (int t = tid; t < nscan; t += kArgmaxThreads) first = (gb[t] >= T && t < first) ? t : first;
    first = wave_min_int(first);
    if (lane == 0) red_i[wave] = first;
    __syncthreads();
    first = red_i[0];
#pragma unroll
    for (int i = 1; i < kW; ++i) first = min(first, red_i[i]);
    __syncthreads();
    if (first == INT_MAX) {   // only with NaN logits
        if (tid == 0) ids[b] = 0xffffffffu;
        return;
    }
    if (gmax) {   // the first task of group `first` reaching T (the group's maximum does)
        const int t = first * kWave + lane;
        const bool hit = t < ntasks && pb[t] >= T;
        const uint64_t mask = __builtin_amdgcn_ballot_w64(hit);
        first = first * kWave + (mask ? (int)__builtin_ctzll(mask) : 0);
    }
    // 3. lowest row of that task with logit >= T
    const int r0 = first * rows_per_task, r1 = min(r0 + rows_per_task, vocab);
    int best = INT_MAX;
#pragma unroll 4
    for (int r = r0 + tid; r < r1; r += kArgmaxThreads) best = (lb[r] >= T && r < best) ? r : best;
    best = wave_min_int(best);
    if (lane == 0) red_i[wave] = best;
    __syncthreads();
    if (tid == 0) {
        for (int i = 1; i < kW; ++i) best = min(best, red_i[i]);
        ids[b] = (uint32_t)min(best, red_i[0]);
    }
}

// ----------------------------------------------------------- launch plumbing ----
// y[b, r] (=|+=) ys[b, m.source_row(r)]: the gather epilogue of a row-remapped
// projection, ys [batch, ld] holding the readout of every source row once.
template <bool ACC>
__global__ void __launch_bounds__(256) remap_gather_kernel(const float* __restrict__ ys, int ld, int rows, int batch,
                                                           const Remap m, float* __restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)rows * batch) return;
    const int64_t b = i / rows, r = i - b * rows;
    const float v = ys[b * ld + m.source_row(r)];
    if (ACC) y[i] += v;
    else y[i] = v;
}

// xp[b, j] = x[b, a] for the logical axis a whose source column is j (mode 4):
// sum_a W[r, src(a)] x[a] = sum_j W[r, j] xp[j].
__global__ void __launch_bounds__(256) remap_axes_kernel(const float* __restrict__ x, int cols, int batch,
                                                         const Remap m, float* __restrict__ xp) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)cols * batch) return;
    const int64_t b = i / cols;
    const int j = (int)(i - b * cols), h = j / m.hd;
    xp[i] = x[b * cols + (int64_t)h * m.hd + m.rot_inv(j - h * m.hd)];
}

static int pow2ceil(int v) {
    int p = 1;
    while (p < v) p <<= 1;
    return p;
}

static bool is_kquant(int fmt) { return fmt == RTA_Q4_K || fmt == RTA_Q6_K; }

constexpr int kPlanCUs = 256;      // CUs the work split is planned for (MI355X)

struct Plan {
    bool b1;          // batch-1 kernel
    int nb, r, kw, lpr, ntasks, grid, block, rows_per_task;
};

// Launch plan of one K-quant projection over `batch` (<= 8) x rows; row_bytes of one
// matrix row (both matrices' rows are streamed in the dual case).
static Plan plan_kquant(int rows, int cols, int batch, bool dual, int64_t row_bytes) {
    Plan p{};
    const int S = cols / 64;
    p.b1 = batch == 1 && S <= 4 * kWave;
    if (p.b1) {
        p.nb = 1;
        p.r = dual ? 1 : 2;
        p.kw = S <= kWave ? 1 : (S + kWave - 1) / kWave;
        p.lpr = S >= kWave ? kWave : pow2ceil(S);
        p.rows_per_task = (kWave / p.lpr) * p.r;
        p.ntasks = (rows + p.rows_per_task - 1) / p.rows_per_task;
        const int groups = p.kw == 3 ? 1 : 4 / p.kw;
        p.block = p.kw == 3 ? 192 : 256;
        const int blocks = (p.ntasks + groups - 1) / groups;
        // Every block stages x (cols x 4 B) once and then streams its tasks: the grid keeps
        // that traffic near an eighth of the weights' bytes, within 3 to 8 blocks per CU
        // (measured: 4096x12288 down 14.5 -> 11.1 us at 768 blocks, 151936x2048 LM head
        // 58 us at 2048 and 65 us at 768).
        const int64_t wbytes = (int64_t)rows * row_bytes * (dual ? 2 : 1);
        int64_t cap = wbytes / (8 * (int64_t)cols * 4);
        cap = cap < 3 * kPlanCUs ? 3 * kPlanCUs : cap > 8 * kPlanCUs ? 8 * kPlanCUs : cap;
        p.grid = blocks < cap ? blocks : (int)cap;
        return p;
    }
    p.nb = batch <= 1 ? 1 : batch <= 2 ? 2 : batch <= 4 ? 4 : 8;
    p.r = p.nb >= 8 ? 2 : 4;
    if (dual) p.r = p.r / 2 > 0 ? p.r / 2 : 1;
    p.kw = 1;
    p.lpr = S >= kWave ? kWave : pow2ceil(S);
    p.rows_per_task = (kWave / p.lpr) * p.r;
    p.ntasks = (rows + p.rows_per_task - 1) / p.rows_per_task;
    const int wgs = (p.ntasks + 3) / 4;
    p.grid = wgs < 2048 ? wgs : 2048;
    p.block = 256;
    return p;
}

struct Launch {
    const uint8_t* w;
    const uint8_t* w2;
    int64_t row_bytes;
    int rows, cols;
    const float* x;
    float* y;
    float* partial;
    int batch;
    RowNorm rn;   // packed readouts only
    XNorm xn;     // batch-1 readouts only
};

template <int FMT, int R, int MODE, int KW>
static void launch_b1(const Plan& p, const Launch& l, hipStream_t s) {
    const size_t lds = b1_lds_bytes(l.cols / 64);
    if (lds > 65536) {   // above the default dynamic LDS limit (at most 16384 columns: 68 KB)
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&gemv_b1_kernel<FMT, R, MODE, KW>),
            hipFuncAttributeMaxDynamicSharedMemorySize, b1_lds_bytes(4 * kWave));
        (void)attr;   // a failure surfaces as the launch error
    }
    hipLaunchKernelGGL((gemv_b1_kernel<FMT, R, MODE, KW>), dim3(p.grid), dim3(p.block), lds, s, l.w, l.w2,
                       l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, p.lpr, p.ntasks, l.xn.w, l.xn.eps);
}

template <int FMT, int MODE, int R>
static void launch_b1_kw(const Plan& p, const Launch& l, hipStream_t s) {
    switch (p.kw) {
    case 1: launch_b1<FMT, R, MODE, 1>(p, l, s); break;
    case 2: launch_b1<FMT, R, MODE, 2>(p, l, s); break;
    case 3: launch_b1<FMT, R, MODE, 3>(p, l, s); break;
    default: launch_b1<FMT, R, MODE, 4>(p, l, s); break;
    }
}

template <int FMT, int MODE>
static void launch_kquant_fmt(const Plan& p, const Launch& l, hipStream_t s) {
    if (p.b1) {
        if (p.r == 1) launch_b1_kw<FMT, MODE, 1>(p, l, s);
        else launch_b1_kw<FMT, MODE, 2>(p, l, s);
        return;
    }
    const dim3 g(p.grid), b(256);
    constexpr bool dual = MODE == kSwiglu;
    switch (p.nb) {
    case 1: hipLaunchKernelGGL((gemv_kquant_kernel<FMT, 1, dual ? 2 : 4, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch, p.lpr, p.ntasks); break;
    case 2: hipLaunchKernelGGL((gemv_kquant_kernel<FMT, 2, dual ? 2 : 4, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch, p.lpr, p.ntasks); break;
    case 4: hipLaunchKernelGGL((gemv_kquant_kernel<FMT, 4, dual ? 2 : 4, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch, p.lpr, p.ntasks); break;
    default: hipLaunchKernelGGL((gemv_kquant_kernel<FMT, 8, dual ? 1 : 2, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch, p.lpr, p.ntasks); break;
    }
}

template <int MODE>
static hipError_t launch_kquant(int fmt, const Plan& p, const Launch& l, hipStream_t s) {
    if (fmt == RTA_Q4_K) launch_kquant_fmt<RTA_Q4_K, MODE>(p, l, s);
    else launch_kquant_fmt<RTA_Q6_K, MODE>(p, l, s);
    return hipGetLastError();
}

template <int MODE>
static hipError_t launch_plain(int fmt, const Launch& l, int grid, hipStream_t s) {
    const dim3 g(grid), b(256);
    if (fmt == RTA_F32) hipLaunchKernelGGL((gemv_plain_kernel<RTA_F32, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch);
    else if (fmt == RTA_F16) hipLaunchKernelGGL((gemv_plain_kernel<RTA_F16, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch);
    else hipLaunchKernelGGL((gemv_plain_kernel<RTA_BF16, MODE>), g, b, 0, s, l.w, l.w2, l.row_bytes, l.rows, l.cols, l.x, l.y, l.partial, l.batch);
    return hipGetLastError();
}

static bool is_tiled(int fmt) { return fmt == (RTA_Q4_K | kTiled) || fmt == (RTA_Q6_K | kTiled); }

static int check_matrix(int fmt, const void* w, int rows, int cols) {
    if (is_tiled(fmt)) {   // packed by rta_pack: 16-byte aligned tiles
        if (!w) return RTA_ERR_NULL;
        if (rows <= 0 || cols <= 0 || cols % 256) return RTA_ERR_SHAPE;
        return reinterpret_cast<uintptr_t>(w) % 16 ? RTA_ERR_ALIGN : RTA_OK;
    }
    if (!host::valid_format(fmt)) return RTA_ERR_FORMAT;
    if (!w) return RTA_ERR_NULL;
    if (rows <= 0 || cols <= 0) return RTA_ERR_SHAPE;
    if (is_kquant(fmt) && cols % 256) return RTA_ERR_SHAPE;
    if (!is_kquant(fmt) && cols % 4) return RTA_ERR_SHAPE;
    const uintptr_t p = reinterpret_cast<uintptr_t>(w);
    const uintptr_t need = fmt == RTA_Q4_K ? 16 : fmt == RTA_F32 ? 4 : 2;
    if (p % need) return RTA_ERR_ALIGN;
    return RTA_OK;
}

// ------------------------------------------------------------ MFMA path ----
// Whether a GGUF-row K-quant readout of `weights` values (rows x cols, both matrices of a
// SwiGLU pair) over `batch` rows runs on the matrix cores rather than the vector ALUs.
// Measured per call on MI355X against the vector-ALU kernel (gemv_kquant_kernel, batch
// tiles of up to 8 rows), row layout:
//   4096x4096 Q4_K      b2 9.5 / 19.6 us, b3 12.5 / 19.8, b4 14.3 / 20.0, b5 24.3 / 19.9
//   12288x4096 Q4_K     b2 20.1 / 27.0, b3 27.4 / 27.3, b4 32.8 / 27.3, b5 61.2 / 27.5
//   151936x2048 Q6_K LM head   b2 101.7 / 90.4, b4 154.5 / 90.7, b5 228.9 / 90.6,
//                              b16 638.6 / 91.7 (vector ALUs: 135 M VALU instructions)
//   SwiGLU MLP 2048x6144 (config 2)   b4 46.4 / 42.1, b8 78.7 / 43.8, b32 307.9 / 50.9
// The vector path issues NB fma per weight and batch tile, so its time grows with the
// batch; the matrix cores' does not up to 32 rows.
constexpr int64_t kMmaAnyWeights = 0;               // from batch 5: every matrix
constexpr int64_t kMmaMidWeights = 32ll << 20;      // from batch 3
constexpr int64_t kMmaTallWeights = 128ll << 20;    // from batch 2
__host__ __device__ constexpr bool mma_batch(int64_t weights, int batch) {
    return (batch >= 5 && weights >= kMmaAnyWeights) || (batch >= 3 && weights >= kMmaMidWeights) ||
           (batch >= 2 && weights >= kMmaTallWeights);
}
constexpr int kMfmaRT = 2;         // 16-row tiles per wave

struct MmaPlan {
    int nbt, total_rows, ntg, nslab, sb_per_slab, wgs_per_slab, grid;
    size_t x_bytes, part_bytes;
};

// Work split of one projection over a batch tile: K slabs that fit the LDS, doubled
// while the (tile, slab) units would leave waves idle.  Independent of the device so
// that workspace sizes are host queries.
static MmaPlan plan_mfma(int rows, int cols, int nbt, bool dual) {
    MmaPlan p{};
    p.nbt = nbt;
    p.total_rows = dual ? 2 * rows : rows;
    p.ntg = (p.total_rows + 16 * kMfmaRT - 1) / (16 * kMfmaRT);
    const int nsbt = cols / 256;
    const int sbmax = kSlabRowSb / (16 * nbt);
    int nslab = (nsbt + sbmax - 1) / sbmax;
    while (nslab < nsbt && (int64_t)p.ntg * nslab < (int64_t)kPlanCUs * kGemmWaves) nslab *= 2;
    if (nslab > nsbt) nslab = nsbt;
    p.sb_per_slab = (nsbt + nslab - 1) / nslab;
    p.nslab = (nsbt + p.sb_per_slab - 1) / p.sb_per_slab;
    int wps = (kPlanCUs + p.nslab - 1) / p.nslab;
    const int need = (p.ntg + kGemmWaves - 1) / kGemmWaves;
    p.wgs_per_slab = wps < need ? wps : need;
    p.grid = p.nslab * p.wgs_per_slab;
    p.x_bytes = (size_t)kMaxBatchTile * cols * 2 * 2                 // hi, lo
              + (size_t)kMaxBatchTile * nsbt * 64                    // group-sum operands
              + (size_t)kMaxBatchTile * nsbt * sizeof(float);        // 1 / scale
    p.x_bytes = (p.x_bytes + 255) & ~(size_t)255;
    p.part_bytes = p.nslab > 1 ? (size_t)p.nslab * kMaxBatchTile * p.total_rows * sizeof(float) : 0;
    return p;
}

static GemmX carve_x(void* ws, int cols) {
    uint8_t* b = static_cast<uint8_t*>(ws);
    GemmX x;
    const size_t n = (size_t)kMaxBatchTile * cols;
    const size_t nsbt = cols / 256;
    x.hi = reinterpret_cast<_Float16*>(b);
    x.lo = reinterpret_cast<_Float16*>(b + 2 * n);
    x.g = reinterpret_cast<h8_t*>(b + 4 * n);
    x.inv = reinterpret_cast<float*>(b + 4 * n + (size_t)kMaxBatchTile * nsbt * 64);
    return x;
}

// Work split of a projection over packed tiles: 16-row tiles are shared out to the
// waves of each K slab in balanced contiguous ranges and multiplied in pairs (the
// gate and up tiles of one row range in kSwiglu).
static MmaPlan plan_tiled(int rows, int cols, int nbt, bool dual) {
    MmaPlan p{};
    p.nbt = nbt;
    p.total_rows = dual ? 2 * rows : rows;
    const int ntile = (rows + 15) / 16;
    const int units = dual ? ntile : (ntile + 1) / 2;
    p.ntg = ntile;
    const int nsbt = cols / 256;
    const int sbmax = kSlabRowSb / (16 * nbt);
    int nslab = (nsbt + sbmax - 1) / sbmax;
    while (nslab < nsbt && (int64_t)units * nslab < (int64_t)kPlanCUs * kGemmWaves) nslab *= 2;
    if (nslab > nsbt) nslab = nsbt;
    p.sb_per_slab = (nsbt + nslab - 1) / nslab;
    p.nslab = (nsbt + p.sb_per_slab - 1) / p.sb_per_slab;
    // one workgroup per CU (the LDS slab fills a CU): never plan a second round
    const int wps = kPlanCUs / p.nslab > 0 ? kPlanCUs / p.nslab : 1;
    const int need = (units + kGemmWaves - 1) / kGemmWaves;
    p.wgs_per_slab = wps < need ? wps : need;
    p.grid = p.nslab * p.wgs_per_slab;
    p.x_bytes = 0;   // x is prepared in LDS by the kernel
    p.part_bytes = p.nslab > 1 ? (size_t)p.nslab * kMaxBatchTile * p.total_rows * sizeof(float) : 0;
    return p;
}

// Bytes of workspace one projection needs (0 when the VALU paths serve it); covers
// batch tiles of either width.
static size_t projection_ws(int fmt, int rows, int cols, int batch, bool dual) {
    if (is_tiled(fmt)) {
        const MmaPlan a = plan_tiled(rows, cols, 1, dual), b = plan_tiled(rows, cols, 2, dual);
        return a.x_bytes + (a.part_bytes > b.part_bytes ? a.part_bytes : b.part_bytes);
    }
    if (!(fmt == RTA_Q4_K || fmt == RTA_Q6_K) || !mma_batch((int64_t)rows * cols * (dual ? 2 : 1), batch)) return 0;
    const MmaPlan a = plan_mfma(rows, cols, 1, dual), b = plan_mfma(rows, cols, 2, dual);
    return a.x_bytes + (a.part_bytes > b.part_bytes ? a.part_bytes : b.part_bytes);
}

// The fixed-order slab reduce (gemm_reduce_kernel), its loads all in flight at once for
// up to 16 slabs.
template <int MODE>
static void launch_reduce(dim3 grid, const float* part, int nslab, int rows, int batch, float* y, float* pmax,
                          hipStream_t s) {
    with_slab_count(nslab, [&](auto ns) {
        hipLaunchKernelGGL((gemm_reduce_kernel<MODE, decltype(ns)::value>), grid, dim3(256), 0, s, part, nslab, rows,
                           batch, y, pmax);
    });
}

template <int FMT, int NBT, int MODE>
static void launch_gemm(const MmaPlan& p, const Launch& l, const GemmX& xp, float* part, float* pmax,
                        hipStream_t s) {
    hipLaunchKernelGGL((xprep_kernel<FMT == RTA_Q6_K ? kXpQ6Row : kXpQ4Row>), dim3(l.cols / 256, 8 * NBT), dim3(64), 0, s, l.x, l.cols,
                       l.batch, xp);
    hipLaunchKernelGGL((gemm_mfma_kernel<FMT, kMfmaRT, NBT, MODE>), dim3(p.grid), dim3(64 * kGemmWaves), 0, s, l.w,
                       l.w2, l.row_bytes, l.rows, l.cols, xp, l.batch, l.y, part, pmax, p.sb_per_slab,
                       p.wgs_per_slab);
}

// One batch tile (<= 32 rows): xprep -> MFMA GEMM (-> fixed-order slab reduce).
// For kLogits, pmax receives per-task maxima [batch][*ntasks_out], tasks of
// *rpt_out rows.
template <int MODE>
static hipError_t run_mfma(int fmt, const Launch& l, void* ws, float* pmax, int* ntasks_out, int* rpt_out,
                           hipStream_t s) {
    const int nbt = l.batch > 16 ? 2 : 1;
    const MmaPlan p = plan_mfma(l.rows, l.cols, nbt, MODE == kSwiglu);
    GemmX xp = carve_x(ws, l.cols);
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + p.x_bytes);
    if (fmt == RTA_Q4_K) {
        if (nbt == 1) launch_gemm<RTA_Q4_K, 1, MODE>(p, l, xp, part, pmax, s);
        else launch_gemm<RTA_Q4_K, 2, MODE>(p, l, xp, part, pmax, s);
    } else {
        if (nbt == 1) launch_gemm<RTA_Q6_K, 1, MODE>(p, l, xp, part, pmax, s);
        else launch_gemm<RTA_Q6_K, 2, MODE>(p, l, xp, part, pmax, s);
    }
    if (p.nslab > 1) {
        const dim3 rg((l.rows + 255) / 256, l.batch);
        launch_reduce<MODE>(rg, part, p.nslab, l.rows, l.batch, l.y, pmax, s);
        if (ntasks_out) *ntasks_out = (int)rg.x;
        if (rpt_out) *rpt_out = 256;
    } else {
        if (ntasks_out) *ntasks_out = p.ntg;
        if (rpt_out) *rpt_out = 16 * kMfmaRT;
    }
    return hipGetLastError();
}

template <int FMT, int NBT, int MODE>
static void launch_tiled(const MmaPlan& p, const Launch& l, float* part, float* pmax, hipStream_t s) {
    hipLaunchKernelGGL((gemm_tiled_kernel<FMT, NBT, MODE>), dim3(p.wgs_per_slab, p.nslab), dim3(64 * kGemmWaves), 0,
                       s, l.w, l.w2, l.rows, l.cols, l.x, l.batch, l.y, part, pmax, p.sb_per_slab, p.wgs_per_slab,
                       l.rn);
}

// One batch tile (<= 32 rows) over packed weights: the tiled GEMM prepares x in LDS
// itself; with several K slabs, gemm_reduce_kernel adds the partials in slab order.
template <int MODE>
static hipError_t run_tiled(int fmt, const Launch& l, void* ws, float* pmax, int* ntasks_out, int* rpt_out,
                            hipStream_t s) {
    const int nbt = l.batch > 16 ? 2 : 1;
    const MmaPlan p = plan_tiled(l.rows, l.cols, nbt, MODE == kSwiglu);
    float* part = static_cast<float*>(ws);
    if ((fmt & 0xff) == RTA_Q4_K) {
        if (nbt == 1) launch_tiled<RTA_Q4_K, 1, MODE>(p, l, part, pmax, s);
        else launch_tiled<RTA_Q4_K, 2, MODE>(p, l, part, pmax, s);
    } else {
        if (nbt == 1) launch_tiled<RTA_Q6_K, 1, MODE>(p, l, part, pmax, s);
        else launch_tiled<RTA_Q6_K, 2, MODE>(p, l, part, pmax, s);
    }
    if (p.nslab > 1) {
        const dim3 rg((l.rows + 255) / 256, l.batch);
        launch_reduce<MODE>(rg, part, p.nslab, l.rows, l.batch, l.y, pmax, s);
        if (ntasks_out) *ntasks_out = (int)rg.x;
        if (rpt_out) *rpt_out = 256;
    } else {
        if (ntasks_out) *ntasks_out = (l.rows + 15) / 16;
        if (rpt_out) *rpt_out = 16;
    }
    return hipGetLastError();
}

// Runs one projection over the whole batch: K-quant tiles of >= 8 rows on the matrix
// cores (32 rows per tile), smaller ones on the VALU kernels (8 rows per tile).
// For kLogits, partial receives per-task maxima laid out [tile row][ntasks] inside the
// tile's [tile x rows] region; *ntasks_out / *rows_per_task_out describe the last tile.
template <int MODE>
static int run_projection(int fmt, const void* w, const void* w2, int rows, int cols, const float* x, int batch,
                          float* y, float* partial, int* ntasks_out, int* rows_per_task_out, void* ws,
                          size_t ws_bytes, hipStream_t s, int path_batch = 0, const RowNorm& rn = RowNorm{},
                          const XNorm& xn = XNorm{}) {
    if (rn.part && !is_tiled(fmt)) return RTA_ERR_FORMAT;   // only the packed readout applies it
    if (xn.w && !b1_norm_fusable(fmt, cols, batch)) return RTA_ERR_FORMAT;   // only the batch-1 readout
    const bool tiled = is_tiled(fmt);
    const int64_t row_bytes = tiled ? 0 : host::row_bytes(fmt, cols);
    int b0 = 0;
    // The path depends on the whole batch (and the matrix), so a row's result never
    // depends on tiling.
    const bool mma = is_kquant(fmt) &&
                     mma_batch((int64_t)rows * cols * (MODE == kSwiglu ? 2 : 1), path_batch > 0 ? path_batch : batch);
    while (b0 < batch) {
        const int cap = (mma || tiled) ? kMaxBatchTile : 8;
        const int chunk = batch - b0 < cap ? batch - b0 : cap;
        Launch l{};
        l.w = static_cast<const uint8_t*>(w);
        l.w2 = static_cast<const uint8_t*>(w2);
        l.row_bytes = row_bytes;
        l.rows = rows;
        l.cols = cols;
        l.x = x + (int64_t)b0 * cols;
        l.y = y + (int64_t)b0 * rows;
        l.batch = chunk;
        l.partial = partial ? partial + (int64_t)b0 * rows : nullptr;
        l.rn = rn;
        if (rn.part) l.rn.part = rn.part + b0;
        l.xn = xn;
        hipError_t e;
        if (tiled) {
            if (!ws || ws_bytes < projection_ws(fmt, rows, cols, chunk, MODE == kSwiglu)) return RTA_ERR_WORKSPACE;
            e = run_tiled<MODE>(fmt, l, ws, l.partial, ntasks_out, rows_per_task_out, s);
        } else if (mma) {
            if (!ws || ws_bytes < projection_ws(fmt, rows, cols, chunk, MODE == kSwiglu)) return RTA_ERR_WORKSPACE;
            e = run_mfma<MODE>(fmt, l, ws, l.partial, ntasks_out, rows_per_task_out, s);
        } else if (is_kquant(fmt)) {
            const Plan p = plan_kquant(rows, cols, chunk, MODE == kSwiglu, row_bytes);
            if (ntasks_out) *ntasks_out = p.ntasks;
            if (rows_per_task_out) *rows_per_task_out = p.rows_per_task;
            e = launch_kquant<MODE>(fmt, p, l, s);
        } else {
            if (ntasks_out) *ntasks_out = rows;
            if (rows_per_task_out) *rows_per_task_out = 1;
            const int wgs = (rows + 3) / 4;
            e = launch_plain<MODE>(fmt, l, wgs < 2048 ? wgs : 2048, s);
        }
        if (e != hipSuccess) return RTA_ERR_LAUNCH;
        b0 += chunk;
    }
    return RTA_OK;
}

// ---- readouts of a staged x image (rta_packed.hpp), used by the decode step -------
// Kernel shape: tiles per wave and superblock, waves per workgroup, superblocks of
// weights in flight per wave.
constexpr int kPkTpw = 2, kPkWaves = 8, kPkDepth = 2;

// Work split: units of kPkTpw tiles (kSwiglu: gate and up tiles of the same rows) are
// shared out to the waves of each K slab in balanced contiguous ranges.  The K range is
// cut into as few slabs as the LDS image capacity allows, and into more (up to one per
// superblock) while the units of all slabs would not occupy every wave once.
static MmaPlan plan_packed(int rows, int cols, int nbt, bool dual) {
    MmaPlan p{};
    p.nbt = nbt;
    p.total_rows = dual ? 2 * rows : rows;
    const int ntile = (rows + 15) / 16;
    const int tpu = dual ? kPkTpw / 2 : kPkTpw;
    const int units = (ntile + tpu - 1) / tpu;
    p.ntg = ntile;
    const int nsbt = cols / 256;
    const int cap = nbt == 1 ? slab_capacity<1>() : slab_capacity<2>();
    int nslab = (nsbt + cap - 1) / cap;
    while (nslab < nsbt && (int64_t)units * nslab < (int64_t)kPlanCUs * kPkWaves) ++nslab;
    p.sb_per_slab = (nsbt + nslab - 1) / nslab;
    p.nslab = (nsbt + p.sb_per_slab - 1) / p.sb_per_slab;
    const int wps = kPlanCUs / p.nslab > 0 ? kPlanCUs / p.nslab : 1;   // one workgroup per CU
    const int need = (units + kPkWaves - 1) / kPkWaves;
    p.wgs_per_slab = wps < need ? wps : need;
    p.grid = p.nslab * p.wgs_per_slab;
    p.x_bytes = 0;
    p.part_bytes = p.nslab > 1 ? (size_t)p.nslab * kMaxBatchTile * p.total_rows * sizeof(float) : 0;
    return p;
}

size_t image_bytes(int cols, int batch) {
    if (cols <= 0 || cols % 256 || batch <= 0 || batch > kMaxBatchTile) return 0;
    const size_t one = batch > 16 ? sizeof(XImage<2>) : sizeof(XImage<1>);
    return ((size_t)(cols / 256) * one + 255) & ~(size_t)255;
}

size_t image_readout_ws_bytes(int rows, int cols, bool dual) {
    const MmaPlan a = plan_packed(rows, cols, 1, dual), b = plan_packed(rows, cols, 2, dual);
    return a.part_bytes > b.part_bytes ? a.part_bytes : b.part_bytes;
}

static bool image_format(int fmt) { return fmt == (RTA_Q4_K | kTiled) || fmt == (RTA_Q6_K | kTiled); }

int residual_norm_image(int fmt, float* hidden, const float* part, int nslab, const float* w, int batch, int width,
                        float* ss, float* out, void* img, hipStream_t s) {
    if (!image_format(fmt)) return RTA_ERR_FORMAT;
    if (!hidden || !w || !ss || !img || (nslab > 0 && !part)) return RTA_ERR_NULL;
    if (batch <= 0 || batch > kMaxBatchTile || width <= 0 || width % 256 || width > 4096 || nslab < 0)
        return RTA_ERR_SHAPE;
    if (!host::aligned(hidden, 16) || !host::aligned(w, 16) || !host::aligned(ss, 16) || !host::aligned(img, 16) ||
        (part && !host::aligned(part, 16)) || (out && !host::aligned(out, 16)))
        return RTA_ERR_ALIGN;
    const int nbt = batch > 16 ? 2 : 1;
    const dim3 g((width + 1023) / 1024, 16 * nbt), b(256);
    const bool q4 = (fmt & 0xff) == RTA_Q4_K;
    with_slab_count(nslab, [&](auto ns) {
        constexpr int NS = decltype(ns)::value;
        if (nbt == 1) {
            if (q4) hipLaunchKernelGGL((residual_norm_image_kernel<RTA_Q4_K, 1, NS>), g, b, 0, s, hidden, part, nslab,
                                       w, width, batch, ss, out, static_cast<XImage<1>*>(img));
            else hipLaunchKernelGGL((residual_norm_image_kernel<RTA_Q6_K, 1, NS>), g, b, 0, s, hidden, part, nslab, w,
                                    width, batch, ss, out, static_cast<XImage<1>*>(img));
        } else {
            if (q4) hipLaunchKernelGGL((residual_norm_image_kernel<RTA_Q4_K, 2, NS>), g, b, 0, s, hidden, part, nslab,
                                       w, width, batch, ss, out, static_cast<XImage<2>*>(img));
            else hipLaunchKernelGGL((residual_norm_image_kernel<RTA_Q6_K, 2, NS>), g, b, 0, s, hidden, part, nslab, w,
                                    width, batch, ss, out, static_cast<XImage<2>*>(img));
        }
    });
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int swiglu_image(int fmt, const float* part, int nslab, int width, int batch, void* img, hipStream_t s) {
    if (!image_format(fmt)) return RTA_ERR_FORMAT;
    if (!part || !img) return RTA_ERR_NULL;
    if (batch <= 0 || batch > kMaxBatchTile || width <= 0 || width % 256 || nslab <= 0) return RTA_ERR_SHAPE;
    if (!host::aligned(part, 16) || !host::aligned(img, 16)) return RTA_ERR_ALIGN;
    const int nbt = batch > 16 ? 2 : 1;
    const dim3 g((width + 1023) / 1024, 16 * nbt), b(256);
    const bool q4 = (fmt & 0xff) == RTA_Q4_K;
    with_slab_count(nslab, [&](auto ns) {
        constexpr int NS = decltype(ns)::value;
        if (nbt == 1) {
            if (q4) hipLaunchKernelGGL((swiglu_image_kernel<RTA_Q4_K, 1, NS>), g, b, 0, s, part, nslab, width, batch,
                                       static_cast<XImage<1>*>(img));
            else hipLaunchKernelGGL((swiglu_image_kernel<RTA_Q6_K, 1, NS>), g, b, 0, s, part, nslab, width, batch,
                                    static_cast<XImage<1>*>(img));
        } else {
            if (q4) hipLaunchKernelGGL((swiglu_image_kernel<RTA_Q4_K, 2, NS>), g, b, 0, s, part, nslab, width, batch,
                                       static_cast<XImage<2>*>(img));
            else hipLaunchKernelGGL((swiglu_image_kernel<RTA_Q6_K, 2, NS>), g, b, 0, s, part, nslab, width, batch,
                                    static_cast<XImage<2>*>(img));
        }
    });
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

template <int FMT, int NBT, int MODE>
static void launch_packed(const MmaPlan& p, const uint8_t* w, const uint8_t* w2, int rows, int cols, const void* img,
                          int batch, float* y, float* part, const RowNorm& rn, hipStream_t s) {
    hipLaunchKernelGGL((gemm_packed_kernel<FMT, NBT, MODE, kPkTpw, kPkWaves, kPkDepth>),
                       dim3(p.wgs_per_slab, p.nslab), dim3(64 * kPkWaves), 0, s, w, w2, rows, cols, static_cast<const XImage<NBT>*>(img), batch, y,
                       part, p.sb_per_slab, p.wgs_per_slab, rn);
}

template <int MODE>
static int image_readout_mode(int fmt, const void* w, const void* w2, int rows, int cols, const void* img, int batch,
                              float* y, bool reduce, void* ws, size_t ws_bytes, hipStream_t s, int* nslab,
                              const RowNorm& rn) {
    if (!image_format(fmt)) return RTA_ERR_FORMAT;
    if (!w || !img || !y || (MODE == kSwiglu && !w2)) return RTA_ERR_NULL;
    if (batch <= 0 || batch > kMaxBatchTile || rows <= 0 || cols <= 0 || cols % 256) return RTA_ERR_SHAPE;
    const int nbt = batch > 16 ? 2 : 1;
    const MmaPlan p = plan_packed(rows, cols, nbt, MODE == kSwiglu);
    if (p.part_bytes && (!ws || ws_bytes < p.part_bytes)) return RTA_ERR_WORKSPACE;
    float* part = static_cast<float*>(ws);
    const uint8_t* a = static_cast<const uint8_t*>(w);
    const uint8_t* a2 = static_cast<const uint8_t*>(w2);
    if ((fmt & 0xff) == RTA_Q4_K) {
        if (nbt == 1) launch_packed<RTA_Q4_K, 1, MODE>(p, a, a2, rows, cols, img, batch, y, part, rn, s);
        else launch_packed<RTA_Q4_K, 2, MODE>(p, a, a2, rows, cols, img, batch, y, part, rn, s);
    } else {
        if (nbt == 1) launch_packed<RTA_Q6_K, 1, MODE>(p, a, a2, rows, cols, img, batch, y, part, rn, s);
        else launch_packed<RTA_Q6_K, 2, MODE>(p, a, a2, rows, cols, img, batch, y, part, rn, s);
    }
    if (reduce && p.nslab > 1)
        launch_reduce<MODE>(dim3((rows + 255) / 256, batch), part, p.nslab, rows, batch, y, nullptr, s);
    if (nslab) *nslab = reduce ? 1 : p.nslab;
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

static_assert(kReadStore == kStore && kReadAccumulate == kAccumulate && kReadSwiglu == kSwiglu, "readout modes");

int image_readout(int fmt, int mode, const void* w, const void* w2, int rows, int cols, const void* img, int batch,
                  float* y, bool reduce, void* ws, size_t ws_bytes, hipStream_t s, int* nslab, const RowNorm& rn) {
    switch (mode) {
    case kStore:
        return image_readout_mode<kStore>(fmt, w, w2, rows, cols, img, batch, y, reduce, ws, ws_bytes, s, nslab, rn);
    case kAccumulate:
        return image_readout_mode<kAccumulate>(fmt, w, w2, rows, cols, img, batch, y, reduce, ws, ws_bytes, s, nslab,
                                               rn);
    case kSwiglu:
        return image_readout_mode<kSwiglu>(fmt, w, w2, rows, cols, img, batch, y, reduce, ws, ws_bytes, s, nslab, rn);
    default: return RTA_ERR_RANGE;
    }
}

static_assert(kSlabBatch == kMaxBatchTile, "partial blocks hold one batch tile");

int tiled_partials(int fmt, const void* w, int rows, int cols, const float* x, int batch, float* y, bool accumulate,
                   void* ws, size_t ws_bytes, hipStream_t s, int* nslab, const RowNorm& rn) {
    if (!is_tiled(fmt) || batch <= 0 || batch > kMaxBatchTile || !nslab) return RTA_ERR_RANGE;
    if (!ws || ws_bytes < projection_ws(fmt, rows, cols, batch, false)) return RTA_ERR_WORKSPACE;
    const int nbt = batch > 16 ? 2 : 1;
    const MmaPlan p = plan_tiled(rows, cols, nbt, false);
    Launch l{};
    l.w = static_cast<const uint8_t*>(w);
    l.rows = rows;
    l.cols = cols;
    l.x = x;
    l.y = y;
    l.batch = batch;
    l.rn = rn;
    float* part = static_cast<float*>(ws);
    if (accumulate) {
        if ((fmt & 0xff) == RTA_Q4_K) {
            if (nbt == 1) launch_tiled<RTA_Q4_K, 1, kAccumulate>(p, l, part, nullptr, s);
            else launch_tiled<RTA_Q4_K, 2, kAccumulate>(p, l, part, nullptr, s);
        } else {
            if (nbt == 1) launch_tiled<RTA_Q6_K, 1, kAccumulate>(p, l, part, nullptr, s);
            else launch_tiled<RTA_Q6_K, 2, kAccumulate>(p, l, part, nullptr, s);
        }
    } else {
        if ((fmt & 0xff) == RTA_Q4_K) {
            if (nbt == 1) launch_tiled<RTA_Q4_K, 1, kStore>(p, l, part, nullptr, s);
            else launch_tiled<RTA_Q4_K, 2, kStore>(p, l, part, nullptr, s);
        } else {
            if (nbt == 1) launch_tiled<RTA_Q6_K, 1, kStore>(p, l, part, nullptr, s);
            else launch_tiled<RTA_Q6_K, 2, kStore>(p, l, part, nullptr, s);
        }
    }
    *nslab = p.nslab;
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int swiglu_activation(int fmt, const void* wg, const void* wu, int inter, int hidden, const float* x, int batch,
                      float* act, void* ws, size_t ws_bytes, hipStream_t s, const RowNorm& rn, const XNorm& xn) {
    return run_projection<kSwiglu>(fmt, wg, wu, inter, hidden, x, batch, act, nullptr, nullptr, nullptr, ws, ws_bytes,
                                   s, 0, rn, xn);
}

int projection_store(int fmt, const void* w, int rows, int cols, const float* x, int batch, float* y, void* ws,
                     size_t ws_bytes, hipStream_t s, const RowNorm& rn, const XNorm& xn) {
    const int rc = check_matrix(fmt, w, rows, cols);
    if (rc) return rc;
    return run_projection<kStore>(fmt, w, nullptr, rows, cols, x, batch, y, nullptr, nullptr, nullptr, ws, ws_bytes, s,
                                  0, rn, xn);
}

bool b1_norm_fusable(int fmt, int cols, int batch) {
    return batch == 1 && is_kquant(fmt) && cols > 0 && cols % 256 == 0 && cols / 64 <= 4 * kWave;
}

// Validates a remap against the matrix and gives the source rows one readout covers
// (rows of ys for the row modes).
static int check_remap(const rta_remap* rp, int src_rows, int rows, int cols, Remap* m, int* need) {
    if (!rp) return RTA_ERR_NULL;
    if (rp->mode < RTA_REMAP_NONE || rp->mode > RTA_REMAP_KEY_REPEAT) return RTA_ERR_RANGE;
    Remap r;
    r.mode = rp->mode;
    r.hd = rp->head_dim;
    r.rotary = rp->rotary_dim;
    r.key_rows = rp->key_rows;
    if (rows <= 0 || cols <= 0 || src_rows <= 0) return RTA_ERR_SHAPE;
    int64_t n = rows;
    if (r.mode >= RTA_REMAP_QUERY && r.mode <= RTA_REMAP_AXES) {
        if (r.hd <= 0 || r.rotary < 0 || r.rotary > r.hd || r.rotary % 2) return RTA_ERR_RANGE;
        if (r.mode == RTA_REMAP_AXES ? cols % r.hd : rows % r.hd) return RTA_ERR_SHAPE;
        if (r.mode == RTA_REMAP_QUERY || r.mode == RTA_REMAP_GATE) n = 2 * (int64_t)rows;
    } else if (r.mode == RTA_REMAP_KEY_REPEAT) {
        if (r.key_rows <= 0) return RTA_ERR_RANGE;
        n = rows < r.key_rows ? rows : r.key_rows;
    }
    if (n > src_rows) return RTA_ERR_SHAPE;
    *m = r;
    *need = (int)n;
    return RTA_OK;
}

static size_t floats256(int64_t n) { return ((size_t)n * sizeof(float) + 255) & ~(size_t)255; }

}  // namespace rta

using namespace rta;

extern "C" {

int rta_version(void) { return 1; }

const char* rta_status_string(int status) {
    switch (status) {
    case RTA_OK: return "ok";
    case RTA_ERR_NULL: return "null pointer argument";
    case RTA_ERR_SHAPE: return "invalid shape";
    case RTA_ERR_FORMAT: return "unsupported format";
    case RTA_ERR_ALIGN: return "misaligned pointer";
    case RTA_ERR_WORKSPACE: return "workspace missing or too small";
    case RTA_ERR_LAUNCH: return "HIP launch error";
    case RTA_ERR_RANGE: return "argument out of supported range";
    case RTA_ERR_DEVICE: return "device error word set";
    case RTA_ERR_SCRATCH: return "call needs more scratch than the no-alloc variant holds (RTA_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
    }
}

int rta_device_error(uint32_t* bits, int clear) {
    if (!bits) return RTA_ERR_NULL;
    if (hipDeviceSynchronize() != hipSuccess) return RTA_ERR_LAUNCH;
    uint32_t v = 0;
    if (hipMemcpyFromSymbol(&v, HIP_SYMBOL(g_error_word), sizeof(v), 0, hipMemcpyDeviceToHost) != hipSuccess)
        return RTA_ERR_LAUNCH;
    *bits = v;
    if (clear) {
        const uint32_t zero = 0;
        if (hipMemcpyToSymbol(HIP_SYMBOL(g_error_word), &zero, sizeof(zero), 0, hipMemcpyHostToDevice) != hipSuccess)
            return RTA_ERR_LAUNCH;
    }
    return RTA_OK;
}

int64_t rta_row_bytes(int fmt, int64_t cols) { return host::row_bytes(fmt, cols); }

int rta_dequant(int fmt, const void* src, int64_t n, float* out, rta_stream_t stream) {
    if (!host::valid_format(fmt)) return RTA_ERR_FORMAT;
    if (!src || !out) return RTA_ERR_NULL;
    if (n < 0 || (is_kquant(fmt) && n % 256)) return RTA_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(src) % (fmt == RTA_F32 || fmt == RTA_Q4_K ? 4 : 2) ||
        reinterpret_cast<uintptr_t>(out) % 4)
        return RTA_ERR_ALIGN;
    if (n == 0) return RTA_OK;
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(dequant_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, fmt,
                       static_cast<const uint8_t*>(src), n, out);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

size_t rta_gemv_workspace_bytes(int fmt, int rows, int cols, int batch) {
    if (rows <= 0 || cols <= 0 || batch <= 0 || ((is_kquant(fmt) || is_tiled(fmt)) && cols % 256)) return 0;
    return projection_ws(fmt, rows, cols, batch < kMaxBatchTile ? batch : kMaxBatchTile, false);
}

int rta_gemv(int fmt, const void* w, int rows, int cols, const float* x, int batch, float* y, int epilogue,
             void* workspace, size_t workspace_bytes, rta_stream_t stream) {
    int rc = check_matrix(fmt, w, rows, cols);
    if (rc) return rc;
    if (!x || !y) return RTA_ERR_NULL;
    if (batch <= 0) return RTA_ERR_SHAPE;
    if (epilogue != RTA_EPI_STORE && epilogue != RTA_EPI_ACCUMULATE) return RTA_ERR_RANGE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 4 ||
        reinterpret_cast<uintptr_t>(workspace) % 256)
        return RTA_ERR_ALIGN;
    if (workspace_bytes < rta_gemv_workspace_bytes(fmt, rows, cols, batch)) return RTA_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    if (epilogue == RTA_EPI_STORE)
        return run_projection<kStore>(fmt, w, nullptr, rows, cols, x, batch, y, nullptr, nullptr, nullptr, workspace,
                                      workspace_bytes, s);
    return run_projection<kAccumulate>(fmt, w, nullptr, rows, cols, x, batch, y, nullptr, nullptr, nullptr, workspace,
                                       workspace_bytes, s);
}

size_t rta_gemv_remap_workspace_bytes(int fmt, const rta_remap* remap, int rows, int cols, int batch) {
    Remap m;
    int need = 0;
    if (batch <= 0 || check_remap(remap, INT_MAX, rows, cols, &m, &need)) return 0;
    const size_t inner = rta_gemv_workspace_bytes(fmt, need, cols, batch);
    if (m.mode == RTA_REMAP_NONE) return inner;
    if ((is_kquant(fmt) || is_tiled(fmt)) && cols % 256) return 0;
    return (m.moves_rows() ? floats256((int64_t)batch * need) : floats256((int64_t)batch * cols)) + inner;
}

int rta_gemv_remap(int fmt, const void* w, int src_rows, int rows, int cols, const rta_remap* remap, const float* x,
                   int batch, float* y, int epilogue, void* workspace, size_t workspace_bytes, rta_stream_t stream) {
    Remap m;
    int need = 0;
    int rc = check_remap(remap, src_rows, rows, cols, &m, &need);
    if (rc) return rc;
    if (m.mode == RTA_REMAP_NONE)
        return rta_gemv(fmt, w, rows, cols, x, batch, y, epilogue, workspace, workspace_bytes, stream);
    rc = check_matrix(fmt, w, need, cols);
    if (rc) return rc;
    if (!x || !y) return RTA_ERR_NULL;
    if (batch <= 0) return RTA_ERR_SHAPE;
    if (epilogue != RTA_EPI_STORE && epilogue != RTA_EPI_ACCUMULATE) return RTA_ERR_RANGE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(y) % 4 ||
        reinterpret_cast<uintptr_t>(workspace) % 256)
        return RTA_ERR_ALIGN;
    if (workspace_bytes < rta_gemv_remap_workspace_bytes(fmt, remap, rows, cols, batch)) return RTA_ERR_WORKSPACE;
    if (!workspace) return RTA_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    if (!m.moves_rows()) {   // mode 4: the permuted x, then the plain readout with the caller's epilogue
        float* xp = reinterpret_cast<float*>(ws);
        const size_t xb = floats256((int64_t)batch * cols);
        const int64_t n = (int64_t)batch * cols;
        hipLaunchKernelGGL(remap_axes_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, x, cols, batch, m,
                           xp);
        if (hipGetLastError() != hipSuccess) return RTA_ERR_LAUNCH;
        return rta_gemv(fmt, w, rows, cols, xp, batch, y, epilogue, ws + xb, workspace_bytes - xb, stream);
    }
    // row modes: every source row read once into ys, then gathered into y
    float* ys = reinterpret_cast<float*>(ws);
    const size_t yb = floats256((int64_t)batch * need);
    rc = rta_gemv(fmt, w, need, cols, x, batch, ys, RTA_EPI_STORE, ws + yb, workspace_bytes - yb, stream);
    if (rc) return rc;
    const int64_t n = (int64_t)batch * rows;
    if (epilogue == RTA_EPI_STORE)
        hipLaunchKernelGGL(remap_gather_kernel<false>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ys, need,
                           rows, batch, m, y);
    else
        hipLaunchKernelGGL(remap_gather_kernel<true>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ys, need,
                           rows, batch, m, y);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

size_t rta_mlp_workspace_bytes(int fmt_g, int fmt_d, int hidden, int inter, int batch) {
    if (hidden <= 0 || inter <= 0 || batch <= 0) return 0;
    if (((is_kquant(fmt_g) || is_tiled(fmt_g)) && hidden % 256) || ((is_kquant(fmt_d) || is_tiled(fmt_d)) && inter % 256))
        return 0;
    const int tile = batch < kMaxBatchTile ? batch : kMaxBatchTile;
    const size_t a = projection_ws(fmt_g, inter, hidden, tile, true);
    const size_t b = projection_ws(fmt_d, hidden, inter, tile, false);
    return a > b ? a : b;
}

int rta_mlp_swiglu(int fmt_g, const void* wg, int fmt_u, const void* wu, int fmt_d, const void* wd, int hidden,
                   int inter, const float* x, int batch, float* act, float* y, int epilogue, void* workspace,
                   size_t workspace_bytes, rta_stream_t stream) {
    int rc = check_matrix(fmt_g, wg, inter, hidden);
    if (rc) return rc;
    if ((rc = check_matrix(fmt_u, wu, inter, hidden))) return rc;
    if ((rc = check_matrix(fmt_d, wd, hidden, inter))) return rc;
    if (fmt_g != fmt_u) return RTA_ERR_FORMAT;  // the fused gate/up pass streams both in one format
    if (!x || !act || !y) return RTA_ERR_NULL;
    if (batch <= 0) return RTA_ERR_SHAPE;
    if (epilogue != RTA_EPI_STORE && epilogue != RTA_EPI_ACCUMULATE) return RTA_ERR_RANGE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(act) % 16 ||
        reinterpret_cast<uintptr_t>(y) % 4 || reinterpret_cast<uintptr_t>(workspace) % 256)
        return RTA_ERR_ALIGN;
    if (workspace_bytes < rta_mlp_workspace_bytes(fmt_g, fmt_d, hidden, inter, batch)) return RTA_ERR_WORKSPACE;
    hipStream_t s = (hipStream_t)stream;
    rc = run_projection<kSwiglu>(fmt_g, wg, wu, inter, hidden, x, batch, act, nullptr, nullptr, nullptr, workspace,
                                 workspace_bytes, s);
    if (rc) return rc;
    if (epilogue == RTA_EPI_STORE)
        return run_projection<kStore>(fmt_d, wd, nullptr, hidden, inter, act, batch, y, nullptr, nullptr, nullptr,
                                      workspace, workspace_bytes, s);
    return run_projection<kAccumulate>(fmt_d, wd, nullptr, hidden, inter, act, batch, y, nullptr, nullptr, nullptr,
                                       workspace, workspace_bytes, s);
}

int rta_swiglu(int fmt, const void* wg, const void* wu, int hidden, int inter, const float* x, int batch, float* act,
               void* workspace, size_t workspace_bytes, rta_stream_t stream) {
    int rc = check_matrix(fmt, wg, inter, hidden);
    if (rc) return rc;
    if ((rc = check_matrix(fmt, wu, inter, hidden))) return rc;
    if (!x || !act) return RTA_ERR_NULL;
    if (batch <= 0) return RTA_ERR_SHAPE;
    if (reinterpret_cast<uintptr_t>(x) % 16 || reinterpret_cast<uintptr_t>(act) % 16 ||
        reinterpret_cast<uintptr_t>(workspace) % 256)
        return RTA_ERR_ALIGN;
    if (workspace_bytes < rta_mlp_workspace_bytes(fmt, fmt, hidden, inter, batch)) return RTA_ERR_WORKSPACE;
    return run_projection<kSwiglu>(fmt, wg, wu, inter, hidden, x, batch, act, nullptr, nullptr, nullptr, workspace,
                                   workspace_bytes, (hipStream_t)stream);
}

size_t rta_lm_head_workspace_bytes(int fmt, int vocab, int hidden, int batch) {
    if (vocab <= 0 || hidden <= 0 || batch <= 0 || !(host::valid_format(fmt) || is_tiled(fmt))) return 0;
    if ((is_kquant(fmt) || is_tiled(fmt)) && hidden % 256) return 0;
    // per-task maxima [batch][vocab] (upper bound), then the matrix-core scratch of one tile
    const size_t maxima = ((size_t)vocab * (size_t)batch * sizeof(float) + 255) & ~(size_t)255;
    return maxima + projection_ws(fmt, vocab, hidden, batch < kMaxBatchTile ? batch : kMaxBatchTile, false);
}

int rta_lm_head(int fmt, const void* w, int vocab, int hidden, const float* h, int batch, float margin, float* logits,
                uint32_t* ids, void* workspace, size_t workspace_bytes, rta_stream_t stream) {
    return lm_head_rownorm(fmt, w, vocab, hidden, h, batch, margin, logits, ids, workspace, workspace_bytes,
                           (hipStream_t)stream, RowNorm{});
}

}  // extern "C"

namespace rta {

int lm_head_rownorm(int fmt, const void* w, int vocab, int hidden, const float* h, int batch, float margin,
                    float* logits, uint32_t* ids, void* workspace, size_t workspace_bytes, hipStream_t s,
                    const RowNorm& rn, const XNorm& xn, hipEvent_t readout_done) {
    int rc = check_matrix(fmt, w, vocab, hidden);
    if (rc) return rc;
    if (!h || !logits || !ids) return RTA_ERR_NULL;
    if (batch <= 0) return RTA_ERR_SHAPE;
    if (!(margin >= 0.0f) || !(margin < 1.0f)) return RTA_ERR_RANGE;
    const size_t maxima = ((size_t)vocab * (size_t)batch * sizeof(float) + 255) & ~(size_t)255;
    const size_t mma = projection_ws(fmt, vocab, hidden, batch < kMaxBatchTile ? batch : kMaxBatchTile, false);
    if (!workspace || workspace_bytes < rta_lm_head_workspace_bytes(fmt, vocab, hidden, batch)) return RTA_ERR_WORKSPACE;
    if (reinterpret_cast<uintptr_t>(h) % 16 || reinterpret_cast<uintptr_t>(logits) % 4 ||
        reinterpret_cast<uintptr_t>(ids) % 4 || reinterpret_cast<uintptr_t>(workspace) % 256)
        return RTA_ERR_ALIGN;
    float* partial = static_cast<float*>(workspace);
    void* scratch = static_cast<uint8_t*>(workspace) + maxima;
    // Argmax per batch tile, with the plan that tile was written with.
    int b0 = 0;
    while (b0 < batch) {
        const bool cores = is_kquant(fmt) && mma_batch((int64_t)vocab * hidden, batch);
        const int cap = (cores || is_tiled(fmt)) ? kMaxBatchTile : 8;
        const int chunk = batch - b0 < cap ? batch - b0 : cap;
        int ntasks = 0, rpt = 1;
        RowNorm rc_rn = rn;
        if (rn.part) rc_rn.part = rn.part + b0;
        rc = run_projection<kLogits>(fmt, w, nullptr, vocab, hidden, h + (int64_t)b0 * hidden, chunk,
                                     logits + (int64_t)b0 * vocab, partial + (int64_t)b0 * vocab, &ntasks, &rpt,
                                     scratch, mma, s, batch, rc_rn, xn);
        if (rc) return rc;
        if (readout_done && b0 + chunk == batch && hipEventRecord(readout_done, s) != hipSuccess) return RTA_ERR_LAUNCH;
        // many small tasks: their group maxima go into the maxima region after the tasks'
        // (the chunk's [chunk][ntasks] task maxima leave chunk x (vocab - ntasks) floats)
        const int ngroups = (ntasks + kWave - 1) / kWave;
        float* gm = nullptr;
        if (ntasks > 4 * kArgmaxThreads && (int64_t)chunk * (ntasks + ngroups) <= (int64_t)chunk * vocab) {
            gm = partial + (int64_t)b0 * vocab + (int64_t)chunk * ntasks;
            hipLaunchKernelGGL(group_max_kernel, dim3((ngroups + 3) / 4, chunk), dim3(256), 0, s,
                               partial + (int64_t)b0 * vocab, ntasks, ngroups, gm);
        }
        hipLaunchKernelGGL(argmax_margin_kernel, dim3(chunk), dim3(kArgmaxThreads), 0, s, logits + (int64_t)b0 * vocab,
                           vocab, partial + (int64_t)b0 * vocab, ntasks, rpt, margin, ids + b0, gm, ngroups);
        if (hipGetLastError() != hipSuccess) return RTA_ERR_LAUNCH;
        b0 += chunk;
    }
    return RTA_OK;
}

}  // namespace rta

extern "C" {

int64_t rta_pack_bytes(int fmt, int rows, int cols) {
    if (rows <= 0 || cols <= 0 || cols % 256) return -1;
    const int64_t tiles = (int64_t)((rows + 15) / 16) * (cols / 256);
    if (fmt == RTA_Q4_K) return tiles * TileFmt<RTA_Q4_K>::kBytes;
    if (fmt == RTA_Q6_K) return tiles * TileFmt<RTA_Q6_K>::kBytes;
    return -1;
}

static int pack_rows(int fmt, const void* src, int rows, int cols, const Remap& m, void* dst, hipStream_t s) {
    if (!dst) return RTA_ERR_NULL;
    if (reinterpret_cast<uintptr_t>(dst) % 16) return RTA_ERR_ALIGN;
    const int64_t n2 = rta_pack_bytes(fmt, rows, cols) / 2;
    const dim3 g((unsigned)((n2 + 255) / 256)), b(256);
    if (fmt == RTA_Q4_K)
        hipLaunchKernelGGL(pack_kernel<RTA_Q4_K>, g, b, 0, s, static_cast<const uint8_t*>(src), rows, cols,
                           static_cast<uint8_t*>(dst), n2, m);
    else
        hipLaunchKernelGGL(pack_kernel<RTA_Q6_K>, g, b, 0, s, static_cast<const uint8_t*>(src), rows, cols,
                           static_cast<uint8_t*>(dst), n2, m);
    return hipGetLastError() == hipSuccess ? RTA_OK : RTA_ERR_LAUNCH;
}

int rta_pack(int fmt, const void* src, int rows, int cols, void* dst, rta_stream_t stream) {
    if (fmt != RTA_Q4_K && fmt != RTA_Q6_K) return RTA_ERR_FORMAT;
    int rc = check_matrix(fmt, src, rows, cols);
    if (rc) return rc;
    return pack_rows(fmt, src, rows, cols, Remap{}, dst, (hipStream_t)stream);
}

int rta_pack_remap(int fmt, const void* src, int src_rows, int cols, const rta_remap* remap, int rows, void* dst,
                   rta_stream_t stream) {
    if (fmt != RTA_Q4_K && fmt != RTA_Q6_K) return RTA_ERR_FORMAT;
    Remap m;
    int need = 0;
    int rc = check_remap(remap, src_rows, rows, cols, &m, &need);
    if (rc) return rc;
    if (m.mode == RTA_REMAP_AXES) return RTA_ERR_RANGE;
    rc = check_matrix(fmt, src, need, cols);
    if (rc) return rc;
    return pack_rows(fmt, src, rows, cols, m, dst, (hipStream_t)stream);
}

size_t rta_image_bytes(int cols, int batch) { return image_bytes(cols, batch); }

size_t rta_image_readout_workspace_bytes(int rows, int cols, int dual) {
    if (rows <= 0 || cols <= 0 || cols % 256) return 0;
    return image_readout_ws_bytes(rows, cols, dual != 0);
}

int rta_image_from_rows(int fmt, const float* x, const float* w, int batch, int cols, float* ss, void* img,
                        rta_stream_t stream) {
    if (!x || !w || !ss || !img) return RTA_ERR_NULL;
    // with no slabs the kernel reads x and never writes it
    return residual_norm_image(fmt, const_cast<float*>(x), nullptr, 0, w, batch, cols, ss, nullptr, img,
                               (hipStream_t)stream);
}

int rta_image_from_swiglu(int fmt, const float* part, int nslab, int width, int batch, void* img,
                          rta_stream_t stream) {
    if (!part || !img) return RTA_ERR_NULL;
    if (nslab <= 0 || image_bytes(width, batch) == 0) return RTA_ERR_SHAPE;
    if (!host::aligned(part, 16) || !host::aligned(img, 16)) return RTA_ERR_ALIGN;
    return swiglu_image(fmt, part, nslab, width, batch, img, (hipStream_t)stream);
}

int rta_image_readout(int fmt, int mode, const void* w, const void* w2, int rows, int cols, const void* img,
                      int batch, const float* ss, float eps, float* y, int reduce, void* workspace,
                      size_t workspace_bytes, int* nslab, rta_stream_t stream) {
    if (mode != RTA_EPI_STORE && mode != RTA_EPI_ACCUMULATE && mode != RTA_IMAGE_SWIGLU) return RTA_ERR_RANGE;
    if (image_bytes(cols, batch) == 0) return RTA_ERR_SHAPE;
    // ss holds the four 1024-column chunk sums rta_image_from_rows writes (cols <= 4096)
    if (ss && cols > 4096) return RTA_ERR_SHAPE;
    // img and the K slabs are read with 16-byte loads; y is written per element
    if ((ss && !host::aligned(ss, 16)) || !host::aligned(img, 16) || !host::aligned(workspace, 16) ||
        !host::aligned(y, 4))
        return RTA_ERR_ALIGN;
    RowNorm rn;
    if (ss) rn = RowNorm{reinterpret_cast<const float4*>(ss), (float)cols, eps};
    const int m = mode == RTA_EPI_STORE ? kReadStore : mode == RTA_EPI_ACCUMULATE ? kReadAccumulate : kReadSwiglu;
    return image_readout(fmt, m, w, w2, rows, cols, img, batch, y, reduce != 0, workspace, workspace_bytes,
                         (hipStream_t)stream, nslab, rn);
}

}  // extern "C"
