// gsr_bin.hip — tile binning (a3-a5), tile ranges (a7) and the per-Gaussian
// blend records.
//
// Ordering design.  The reference emits 64-bit (tile << 32 | depth bits) keys
// in Gaussian-major order and stable-sorts all of them (rasterize.cu:124-135,
// :423-435), which orders pairs by (tile, depth bits, Gaussian id).  Here the
// Gaussians are first stable-sorted by depth bits (N keys, 32 bits), pairs are
// emitted in that depth order carrying only the tile id, and the pairs are
// then stable-sorted by the tile id's significant bits.  Stability makes the
// result the same (tile, depth bits, Gaussian id) order, bit for bit, while
// the M-sized sort moves 8 B per pair per pass over ceil(log2 T / 8) passes
// instead of 12 B over ceil((32 + log2 T) / 8).
#include "gsr_internal.h"
#include "gsr_common.h"

namespace gsr {

namespace {

constexpr int kThreads = 256;

struct TileRect {
    int x0, x1, y0, y1;
    bool ok;
};

// rasterize.cu:19-59: radius from the larger eigenvalue of the 2D covariance,
// pixel box clamped to the screen, tile box clamped to the grid.
__device__ __forceinline__ TileRect tile_rect(float mx, float my, float a, float b, float c,
                                              int W, int H) {
    TileRect r{0, 0, 0, 0, false};
    const float det = a * c - b * b;
    if (det <= 0.0f) return r;
    const float mid = 0.5f * (a + c);
    const float lambda_max = mid + __builtin_sqrtf(fmaxf(0.1f, mid * mid - det));
    const float radius = __builtin_ceilf(3.0f * __builtin_sqrtf(lambda_max));
    const int min_x = max(0, f2i_sat(__builtin_floorf(mx - radius)));
    const int max_x = min(W, f2i_sat(__builtin_ceilf(mx + radius)));
    const int min_y = max(0, f2i_sat(__builtin_floorf(my - radius)));
    const int max_y = min(H, f2i_sat(__builtin_ceilf(my + radius)));
    const int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
    r.x0 = max(0, min(tiles_x, min_x / 16));
    r.x1 = max(0, min(tiles_x, (max_x + 15) / 16));
    r.y0 = max(0, min(tiles_y, min_y / 16));
    r.y1 = max(0, min(tiles_y, (max_y + 15) / 16));
    r.ok = true;
    return r;
}

__global__ __launch_bounds__(kThreads) void bin_count_kernel(
    int n, const float* __restrict__ mean2d, const float* __restrict__ cov2d,
    const float* __restrict__ depth, int H, int W, uint32_t* __restrict__ counts,
    uint2* __restrict__ rects, uint32_t* __restrict__ dkeys, uint32_t* __restrict__ dvals) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const TileRect r = tile_rect(mean2d[2 * (size_t)i], mean2d[2 * (size_t)i + 1],
                                 cov2d[3 * (size_t)i], cov2d[3 * (size_t)i + 1],
                                 cov2d[3 * (size_t)i + 2], W, H);
    const uint32_t cnt = r.ok ? (uint32_t)(max(0, r.x1 - r.x0) * max(0, r.y1 - r.y0)) : 0u;
    counts[i] = cnt;
    rects[i] = make_uint2((uint32_t)r.x0 | ((uint32_t)r.x1 << 16),
                          (uint32_t)r.y0 | ((uint32_t)r.y1 << 16));
    // Gaussians without tiles sort last; they emit nothing, so their place
    // in the depth order never shows.
    dkeys[i] = cnt ? __float_as_uint(depth[i]) : 0xffffffffu;
    dvals[i] = (uint32_t)i;
}

// One thread per depth rank: write the Gaussian's tiles, ty outer, tx inner.
__global__ __launch_bounds__(kThreads) void emit_pairs_kernel(
    int n, const uint32_t* __restrict__ perm, const uint32_t* __restrict__ counts,
    const uint2* __restrict__ rects, const uint32_t* __restrict__ offsets, int tiles_x,
    uint64_t m, uint32_t* __restrict__ tile_keys, uint32_t* __restrict__ ids) {
    const int r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= n) return;
    const uint32_t g = perm[r];
    if (g >= (uint32_t)n || counts[g] == 0) return;
    if ((uint64_t)offsets[r] + counts[g] > m) return;  // inconsistent scan: write nothing
    const uint2 rc = rects[g];
    const int x0 = rc.x & 0xffff, x1 = rc.x >> 16, y0 = rc.y & 0xffff, y1 = rc.y >> 16;
    size_t o = offsets[r];
    for (int ty = y0; ty < y1; ++ty) {
        const uint32_t row = (uint32_t)(ty * tiles_x);
        for (int tx = x0; tx < x1; ++tx, ++o) {
            tile_keys[o] = row + (uint32_t)tx;
            ids[o] = g;
        }
    }
}

// identify_tile_ranges_kernel (rasterize.cu:140-166): tile boundaries in the
// sorted tile keys; tiles without pairs keep the zeros written before.
__global__ __launch_bounds__(kThreads) void tile_ranges_kernel(uint64_t m, uint32_t T,
                                                               const uint32_t* __restrict__ tiles,
                                                               int32_t* __restrict__ ranges) {
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= m) return;
    const uint32_t cur = tiles[i];
    if (cur >= T || (i > 0 && tiles[i - 1] >= T)) return;  // keys come from [0, T)
    if (i == 0) {
        ranges[2 * (size_t)cur] = 0;
    } else {
        const uint32_t prev = tiles[i - 1];
        if (cur != prev) {
            ranges[2 * (size_t)prev + 1] = (int32_t)i;
            ranges[2 * (size_t)cur] = (int32_t)i;
        }
    }
    if (i == m - 1) ranges[2 * (size_t)cur + 1] = (int32_t)m;
}

__global__ __launch_bounds__(kThreads) void full_keys_kernel(uint64_t m,
                                                             const uint32_t* __restrict__ tiles,
                                                             const int32_t* __restrict__ ids,
                                                             const float* __restrict__ depth,
                                                             int n, uint64_t* __restrict__ keys) {
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= m) return;
    const int g = ids[i];
    const uint32_t dbits = (g >= 0 && g < n) ? __float_as_uint(depth[g]) : 0xffffffffu;
    keys[i] = ((uint64_t)tiles[i] << 32) | (uint64_t)dbits;
}

// Squared distance d^2 beyond which o * exp(-q/2) < 1/255 for every pixel, with
// q = d^T C d >= lambda_min(C) |d|^2.  Computed in double from the fp32 conic and
// opacity; lambda_min is lowered by 2e-5 (mid + |cy|) to cover the fp32
// rounding of q in the per-pixel evaluation (~4e-7 of the same scale), and the
// threshold raised by 0.1% + 1e-4 to cover exp and the o*G product, so an entry
// is skipped only where the reference's per-pixel tests skip it too.
__device__ __forceinline__ float alpha_cut_radius2(float cx, float cy, float cz, float o) {
    if (!(o >= kAlphaMin)) return -1.0f;  // alpha <= o < 1/255 for every pixel
    const double mid = 0.5 * ((double)cx + (double)cz);
    const double det = (double)cx * cz - (double)cy * cy;
    if (!(det > 0.0) || !(mid > 0.0)) return __builtin_inff();
    const double lmax = mid + sqrt(fmax(0.0, mid * mid - det));
    const double k = 0.5 * (det / lmax - 2e-5 * (mid + fabs((double)cy)));
    if (!(k > 0.0)) return __builtin_inff();
    const double r2 = (log(255.0 * (double)o) * 1.001 + 1e-4) / k;
    return nextafterf((float)r2, __builtin_inff());
}

// Conic = cov^-1 with 1/det first (rasterize.cu:224-232), packed with mean,
// opacity and colour so the blend loads one 48 B record per list entry.
__global__ __launch_bounds__(kThreads) void blend_records_kernel(
    int n, const float* __restrict__ mean2d, const float* __restrict__ cov2d,
    const float* __restrict__ colors, const float* __restrict__ alpha,
    BlendRec* __restrict__ recs) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float a = cov2d[3 * (size_t)i], b = cov2d[3 * (size_t)i + 1], c = cov2d[3 * (size_t)i + 2];
    const float det = a * c - b * b;
    const float det_inv = (det > 0.0f) ? (1.0f / det) : 0.0f;
    const float cx = c * det_inv, cy = -b * det_inv, cz = a * det_inv;
    BlendRec r;
    r.a = make_float4(mean2d[2 * (size_t)i], mean2d[2 * (size_t)i + 1], cx, 2.0f * cy);
    r.b = make_float4(cz, alpha[i], colors[3 * (size_t)i], colors[3 * (size_t)i + 1]);
    r.c = make_float4(colors[3 * (size_t)i + 2], cy, alpha_cut_radius2(cx, cy, cz, alpha[i]),
                      0.0f);
    recs[i] = r;
}

inline unsigned blocks_for(uint64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_bin_count(int n, const float* mean2d, const float* cov2d, const float* depth,
                            int H, int W, uint32_t* counts, uint2* rects, uint32_t* dkeys,
                            uint32_t* dvals, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(bin_count_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, mean2d,
                       cov2d, depth, H, W, counts, rects, dkeys, dvals);
    return hipGetLastError();
}

hipError_t launch_emit_pairs(int n, const uint32_t* perm, const uint32_t* counts,
                             const uint2* rects, const uint32_t* offsets, int tiles_x, uint64_t m,
                             uint32_t* tile_keys, uint32_t* ids, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(emit_pairs_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, perm,
                       counts, rects, offsets, tiles_x, m, tile_keys, ids);
    return hipGetLastError();
}

hipError_t launch_tile_ranges(uint64_t m, uint32_t T, const uint32_t* sorted_tiles,
                              int32_t* ranges, hipStream_t st) {
    if (m == 0) return hipSuccess;
    hipLaunchKernelGGL(tile_ranges_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, m, T,
                       sorted_tiles, ranges);
    return hipGetLastError();
}

hipError_t launch_full_keys(uint64_t m, const uint32_t* sorted_tiles, const int32_t* ids,
                            const float* depth, int n, uint64_t* keys, hipStream_t st) {
    if (m == 0) return hipSuccess;
    hipLaunchKernelGGL(full_keys_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, m,
                       sorted_tiles, ids, depth, n, keys);
    return hipGetLastError();
}

hipError_t launch_blend_records(int n, const float* mean2d, const float* cov2d,
                                const float* colors, const float* alpha, void* recs,
                                hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(blend_records_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n,
                       mean2d, cov2d, colors, alpha, static_cast<BlendRec*>(recs));
    return hipGetLastError();
}

}  // namespace gsr
