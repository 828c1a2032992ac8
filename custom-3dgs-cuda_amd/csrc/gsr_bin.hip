// gsr_bin.hip — tile binning, tile ranges and the per-Gaussian blend records.
//
// Ordering design.  The reference emits 64-bit (tile << 32 | depth bits) keys
// in Gaussian-major order and stable-sorts all of them (rasterize.cu:124-135,
// :423-435), which orders pairs by (tile, depth bits, Gaussian id).  Here the
// Gaussians are first stable-sorted by depth bits (N keys, 32 bits), pairs are
// laid out in that depth order carrying only the tile id, and the pairs are
// then stable-sorted by the tile id's significant bits.  Stability makes the
// result the same (tile, depth bits, Gaussian id) order, bit for bit, while
// the M-sized sort moves 8 B per pair per pass over ceil(log2 T / 8) passes
// instead of 12 B over ceil((32 + log2 T) / 8).  The pairs are never written
// in depth order: the first tile-sort pass generates them per partition from
// the depth order, the per-Gaussian offsets and tile rectangles, and the
// passes' digit histograms come from the rectangles here, so no pass reads
// the keys only to count them.
#include <algorithm>

#include "gsr_internal.h"
#include "gsr_common.h"
#include "gsr_group.h"
#include "gsr_schedule.h"

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

// Adds the digit counts of the tile ids in the row range [a, a + w) to the
// work-group histograms: digit 0 through a difference array over the 256 bins
// (w >> 8 full cycles are counted once per row in *full), digits 1..passes-1
// per aligned block of 256^p ids the range meets.
__device__ __forceinline__ void hist_row(uint32_t a, uint32_t w, int passes, int* s_d0,
                                         uint32_t (*s_h)[kRadixBins], uint32_t* full) {
    *full += w >> 8;
    const uint32_t rem = w & 255u;
    if (rem) {
        const uint32_t st = a & 255u, en = st + rem;
        atomicAdd(&s_d0[st], 1);
        if (en <= 256u) {
            atomicSub(&s_d0[en], 1);
        } else {
            atomicAdd(&s_d0[0], 1);
            atomicSub(&s_d0[en - 256u], 1);
        }
    }
    for (int p = 1; p < passes; ++p) {
        const int sh = 8 * p;
        const uint64_t lo = a, hi = (uint64_t)a + w;
        for (uint64_t b = lo >> sh; b <= (hi - 1) >> sh; ++b) {
            const uint64_t bl = max(lo, b << sh), bh = min(hi, (b + 1) << sh);
            atomicAdd(&s_h[p - 1][b & 255u], (uint32_t)(bh - bl));
        }
    }
}

constexpr int kBinUnroll = 4;

// Per Gaussian: tile rectangle and count (rasterize.cu:19-59, :98-105), the
// depth sort's key and value, and the Gaussian's share of both sorts' global
// digit histograms (depth_hist[p][d]: keys with digit d in pass p;
// tile_hist[p][d]: pairs whose tile id has digit d in pass p), accumulated per
// work-group and flushed with one global atomic per non-zero bin.
__global__ __launch_bounds__(kThreads) void bin_count_kernel(
    int n, const float* __restrict__ mean2d, const float* __restrict__ cov2d,
    const float* __restrict__ depth, int H, int W, uint32_t* __restrict__ counts,
    uint2* __restrict__ rects, uint32_t* __restrict__ dkeys, uint32_t* __restrict__ dvals,
    int passes, uint32_t* __restrict__ tile_hist, uint32_t* __restrict__ depth_hist,
    BlockGrid bg, uint32_t* __restrict__ block_hist, uint64_t* __restrict__ pair_total) {
    __shared__ int s_d0[kRadixBins + 1];
    __shared__ uint32_t s_h[3][kRadixBins];
    __shared__ uint32_t s_dh[4][kRadixBins];
    __shared__ int s_bh[kMaxBlocks];  // block histogram, first as a 2D difference array
    __shared__ uint32_t s_full[kThreads / kWave];
    __shared__ uint32_t s_scan[kThreads / kWave];
    const int tid = threadIdx.x;
    const bool blocks = block_hist != nullptr;
    for (int j = tid; j <= kRadixBins; j += kThreads) s_d0[j] = 0;
    for (int j = tid; j < 3 * kRadixBins; j += kThreads) (&s_h[0][0])[j] = 0;
    for (int j = tid; j < 4 * kRadixBins; j += kThreads) (&s_dh[0][0])[j] = 0;
    if (blocks)
        for (int j = tid; j < bg.nb; j += kThreads) s_bh[j] = 0;
    __syncthreads();
    const int tiles_x = (W + 15) / 16;
    uint32_t full = 0;
    uint64_t pairs = 0;
    // the grid-strided loop takes kBinUnroll Gaussians per step, their loads
    // issued together
    const int64_t stride = (int64_t)gridDim.x * kThreads;
    for (int64_t i0 = (int64_t)blockIdx.x * kThreads + tid; i0 < n; i0 += kBinUnroll * stride) {
        float in[kBinUnroll][6];
#pragma unroll
        for (int u = 0; u < kBinUnroll; ++u) {
            const int64_t i = i0 + u * stride;
            const bool ok = i < n;
            in[u][0] = ok ? mean2d[2 * (size_t)i] : 0.0f;
            in[u][1] = ok ? mean2d[2 * (size_t)i + 1] : 0.0f;
            in[u][2] = ok ? cov2d[3 * (size_t)i] : 0.0f;
            in[u][3] = ok ? cov2d[3 * (size_t)i + 1] : 0.0f;
            in[u][4] = ok ? cov2d[3 * (size_t)i + 2] : 0.0f;
            in[u][5] = (ok && dkeys) ? depth[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kBinUnroll; ++u) {
            const int64_t i = i0 + u * stride;
            if (i >= n) break;
            const TileRect r = tile_rect(in[u][0], in[u][1], in[u][2], in[u][3], in[u][4], W, H);
            const uint32_t cnt = r.ok ? (uint32_t)(max(0, r.x1 - r.x0) * max(0, r.y1 - r.y0)) : 0u;
            counts[i] = cnt;
            rects[i] = make_uint2((uint32_t)r.x0 | ((uint32_t)r.x1 << 16),
                                  (uint32_t)r.y0 | ((uint32_t)r.y1 << 16));
            if (dkeys) {
                // Gaussians without tiles sort last; they emit nothing, so their
                // place in the depth order never shows.
                const uint32_t dk = cnt ? __float_as_uint(in[u][5]) : 0xffffffffu;
                dkeys[i] = dk;
                dvals[i] = (uint32_t)i;
#pragma unroll
                for (int p = 0; p < 4; ++p) lds_hist_add(s_dh[p], (dk >> (8 * p)) & 0xffu);
            }
            pairs += cnt;
            if (cnt && passes > 0) {
                const uint32_t w = (uint32_t)(r.x1 - r.x0);
                for (int y = r.y0; y < r.y1; ++y)
                    hist_row((uint32_t)y * (uint32_t)tiles_x + (uint32_t)r.x0, w, passes, s_d0, s_h,
                             &full);
            }
            if (cnt && blocks) {
                // the 8x8-tile blocks the rectangle meets, [bx0, bx1) x
                // [by0, by1): +1 at its first corner, -1 past its right and
                // bottom edges, +1 past both (corners off the grid dropped);
                // the 2D prefix sum below turns these into the counts
                const int bx0 = r.x0 >> 3, bx1 = (r.x1 + 7) >> 3;
                const int by0 = r.y0 >> 3, by1 = (r.y1 + 7) >> 3;
                atomicAdd(&s_bh[by0 * bg.bw + bx0], 1);
                if (bx1 < bg.bw) atomicAdd(&s_bh[by0 * bg.bw + bx1], -1);
                if (by1 < bg.bh) {
                    atomicAdd(&s_bh[by1 * bg.bw + bx0], -1);
                    if (bx1 < bg.bw) atomicAdd(&s_bh[by1 * bg.bw + bx1], 1);
                }
            }
        }
    }
    const uint32_t wfull = (uint32_t)wave_sum_u32(full);
    if ((tid & 63) == 0) s_full[tid >> 6] = wfull;
    __syncthreads();
    // digit-0 bin d = full cycles + prefix of the difference array
    const uint32_t all = s_full[0] + s_full[1] + s_full[2] + s_full[3];
    const uint32_t inc = wave_inclusive_scan((uint32_t)s_d0[tid]);
    if ((tid & 63) == 63) s_scan[tid >> 6] = inc;
    __syncthreads();
    uint32_t pre = 0;
    for (int w = 0; w < (tid >> 6); ++w) pre += s_scan[w];
    const uint32_t d0 = all + pre + inc;
    if (passes > 0 && d0) atomicAdd(&tile_hist[tid], d0);
    for (int p = 1; p < passes; ++p) {
        const uint32_t v = s_h[p - 1][tid];
        if (v) atomicAdd(&tile_hist[p * kRadixBins + tid], v);
    }
    if (blocks) {
        // 2D inclusive prefix sum of the difference array: along each block
        // row, then down each block column, one wave per row / column and 64
        // entries per wave scan
        const int lane = tid & 63, wave = tid >> 6;
        for (int rr = wave; rr < bg.bh; rr += kThreads / kWave) {
            uint32_t carry = 0;
            for (int c0 = 0; c0 < bg.bw; c0 += kWave) {
                const int c = c0 + lane;
                const uint32_t v = (c < bg.bw) ? (uint32_t)s_bh[rr * bg.bw + c] : 0u;
                const uint32_t inc = wave_inclusive_scan(v) + carry;
                if (c < bg.bw) s_bh[rr * bg.bw + c] = (int)inc;
                carry = (uint32_t)__builtin_amdgcn_readlane((int)inc, kWave - 1);
            }
        }
        __syncthreads();
        for (int cc = wave; cc < bg.bw; cc += kThreads / kWave) {
            uint32_t carry = 0;
            for (int r0 = 0; r0 < bg.bh; r0 += kWave) {
                const int rr = r0 + lane;
                const uint32_t v = (rr < bg.bh) ? (uint32_t)s_bh[rr * bg.bw + cc] : 0u;
                const uint32_t inc = wave_inclusive_scan(v) + carry;
                if (rr < bg.bh) s_bh[rr * bg.bw + cc] = (int)inc;
                carry = (uint32_t)__builtin_amdgcn_readlane((int)inc, kWave - 1);
            }
        }
        __syncthreads();
        for (int j = tid; j < bg.nb; j += kThreads) {
            const uint32_t v = (uint32_t)s_bh[j];
            if (v) atomicAdd(&block_hist[j], v);
        }
        const uint64_t wp = wave_sum_u64(pairs);
        if ((tid & 63) == 0 && wp) atomicAdd(reinterpret_cast<unsigned long long*>(pair_total),
                                             (unsigned long long)wp);
    }
    if (dkeys) {
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t v = s_dh[p][tid];
            if (v) atomicAdd(&depth_hist[p * kRadixBins + tid], v);
        }
    }
}

// Behind bin_count_kernel (block histogram mode), one work-group: the hand-off
// (bin_finish_body: the pair count and status word to the host, the block and
// segment starts).  A kernel of its own, or a work-group of the depth sort's
// first pass, rather than bin_count's last work-group: on this chip every
// work-group's agent-scope release would write the L2 back once more.
__global__ __launch_bounds__(kThreads) void bin_finish_kernel(BinFinish f) {
    __shared__ uint32_t s_scan[kThreads / kWave];
    __shared__ uint32_t s_v[kThreads / kWave];
    bin_finish_body<kThreads>(f, s_scan, s_v);
}

// Pairs per tile row of the frame, for planning screen bands: each Gaussian's
// rectangle (tile_rect, as bin_count_kernel forms it) adds its width to the
// rows it spans, through a per-work-group difference array in LDS flushed
// with one 64-bit atomic per non-zero entry into diff[0 .. tiles_y].
constexpr int kMaxRowTiles = 4096;  // 65535 rows / 16
__global__ __launch_bounds__(kThreads) void row_pairs_kernel(int n,
                                                             const float* __restrict__ mean2d,
                                                             const float* __restrict__ cov2d,
                                                             int H, int W,
                                                             unsigned long long* __restrict__ diff) {
    __shared__ unsigned long long s_diff[kMaxRowTiles + 1];
    const int tiles_y = (H + 15) / 16;
    for (int j = threadIdx.x; j <= tiles_y; j += kThreads) s_diff[j] = 0ull;
    __syncthreads();
    for (int i = blockIdx.x * kThreads + threadIdx.x; i < n; i += gridDim.x * kThreads) {
        const TileRect r = tile_rect(mean2d[2 * (size_t)i], mean2d[2 * (size_t)i + 1],
                                     cov2d[3 * (size_t)i], cov2d[3 * (size_t)i + 1],
                                     cov2d[3 * (size_t)i + 2], W, H);
        const int w = r.ok ? max(0, r.x1 - r.x0) : 0;
        if (w > 0 && r.y1 > r.y0) {
            atomicAdd(&s_diff[r.y0], (unsigned long long)w);
            atomicAdd(&s_diff[r.y1], (unsigned long long)(-(long long)w));
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j <= tiles_y; j += kThreads) {
        const unsigned long long v = s_diff[j];
        if (v) atomicAdd(&diff[j], v);
    }
}

// flags[i] = 1 when Gaussian i's tile rectangle (tile_rect, as bin_count_kernel
// forms it on this H x W frame), widened by one tile row above and below, holds
// a marked tile, else 0.  sat is the summed-area table of the marked tiles:
// (tiles_y + 1) x (tiles_x + 1) int32, row-major, row 0 and column 0 zero.
// The widening covers a render of the same Gaussians in a screen band, whose
// means are moved by the band's first row: the move can round a mean far above
// the band in its last bit, which moves its rectangle's rows by at most one.
__global__ __launch_bounds__(kThreads) void tiles_touch_kernel(int n,
                                                               const float* __restrict__ mean2d,
                                                               const float* __restrict__ cov2d,
                                                               int H, int W,
                                                               const int32_t* __restrict__ sat,
                                                               uint8_t* __restrict__ flags) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const TileRect r = tile_rect(mean2d[2 * (size_t)i], mean2d[2 * (size_t)i + 1],
                                 cov2d[3 * (size_t)i], cov2d[3 * (size_t)i + 1],
                                 cov2d[3 * (size_t)i + 2], W, H);
    const int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
    const int y0 = max(0, r.y0 - 1), y1 = min(tiles_y, r.y1 + 1);
    bool hit = false;
    if (r.ok && r.x1 > r.x0 && y1 > y0) {
        const int sx = tiles_x + 1;
        hit = sat[y1 * sx + r.x1] - sat[y0 * sx + r.x1] - sat[y1 * sx + r.x0] +
                  sat[y0 * sx + r.x0] >
              0;
    }
    flags[i] = hit ? 1 : 0;
}

// In place: diff[0 .. tiles_y) becomes its inclusive prefix sums (the pairs of
// each tile row).  One work-group.
__global__ __launch_bounds__(kThreads) void row_pairs_scan_kernel(
    int tiles_y, unsigned long long* __restrict__ rows) {
    __shared__ unsigned long long s_carry;
    __shared__ unsigned long long s_w[kThreads / kWave];
    if (threadIdx.x == 0) s_carry = 0ull;
    __syncthreads();
    for (int b = 0; b < tiles_y; b += kThreads) {
        const int j = b + (int)threadIdx.x;
        unsigned long long v = j < tiles_y ? rows[j] : 0ull;
        // inclusive scan over the work-group: waves, then wave totals
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        for (int off = 1; off < 64; off <<= 1) {
            const unsigned long long o = __shfl_up(v, off, kWave);
            if (lane >= off) v += o;
        }
        if (lane == 63) s_w[wave] = v;
        __syncthreads();
        unsigned long long pre = s_carry;
        for (int k = 0; k < wave; ++k) pre += s_w[k];
        if (j < tiles_y) rows[j] = pre + v;
        __syncthreads();
        if (threadIdx.x == kThreads - 1) s_carry = pre + v;
        __syncthreads();
    }
}

// part_rank[p] = the depth rank whose pairs include sort slot p * kSortPartition;
// part_rank[nparts] = one past the last rank with pairs.
__global__ __launch_bounds__(kThreads) void partition_starts_kernel(
    int n, const uint32_t* __restrict__ perm, const uint32_t* __restrict__ counts,
    const uint32_t* __restrict__ offsets, uint64_t m, uint32_t nparts,
    uint32_t* __restrict__ part_rank) {
    const int r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= n) return;
    const uint32_t g = perm[r];
    if (g >= (uint32_t)n) return;
    const uint64_t c = counts[g];
    if (c == 0) return;
    const uint64_t off = offsets[r], end = off + c;
    if (end > m) return;  // inconsistent scan: write nothing
    for (uint64_t p = (off + kSortPartition - 1) / kSortPartition; p <= (end - 1) / kSortPartition;
         ++p)
        part_rank[p] = (uint32_t)r;
    if (end == m) part_rank[nparts] = (uint32_t)r + 1;
}

// identify_tile_ranges_kernel (rasterize.cu:140-166): tile boundaries in the
// sorted tile keys; tiles without pairs keep the zeros written before.
__global__ __launch_bounds__(kThreads) void tile_ranges_kernel(uint64_t m, uint32_t T,
                                                               const uint32_t* __restrict__ tiles,
                                                               int shift,
                                                               int32_t* __restrict__ ranges) {
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= m) return;
    const uint32_t cur = tiles[i] >> shift;
    if (cur >= T || (i > 0 && (tiles[i - 1] >> shift) >= T)) return;  // keys come from [0, T)
    if (i == 0) {
        ranges[2 * (size_t)cur] = 0;
    } else {
        const uint32_t prev = tiles[i - 1] >> shift;
        if (cur != prev) {
            ranges[2 * (size_t)prev + 1] = (int32_t)i;
            ranges[2 * (size_t)cur] = (int32_t)i;
        }
    }
    if (i == m - 1) ranges[2 * (size_t)cur + 1] = (int32_t)m;
}

__global__ __launch_bounds__(kThreads) void full_keys_kernel(uint64_t m,
                                                             const uint32_t* __restrict__ tiles,
                                                             int shift,
                                                             const int32_t* __restrict__ ids,
                                                             const float* __restrict__ depth,
                                                             int n, uint64_t* __restrict__ keys) {
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    if (i >= m) return;
    const int g = ids[i];
    const uint32_t dbits = (g >= 0 && g < n) ? __float_as_uint(depth[g]) : 0xffffffffu;
    keys[i] = ((uint64_t)(tiles[i] >> shift) << 32) | (uint64_t)dbits;
}

__device__ __forceinline__ uint32_t rect_count(const TileRect& tr) {
    return tr.ok ? (uint32_t)(max(0, tr.x1 - tr.x0) * max(0, tr.y1 - tr.y0)) : 0u;
}

__device__ __forceinline__ uint2 rect_word(const TileRect& tr) {
    return make_uint2((uint32_t)tr.x0 | ((uint32_t)tr.x1 << 16),
                      (uint32_t)tr.y0 | ((uint32_t)tr.y1 << 16));
}

__global__ __launch_bounds__(kThreads) void blend_records_kernel(
    int n, const float* __restrict__ mean2d, const float* __restrict__ cov2d,
    const float* __restrict__ colors, const float* __restrict__ alpha,
    BlendRec* __restrict__ recs, int H, int W, uint32_t* __restrict__ counts,
    uint2* __restrict__ rects) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const float mx = mean2d[2 * (size_t)i], my = mean2d[2 * (size_t)i + 1];
    const float a = cov2d[3 * (size_t)i], b = cov2d[3 * (size_t)i + 1], c = cov2d[3 * (size_t)i + 2];
    if (counts) {
        const TileRect tr = tile_rect(mx, my, a, b, c, W, H);
        counts[i] = rect_count(tr);
        rects[i] = rect_word(tr);
    }
    recs[i] = blend_record(mx, my, a, b, c, alpha[i], colors[3 * (size_t)i],
                           colors[3 * (size_t)i + 1], colors[3 * (size_t)i + 2]);
}

// The backward's per-Gaussian pass in one kernel: blend records, tile
// rectangles and counts (as blend_records_kernel forms them), and the
// Gaussian-major slot offsets goff[i] = counts[0] + ... + counts[i - 1] (the
// total to *total) over partitions of kSlotItems x 256 Gaussians (at most
// 512: up to 2^18 Gaussians).  The partition is the work-group's index: a
// partition waits only on the ones before it, which were dispatched before it
// and publish their counts before they wait on anything.  Its offset is a
// fan-in of their published counts (wave_fanin), during which the other
// waves form the records.  Work-groups from `parts` on compute the backward
// blend's per-tile work estimate instead (tile_work_bwd_wave, one wave per
// tile): work independent of the records, in the same launch.
constexpr int kSlotItems = 2;
constexpr int kSlotPartition = kThreads * kSlotItems;

__global__ __launch_bounds__(kThreads) void records_slots_kernel(
    int n, const float* __restrict__ mean2d, const float* __restrict__ cov2d,
    const float* __restrict__ colors, const float* __restrict__ alpha,
    BlendRec* __restrict__ recs, int H, int W, uint32_t* __restrict__ counts,
    uint2* __restrict__ rects, uint32_t* __restrict__ goff, uint64_t* __restrict__ total,
    uint64_t* __restrict__ status, int* __restrict__ err, uint32_t parts, BwdWork bw) {
    __shared__ uint32_t s_wsum[kThreads / kWave];
    __shared__ uint64_t s_base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (blockIdx.x >= parts) {  // whole work-groups: no barriers in this branch
        const int tile = (int)(blockIdx.x - parts) * kWorkTilesPerBlock + wave;
        if (tile < bw.T) tile_work_bwd_wave(bw, tile);
        return;
    }
    const uint64_t part = blockIdx.x;
    const int64_t first = (int64_t)part * kSlotPartition + (int64_t)tid * kSlotItems;
    // every input loaded up front, all loads in flight together
    float in[kSlotItems][9];
#pragma unroll
    for (int j = 0; j < kSlotItems; ++j) {
        const int64_t i = first + j;
        const bool ok = i < n;
        in[j][0] = ok ? mean2d[2 * (size_t)i] : 0.0f;
        in[j][1] = ok ? mean2d[2 * (size_t)i + 1] : 0.0f;
        in[j][2] = ok ? cov2d[3 * (size_t)i] : 0.0f;
        in[j][3] = ok ? cov2d[3 * (size_t)i + 1] : 0.0f;
        in[j][4] = ok ? cov2d[3 * (size_t)i + 2] : 0.0f;
        in[j][5] = ok ? alpha[i] : 0.0f;
        in[j][6] = ok ? colors[3 * (size_t)i] : 0.0f;
        in[j][7] = ok ? colors[3 * (size_t)i + 1] : 0.0f;
        in[j][8] = ok ? colors[3 * (size_t)i + 2] : 0.0f;
    }
    uint32_t cnt[kSlotItems];
    uint32_t sum = 0;
#pragma unroll
    for (int j = 0; j < kSlotItems; ++j) {
        const int64_t i = first + j;
        cnt[j] = 0u;
        if (i < n) {
            const TileRect tr = tile_rect(in[j][0], in[j][1], in[j][2], in[j][3], in[j][4], W, H);
            cnt[j] = rect_count(tr);
            counts[i] = cnt[j];
            rects[i] = rect_word(tr);
        }
        sum += cnt[j];
    }
    const uint32_t inc = wave_inclusive_scan(sum);
    if (lane == 63) s_wsum[wave] = inc;
    __syncthreads();
    uint32_t wpre = 0, btot = 0;
#pragma unroll
    for (int w = 0; w < kThreads / kWave; ++w) {
        if (w < wave) wpre += s_wsum[w];
        btot += s_wsum[w];
    }
    if (wave == 0) {
        const uint64_t excl = wave_fanin(status, (uint32_t)part, (uint64_t)btot, err);
        if (lane == 0) {
            s_base = excl;
            if (part * kSlotPartition + kSlotPartition >= (uint64_t)n) *total = excl + btot;
        }
    }
#pragma unroll
    for (int j = 0; j < kSlotItems; ++j) {
        const int64_t i = first + j;
        if (i < n)
            recs[i] = blend_record(in[j][0], in[j][1], in[j][2], in[j][3], in[j][4], in[j][5],
                                   in[j][6], in[j][7], in[j][8]);
    }
    __syncthreads();
    uint64_t run = s_base + wpre + inc - sum;
#pragma unroll
    for (int j = 0; j < kSlotItems; ++j) {
        const int64_t i = first + j;
        if (i < n) goff[i] = (uint32_t)run;
        run += cnt[j];
    }
}

inline unsigned blocks_for(uint64_t n) { return (unsigned)((n + kThreads - 1) / kThreads); }

}  // namespace

hipError_t launch_bin_count(int n, const float* mean2d, const float* cov2d, const float* depth,
                            int H, int W, uint32_t* counts, uint2* rects, uint32_t* dkeys,
                            uint32_t* dvals, int tile_passes, uint32_t* tile_hist,
                            uint32_t* depth_hist, uint32_t* block_hist, uint64_t* pair_total,
                            uint32_t* block_start, uint32_t* seg_start, uint64_t* host_total,
                            int* status, hipStream_t st, bool finish) {
    if (n <= 0) return hipSuccess;
    if (tile_passes < 0 || tile_passes > 4) return hipErrorInvalidValue;
    const BlockGrid bg = block_grid((W + 15) / 16, (H + 15) / 16);
    if (block_hist && (bg.nb > kMaxBlocks || !pair_total || !block_start || !seg_start))
        return hipErrorInvalidValue;
    // few work-groups: each flushes its histograms with one global atomic per
    // bin.  One per two CUs up to 2^19 Gaussians; beyond, one per CU, so that
    // each thread's grid-strided loop stays short (its loads are not
    // overlapped across iterations).  At 1M Gaussians: 128 groups 170 us, 256
    // 150 us, 512 157 us, 1024 199 us (bin_count + depth sort); at 100k, 64
    // groups 21.0 us, 128 20.0, 256 27.5 (bin_count).
    const unsigned blocks = std::min(blocks_for(n), n >= (1 << 19) ? 256u : 128u);
    hipLaunchKernelGGL(bin_count_kernel, dim3(blocks), dim3(kThreads), 0, st, n, mean2d, cov2d,
                       depth, H, W, counts, rects, dkeys, dvals, tile_passes, tile_hist,
                       depth_hist, bg, block_hist, pair_total);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !block_hist || !finish) return e;
    const BinFinish f{bg.nb, block_hist, pair_total, block_start, seg_start, host_total, status};
    hipLaunchKernelGGL(bin_finish_kernel, dim3(1), dim3(kThreads), 0, st, f);
    return hipGetLastError();
}

hipError_t launch_row_pairs(int n, const float* mean2d, const float* cov2d, int H, int W,
                            uint64_t* rows, hipStream_t st) {
    const int tiles_y = (H + 15) / 16;
    if (tiles_y > kMaxRowTiles) return hipErrorInvalidValue;
    hipError_t e = zero_fill(rows, (size_t)(tiles_y + 1) * sizeof(uint64_t), st);
    if (e != hipSuccess) return e;
    if (n > 0) {
        const unsigned blocks = std::min(blocks_for(n), 1024u);
        hipLaunchKernelGGL(row_pairs_kernel, dim3(blocks), dim3(kThreads), 0, st, n, mean2d,
                           cov2d, H, W, reinterpret_cast<unsigned long long*>(rows));
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(row_pairs_scan_kernel, dim3(1), dim3(kThreads), 0, st, tiles_y,
                       reinterpret_cast<unsigned long long*>(rows));
    return hipGetLastError();
}

hipError_t launch_tiles_touch(int n, const float* mean2d, const float* cov2d, int H, int W,
                              const int32_t* sat, uint8_t* flags, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(tiles_touch_kernel, dim3(blocks_for((uint64_t)n)), dim3(kThreads), 0, st,
                       n, mean2d, cov2d, H, W, sat, flags);
    return hipGetLastError();
}

hipError_t launch_partition_starts(int n, const uint32_t* perm, const uint32_t* counts,
                                   const uint32_t* offsets, uint64_t m, uint32_t* part_rank,
                                   hipStream_t st) {
    if (n <= 0 || m == 0) return hipSuccess;
    const uint32_t nparts = (uint32_t)((m + kSortPartition - 1) / kSortPartition);
    hipLaunchKernelGGL(partition_starts_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n,
                       perm, counts, offsets, m, nparts, part_rank);
    return hipGetLastError();
}

hipError_t launch_tile_ranges(uint64_t m, uint32_t T, const uint32_t* sorted_tiles, int shift,
                              int32_t* ranges, hipStream_t st) {
    if (m == 0) return hipSuccess;
    hipLaunchKernelGGL(tile_ranges_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, m, T,
                       sorted_tiles, shift, ranges);
    return hipGetLastError();
}

hipError_t launch_full_keys(uint64_t m, const uint32_t* sorted_tiles, int shift,
                            const int32_t* ids, const float* depth, int n, uint64_t* keys,
                            hipStream_t st) {
    if (m == 0) return hipSuccess;
    hipLaunchKernelGGL(full_keys_kernel, dim3(blocks_for(m)), dim3(kThreads), 0, st, m,
                       sorted_tiles, shift, ids, depth, n, keys);
    return hipGetLastError();
}

// One kernel up to 2^18 Gaussians (at 100k: 12.2 us against 7.0 + 9.5); beyond,
// the records kernel and the 4096-Gaussian-partition scan, whose look-back
// chain is 8x shorter (at 1M: 45 us against 75 for the one kernel).
constexpr int kRecordsSlotsFusedMax = 1 << 18;

size_t records_slots_control_bytes(int n) {
    const size_t parts = ((size_t)std::max(n, 1) + kSlotPartition - 1) / kSlotPartition;
    return std::max(256 + parts * 8, scan_control_bytes(n));
}

hipError_t launch_records_slots(int n, const float* mean2d, const float* cov2d,
                                const float* colors, const float* alpha, void* recs, int H, int W,
                                uint32_t* counts, uint2* rects, uint32_t* goff, uint64_t* total,
                                void* control, int* err, hipStream_t st, const int32_t* ranges,
                                uint64_t num_pairs, const int32_t* ncontrib, uint32_t* work,
                                bool* work_done) {
    if (work_done) *work_done = false;
    if (n <= 0) return hipSuccess;
    if (n > kRecordsSlotsFusedMax) {
        hipLaunchKernelGGL(blend_records_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n,
                           mean2d, cov2d, colors, alpha, static_cast<BlendRec*>(recs), H, W,
                           counts, rects);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        return launch_scan_counts(n, nullptr, counts, goff, total, control, err, st);
    }
    const unsigned parts = (unsigned)(((size_t)n + kSlotPartition - 1) / kSlotPartition);
    static_assert(kRecordsSlotsFusedMax / kSlotPartition <= 64 * kFanPerLane,
                  "the fan-in covers every partition");
    uint64_t* status = reinterpret_cast<uint64_t*>(static_cast<char*>(control) + 256);
    BwdWork bw{};
    unsigned work_groups = 0;
    if (work && ranges && ncontrib) {
        static_assert(kThreads == kWorkTilesPerBlock * kWave, "one wave per tile");
        bw = make_bwd_work(H, W, ranges, num_pairs, ncontrib, work);
        work_groups = (unsigned)((bw.T + kWorkTilesPerBlock - 1) / kWorkTilesPerBlock);
    }
    hipLaunchKernelGGL(records_slots_kernel, dim3(parts + work_groups), dim3(kThreads), 0, st, n,
                       mean2d, cov2d, colors, alpha, static_cast<BlendRec*>(recs), H, W, counts,
                       rects, goff, total, status, err, parts, bw);
    if (work_done) *work_done = work_groups > 0;
    return hipGetLastError();
}

hipError_t launch_blend_records(int n, const float* mean2d, const float* cov2d,
                                const float* colors, const float* alpha, void* recs,
                                hipStream_t st, int H, int W, uint32_t* counts, uint2* rects) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(blend_records_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n,
                       mean2d, cov2d, colors, alpha, static_cast<BlendRec*>(recs), H, W, counts,
                       rects);
    return hipGetLastError();
}

}  // namespace gsr
