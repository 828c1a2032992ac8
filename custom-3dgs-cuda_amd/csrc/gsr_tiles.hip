// gsr_tiles.hip — two-level tile binning: the (tile, Gaussian) pairs in
// (tile, depth rank) order without a sort over the pairs.
//
// The pairs are the tiles of each Gaussian's tile rectangle (rasterize.cu:
// 98-135); the reference sorts them on (tile << 32 | depth bits), which with
// the depth-ordered Gaussians (stable on the Gaussian index) is a stable
// partition of the depth order into one list per tile.  Here that partition
// is done in two levels of 64-way buckets:
//   level 1: each Gaussian, in depth order, goes to the 8x8-tile blocks its
//            rectangle meets;
//   level 2: each block's list goes to the block's 64 tiles.
// Every level is three kernels without inter-work-group waits:
//   count   — one wave per 64 consecutive list entries; a ballot of "this
//             lane's rectangle covers bucket b" gives the bucket's count for
//             the wave and, through the lanes below, each lane's rank in it;
//   scan    — per bucket, the exclusive prefix of the counts over the waves
//             in list order (plus the bucket's start);
//   scatter — each lane writes its entry at start + prefix + rank.
// Ranks follow lane order and prefixes follow wave order, so each bucket's
// list keeps the input order: the result is the reference's sorted ids, and
// the tile ranges come from the per-tile totals.
//
// HBM traffic: level 1 reads the depth order and rectangles twice and writes
// M_1 block entries (M_1 = sum over Gaussians of blocks met, ~5 per Gaussian
// at 1080p); level 2 reads the block lists twice and writes the M pair ids
// once, in runs of consecutive addresses (one run per wave and tile).
#include <algorithm>

#include "gsr_internal.h"
#include "gsr_common.h"
#include "gsr_group.h"

namespace gsr {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPer = kThreads / kWave;

struct Rect {
    int x0, x1, y0, y1;  // tiles [x0, x1) x [y0, y1)
};

__device__ __forceinline__ Rect unpack_rect(uint2 rc) {
    return Rect{(int)(rc.x & 0xffffu), (int)(rc.x >> 16), (int)(rc.y & 0xffffu),
                (int)(rc.y >> 16)};
}

__device__ __forceinline__ uint32_t uniform(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

// The work-group's index with the work-groups of one XCD made consecutive.
// Work-groups are dealt to the 8 XCDs round-robin (work-group i runs on XCD
// i % 8); renumbered, the XCD of work-group i takes a contiguous share of the
// indices, so neighbouring segments (whose runs of a tile share cache lines)
// are written through the same L2, which merges them into whole lines.
// Grids that are not a multiple of 8 keep their order.
__device__ __forceinline__ uint32_t xcd_group() {
    const uint32_t g = blockIdx.x, n = gridDim.x;
    return (n % 8u == 0u) ? (g % 8u) * (n / 8u) + g / 8u : g;
}

// tile_scatter's 32-bit addressing.  A tile's run starts at list position
// base and holds up to kWave entries (rank 0..63).  The run's stores take the
// byte offset (base - b0) * 4 + rank * 4 from ids + b0 in uint32 arithmetic,
// which is exact only when the whole run, not just its start, lies within
// 2^30 entries of b0.  run_fits is the condition; run_byte_offset the offset.
constexpr uint32_t kRunSpan = 1u << 30;
__host__ __device__ constexpr bool run_fits(uint32_t base, uint32_t b0, uint64_t m) {
    return base >= b0 && base - b0 <= kRunSpan - (uint32_t)kWave &&
           (uint64_t)base + (uint64_t)kWave <= m;
}
__host__ __device__ constexpr uint32_t run_byte_offset(uint32_t base, uint32_t b0,
                                                       uint32_t rank) {
    return ((base - b0) << 2) + (rank << 2);
}
// The largest admitted run's last store is exact; one entry further is
// refused (the run would reach 2^30 entries from b0, whose byte offset wraps).
static_assert(run_fits(7u + kRunSpan - 64u, 7u, 1ull << 40), "largest run admitted");
static_assert(!run_fits(7u + kRunSpan - 63u, 7u, 1ull << 40), "a run reaching 2^30 refused");
static_assert(!run_fits(7u + kRunSpan - 1u, 7u, 1ull << 40), "a run wrapping refused");
static_assert((uint64_t)run_byte_offset(7u + kRunSpan - 64u, 7u, 63u) ==
                  ((uint64_t)(kRunSpan - 64u) + 63u) * 4u,
              "the largest admitted offset does not wrap");
static_assert(!run_fits(6u, 7u, 1ull << 40), "a run before b0 refused");
static_assert(!run_fits(100u, 7u, 163u) && run_fits(99u, 7u, 163u), "runs end at m");

// Lanes of m below this one.
__device__ __forceinline__ uint32_t rank_in(uint64_t m) {
    return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                     __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// ---- level 1: depth order -> block lists -----------------------------------

// One lane's depth rank: its Gaussian and the block rectangle of its tile
// rectangle as origin and extent (has: the Gaussian has tiles).
struct RankLane {
    uint32_t g;
    int bx0, by0;
    uint32_t bw, bh;
    bool has;
    Rect t;  // the tile rectangle
};

// A tile rectangle clipped to the 8x8-tile block at tile (ox, oy), which it
// meets, in 12 bits: x0 and y0 in [0, 8) and the extents less one.
__device__ __forceinline__ uint16_t local_rect(const Rect& t, int ox, int oy) {
    const int lx0 = max(t.x0 - ox, 0), lx1 = min(t.x1 - ox, 8);
    const int ly0 = max(t.y0 - oy, 0), ly1 = min(t.y1 - oy, 8);
    return (uint16_t)(lx0 | ((lx1 - lx0 - 1) << 3) | (ly0 << 6) | ((ly1 - ly0 - 1) << 9));
}

// drects: the rectangles already in depth order (rank_rects_kernel), read in
// rank order instead of by Gaussian id.
__device__ __forceinline__ RankLane rank_lane(int n, const uint32_t* __restrict__ perm,
                                              const uint2* __restrict__ rects,
                                              const uint2* __restrict__ drects, int64_t r) {
    RankLane L{0u, 0, 0, 0u, 0u, false, Rect{0, 0, 0, 0}};
    if (r < n) {
        const uint32_t g = perm[r];
        if (g < (uint32_t)n) {
            const Rect t = unpack_rect(drects ? drects[r] : rects[g]);
            if (t.x1 > t.x0 && t.y1 > t.y0) {
                L.g = g;
                L.t = t;
                L.bx0 = t.x0 >> 3;
                L.by0 = t.y0 >> 3;
                L.bw = (uint32_t)(((t.x1 + 7) >> 3) - L.bx0);
                L.bh = (uint32_t)(((t.y1 + 7) >> 3) - L.by0);
                L.has = true;
            }
        }
    }
    return L;
}

// Level-1 work item of one wave: chunk c of 64 depth ranks against window w
// of 64 consecutive block indices.  Adjacent waves share the chunk.
struct ChunkWindow {
    int chunk, window;
};

__device__ __forceinline__ ChunkWindow chunk_window(int windows) {
    const int id = (int)uniform(blockIdx.x * kWavesPer + (threadIdx.x >> 6));
    return ChunkWindow{id / windows, id - (id / windows) * windows};
}

// 64-bit value of lane src (all lanes active).
__device__ __forceinline__ uint64_t lane_u64(uint64_t v, int src) {
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, kWave);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, kWave);
    return ((uint64_t)hi << 32) | lo;
}

// The lanes whose rectangle meets block (row sy, column sx) are
// rows[sy] & cols[sx]: one ballot per block row and per block column of the
// window gives every block's count and every lane's rank.  Lane j holds the
// mask of the window's j-th row (rowv) and j-th column (colv); the window's
// blocks [s0, s1) span rows sy_a.. and, in order, the columns col_base + j
// (mod bw): all bw columns when bw <= 64, else 64 distinct ones.
struct WindowMasks {
    int s0, s1, sy_a, sx_a, col_base, nrows, ncols;
    uint64_t rowv, colv;
};

__device__ __forceinline__ WindowMasks window_masks(const RankLane& L, const BlockGrid& bg,
                                                    int w) {
    const int lane = lane_id();
    WindowMasks W;
    W.s0 = w * kWave;
    W.s1 = min(W.s0 + kWave, bg.nb);
    W.sy_a = W.s0 / bg.bw;
    W.sx_a = W.s0 - W.sy_a * bg.bw;
    W.nrows = (W.s1 - 1) / bg.bw - W.sy_a + 1;
    W.ncols = min(bg.bw, kWave);
    W.col_base = (bg.bw <= kWave) ? 0 : W.sx_a;
    W.rowv = 0;
    W.colv = 0;
    const uint64_t lanes = ballot(L.has);
    if (lanes == 0) return W;
    for (int j = 0; j < W.nrows; ++j) {
        const uint64_t m = lanes & ballot((uint32_t)(W.sy_a + j - L.by0) < L.bh);
        W.rowv = (lane == j) ? m : W.rowv;
    }
    for (int j = 0; j < W.ncols; ++j) {
        int c = W.col_base + j;
        c -= (c >= bg.bw) ? bg.bw : 0;
        const uint64_t m = ballot((uint32_t)(c - L.bx0) < L.bw);
        W.colv = (lane == j) ? m : W.colv;
    }
    return W;
}

// Index of block column sx among the window's columns.
__device__ __forceinline__ int window_col(const WindowMasks& W, const BlockGrid& bg, int sx) {
    const int d = sx - W.col_base;
    return d < 0 ? d + bg.bw : d;
}

// counts[b * cstride + c] = how many of chunk c's 64 ranks meet block b, for
// every block (zeros included); lane l counts block 64 w + l.
// Records of the blends, formed by the count kernel's work-groups from
// `first` on (one Gaussian per thread), when `recs` is set.
struct RecordArgs {
    const float* mean2d;
    const float* cov2d;
    const float* colors;
    const float* alpha;
    BlendRec* recs;
    uint32_t first;
};

__global__ __launch_bounds__(kThreads) void block_count_kernel(
    int n, const uint32_t* __restrict__ perm, const uint2* __restrict__ rects,
    const uint2* __restrict__ drects, BlockGrid bg,
    int chunks, int windows, int cstride, uint32_t* __restrict__ counts, RecordArgs ra) {
    if (ra.recs && blockIdx.x >= ra.first) {
        const int i = (int)(blockIdx.x - ra.first) * kThreads + (int)threadIdx.x;
        if (i < n) {
            const float mx = ra.mean2d[2 * (size_t)i], my = ra.mean2d[2 * (size_t)i + 1];
            const float a = ra.cov2d[3 * (size_t)i], b = ra.cov2d[3 * (size_t)i + 1],
                        c = ra.cov2d[3 * (size_t)i + 2];
            ra.recs[i] = blend_record(mx, my, a, b, c, ra.alpha[i], ra.colors[3 * (size_t)i],
                                      ra.colors[3 * (size_t)i + 1], ra.colors[3 * (size_t)i + 2]);
        }
        return;
    }
    const int lane = lane_id();
    const ChunkWindow cw = chunk_window(windows);
    if (cw.chunk >= chunks) return;
    const RankLane L = rank_lane(n, perm, rects, drects, (int64_t)cw.chunk * kWave + lane);
    const WindowMasks W = window_masks(L, bg, cw.window);
    const int s = W.s0 + lane;
    const int sy = (W.sx_a + lane) / bg.bw;  // rows below sy_a
    const int sx = W.sx_a + lane - sy * bg.bw;
    const uint64_t m = lane_u64(W.rowv, min(sy, kWave - 1)) &
                       lane_u64(W.colv, min(window_col(W, bg, sx), kWave - 1));
    if (s < W.s1) counts[(size_t)s * cstride + cw.chunk] = (uint32_t)popc64(m);
}

// Per block b: the chunk counts replaced by block_start[b] + their exclusive
// prefix (the list position of each chunk's first entry in b), and
// seg_owner[k] = b for b's level-2 segments.  A column total that differs
// from the binning's block histogram sets err bit 2.
__global__ __launch_bounds__(kThreads) void block_scan_kernel(
    int chunks, int cstride, uint32_t* __restrict__ counts, const uint32_t* __restrict__ hist,
    const uint32_t* __restrict__ block_start, const uint32_t* __restrict__ seg_start,
    uint32_t* __restrict__ seg_owner, uint32_t seg_cap, int* __restrict__ err) {
    __shared__ uint32_t s_w[kWavesPer];
    const int b = blockIdx.x, tid = threadIdx.x;
    uint4* col = reinterpret_cast<uint4*>(counts + (size_t)b * cstride);
    const uint32_t start = block_start[b];
    uint32_t carry = start;
    for (int base = 0; base < chunks; base += 4 * kThreads) {
        const int i = base + 4 * tid;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (i < chunks) v = col[i / 4];
        if (i + 1 >= chunks) v.y = 0u;
        if (i + 2 >= chunks) v.z = 0u;
        if (i + 3 >= chunks) v.w = 0u;
        uint32_t tot;
        const uint32_t ex = group_exclusive_scan<kThreads>(v.x + v.y + v.z + v.w, s_w, &tot);
        if (i < chunks) {
            const uint32_t p0 = carry + ex;
            col[i / 4] = make_uint4(p0, p0 + v.x, p0 + v.x + v.y, p0 + v.x + v.y + v.z);
        }
        carry += tot;
    }
    if (tid == 0 && carry - start != hist[b]) atomicOr(err, 2);
    const uint32_t k1 = min(seg_start[b + 1], seg_cap);
    for (uint32_t k = seg_start[b] + tid; k < k1; k += kThreads) seg_owner[k] = b;
}

// Each rank's Gaussian id into the lists of the blocks it meets, at the
// chunk's position in the block plus the lane's rank among the chunk's lanes
// meeting the block.  Each lane walks its own blocks in the window.  Positions
// at or beyond cap are dropped.
__global__ __launch_bounds__(kThreads) void block_scatter_kernel(
    int n, const uint32_t* __restrict__ perm, const uint2* __restrict__ rects,
    const uint2* __restrict__ drects, BlockGrid bg,
    int chunks, int windows, int cstride, const uint32_t* __restrict__ pos,
    uint32_t* __restrict__ lists, uint16_t* __restrict__ lrects, uint64_t cap) {
    __shared__ uint64_t s_row[kWavesPer][kWave];
    __shared__ uint64_t s_col[kWavesPer][kWave];
    __shared__ uint32_t s_base[kWavesPer][kWave];
    const int lane = lane_id(), wave = threadIdx.x >> 6;
    const ChunkWindow cw = chunk_window(windows);
    if (cw.chunk >= chunks) return;
    const RankLane L = rank_lane(n, perm, rects, drects, (int64_t)cw.chunk * kWave + lane);
    const WindowMasks W = window_masks(L, bg, cw.window);
    const int b = W.s0 + lane;
    s_row[wave][lane] = W.rowv;
    s_col[wave][lane] = W.colv;
    s_base[wave][lane] = (b < W.s1) ? pos[(size_t)b * cstride + cw.chunk] : 0u;
    __builtin_amdgcn_wave_barrier();
    if (!L.has) return;
    const uint64_t below = lanemask_lt();
    const int y1 = min(L.by0 + (int)L.bh, W.sy_a + W.nrows);
    for (int sy = max(L.by0, W.sy_a); sy < y1; ++sy) {
        const uint64_t rm = s_row[wave][sy - W.sy_a];
        for (int sx = L.bx0; sx < L.bx0 + (int)L.bw; ++sx) {
            const int s = sy * bg.bw + sx;
            if (s < W.s0 || s >= W.s1) continue;
            const uint64_t m = rm & s_col[wave][window_col(W, bg, sx)];
            const uint64_t p = (uint64_t)s_base[wave][s - W.s0] + (uint64_t)popc64(m & below);
            if (p < cap) {
                lists[p] = L.g;
                lrects[p] = local_rect(L.t, sx * 8, sy * 8);
            }
        }
    }
}

// drects[r] = rects[perm[r]]: the depth order's rectangles, gathered once so
// that both level-1 passes read them in rank order.
__global__ __launch_bounds__(kThreads) void rank_rects_kernel(int n,
                                                              const uint32_t* __restrict__ perm,
                                                              const uint2* __restrict__ rects,
                                                              uint2* __restrict__ drects) {
    const int r = blockIdx.x * kThreads + threadIdx.x;
    if (r >= n) return;
    const uint32_t g = perm[r];
    drects[r] = (g < (uint32_t)n) ? rects[g] : make_uint2(0u, 0u);
}

// ---- level 2: block lists -> tile lists ------------------------------------

// One lane of a level-2 segment (64 consecutive entries of one block's list):
// its Gaussian and its rectangle within the block's 8x8 tiles (origin and
// extent; extent 0 when the lane holds no entry).
struct SegLane {
    uint32_t g;
    int lx0, ly0;
    uint32_t lw, lh;
};

// The entry's id (with_id) and its local rectangle, written beside it by the
// level-1 scatter, so level 2 reads both in list order.
template <bool with_id>
__device__ __forceinline__ SegLane seg_lane(const uint32_t* __restrict__ lists,
                                            const uint16_t* __restrict__ lrects, uint32_t first,
                                            uint32_t end, uint64_t cap, int n) {
    SegLane S{0u, 0, 0, 0u, 0u};
    const uint32_t e = first + (uint32_t)lane_id();
    if (e < end && e < cap) {
        if constexpr (with_id) {
            const uint32_t g = lists[e];
            if (g >= (uint32_t)n) return S;
            S.g = g;
        }
        const uint32_t lr = lrects[e];
        S.lx0 = (int)(lr & 7u);
        S.lw = ((lr >> 3) & 7u) + 1u;
        S.ly0 = (int)((lr >> 6) & 7u);
        S.lh = ((lr >> 9) & 7u) + 1u;
    }
    return S;
}

// Lanes covering tile row r / tile column c of the block.
__device__ __forceinline__ uint64_t seg_row(const SegLane& S, int r) {
    return ballot((uint32_t)(r - S.ly0) < S.lh);
}
__device__ __forceinline__ uint64_t seg_col(const SegLane& S, int c) {
    return ballot((uint32_t)(c - S.lx0) < S.lw);
}

struct SegInfo {
    uint32_t first, end;  // the segment's entries in the block lists
    int ox, oy;           // the block's first tile
};

__device__ __forceinline__ SegInfo seg_info(uint32_t k, const uint32_t* __restrict__ seg_owner,
                                            const uint32_t* __restrict__ seg_start,
                                            const uint32_t* __restrict__ block_start,
                                            int bw, int nb) {
    const uint32_t b = min(uniform(seg_owner[k]), (uint32_t)(nb - 1));
    SegInfo I;
    I.first = uniform(block_start[b]) + (k - uniform(seg_start[b])) * (uint32_t)kWave;
    I.end = uniform(block_start[b + 1]);
    const int by = (int)b / bw;
    I.ox = ((int)b - by * bw) * 8;
    I.oy = by * 8;
    return I;
}

// Whether the block's tile of this lane (lane t: tile t of the 8 x 8 block at
// (ox, oy)) is on the screen and its list is to be built: skip (optional) marks
// tiles whose lists stay empty.
__device__ __forceinline__ bool lane_tile_live(const BlockGrid& bg, int ox, int oy,
                                               const uint8_t* __restrict__ skip) {
    const int lane = lane_id();
    const int tx = ox + (lane & 7), ty = oy + (lane >> 3);
    const bool on = tx < bg.tiles_x && ty < bg.tiles_y;
    return on && !(skip && skip[(size_t)ty * bg.tiles_x + tx]);
}

// tcount[k * 64 + t] = entries of segment k covering the block's tile t
// (rows[t / 8] & cols[t % 8]; 0 for a skipped tile).  Segments k <
// seg_start[nb] (at most seg_cap), grid-strided.
__global__ __launch_bounds__(kThreads) void tile_count_kernel(
    int n, BlockGrid bg, const uint32_t* __restrict__ seg_owner,
    const uint32_t* __restrict__ seg_start, const uint32_t* __restrict__ block_start,
    const uint32_t* __restrict__ lists, uint64_t cap, const uint16_t* __restrict__ lrects,
    uint32_t seg_cap, uint32_t* __restrict__ tcount, const uint8_t* __restrict__ skip) {
    const uint32_t nseg = min(uniform(seg_start[bg.nb]), seg_cap);
    const uint32_t stride = gridDim.x * kWavesPer;
    const int lane = lane_id();
    for (uint32_t k = uniform(blockIdx.x * kWavesPer + (threadIdx.x >> 6)); k < nseg;
         k += stride) {
        const SegInfo I = seg_info(k, seg_owner, seg_start, block_start, bg.bw, bg.nb);
        const SegLane S = seg_lane<false>(lists, lrects, I.first, I.end, cap, n);
        uint64_t rowv = 0, colv = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint64_t r = seg_row(S, j), c = seg_col(S, j);
            rowv = (lane == j) ? r : rowv;
            colv = (lane == j) ? c : colv;
        }
        const uint64_t m = lane_u64(rowv, lane >> 3) & lane_u64(colv, lane & 7);
        const bool keep = !skip || lane_tile_live(bg, I.ox, I.oy, skip);
        tcount[(size_t)k * kWave + lane] = keep ? (uint32_t)popc64(m) : 0u;
    }
}

// Per block: each tile's segment counts replaced by their exclusive prefix
// over the block's segments, and the tile's total to ttotal (tiles on the
// screen only).  kScanWaves waves split the segments into consecutive runs
// (one work-group per block: a block's run is the serial part).
constexpr int kScanWaves = 16;
__global__ __launch_bounds__(kScanWaves * kWave) void tile_scan_kernel(
    BlockGrid bg, const uint32_t* __restrict__ seg_start, uint32_t seg_cap,
    uint32_t* __restrict__ tcount, uint32_t* __restrict__ ttotal) {
    __shared__ uint32_t s_sum[kScanWaves][kWave];
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t k0 = min(seg_start[b], seg_cap);
    const uint32_t R = min(seg_start[b + 1], seg_cap) - k0;
    const uint32_t per = (R + kScanWaves - 1) / kScanWaves;
    const uint32_t r0 = k0 + min(R, (uint32_t)wave * per);
    const uint32_t r1 = k0 + min(R, (uint32_t)(wave + 1) * per);
    uint32_t sum = 0;
#pragma unroll 8
    for (uint32_t k = r0; k < r1; ++k) sum += tcount[(size_t)k * kWave + lane];
    s_sum[wave][lane] = sum;
    __syncthreads();
    uint32_t run = 0, total = 0;
#pragma unroll
    for (int w = 0; w < kScanWaves; ++w) {
        run += (w < wave) ? s_sum[w][lane] : 0u;
        total += s_sum[w][lane];
    }
#pragma unroll 8
    for (uint32_t k = r0; k < r1; ++k) {
        const uint32_t v = tcount[(size_t)k * kWave + lane];
        tcount[(size_t)k * kWave + lane] = run;
        run += v;
    }
    if (wave == 0) {
        const int by = b / bg.bw;
        const int tx = (b - by * bg.bw) * 8 + (lane & 7), ty = by * 8 + (lane >> 3);
        if (tx < bg.tiles_x && ty < bg.tiles_y) ttotal[(size_t)ty * bg.tiles_x + tx] = total;
    }
}

// The tile ranges from the tile totals: one work-group of 1024 threads.
constexpr int kStartsThreads = 1024;
__global__ __launch_bounds__(kStartsThreads) void tile_starts_kernel(
    int T, const uint32_t* __restrict__ ttotal, uint64_t m, int2* __restrict__ ranges,
    int* __restrict__ err, bool at_most) {
    __shared__ uint32_t s_w[kStartsThreads / kWave];
    tile_starts_body<kStartsThreads>(T, ttotal, m, ranges, err, s_w, at_most);
}

// Each segment entry's Gaussian id into the lists of the tiles it covers, at
// the tile's start + the segment's prefix + the lane's rank.  The tile masks
// rows[t / 8] & cols[t % 8] are wave-uniform.  Positions at or beyond m are
// dropped, and so are the entries of skipped tiles (skip optional).
__global__ __launch_bounds__(kThreads) void tile_scatter_kernel(
    int n, BlockGrid bg, const uint32_t* __restrict__ seg_owner,
    const uint32_t* __restrict__ seg_start, const uint32_t* __restrict__ block_start,
    const uint32_t* __restrict__ lists, uint64_t cap, const uint16_t* __restrict__ lrects,
    uint32_t seg_cap, const uint32_t* __restrict__ tcount, const int2* __restrict__ ranges,
    uint64_t m, uint32_t* __restrict__ ids, const uint8_t* __restrict__ skip) {
    const uint32_t nseg = min(uniform(seg_start[bg.nb]), seg_cap);
    const uint32_t stride = gridDim.x * kWavesPer;
    const int lane = lane_id();
    for (uint32_t k = uniform(xcd_group() * kWavesPer + (threadIdx.x >> 6)); k < nseg;
         k += stride) {
        const SegInfo I = seg_info(k, seg_owner, seg_start, block_start, bg.bw, bg.nb);
        const SegLane S = seg_lane<true>(lists, lrects, I.first, I.end, cap, n);
        // lane t: where segment k's entries of tile t begin (its list start
        // plus the segment's prefix); the block's first built tile (lists are
        // laid out in row-major tile order) has the lowest list start, b0,
        // and each run is addressed from ids + b0
        const int tx = I.ox + (lane & 7), ty = I.oy + (lane >> 3);
        const bool on = lane_tile_live(bg, I.ox, I.oy, skip);
        // bit t: tile t's list is built (scalar)
        const uint64_t live = ballot(on);
        uint32_t lstart = 0, base = 0;
        if (on) {
            lstart = (uint32_t)ranges[(size_t)ty * bg.tiles_x + tx].x;
            base = lstart + tcount[(size_t)k * kWave + lane];
        }
        const uint32_t b0 = (uint32_t)__builtin_amdgcn_readlane(
            (int)lstart, live ? (int)__builtin_ctzll(live) : 0);
        // in_row[r] / in_col[c]: this lane covers tile row r / column c; as
        // lane masks they are the ballots, so the lanes of tile (r, c) are
        // selected with scalar ANDs
        bool in_row[8], in_col[8];
        uint64_t rows[8], cols[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            in_row[j] = (uint32_t)(j - S.ly0) < S.lh;
            in_col[j] = (uint32_t)(j - S.lx0) < S.lw;
            rows[j] = ballot(in_row[j]);
            cols[j] = ballot(in_col[j]);
        }
        // The lanes of tile t's mask write positions b_t + their rank in it.
        // When every run b_t + [0, 64) lies in [b0, m) and within 2^30 entries
        // of b0 (all but the list's last entries, for consistent counts), the
        // stores take a 32-bit byte offset from ids + b0 and no position needs
        // its own check.
        const bool fits = ballot(on && !run_fits(base, b0, m)) == 0ull;
        if (fits) {
            uint32_t* run0 = ids + b0;
            const uint32_t dq = run_byte_offset(base, b0, 0u);  // this lane's tile's run
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                if (((live >> t) & 1u) && in_row[t >> 3] && in_col[t & 7]) {
                    const uint32_t rank = rank_in(rows[t >> 3] & cols[t & 7]);
                    const uint32_t off =
                        (rank << 2) + (uint32_t)__builtin_amdgcn_readlane((int)dq, t);
                    *reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(run0) + off) = S.g;
                }
            }
        } else {
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                const uint64_t mk = rows[t >> 3] & cols[t & 7];
                if (mk == 0 || !((live >> t) & 1u)) continue;
                const uint64_t p = (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)base, t) +
                                   (uint64_t)rank_in(mk);
                if (in_row[t >> 3] && in_col[t & 7] && p < m) ids[p] = S.g;
            }
        }
    }
}

// keys[i] = (tile << 32) | depth bits of ids[i], one wave per tile.
__global__ __launch_bounds__(kThreads) void range_keys_kernel(int T,
                                                              const int2* __restrict__ ranges,
                                                              const int32_t* __restrict__ ids,
                                                              const float* __restrict__ depth,
                                                              int n, uint64_t m,
                                                              uint64_t* __restrict__ keys) {
    const int t = (int)uniform(blockIdx.x * kWavesPer + (threadIdx.x >> 6));
    if (t >= T) return;
    const int2 r = ranges[t];
    for (int64_t i = (int64_t)r.x + lane_id(); i < (int64_t)r.y && i < (int64_t)m; i += kWave) {
        const int g = ids[i];
        const uint32_t dbits = (g >= 0 && g < n) ? __float_as_uint(depth[g]) : 0xffffffffu;
        keys[i] = ((uint64_t)(uint32_t)t << 32) | (uint64_t)dbits;
    }
}

inline unsigned groups_for(uint64_t waves) {
    return (unsigned)((waves + kWavesPer - 1) / kWavesPer);
}

// Work-groups of the grid-strided segment kernels: enough for the bound on
// segments, at most 8 per CU of a 256-CU device.
// Pair lists beyond which tile_scatter runs fewer work-groups (1 GB of ids).
constexpr uint64_t kScatterThrottlePairs = 1ull << 28;

inline unsigned seg_groups(uint64_t seg_bound) {
    return (unsigned)std::max<uint64_t>(1, std::min<uint64_t>(groups_for(seg_bound), 2048));
}

}  // namespace

BlockGrid block_grid(int tiles_x, int tiles_y) {
    BlockGrid g;
    g.tiles_x = tiles_x;
    g.tiles_y = tiles_y;
    g.bw = (tiles_x + 7) / 8;
    g.bh = (tiles_y + 7) / 8;
    g.nb = g.bw * g.bh;
    return g;
}

size_t block_count_stride(int n) {
    const size_t chunks = ((size_t)std::max(n, 0) + kWave - 1) / kWave;
    return (chunks + 3) / 4 * 4;
}

uint64_t segment_bound(uint64_t m, const BlockGrid& bg) {
    return m / kWave + (uint64_t)bg.nb + 1;
}

hipError_t launch_tile_binning(const TileBinning& tb, hipStream_t st) {
    const BlockGrid& bg = tb.grid;
    if (tb.m == 0 || tb.n <= 0 || bg.nb <= 0) return hipSuccess;
    const int chunks = (int)(((size_t)tb.n + kWave - 1) / kWave);
    const int windows = (bg.nb + kWave - 1) / kWave;
    const int cstride = (int)block_count_stride(tb.n);
    const uint64_t segs = segment_bound(tb.m, bg);
    if (segs > 0xffffffffull) return hipErrorInvalidValue;
    const uint32_t seg_cap = (uint32_t)segs;
    hipError_t e;
    const uint64_t l1_waves = (uint64_t)chunks * (uint64_t)windows;
    if (tb.drects) {
        hipLaunchKernelGGL(rank_rects_kernel, dim3(groups_for(((uint64_t)tb.n + kWave - 1) / kWave)),
                           dim3(kThreads), 0, st, tb.n, tb.perm, tb.rects, tb.drects);
        if ((e = hipGetLastError()) != hipSuccess) return e;
    }
    RecordArgs ra{tb.rec_mean2d, tb.rec_cov2d, tb.rec_colors, tb.rec_alpha,
                  static_cast<BlendRec*>(tb.recs), groups_for(l1_waves)};
    const unsigned rec_groups =
        ra.recs ? (unsigned)(((size_t)tb.n + kThreads - 1) / kThreads) : 0u;
    hipLaunchKernelGGL(block_count_kernel, dim3(ra.first + rec_groups), dim3(kThreads), 0, st,
                       tb.n, tb.perm, tb.rects, tb.drects, bg, chunks, windows, cstride,
                       tb.bcount, ra);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(block_scan_kernel, dim3(bg.nb), dim3(kThreads), 0, st, chunks, cstride,
                       tb.bcount, tb.block_hist, tb.block_start, tb.seg_start, tb.seg_owner,
                       seg_cap, tb.err);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(block_scatter_kernel, dim3(groups_for(l1_waves)), dim3(kThreads), 0, st,
                       tb.n, tb.perm, tb.rects, tb.drects, bg, chunks, windows, cstride, tb.bcount,
                       tb.lists, tb.lrects, tb.m);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(tile_count_kernel, dim3(seg_groups(segs)), dim3(kThreads), 0, st, tb.n, bg,
                       tb.seg_owner, tb.seg_start, tb.block_start, tb.lists, tb.m, tb.lrects,
                       seg_cap, tb.tcount, tb.skip);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(tile_scan_kernel, dim3(bg.nb), dim3(kScanWaves * kWave), 0, st, bg,
                       tb.seg_start, seg_cap, tb.tcount, tb.ttotal);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(tile_starts_kernel, dim3(1), dim3(kStartsThreads), 0, st,
                       bg.tiles_x * bg.tiles_y, tb.ttotal, tb.m,
                       reinterpret_cast<int2*>(tb.ranges), tb.err, tb.skip != nullptr);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // Each wave writes its segment's 64 runs to 64 lists.  Once the lists
    // are gigabytes (config c5: 7.4 GB per band, runs of ~13 ids), fewer
    // waves in flight write faster: 2 work-groups per CU took c5's binning
    // from 24.3 to 21.7 ms per frame, while 8 stay best at c4 (166 MB of ids:
    // 166 us against 194) and at 1080p.
    const unsigned scatter_groups =
        tb.m > kScatterThrottlePairs ? std::min(seg_groups(segs), 512u) : seg_groups(segs);
    hipLaunchKernelGGL(tile_scatter_kernel, dim3(scatter_groups), dim3(kThreads), 0, st, tb.n,
                       bg, tb.seg_owner, tb.seg_start, tb.block_start, tb.lists, tb.m, tb.lrects,
                       seg_cap, tb.tcount, reinterpret_cast<const int2*>(tb.ranges), tb.m,
                       tb.ids, tb.skip);
    return hipGetLastError();
}

hipError_t launch_range_keys(int T, const int32_t* ranges, const int32_t* ids, const float* depth,
                             int n, uint64_t m, uint64_t* keys, hipStream_t st) {
    if (m == 0 || T <= 0) return hipSuccess;
    hipLaunchKernelGGL(range_keys_kernel, dim3(groups_for((uint64_t)T)), dim3(kThreads), 0, st, T,
                       reinterpret_cast<const int2*>(ranges), ids, depth, n, m, keys);
    return hipGetLastError();
}

}  // namespace gsr
