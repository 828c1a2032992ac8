// gsr_schedule.h — the backward blend's per-tile work estimate, shared by the
// schedule kernel (gsr_blend.hip) and the backward records kernel
// (gsr_bin.hip), which runs it in extra work-groups of its own launch.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "gsr_common.h"

namespace gsr {

// [start, end) of a tile's list, clamped to [0, m].
__device__ __forceinline__ void clamp_range(int2 rg, uint64_t m, int& start, int& end) {
    const int64_t s = min<int64_t>(max<int64_t>(rg.x, 0), (int64_t)m);
    const int64_t e = min<int64_t>(max<int64_t>(rg.y, s), (int64_t)m);
    start = (int)s;
    end = (int)e;
}

// The inputs of the backward's per-tile work: its list entries up to the
// largest n_contrib of its pixels.
struct BwdWork {
    int T, H, W, tiles_x;
    uint64_t m;
    const int2* ranges;
    const int32_t* ncontrib;
    uint32_t* work;
    int vec4;  // n_contrib rows 16-byte aligned: one 16-byte load per lane
};

inline BwdWork make_bwd_work(int H, int W, const int32_t* ranges, uint64_t num_pairs,
                             const int32_t* ncontrib, uint32_t* work) {
    BwdWork b;
    b.tiles_x = (W + kTileSize - 1) / kTileSize;
    b.T = b.tiles_x * ((H + kTileSize - 1) / kTileSize);
    b.H = H;
    b.W = W;
    b.m = num_pairs;
    b.ranges = reinterpret_cast<const int2*>(ranges);
    b.ncontrib = ncontrib;
    b.work = work;
    b.vec4 = (W % 4 == 0) && ((reinterpret_cast<uintptr_t>(ncontrib) & 15) == 0);
    return b;
}

// Tiles per 256-thread work-group of the work estimate: one wave per tile.
constexpr int kWorkTilesPerBlock = 4;

// One wave: tile `tile`'s work.  Lane l reads row l / 4, columns 4 (l % 4) ..
// + 3 of the tile.
__device__ __forceinline__ void tile_work_bwd_wave(const BwdWork& b, int tile) {
    const int lane = threadIdx.x & 63;
    const int py = (tile / b.tiles_x) * kTileSize + (lane >> 2);
    const int px = (tile % b.tiles_x) * kTileSize + 4 * (lane & 3);
    int c = 0;
    if (py < b.H) {
        const int32_t* row = b.ncontrib + (size_t)py * b.W;
        if (b.vec4 && px + 3 < b.W) {
            const int4 v = *reinterpret_cast<const int4*>(row + px);
            c = max(max(v.x, v.y), max(v.z, v.w));
        } else {
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (px + k < b.W) c = max(c, row[px + k]);
        }
    }
    const uint32_t mx = wave_max_u32((uint32_t)max(c, 0));
    if (lane == 0) {
        int start, end;
        clamp_range(b.ranges[tile], b.m, start, end);
        b.work[tile] = min(mx, (uint32_t)(end - start));
    }
}

}  // namespace gsr
