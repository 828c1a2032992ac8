// gsr_group.h — work-group scans and the one-wave decoupled look-back shared
// by the binning and scan kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gsr_common.h"

namespace gsr {

// Work-group exclusive scan of one value per thread (kT threads); *total
// receives the sum.  s_w holds kT / 64 words.  Ends with the LDS free for reuse.
template <int kT>
__device__ __forceinline__ uint32_t group_exclusive_scan(uint32_t v, uint32_t* s_w,
                                                         uint32_t* total) {
    constexpr int kW = kT / kWave;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t inc = wave_inclusive_scan(v);
    if (lane == 63) s_w[wave] = inc;
    __syncthreads();
    uint32_t pre = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kW; ++w) {
        const uint32_t x = s_w[w];
        pre += (w < wave) ? x : 0u;
        all += x;
    }
    __syncthreads();
    *total = all;
    return pre + inc - v;
}

// Device-coherent 32-bit accesses for values one work-group hands to another
// within a kernel (every XCD sees the latest value).
__device__ __forceinline__ uint32_t load_agent_u32(const uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void store_agent_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Decoupled look-back over 64-bit status words (flag in the top two bits,
// value below), run by one whole wave: publishes agg as partition part's
// aggregate (its inclusive prefix when part is 0), sums the published values
// of partitions part - 1 downwards, 64 per step, to the nearest one with an
// inclusive prefix (waiting only while one of those is unpublished), publishes
// part's inclusive prefix and returns its exclusive prefix in every lane.  A
// wait beyond kSpinLimit sets bit 0 of *err and ends it (the prefix is then
// incomplete), so no wave can hang.
__device__ inline uint64_t wave_lookback(uint64_t* status, uint64_t part, uint64_t agg,
                                         int* err) {
    const int lane = lane_id();
    uint64_t* mine = status + part;
    if (lane == 0) store_agent(mine, (part == 0 ? kFlagInclusive : kFlagAggregate) | agg);
    uint64_t excl = 0;
    if (part > 0) {
        int64_t hi = (int64_t)part - 1;
        uint32_t spins = 0;
        while (true) {
            const int64_t q = hi - lane;
            // below partition 0: an inclusive zero, which ends the walk
            const uint64_t s = (q >= 0) ? load_agent(status + q) : kFlagInclusive;
            const uint64_t flag = s & ~kValueMask;
            const uint64_t incl = ballot(flag == kFlagInclusive);
            const int last = incl ? (int)__builtin_ctzll(incl) : 63;
            const uint64_t need = (last == 63) ? ~0ull : ((2ull << last) - 1ull);
            if (ballot(flag == 0) & need) {
                if (++spins > kSpinLimit) {
                    if (lane == 0) atomicOr(err, 1);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
                continue;
            }
            excl += wave_sum_u64(lane <= last ? (s & kValueMask) : 0ull);
            if (incl) break;
            hi -= 64;
        }
        if (lane == 0) store_agent(mine, kFlagInclusive | (excl + agg));
    }
    return excl;
}

// Fan-in over 64-bit status words (flag in the top two bits, value below),
// run by one whole wave: publishes agg as partition part's aggregate and
// returns, in every lane, the sum of the aggregates of partitions
// 0 .. part - 1 (lane l reads partitions l, l + 64, ..., all its loads in
// flight together), waiting only for those not yet published.  No partition
// publishes a prefix, so no partition waits on another's wait.  For at most
// 64 kFanPerLane partitions.  A wait beyond kSpinLimit sets bit 0 of *err and
// ends it (the sum is then incomplete), so no wave can hang.
constexpr int kFanPerLane = 8;
__device__ inline uint64_t wave_fanin(uint64_t* status, uint32_t part, uint64_t agg, int* err) {
    const int lane = lane_id();
    if (lane == 0) store_agent(status + part, kFlagAggregate | agg);
    uint64_t v[kFanPerLane];
#pragma unroll
    for (int k = 0; k < kFanPerLane; ++k) {
        const uint32_t q = (uint32_t)lane + 64u * (uint32_t)k;
        v[k] = q < part ? load_agent(status + q) : kFlagAggregate;
    }
    for (uint32_t spins = 0;; ++spins) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < kFanPerLane; ++k) all &= (v[k] & ~kValueMask) != 0;
        if (all) break;
        if (spins >= kSpinLimit) {
            atomicOr(err, 1);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < kFanPerLane; ++k)
            if ((v[k] & ~kValueMask) == 0)
                v[k] = load_agent(status + (uint32_t)lane + 64u * (uint32_t)k);
    }
    uint64_t sum = 0;
#pragma unroll
    for (int k = 0; k < kFanPerLane; ++k) sum += v[k] & kValueMask;
    return wave_sum_u64(sum);
}

// block_start[b] / seg_start[b] (nb + 1 entries each): exclusive prefixes of
// the block histogram and of its 64-entry segment counts.  One work-group of
// kT threads; s_w and s_v hold kT / 64 words each.
template <int kT>
__device__ void block_starts_body(int nb, const uint32_t* hist, uint32_t* block_start,
                                  uint32_t* seg_start, uint32_t* s_w, uint32_t* s_v) {
    const int tid = threadIdx.x;
    uint32_t carry = 0, scarry = 0;
    for (int base = 0; base < nb; base += 4 * kT) {
        const int i = base + 4 * tid;
        uint32_t v[4], s[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v[j] = (i + j < nb) ? load_agent_u32(hist + i + j) : 0u;
            s[j] = (v[j] + kWave - 1) / kWave;
        }
        uint32_t tot, stot;
        uint32_t p = carry + group_exclusive_scan<kT>(v[0] + v[1] + v[2] + v[3], s_w, &tot);
        uint32_t q = scarry + group_exclusive_scan<kT>(s[0] + s[1] + s[2] + s[3], s_v, &stot);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            if (i + j < nb) {
                block_start[i + j] = p;
                seg_start[i + j] = q;
            }
            p += v[j];
            q += s[j];
        }
        carry += tot;
        scarry += stot;
    }
    if (tid == 0) {
        block_start[nb] = carry;
        seg_start[nb] = scarry;
    }
}

// The binning's hand-off after its count kernel (one work-group of kT
// threads): the final pair count and the device status word (read and
// cleared: each error is reported once) stored to the host-mapped words
// host_total[0, 1] with system scope, then the block and segment starts from
// the block histogram.
template <int kT>
__device__ void bin_finish_body(const BinFinish& f, uint32_t* s_w, uint32_t* s_v) {
    if (threadIdx.x == 0 && f.host_total) {
        const uint64_t total = *f.pair_total;
        const int stat = f.status ? atomicExch(f.status, 0) : 0;
        __hip_atomic_store(f.host_total + 1, (uint64_t)(uint32_t)stat, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
        __hip_atomic_store(f.host_total, total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __threadfence_system();
    }
    block_starts_body<kT>(f.nb, f.block_hist, f.block_start, f.seg_start, s_w, s_v);
}

// ranges[t] = [start, start + count) from the tile totals in tile order,
// (0, 0) for tiles without pairs (rasterize.cu:140-166); a grand total other
// than m (above m, with at_most: skipped tiles' lists stay empty) sets err bit 2.  One work-group of kT threads; s_w holds kT / 64 words.
// Each thread takes 8 consecutive tiles per step, their loads issued together
// (8192 tiles, 1080p's 8160, in one step of 1024 threads).
template <int kT>
__device__ void tile_starts_body(int T, const uint32_t* __restrict__ ttotal, uint64_t m,
                                 int2* __restrict__ ranges, int* err, uint32_t* s_w,
                                 bool at_most = false) {
    constexpr int kItems = 8;
    const int tid = threadIdx.x;
    uint32_t carry = 0;
    for (int base = 0; base < T; base += kItems * kT) {
        const int i = base + kItems * tid;
        uint32_t v[kItems];
        if (i + kItems <= T && (reinterpret_cast<uintptr_t>(ttotal) & 15u) == 0u) {
            const uint4 a = *reinterpret_cast<const uint4*>(ttotal + i);
            const uint4 b = *reinterpret_cast<const uint4*>(ttotal + i + 4);
            v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w;
            v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < kItems; ++j) v[j] = (i + j < T) ? ttotal[i + j] : 0u;
        }
        uint32_t sum = 0;
#pragma unroll
        for (int j = 0; j < kItems; ++j) sum += v[j];
        uint32_t tot;
        uint32_t p = carry + group_exclusive_scan<kT>(sum, s_w, &tot);
#pragma unroll
        for (int j = 0; j < kItems; ++j) {
            if (i + j < T)
                ranges[i + j] = v[j] ? make_int2((int)p, (int)(p + v[j])) : make_int2(0, 0);
            p += v[j];
        }
        carry += tot;
    }
    if (tid == 0 && (at_most ? (uint64_t)carry > m : (uint64_t)carry != m)) atomicOr(err, 2);
}

}  // namespace gsr
