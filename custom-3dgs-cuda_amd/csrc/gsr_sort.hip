// gsr_sort.hip — radix sorts of u32 keys carrying u32 values (the depth order
// and the LSD tile sort) and the decoupled look-back scan of per-Gaussian tile
// counts.  Every sort is stable and LSD over 8-bit digits; the kernels differ
// by size.
//
// Ranking (every kernel): stable in-partition ranks from 8 ballots per item
// (the lanes sharing a digit, merged two bits per three-way OR) plus per-wave
// running digit counters in LDS; items are loaded wave-striped (item i of lane
// l in wave w is element w*64*items + i*64 + l), so each wave load is one
// contiguous 256 B access and ranks follow element order.
//
// Depth orders of at most 2^20 keys: onesweep_small_kernel, one kernel per
// pass, over at most 256 partitions (256 threads and 1024 keys per partition
// up to 2^18 keys, 1024 threads and 4096 keys beyond); the partition is the
// work-group's index, and a partition waits only on partitions dispatched
// before it.  Each partition publishes its digit counts and sums those of
// every earlier partition (a fan-in of 512 B per partition, the loads in
// flight together): no partition waits on another's prefix, so there is no
// look-back chain.  The keys and the four passes' digit
// histograms come from the binning's count kernel (or depth_keys_hist_kernel)
// in one pass.  These passes are latency chains (load, rank, look-back,
// scatter).
//
// Larger depth orders (beyond 2^20 keys): reduce-then-scan, three kernels per
// pass with no waits between work-groups (rts_upsweep / rts_scan /
// rts_downsweep).  Their
// partitions are sized so that one round of two 1024-thread work-groups per
// CU covers the keys; with all partitions resident at once, a decoupled
// look-back would walk about half of its predecessors' status words (the
// inclusive prefix spreads only quadratically in round trips).
//
// The LSD tile sort (fallback binning): onesweep_wide_kernel, 1024 threads
// (16 waves) over 8192-element partitions, 16-bit per-wave counters and one
// LDS exchange buffer for keys and then values (42 KB, two work-groups per
// CU); its first pass generates the (tile, Gaussian) pairs in LDS.
//
// Look-back and fan-in spins are bounded by kSpinLimit; a partition that reaches it
// raises the error flag and finishes, so every wave exits.
// HBM traffic per pass: 8 B read + 8 B written per element (+ 4 B read in
// the upsweep, + the status / count words).
#include <algorithm>
#include <cstdlib>

#include "gsr_internal.h"
#include "gsr_common.h"
#include "gsr_group.h"

namespace gsr {

namespace {

constexpr int kHistMaxPasses = 4;
constexpr int kLookback = 4;
// Words of the histogram block: [4][256] digit counts.
constexpr int kHistWords = kHistMaxPasses * kRadixBins;

// Inputs up to this size take onesweep passes over 1024-key partitions of 256
// threads (onesweep_small_kernel).
constexpr uint64_t kSmallSortMax = 1u << 18;
constexpr int kSmallThreads = 256;
constexpr int kSmallItems = 4;
constexpr int kSmallPartition = kSmallThreads * kSmallItems;
// Inputs up to kMediumSortMax keys take the same passes with 1024 threads
// over 4096-key partitions (onesweep_small_kernel<1024>): again at most
// kMaxSmallParts partitions.
constexpr uint64_t kMediumSortMax = 1u << 20;
constexpr int kMediumThreads = 1024;
constexpr int kMediumPartition = kMediumThreads * kSmallItems;
constexpr int kMaxSmallParts = 256;
static_assert(kSmallSortMax / kSmallPartition == kMaxSmallParts &&
                  kMediumSortMax / kMediumPartition == kMaxSmallParts,
              "at most 256 partitions per fan-in pass");
// Small passes' status: a partition's count of a digit (at most 1024) in a
// 16-bit word with this flag once published, two digits per 32-bit store;
// rows of the fan-in in flight per thread.
constexpr uint32_t kSmallPublished = 1u << 15;
constexpr uint64_t kSmallAll = 0x8000800080008000ull;

// The wide onesweep: 1024 threads, 8 items.
constexpr int kWideWaves = kSortThreads / kWave;
static_assert(kSortThreads == 1024 && kWideWaves == 16, "sixteen waves per onesweep work-group");
static_assert(kSortPartition == kSortThreads * kSortItems, "partition of the wide onesweep");


inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct SortCtl {
    uint32_t* hist;      // [4][256]
    uint32_t* counters;  // [passes] (one per 64 B line)
    uint64_t* status;    // [passes][parts][256]
};

inline uint64_t parts_for(uint64_t n) { return (n + kSortPartition - 1) / kSortPartition; }
inline bool small_sort(uint64_t n) { return n <= kSmallSortMax; }
// Fan-in passes (onesweep_small_kernel): up to kMediumSortMax keys.
inline bool fanin_sort(uint64_t n) { return n <= kMediumSortMax; }
// Items per thread of the large depth passes (1024 threads): one round of
// 512 resident work-groups (two per CU) where the partitions allow it.
inline int depth_items(uint64_t n) {
    const uint64_t per = (n + 512 * 1024 - 1) / (512 * 1024);
    return per <= 4 ? 4 : per <= 6 ? 6 : per <= 8 ? 8 : 10;
}
inline uint64_t sort_parts(uint64_t n) {
    const uint64_t part =
        small_sort(n)   ? (uint64_t)kSmallPartition
        : fanin_sort(n) ? (uint64_t)kMediumPartition
                        : (uint64_t)kSortThreads * depth_items(n);
    return (n + part - 1) / part;
}
inline size_t hist_bytes() { return align_up((size_t)kHistWords * 4, 256); }

SortCtl carve(void* control) {
    char* p = static_cast<char*>(control);
    SortCtl c;
    c.hist = reinterpret_cast<uint32_t*>(p);
    p += hist_bytes();
    c.counters = reinterpret_cast<uint32_t*>(p);
    p += align_up((size_t)kHistMaxPasses * 64, 256);
    c.status = reinterpret_cast<uint64_t*>(p);
    return c;
}

// Lanes of `active` whose digit equals this lane's, comparing the low `bits`
// bits (the digit's higher bits are known to be zero in every key).  Per bit:
// y = 0 or ~0 (the lane's bit, sign-extended) and the ballot t of the bit;
// t ^ y holds the lanes whose bit differs, and two bits' mismatches are
// merged per 32-lane half with one three-way OR.
__device__ __forceinline__ uint32_t bit_mask(uint32_t d, int b) {
    return (uint32_t)(((int32_t)(d << (31 - b))) >> 31);
}
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t active, int bits = 8) {
    uint32_t mis_lo = ~(uint32_t)active, mis_hi = ~(uint32_t)(active >> 32);
#pragma unroll
    for (int b = 0; b < 8; b += 2) {
        if (b >= bits) break;
        const uint32_t y0 = bit_mask(d, b);
        const uint64_t t0 = ballot(y0 != 0u);
        const uint32_t lo0 = (uint32_t)t0 ^ y0, hi0 = (uint32_t)(t0 >> 32) ^ y0;
        if (b + 1 < bits) {
            const uint32_t y1 = bit_mask(d, b + 1);
            const uint64_t t1 = ballot(y1 != 0u);
            mis_lo = mis_lo | lo0 | ((uint32_t)t1 ^ y1);
            mis_hi = mis_hi | hi0 | ((uint32_t)(t1 >> 32) ^ y1);
        } else {
            mis_lo |= lo0;
            mis_hi |= hi0;
        }
    }
    return ~(((uint64_t)mis_hi << 32) | (uint64_t)mis_lo);
}

// Zeroes up to kMaxFills regions in one launch: bytes up to the first 16-byte
// boundary, 16-byte stores, then the tail bytes.
__global__ __launch_bounds__(256) void fill_zero_kernel(FillList f) {
    const size_t stride = (size_t)gridDim.x * 256;
    const size_t t = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (int r = 0; r < f.count; ++r) {
        uint8_t* b = static_cast<uint8_t*>(f.ptr[r]);
        const size_t len = f.bytes[r];
        const size_t head = std::min<size_t>(len, (16 - ((uintptr_t)b & 15)) & 15);
        if (t < head) b[t] = 0;
        uint4* p = reinterpret_cast<uint4*>(b + head);
        const size_t n16 = (len - head) / 16;
        for (size_t i = t; i < n16; i += stride) p[i] = make_uint4(0u, 0u, 0u, 0u);
        const size_t tail = len - head - n16 * 16;
        if (t < tail) reinterpret_cast<uint8_t*>(p + n16)[t] = 0;
    }
}

// Global digit histograms of every byte in one read of the keys (LDS atomics
// per work-group, one global atomic per non-zero bin).
constexpr int kHistThreads = 1024;
__global__ __launch_bounds__(kHistThreads) void radix_hist_kernel(const uint32_t* __restrict__ keys,
                                                                  uint64_t n,
                                                                  uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_h[kHistWords];
    for (int j = threadIdx.x; j < kHistWords; j += kHistThreads) s_h[j] = 0;
    __syncthreads();
    const uint64_t stride = (uint64_t)gridDim.x * kHistThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kHistThreads + threadIdx.x; i < n; i += stride) {
        const uint32_t k = keys[i];
#pragma unroll
        for (int p = 0; p < kHistMaxPasses; ++p)
            lds_hist_add(s_h + p * kRadixBins, (k >> (8 * p)) & 0xffu);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < kHistWords; j += kHistThreads) {
        const uint32_t v = s_h[j];
        if (v) atomicAdd(&hist[j], v);
    }
}

// The depth order's keys (the bits of each depth, every Gaussian) and values
// (indices), with the keys' digit histograms, in one read of the depths.
__global__ __launch_bounds__(kHistThreads) void depth_keys_hist_kernel(
    const float* __restrict__ depth, uint64_t n, uint32_t* __restrict__ keys,
    uint32_t* __restrict__ vals, uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_h[kHistWords];
    for (int j = threadIdx.x; j < kHistWords; j += kHistThreads) s_h[j] = 0;
    __syncthreads();
    const uint64_t stride = (uint64_t)gridDim.x * kHistThreads;
    for (uint64_t i = (uint64_t)blockIdx.x * kHistThreads + threadIdx.x; i < n; i += stride) {
        const uint32_t k = __float_as_uint(depth[i]);
        keys[i] = k;
        vals[i] = (uint32_t)i;
#pragma unroll
        for (int p = 0; p < kHistMaxPasses; ++p)
            lds_hist_add(s_h + p * kRadixBins, (k >> (8 * p)) & 0xffu);
    }
    __syncthreads();
    for (int j = threadIdx.x; j < kHistWords; j += kHistThreads) {
        const uint32_t v = s_h[j];
        if (v) atomicAdd(&hist[j], v);
    }
}

// Copies a partition through unchanged (every key has the pass's digit).
// 16-byte copies when every array is 16-byte aligned, the rest word by word.
template <bool kPacked>
__device__ __forceinline__ void copy_partition(const uint32_t* __restrict__ kin,
                                               const uint32_t* __restrict__ vin,
                                               uint32_t* __restrict__ kout,
                                               uint32_t* __restrict__ vout, uint64_t base,
                                               int nvalid, uint32_t mask) {
    const int nthr = (int)blockDim.x;
    const int tid = (int)threadIdx.x;
    const uintptr_t al = reinterpret_cast<uintptr_t>(kin + base) |
                         reinterpret_cast<uintptr_t>(kout + base) |
                         reinterpret_cast<uintptr_t>(vin + base) |
                         reinterpret_cast<uintptr_t>(vout + base);
    const int n4 = (al & 15) ? 0 : nvalid / 4;
    const uint4* k4 = reinterpret_cast<const uint4*>(kin + base);
    uint4* ko4 = reinterpret_cast<uint4*>(kout + base);
#pragma unroll 2
    for (int e = tid; e < n4; e += nthr) {
        const uint4 k = k4[e];
        ko4[e] = k;
        if constexpr (kPacked) {
            if (vout)
                reinterpret_cast<uint4*>(vout + base)[e] =
                    make_uint4(k.x & mask, k.y & mask, k.z & mask, k.w & mask);
        } else {
            reinterpret_cast<uint4*>(vout + base)[e] = reinterpret_cast<const uint4*>(vin + base)[e];
        }
    }
    for (int e = 4 * n4 + tid; e < nvalid; e += nthr) {
        const uint32_t k = kin[base + e];
        kout[base + e] = k;
        if constexpr (kPacked) {
            if (vout) vout[base + e] = k & mask;
        } else {
            vout[base + e] = vin[base + e];
        }
    }
}

// Decoupled look-back for digit d of partition part over earlier partitions,
// kLookback status words per round trip (before partition 0 reads as an
// inclusive 0); publishes part's inclusive prefix and returns its exclusive
// prefix.  A wait beyond kSpinLimit sets *err and ends the walk.
template <int kWindow = kLookback>
__device__ __forceinline__ uint64_t digit_lookback(uint64_t* __restrict__ status, uint64_t part,
                                                   int d, uint64_t total, int* __restrict__ err) {
    uint64_t excl = 0;
    if (part == 0) return 0;
    int64_t p = (int64_t)part - 1;
    uint32_t spins = 0;
    while (true) {
        uint64_t sw[kWindow];
#pragma unroll
        for (int k = 0; k < kWindow; ++k)
            sw[k] = (p - k >= 0) ? load_agent(status + (uint64_t)(p - k) * kRadixBins + d)
                                 : kFlagInclusive;
        int k = 0;
        bool done = false;
        for (; k < kWindow; ++k) {
            const uint64_t flag = sw[k] & ~kValueMask;
            if (flag == 0) break;  // not published yet: reload from here
            excl += sw[k] & kValueMask;
            if (flag == kFlagInclusive) {
                done = true;
                break;
            }
        }
        if (done) break;
        p -= k;
        if (k < kWindow) {
            if (++spins > kSpinLimit) {
                atomicOr(err, 1);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    store_agent(status + part * kRadixBins + d, kFlagInclusive | (excl + total));
    return excl;
}

// Threads below 256 (digit d = threadIdx.x): turns s_cnt[.][d] into the
// exclusive prefix over the waves and returns the digit's total.
__device__ __forceinline__ uint32_t wave_prefix(uint16_t (*s_cnt)[kRadixBins], int waves) {
    const int d = (int)threadIdx.x;
    uint32_t run = 0;
    for (int w = 0; w < waves; ++w) {
        const uint32_t c = s_cnt[w][d];
        s_cnt[w][d] = (uint16_t)run;
        run += c;
    }
    return run;
}

// ---- small inputs: onesweep over 1024-key partitions -----------------------

// A work-group barrier that orders LDS accesses only: global stores and loads
// in flight stay in flight across it (a full __syncthreads waits for them),
// so the published status words travel while the partition scans its digits.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The sum over rows q0, q0 + kStride, ... < part (at most kFan of them) of
// the 16-bit counts in the 64-bit status word col[q * 64] (four digits), once
// every row's four flags are set; rows not yet published are read again, all
// together.  v holds the words as first read.
template <int kFan, int kStride>
__device__ __forceinline__ void small_fan_sum(const uint64_t* col, int q0, int part,
                                              uint64_t (&v)[kFan], uint32_t (&s)[4],
                                              int* __restrict__ err) {
    for (uint32_t spins = 0;; ++spins) {
        bool all = true;
#pragma unroll
        for (int k = 0; k < kFan; ++k) all &= (v[k] & kSmallAll) == kSmallAll;
        if (all) break;
        if (spins >= kSpinLimit) {
            atomicOr(err, 1);
            break;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int k = 0; k < kFan; ++k)
            if ((v[k] & kSmallAll) != kSmallAll)
                v[k] = load_agent(col + (size_t)(q0 + kStride * k) * (kRadixBins / 4));
    }
#pragma unroll
    for (int k = 0; k < kFan; ++k) {
        const uint64_t c = v[k] & ~kSmallAll;
        s[0] += (uint32_t)c & 0xffffu;
        s[1] += (uint32_t)(c >> 16) & 0xffffu;
        s[2] += (uint32_t)(c >> 32) & 0xffffu;
        s[3] += (uint32_t)(c >> 48);
    }
}

template <int kFan, int kStride>
__device__ __forceinline__ void small_fan_issue(const uint64_t* col, int q0, int part,
                                                uint64_t (&v)[kFan]) {
#pragma unroll
    for (int k = 0; k < kFan; ++k) {
        const int q = q0 + kStride * k;
        v[k] = q < part ? load_agent(col + (size_t)q * (kRadixBins / 4)) : kSmallAll;
    }
}

// One LSD pass over (key >> shift) & 0xff, kThreads threads over partitions
// of 4 kThreads keys (at most 256 of them: inputs of at most 2^18 keys with
// 256 threads, 2^20 with 1024): ranks by ballot match and per-wave counters;
// the partition's digit counts are published, the digit starts scanned and
// the keys and values reordered in LDS; the digit offsets are the sums of the
// earlier partitions' published counts (a fan-in, no chain); then keys and
// values are written in digit runs.  The first 256 threads are the digit
// threads (digit d = thread d).
template <int kThreads>
__global__ __launch_bounds__(kThreads) void onesweep_small_kernel(
    const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, uint64_t n, int shift,
    const uint32_t* __restrict__ hist, uint16_t* __restrict__ status, int* __restrict__ err,
    BinFinish fin, uint32_t fin_group) {
    // the binning's hand-off, in a work-group of its own after the partitions'
    // (independent of the pass: one launch fewer than a kernel of its own)
    if (blockIdx.x == fin_group) {
        __shared__ uint32_t s_fw[kThreads / kWave];
        __shared__ uint32_t s_fv[kThreads / kWave];
        bin_finish_body<kThreads>(fin, s_fw, s_fv);
        return;
    }
    constexpr int kItems = kSmallItems;
    constexpr int kPart = kThreads * kItems;
    constexpr int kWaves = kThreads / kWave;
    constexpr int kDigitWaves = kRadixBins / kWave;
    // rows of the fan-in per wave and batch: at most 32 loads in flight
    constexpr int kFan = std::min(32, (kMaxSmallParts + kWaves - 1) / kWaves);
    static_assert(kThreads >= kRadixBins && kThreads % kRadixBins == 0, "digit threads");
    __shared__ uint32_t s_keys[kPart];
    __shared__ uint32_t s_vals[kPart];
    __shared__ uint32_t s_wcnt[kWaves][kRadixBins];
    __shared__ uint32_t s_dstart[kRadixBins];
    __shared__ uint32_t s_gbase[kRadixBins];
    __shared__ uint32_t s_scan[kDigitWaves];
    __shared__ uint32_t s_hscan[kDigitWaves];
    __shared__ uint32_t s_fan[kWaves][kRadixBins];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // A partition waits only on the partitions before it, whose work-groups
    // were dispatched before its own and wait on nothing before publishing,
    // so the partition is the work-group's index (no claim atomic).
    const int part = (int)blockIdx.x;  // scalar
    const uint64_t base = (uint64_t)part * kPart;
    const int nvalid = (int)min((uint64_t)kPart, n - base);
    const bool digit_thread = tid < kRadixBins;
    const int d = tid & (kRadixBins - 1);
    const uint32_t h = hist[d];
    // the keys and values are loaded before the digit check, so its load is
    // in flight with them
    uint32_t key[kItems], val[kItems], rank[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        key[i] = e < nvalid ? kin[base + e] : 0u;
    }
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        val[i] = e < nvalid ? vin[base + e] : 0u;
    }
    for (int j = tid; j < kWaves * kRadixBins; j += kThreads) (&s_wcnt[0][0])[j] = 0;
    if (__syncthreads_or(digit_thread && (uint64_t)h == n)) {
        // every key has the same digit: the stable pass is the identity
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            if (e < nvalid) {
                kout[base + e] = key[i];
                vout[base + e] = val[i];
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        const bool v = e < nvalid;
        const uint32_t dg = (key[i] >> shift) & 0xffu;
        const uint64_t peers = match_digit(dg, ballot(v));
        rank[i] = 0;
        if (v) {
            const uint32_t before = s_wcnt[wave][dg];
            const uint64_t lower = peers & lanemask_lt();
            rank[i] = before + (uint32_t)popc64(lower);
            if (lower == 0) s_wcnt[wave][dg] = before + (uint32_t)popc64(peers);
        }
    }
    lds_barrier();
    // the digit threads: the partition's count (published: digits d and d + 1
    // in one 32-bit word, from the even thread), wave prefixes and the digit's
    // start in the partition
    uint32_t total = 0;
    if (digit_thread) {
        for (int w = 0; w < kWaves; ++w) {
            const uint32_t c = s_wcnt[w][d];
            s_wcnt[w][d] = total;
            total += c;
        }
    }
    uint32_t inc = 0, hinc = 0;
    if (wave < kDigitWaves) {  // whole waves: the shuffles and scans see only digit threads
        const uint32_t other = __shfl_xor(total, 1, kWave);
        if ((d & 1) == 0)
            __hip_atomic_store(
                reinterpret_cast<uint32_t*>(status + (size_t)part * kRadixBins + d),
                (kSmallPublished | total) | ((kSmallPublished | other) << 16), __ATOMIC_RELAXED,
                __HIP_MEMORY_SCOPE_AGENT);
        inc = wave_inclusive_scan(total);
        hinc = wave_inclusive_scan(h);
        if (lane == 63) {
            s_scan[wave] = inc;
            s_hscan[wave] = hinc;
        }
    }
    const uint64_t* col = reinterpret_cast<const uint64_t*>(status) + lane;
    uint64_t fan[kFan];
    lds_barrier();
    uint32_t dstart = 0, hexcl = 0;
    if (digit_thread) {
        uint32_t wpre = 0, hpre = 0;
        for (int w = 0; w < wave; ++w) {
            wpre += s_scan[w];
            hpre += s_hscan[w];
        }
        dstart = wpre + inc - total;
        hexcl = hpre + hinc - h;
        s_dstart[d] = dstart;
    }
    lds_barrier();
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        if (e < nvalid) {
            const uint32_t dg = (key[i] >> shift) & 0xffu;
            const uint32_t pos = s_dstart[dg] + s_wcnt[wave][dg] + rank[i];
            s_keys[pos] = key[i];
            s_vals[pos] = val[i];
        }
    }
    // Fan-in: lane l of wave w sums digits 4l .. 4l + 3 (one 64-bit status
    // word) over rows w, w + kWaves, ..., kFan rows' loads in flight at once.
    // Issued here, after the reorder, rather than right after publishing:
    // fewer rows are then still unpublished and read twice (the pass at 100k
    // keys is about 1 us faster per pass this way).
    small_fan_issue<kFan, kWaves>(col, wave, part, fan);
    {
        uint32_t sum[4] = {0u, 0u, 0u, 0u};
        small_fan_sum<kFan, kWaves>(col, wave, part, fan, sum, err);
        for (int q0 = wave + kWaves * kFan; q0 < part; q0 += kWaves * kFan) {
            small_fan_issue<kFan, kWaves>(col, q0, part, fan);
            small_fan_sum<kFan, kWaves>(col, q0, part, fan, sum, err);
        }
        s_fan[wave][4 * lane] = sum[0];
        s_fan[wave][4 * lane + 1] = sum[1];
        s_fan[wave][4 * lane + 2] = sum[2];
        s_fan[wave][4 * lane + 3] = sum[3];
    }
    __syncthreads();
    if (digit_thread) {
        uint32_t excl = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) excl += s_fan[w][d];
        // element j of digit d's run goes to hexcl + excl + (j - dstart) (32 bits)
        s_gbase[d] = hexcl + excl - dstart;
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int j = tid + k * kThreads;
        if (j < nvalid) {
            const uint32_t kk = s_keys[j];
            const uint32_t o = s_gbase[(kk >> shift) & 0xffu] + (uint32_t)j;
            if ((uint64_t)o < n) {  // always, for consistent histograms; guards the stores
                kout[o] = kk;
                vout[o] = s_vals[j];
            }
        }
    }
}

// ---- large inputs and the tile sort: the wide onesweep ---------------------

// The emission's staging index: one padding word per 16 slots, so a wave's
// blocked writes (kSortItems slots per lane) spread over the banks.
__device__ __forceinline__ int pad16(int slot) { return slot + (slot >> 4); }

// Expands the (tile, Gaussian) pairs of sort slots [base, base + nvalid) into
// s_keys / s_vals at pad16(slot) (kPacked: the one word (tile << gbits) | g in
// s_keys).  Pair slots are laid out by depth rank r at offsets[r] (ty outer,
// tx inner over the rank's tile rectangle), the order in which the reference
// emits keys per Gaussian (rasterize.cu:124-135).  Ranks r_lo..r_lo+nr-1
// overlap the partition; the first kStageRanks of them have their offset,
// Gaussian id and tile rectangle staged in LDS by one parallel load (more
// only occur for partitions of very small Gaussians, or when ranks without
// pairs sit between ranks with pairs, and are read from global memory).
// Each thread expands kSortItems consecutive slots: one binary search, one
// division, then a walk that steps the column and row.
constexpr int kStageRanks = 640;

struct RankStage {
    uint32_t off[kStageRanks];
    uint32_t g[kStageRanks];
    uint2 rect[kStageRanks];
};
constexpr int kRankStageWords = (int)(sizeof(RankStage) / 4);

template <bool kPacked>
__device__ __forceinline__ void expand_pairs(const EmitSource& es, uint64_t base, int nvalid,
                                             uint32_t* s_keys, uint32_t* s_vals,
                                             RankStage* st, int gbits) {
    const int tid = threadIdx.x;
    const uint32_t part = (uint32_t)(base / kSortPartition);
    const uint32_t r_lo = es.part_rank[part];
    const uint32_t r_next = es.part_rank[part + 1];
    // last rank holding a slot of this partition
    const uint64_t next_base = base + (uint64_t)nvalid;
    const uint32_t r_last =
        (part + 1 < es.nparts && (uint64_t)es.offsets[r_next] < next_base) ? r_next : r_next - 1;
    const uint32_t nr = (r_last >= r_lo) ? r_last - r_lo + 1 : 1u;
    const uint32_t nstage = min(nr, (uint32_t)kStageRanks);
    for (uint32_t j = tid; j < nstage; j += kSortThreads) {
        const uint32_t g = es.perm[r_lo + j];
        st->off[j] = es.offsets[r_lo + j];
        st->g[j] = g;
        st->rect[j] = es.rects[g];
    }
    __syncthreads();
    auto off_of = [&](uint32_t j) -> uint64_t {
        return (j < (uint32_t)kStageRanks) ? st->off[j] : es.offsets[r_lo + j];
    };
    const int first = tid * kSortItems;
    if (first < nvalid) {
        const uint64_t s0 = base + (uint64_t)first;
        uint32_t lo = 0, hi = nr - 1;  // last j with offset <= s0
        while (lo < hi) {
            const uint32_t mid = (lo + hi + 1) >> 1;
            if (off_of(mid) <= s0) lo = mid; else hi = mid - 1;
        }
        uint32_t j = lo, g, x0, w, y0;
        auto load_rank = [&](uint32_t jj) {
            uint2 rc;
            if (jj < (uint32_t)kStageRanks) {
                g = st->g[jj];
                rc = st->rect[jj];
            } else {
                g = es.perm[r_lo + jj];
                rc = es.rects[g];
            }
            x0 = rc.x & 0xffffu;
            w = (rc.x >> 16) - x0;
            y0 = rc.y & 0xffffu;
        };
        load_rank(j);
        uint64_t kbase = off_of(j);
        uint64_t next = (j + 1 < nr) ? off_of(j + 1) : ~0ull;
        const uint32_t k0 = (uint32_t)(s0 - kbase);
        uint32_t row = w ? k0 / w : 0u;
        uint32_t col = k0 - row * w;
        for (int i = 0; i < kSortItems; ++i) {
            const int slot = first + i;
            if (slot >= nvalid) break;
            const uint64_t sg = base + (uint64_t)slot;
            while (sg >= next) {  // the next rank with pairs starts at this slot
                ++j;
                load_rank(j);
                kbase = next;
                next = (j + 1 < nr) ? off_of(j + 1) : ~0ull;
                row = 0;
                col = 0;
            }
            const uint32_t tile = (y0 + row) * (uint32_t)es.tiles_x + x0 + col;
            if constexpr (kPacked) {
                s_keys[pad16(slot)] = (tile << gbits) | g;
            } else {
                s_keys[pad16(slot)] = tile;
                s_vals[pad16(slot)] = g;
            }
            if (++col == w) {
                col = 0;
                ++row;
            }
        }
    }
    __syncthreads();
}

// One LSD pass over the digit (key >> shift), digit_bits significant bits.
// kEmit: the partition's (tile, Gaussian) pairs are generated from the depth
// order instead of being read (the first tile pass).  kPacked: each element
// is the one word (tile << gbits) | Gaussian id, sorted on its tile bits; kout
// receives the words and, when vout is not null (the last pass), vout the
// Gaussian ids.  Otherwise keys and values are separate words, both written.
template <bool kEmit, bool kPacked>
__global__ __launch_bounds__(kSortThreads) __attribute__((amdgpu_waves_per_eu(8, 8))) void onesweep_wide_kernel(
    const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, uint64_t n, int shift,
    int digit_bits, const uint32_t* __restrict__ hist, uint64_t* __restrict__ status,
    uint32_t* __restrict__ counter, int* __restrict__ err, EmitSource es, int gbits) {
    constexpr int kThreads = kSortThreads;
    constexpr int kItems = kSortItems;
    constexpr int kPart = kSortPartition;
    constexpr int kWaves = kWideWaves;
    constexpr bool kVals = !kPacked;
    constexpr int kXWords = kEmit ? kPart + kPart / 16 : kPart;
    // after the emission: u16 counters [16][256], digit starts, global bases
    constexpr int kCntWords = kWaves * kRadixBins / 2;
    constexpr int kScanAux = kCntWords + 2 * kRadixBins;
    constexpr int kAuxWords = (kEmit && kRankStageWords > kScanAux) ? kRankStageWords : kScanAux;
    __shared__ uint32_t s_x[kXWords];
    __shared__ uint32_t s_v[(kEmit && kVals) ? kXWords : 1];
    __shared__ __align__(16) uint32_t s_aux[kAuxWords];
    __shared__ uint32_t s_scan[4];
    __shared__ uint32_t s_hscan[4];
    __shared__ uint32_t s_part;
    uint16_t (*s_cnt)[kRadixBins] = reinterpret_cast<uint16_t (*)[kRadixBins]>(s_aux);
    uint32_t* s_dstart = s_aux + kCntWords;
    uint32_t* s_gbase = s_aux + kCntWords + kRadixBins;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_part = atomicAdd(counter, 1u);
    // the digit's global count, fetched while the claim is in flight
    const uint32_t h = tid < kRadixBins ? hist[tid] : 0u;
    const uint32_t gmask = kPacked ? ((1u << gbits) - 1u) : 0u;
    bool same = false;
    if constexpr (!kEmit) same = __syncthreads_or(tid < kRadixBins && (uint64_t)h == n);
    else __syncthreads();
    const uint64_t part = s_part;
    const uint64_t base = part * kPart;
    const int nvalid = (int)min((uint64_t)kPart, n - base);
    if constexpr (!kEmit) {
        // Every key has the same digit: the stable pass is the identity, so the
        // partition is copied through (no ranking, no look-back).
        if (same) {
            copy_partition<kPacked>(kin, vin, kout, vout, base, nvalid, gmask);
            return;
        }
    }

    uint32_t key[kItems], val[kItems], rank[kItems];
    (void)val;
    if constexpr (kEmit) {
        expand_pairs<kPacked>(es, base, nvalid, s_x, s_v, reinterpret_cast<RankStage*>(s_aux),
                              gbits);  // ends with a barrier
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            const bool v = e < nvalid;
            key[i] = v ? s_x[pad16(e)] : 0u;
            if constexpr (kVals) val[i] = v ? s_v[pad16(e)] : 0u;
        }
        __syncthreads();  // the staged ranks' region becomes the counters
    } else {
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            key[i] = e < nvalid ? kin[base + e] : 0u;
        }
    }
    for (int j = tid; j < kCntWords; j += kThreads) s_aux[j] = 0;
    __syncthreads();
    uint32_t total = 0, excl = 0;
    // stable ranks within the wave's slice, in element order
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        const bool v = e < nvalid;
        const uint32_t d = (key[i] >> shift) & 0xffu;
        const uint64_t peers = match_digit(d, ballot(v), digit_bits);
        rank[i] = 0;
        if (v) {
            const uint32_t before = s_cnt[wave][d];
            const uint64_t lower = peers & lanemask_lt();
            rank[i] = before + (uint32_t)popc64(lower);
            if (lower == 0) s_cnt[wave][d] = (uint16_t)(before + (uint32_t)popc64(peers));
        }
    }
    __syncthreads();
    if constexpr (kVals && !kEmit) {
        // the values are needed only for their reorder: their loads are in
        // flight during the scans below and the key reorder
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            val[i] = e < nvalid ? vin[base + e] : 0u;
        }
    }

    // threads below 256, one per digit: the waves' prefixes and the digit's
    // total (published at once), the partition-local digit start and the
    // digit's global start
    uint32_t inc = 0, hinc = 0;
    if (tid < kRadixBins) {
        total = wave_prefix(s_cnt, kWaves);
        store_agent(status + part * kRadixBins + tid,
                    (part == 0 ? kFlagInclusive : kFlagAggregate) | (uint64_t)total);
        inc = wave_inclusive_scan(total);
        hinc = wave_inclusive_scan(h);
        if (lane == 63) {
            s_scan[wave] = inc;
            s_hscan[wave] = hinc;
        }
    }
    __syncthreads();
    uint32_t dstart = 0, hexcl = 0;
    if (tid < kRadixBins) {
        uint32_t wpre = 0, hpre = 0;
        for (int w = 0; w < wave; ++w) {
            wpre += s_scan[w];
            hpre += s_hscan[w];
        }
        dstart = wpre + inc - total;
        hexcl = hpre + hinc - h;
        s_dstart[tid] = dstart;
    }
    __syncthreads();
    // the digit threads look back while every thread reorders its keys
    if (tid < kRadixBins) {
        excl = (uint32_t)digit_lookback(status, part, tid, total, err);
        // element j of digit d's run goes to hexcl + excl + (j - dstart); in
        // 32 bits, exact below 2^32 elements
        s_gbase[tid] = hexcl + excl - dstart;
    }
    uint32_t pos[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        pos[i] = 0xffffffffu;
        if (e < nvalid) {
            const uint32_t d = (key[i] >> shift) & 0xffu;
            pos[i] = s_dstart[d] + s_cnt[wave][d] + rank[i];
            s_x[pos[i]] = key[i];
        }
    }
    __syncthreads();
    uint32_t dst[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int j = tid + k * kThreads;
        dst[k] = 0xffffffffu;
        if (j < nvalid) {
            const uint32_t kk = s_x[j];
            const uint32_t o = s_gbase[(kk >> shift) & 0xffu] + (uint32_t)j;
            if ((uint64_t)o < n) {  // always, for consistent histograms; guards the stores
                dst[k] = o;
                kout[o] = kk;
                if constexpr (kPacked) {
                    if (vout) vout[o] = kk & gmask;
                }
            }
        }
    }
    if constexpr (kVals) {
        __syncthreads();  // every key is read out of the exchange buffer
#pragma unroll
        for (int i = 0; i < kItems; ++i)
            if (pos[i] != 0xffffffffu) s_x[pos[i]] = val[i];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            const int j = tid + k * kThreads;
            if (dst[k] != 0xffffffffu) vout[dst[k]] = s_x[j];
        }
    }
}

// ---- large inputs: reduce-then-scan passes --------------------------------
// One LSD pass as three kernels with no waits between work-groups (no claim
// atomic, no look-back chain):
//   rts_upsweep   — each partition's digit counts, digit-major [256][parts];
//   rts_scan      — per digit, the exclusive prefix over the partitions plus
//                   the digit's global start, partition-major [parts][256];
//   rts_downsweep — stable ranks within the partition (ballot match + per-wave
//                   16-bit counters), keys then values reordered through LDS
//                   and written at the partition's digit offsets.
// The keys are read twice (20 B moved per element instead of 16), but every
// partition proceeds on its own: with all partitions resident at once, a
// look-back walks about half of its predecessors' status words.  A pass whose
// digit is the same for every key copies through in the downsweep; the other
// two kernels return at once.

template <int kItems>
__global__ __launch_bounds__(kSortThreads) void rts_upsweep_kernel(
    const uint32_t* __restrict__ kin, uint64_t n, int shift, const uint32_t* __restrict__ hist,
    uint32_t* __restrict__ part_hist, uint32_t parts) {
    constexpr int kPart = kSortThreads * kItems;
    static_assert(kPart % 4 == 0, "16-byte loads");
    __shared__ uint32_t s_h[kRadixBins];
    const int tid = threadIdx.x;
    const uint32_t h = tid < kRadixBins ? hist[tid] : 0u;
    if (tid < kRadixBins) s_h[tid] = 0;
    if (__syncthreads_or(tid < kRadixBins && (uint64_t)h == n)) return;  // constant digit
    const uint64_t base = (uint64_t)blockIdx.x * kPart;
    const int nvalid = (int)min((uint64_t)kPart, n - base);
    const int n4 = nvalid / 4;
    const uint4* k4 = reinterpret_cast<const uint4*>(kin + base);  // 16-byte aligned
    constexpr int kQ = (kItems + 3) / 4;  // 16-byte loads per thread covering the partition
    uint4 q[kQ];
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
        const int e = i * kSortThreads + tid;
        q[i] = e < n4 ? k4[e] : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int i = 0; i < kQ; ++i) {
        const int e = i * kSortThreads + tid;
        if (e < n4) {
            atomicAdd(&s_h[(q[i].x >> shift) & 0xffu], 1u);
            atomicAdd(&s_h[(q[i].y >> shift) & 0xffu], 1u);
            atomicAdd(&s_h[(q[i].z >> shift) & 0xffu], 1u);
            atomicAdd(&s_h[(q[i].w >> shift) & 0xffu], 1u);
        }
    }
    for (int e = 4 * n4 + tid; e < nvalid; e += kSortThreads)
        atomicAdd(&s_h[(kin[base + e] >> shift) & 0xffu], 1u);
    __syncthreads();
    if (tid < kRadixBins) part_hist[(size_t)tid * parts + blockIdx.x] = s_h[tid];
}

constexpr int kRtsScanThreads = 256;
constexpr int kRtsScanItems = 4;
// Work-group d: digit d's exclusive prefix over the partitions, offset by the
// digit's global start, into part_off[p][d].
__global__ __launch_bounds__(kRtsScanThreads) void rts_scan_kernel(
    const uint32_t* __restrict__ hist, uint64_t n, const uint32_t* __restrict__ part_hist,
    uint32_t parts, uint32_t* __restrict__ part_off) {
    __shared__ uint32_t s_w[kRtsScanThreads / kWave];
    __shared__ uint32_t s_base;
    const int tid = threadIdx.x;
    const int d = blockIdx.x;
    const uint32_t hv = hist[tid];
    if (__syncthreads_or((uint64_t)hv == n)) return;  // constant digit: nothing to place
    uint32_t all = 0;
    const uint32_t below = group_exclusive_scan<kRtsScanThreads>(hv, s_w, &all);
    if (tid == d) s_base = below;  // the keys of the digits below d
    __syncthreads();
    uint32_t carry = s_base;
    const uint32_t* row = part_hist + (size_t)d * parts;
    for (uint32_t c0 = 0; c0 < parts; c0 += kRtsScanThreads * kRtsScanItems) {
        uint32_t v[kRtsScanItems], sum = 0;
        const uint32_t p0 = c0 + (uint32_t)tid * kRtsScanItems;
#pragma unroll
        for (int i = 0; i < kRtsScanItems; ++i) {
            v[i] = p0 + i < parts ? row[p0 + i] : 0u;
            sum += v[i];
        }
        uint32_t chunk = 0;
        uint32_t run = carry + group_exclusive_scan<kRtsScanThreads>(sum, s_w, &chunk);
#pragma unroll
        for (int i = 0; i < kRtsScanItems; ++i) {
            if (p0 + i < parts) part_off[(size_t)(p0 + i) * kRadixBins + d] = run;
            run += v[i];
        }
        carry += chunk;
    }
}

template <bool kPacked, int kItems>
__global__ __launch_bounds__(kSortThreads) __attribute__((amdgpu_waves_per_eu(8, 8))) void
rts_downsweep_kernel(const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
                     uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, uint64_t n,
                     int shift, int digit_bits, const uint32_t* __restrict__ hist,
                     const uint32_t* __restrict__ part_off, int gbits) {
    constexpr int kPart = kSortThreads * kItems;
    constexpr bool kVals = !kPacked;
    __shared__ uint32_t s_x[kPart];
    __shared__ uint16_t s_cnt[kWideWaves][kRadixBins];
    __shared__ uint32_t s_dstart[kRadixBins];
    __shared__ uint32_t s_gbase[kRadixBins];
    __shared__ uint32_t s_scan[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t part = blockIdx.x;
    const uint64_t base = part * kPart;
    const int nvalid = (int)min((uint64_t)kPart, n - base);
    const uint32_t gmask = kPacked ? ((1u << gbits) - 1u) : 0u;
    const uint32_t h = tid < kRadixBins ? hist[tid] : 0u;
    uint32_t* cnt_words = reinterpret_cast<uint32_t*>(&s_cnt[0][0]);
    for (int j = tid; j < kWideWaves * kRadixBins / 2; j += kSortThreads) cnt_words[j] = 0;
    if (__syncthreads_or(tid < kRadixBins && (uint64_t)h == n)) {
        // every key has the same digit: the stable pass is the identity
        copy_partition<kPacked>(kin, vin, kout, vout, base, nvalid, gmask);
        return;
    }
    // where the partition's run of each digit starts (from the scan)
    const uint32_t poff = tid < kRadixBins ? part_off[part * kRadixBins + tid] : 0u;
    uint32_t key[kItems], val[kItems], rank[kItems];
    (void)val;
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        key[i] = e < nvalid ? kin[base + e] : 0u;
    }
    if constexpr (kVals) {
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            val[i] = e < nvalid ? vin[base + e] : 0u;
        }
    }
    // stable ranks within the wave's slice, in element order
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        const bool v = e < nvalid;
        const uint32_t d = (key[i] >> shift) & 0xffu;
        const uint64_t peers = match_digit(d, ballot(v), digit_bits);
        rank[i] = 0;
        if (v) {
            const uint32_t before = s_cnt[wave][d];
            const uint64_t lower = peers & lanemask_lt();
            rank[i] = before + (uint32_t)popc64(lower);
            if (lower == 0) s_cnt[wave][d] = (uint16_t)(before + (uint32_t)popc64(peers));
        }
    }
    __syncthreads();
    uint32_t total = 0, inc = 0;
    if (tid < kRadixBins) {
        total = wave_prefix(s_cnt, kWideWaves);
        inc = wave_inclusive_scan(total);
        if (lane == 63) s_scan[wave] = inc;
    }
    __syncthreads();
    if (tid < kRadixBins) {
        uint32_t wpre = 0;
        for (int w = 0; w < wave; ++w) wpre += s_scan[w];
        const uint32_t dstart = wpre + inc - total;
        s_dstart[tid] = dstart;
        s_gbase[tid] = poff - dstart;  // element j of the digit's run goes to poff + (j - dstart)
    }
    __syncthreads();
    uint32_t pos[kItems];
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        pos[i] = 0xffffffffu;
        if (e < nvalid) {
            const uint32_t d = (key[i] >> shift) & 0xffu;
            pos[i] = s_dstart[d] + s_cnt[wave][d] + rank[i];
            s_x[pos[i]] = key[i];
        }
    }
    __syncthreads();
    uint32_t dst[kItems];
#pragma unroll
    for (int k = 0; k < kItems; ++k) {
        const int j = tid + k * kSortThreads;
        dst[k] = 0xffffffffu;
        if (j < nvalid) {
            const uint32_t kk = s_x[j];
            const uint32_t o = s_gbase[(kk >> shift) & 0xffu] + (uint32_t)j;
            if ((uint64_t)o < n) {  // always, for consistent histograms; guards the stores
                dst[k] = o;
                kout[o] = kk;
                if constexpr (kPacked) {
                    if (vout) vout[o] = kk & gmask;
                }
            }
        }
    }
    if constexpr (kVals) {
        __syncthreads();  // every key is read out of the exchange buffer
#pragma unroll
        for (int i = 0; i < kItems; ++i)
            if (pos[i] != 0xffffffffu) s_x[pos[i]] = val[i];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < kItems; ++k) {
            const int j = tid + k * kSortThreads;
            if (dst[k] != 0xffffffffu) vout[dst[k]] = s_x[j];
        }
    }
}

// ---- exclusive scan of counts[perm[r]] (fan-in, or decoupled look-back) -----
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanPartition = kScanThreads * kScanItems;

__global__ __launch_bounds__(kScanThreads) void scan_counts_kernel(
    int n, const uint32_t* __restrict__ perm, const uint32_t* __restrict__ counts,
    uint32_t* __restrict__ offsets, uint64_t* __restrict__ total, uint64_t* __restrict__ status,
    uint32_t* __restrict__ counter, int* __restrict__ err, int fanin) {
    __shared__ uint32_t s_part;
    __shared__ uint32_t s_wsum[4];
    __shared__ uint64_t s_base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    // fanin (at most 64 kFanPerLane partitions): the partition is the
    // work-group's index and its prefix a fan-in of the earlier partitions'
    // published counts; beyond, partitions claimed in launch order and a
    // look-back
    if (!fanin && tid == 0) s_part = atomicAdd(counter, 1u);
    __syncthreads();
    const uint64_t part = fanin ? (uint64_t)blockIdx.x : (uint64_t)s_part;
    const int64_t first = (int64_t)part * kScanPartition + (int64_t)tid * kScanItems;
    uint32_t c[kScanItems];
    uint32_t sum = 0;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t r = first + i;
        const uint32_t g = (r < n) ? (perm ? perm[r] : (uint32_t)r) : 0xffffffffu;
        c[i] = (g < (uint32_t)n) ? counts[g] : 0u;
        sum += c[i];
    }
    const uint32_t inc = wave_inclusive_scan(sum);
    if (lane == 63) s_wsum[wave] = inc;
    __syncthreads();
    uint32_t wpre = 0, btot = 0;
    for (int w = 0; w < 4; ++w) {
        if (w < wave) wpre += s_wsum[w];
        btot += s_wsum[w];
    }
    // the prefix by the first wave
    if (wave == 0) {
        const uint64_t excl = fanin ? wave_fanin(status, (uint32_t)part, (uint64_t)btot, err)
                                    : wave_lookback(status, part, (uint64_t)btot, err);
        if (lane == 0) {
            s_base = excl;
            const uint64_t pbeg = part * kScanPartition;
            if (pbeg + kScanPartition >= (uint64_t)n) *total = excl + btot;
        }
    }
    __syncthreads();
    uint64_t run = s_base + wpre + inc - sum;
#pragma unroll
    for (int i = 0; i < kScanItems; ++i) {
        const int64_t r = first + i;
        if (r < n) offsets[r] = (uint32_t)run;
        run += c[i];
    }
}

}  // namespace

hipError_t zero_fill(const FillList& f, hipStream_t st) {
    size_t most = 0;
    for (int r = 0; r < f.count; ++r) most = std::max(most, f.bytes[r] / 16);
    if (f.count == 0) return hipSuccess;
    const size_t blocks = std::min<size_t>(std::max<size_t>((most + 255) / 256, 1), 2048);
    hipLaunchKernelGGL(fill_zero_kernel, dim3((unsigned)blocks), dim3(256), 0, st, f);
    return hipGetLastError();
}

hipError_t zero_fill(void* p, size_t bytes, hipStream_t st) {
    FillList f;
    f.add(p, bytes);
    return zero_fill(f, st);
}

size_t sort_control_bytes(uint64_t n) {
    // per partition and pass: 256 16-bit status words (small inputs), or 256
    // digit counts and 256 offsets (reduce-then-scan)
    return hist_bytes() + align_up((size_t)kHistMaxPasses * 64, 256) +
           (size_t)kHistMaxPasses * sort_parts(n) * kRadixBins * (fanin_sort(n) ? 2 : 8);
}

hipError_t launch_depth_keys_hist(uint64_t n, const float* depth, uint32_t* keys, uint32_t* vals,
                                  void* control, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const unsigned blocks =
        (unsigned)std::max<uint64_t>(1, std::min<uint64_t>((n + 8191) / 8192, 1024));
    hipLaunchKernelGGL(depth_keys_hist_kernel, dim3(blocks), dim3(kHistThreads), 0, st, depth, n,
                       keys, vals, carve(control).hist);
    return hipGetLastError();
}

bool radix_sort_takes_finish(uint64_t n) { return n > 0 && fanin_sort(n); }

hipError_t launch_radix_sort(uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1, uint64_t n,
                             void* control, int* err, hipStream_t st, bool hist_ready,
                             const BinFinish* finish, hipEvent_t after_first) {
    if (n == 0) return hipSuccess;
    if (n >= (1ull << 32)) return hipErrorInvalidValue;
    const uint64_t parts = sort_parts(n);
    SortCtl c = carve(control);
    hipError_t e = hipSuccess;
    if (!hist_ready) {
        const unsigned hblocks =
            (unsigned)std::max<uint64_t>(1, std::min<uint64_t>((n + 8191) / 8192, 1024));
        hipLaunchKernelGGL(radix_hist_kernel, dim3(hblocks), dim3(kHistThreads), 0, st, k0, n,
                           c.hist);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    uint32_t *ki = k0, *vi = v0, *ko = k1, *vo = v1;
    const uint32_t np = (uint32_t)parts;
    const int items = fanin_sort(n) ? kSmallItems : depth_items(n);
    for (int p = 0; p < kHistMaxPasses; ++p) {
        const uint32_t* hp = c.hist + p * kRadixBins;
        uint64_t* stat = c.status + (size_t)p * parts * kRadixBins;
        if (fanin_sort(n)) {
            uint16_t* stat16 = reinterpret_cast<uint16_t*>(c.status) + (size_t)p * parts * kRadixBins;
            const bool fin = p == 0 && finish;
            const BinFinish f = fin ? *finish : BinFinish{};
            const uint32_t fin_group = fin ? np : 0xffffffffu;
            const unsigned groups = np + (fin ? 1u : 0u);
            if (small_sort(n))
                hipLaunchKernelGGL(onesweep_small_kernel<kSmallThreads>, dim3(groups),
                                   dim3(kSmallThreads), 0, st, ki, vi, ko, vo, n, 8 * p, hp,
                                   stat16, err, f, fin_group);
            else
                hipLaunchKernelGGL(onesweep_small_kernel<kMediumThreads>, dim3(groups),
                                   dim3(kMediumThreads), 0, st, ki, vi, ko, vo, n, 8 * p, hp,
                                   stat16, err, f, fin_group);
            if (p == 0 && after_first) {
                e = hipGetLastError();
                if (e != hipSuccess) return e;
                e = hipEventRecord(after_first, st);
                if (e != hipSuccess) return e;
            }
        } else {
            // the status words of the pass hold the partitions' digit counts,
            // then their offsets
            uint32_t* part_hist = reinterpret_cast<uint32_t*>(stat);
            uint32_t* part_off = part_hist + (size_t)np * kRadixBins;
#define GSR_RTS_PASS(I)                                                                        \
    hipLaunchKernelGGL((rts_upsweep_kernel<I>), dim3(np), dim3(kSortThreads), 0, st, ki, n, 8 * p, \
                       hp, part_hist, np);                                                     \
    hipLaunchKernelGGL(rts_scan_kernel, dim3(kRadixBins), dim3(kRtsScanThreads), 0, st, hp, n,  \
                       part_hist, np, part_off);                                               \
    hipLaunchKernelGGL((rts_downsweep_kernel<false, I>), dim3(np), dim3(kSortThreads), 0, st,  \
                       ki, vi, ko, vo, n, 8 * p, 8, hp, part_off, 0);
            if (items == 4) {
                GSR_RTS_PASS(4)
            } else if (items == 6) {
                GSR_RTS_PASS(6)
            } else if (items == 8) {
                GSR_RTS_PASS(8)
            } else {
                GSR_RTS_PASS(10)
            }
#undef GSR_RTS_PASS
        }
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        std::swap(ki, ko);
        std::swap(vi, vo);
    }
    return hipSuccess;
}

size_t onesweep_state_bytes(uint64_t n, int passes) {
    return align_up((size_t)passes * 64, 256) + (size_t)passes * parts_for(n) * kRadixBins * 8;
}

hipError_t launch_tile_sort(const EmitSource& es, uint64_t m, int passes, int key_bits,
                            int gbits, const uint32_t* hist, void* state, uint32_t* k0,
                            uint32_t* k1, uint32_t* vbuf, uint32_t* out_vals, uint32_t* out_keys,
                            int* err, hipStream_t st) {
    if (m == 0) return hipSuccess;
    if (passes < 1 || passes > 4 || !out_keys || m >= (1ull << 32)) return hipErrorInvalidValue;
    const bool packed = gbits > 0;
    if (packed && gbits + key_bits > 32) return hipErrorInvalidValue;
    const uint64_t parts = parts_for(m);
    uint32_t* counters = static_cast<uint32_t*>(state);
    uint64_t* status = reinterpret_cast<uint64_t*>(static_cast<char*>(state) +
                                                   align_up((size_t)passes * 64, 256));
    // keys (or packed words): pass p writes kbuf[p & 1], the last pass out_keys
    // values (two-word form): the last pass writes out_vals, earlier passes
    // alternate back from it
    uint32_t* kbuf[2] = {k0, k1};
    uint32_t* vdst[4] = {nullptr, nullptr, nullptr, nullptr};
    if (!packed)
        for (int p = passes - 1, flip = 0; p >= 0; --p, flip ^= 1) vdst[p] = flip ? vbuf : out_vals;
    for (int p = 0; p < passes; ++p) {
        const bool last = p == passes - 1;
        uint32_t* ko = last ? out_keys : kbuf[p & 1];
        const uint32_t* ki = p == 0 ? nullptr : kbuf[(p - 1) & 1];
        const uint32_t* vi = (p == 0 || packed) ? nullptr : vdst[p - 1];
        uint32_t* vo = packed ? (last ? out_vals : nullptr) : vdst[p];
        const dim3 grid((unsigned)parts), block(kSortThreads);
        uint64_t* stat = status + (size_t)p * parts * kRadixBins;
        const uint32_t* h = hist + p * kRadixBins;
        uint32_t* ctr = counters + p * 16;
        const int shift = (packed ? gbits : 0) + 8 * p;
        const int bits = std::max(1, std::min(8, key_bits - 8 * p));  // significant digit bits
        if (p == 0 && packed)
            hipLaunchKernelGGL((onesweep_wide_kernel<true, true>), grid, block, 0, st, ki, vi, ko,
                               vo, m, shift, bits, h, stat, ctr, err, es, gbits);
        else if (p == 0)
            hipLaunchKernelGGL((onesweep_wide_kernel<true, false>), grid, block, 0, st, ki, vi, ko,
                               vo, m, shift, bits, h, stat, ctr, err, es, 0);
        else if (packed)
            hipLaunchKernelGGL((onesweep_wide_kernel<false, true>), grid, block, 0, st, ki, vi, ko,
                               vo, m, shift, bits, h, stat, ctr, err, es, gbits);
        else
            hipLaunchKernelGGL((onesweep_wide_kernel<false, false>), grid, block, 0, st, ki, vi,
                               ko, vo, m, shift, bits, h, stat, ctr, err, es, 0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

size_t scan_control_bytes(int n) {
    const size_t parts = ((size_t)std::max(n, 1) + kScanPartition - 1) / kScanPartition;
    return 256 + parts * 8;
}

hipError_t launch_scan_counts(int n, const uint32_t* perm, const uint32_t* counts,
                              uint32_t* offsets, uint64_t* total, void* control, int* err,
                              hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const unsigned parts = (unsigned)(((size_t)n + kScanPartition - 1) / kScanPartition);
    uint32_t* counter = static_cast<uint32_t*>(control);
    uint64_t* status = reinterpret_cast<uint64_t*>(static_cast<char*>(control) + 256);
    const int fanin = parts <= 64u * (unsigned)kFanPerLane ? 1 : 0;
    hipLaunchKernelGGL(scan_counts_kernel, dim3(parts), dim3(kScanThreads), 0, st, n, perm, counts,
                       offsets, total, status, counter, err, fanin);
    return hipGetLastError();
}

}  // namespace gsr
