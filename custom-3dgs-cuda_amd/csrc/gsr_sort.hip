// gsr_sort.hip — LSD onesweep radix sort (u32 keys carrying u32 values) and
// the decoupled look-back scan of per-Gaussian tile counts.
//
// Sort design (one kernel per 8-bit digit pass, plus one histogram kernel):
//   * A work-group owns a partition of 4096 consecutive elements, claimed in
//     launch order through an atomic counter so that every partition it waits
//     on belongs to a work-group that is already resident.
//   * Items are loaded wave-striped (item i of lane l in wave w is element
//     w*1024 + i*64 + l), so each wave load is one contiguous 256 B access.
//   * Stable in-partition ranks come from 8 ballots per item (lanes sharing a
//     digit) plus per-wave running digit counters in LDS.
//   * Each partition publishes its 256 digit counts, looks back over earlier
//     partitions' published counts (decoupled look-back) and scatters its
//     elements, first reordered in LDS so each digit's run is written with
//     consecutive addresses.
//   * Look-back spins are bounded by kSpinLimit; a partition that reaches it
//     raises the error flag and finishes, so every wave exits.
// HBM traffic per pass: 8 B read + 8 B written per element (+ 8 B per
// partition and digit of status words).
#include <algorithm>

#include "gsr_internal.h"
#include "gsr_common.h"
#include "gsr_group.h"

namespace gsr {

namespace {

constexpr int kHistMaxPasses = 4;
constexpr int kLookback = 4;
static_assert(kSortThreads == kRadixBins, "one thread per digit in the onesweep kernel");
static_assert(kSortThreads == 256, "four waves per onesweep work-group");

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct SortCtl {
    uint32_t* hist;      // [passes][256]
    uint32_t* counters;  // [passes] (one per 64 B line)
    uint64_t* status;    // [passes][parts][256]
};

inline uint64_t parts_for(uint64_t n) { return (n + kSortPartition - 1) / kSortPartition; }

// Items per thread of the key sort (launch_radix_sort): small inputs take
// 1024-element partitions, so a pass runs on more work-groups, each with less
// to rank; larger ones 4096, which keeps the look-back chain short.
constexpr uint64_t kSmallSortMax = 1u << 18;
inline int sort_items(uint64_t n) { return n <= kSmallSortMax ? 4 : kSortItems; }
inline uint64_t sort_parts(uint64_t n) {
    const uint64_t part = (uint64_t)kSortThreads * (uint64_t)sort_items(n);
    return (n + part - 1) / part;
}

SortCtl carve(void* control, uint64_t n, int passes) {
    char* p = static_cast<char*>(control);
    SortCtl c;
    c.hist = reinterpret_cast<uint32_t*>(p);
    p += align_up((size_t)passes * kRadixBins * 4, 256);
    c.counters = reinterpret_cast<uint32_t*>(p);
    p += align_up((size_t)passes * 64, 256);
    c.status = reinterpret_cast<uint64_t*>(p);
    return c;
}

// Lanes of `active` whose digit equals this lane's, comparing the low `bits`
// bits (the digit's higher bits are known to be zero in every key).
__device__ __forceinline__ uint64_t match_digit(uint32_t d, uint64_t active, int bits = 8) {
    uint64_t m = active;
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        if (b >= bits) break;
        const bool bit = (d >> b) & 1u;
        const uint64_t t = ballot(bit);
        m &= bit ? t : ~t;
    }
    return m;
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

// Global digit histograms of every pass in one read of the keys.  Digit
// counts are aggregated per wave (ballot match) before the LDS atomics, and
// per work-group before the global atomics.
__global__ __launch_bounds__(256) void radix_hist_kernel(const uint32_t* __restrict__ keys,
                                                         uint64_t n, int begin_bit, int passes,
                                                         uint32_t* __restrict__ hist) {
    __shared__ uint32_t s_h[kHistMaxPasses][kRadixBins];
    for (int j = threadIdx.x; j < kHistMaxPasses * kRadixBins; j += 256) (&s_h[0][0])[j] = 0;
    __syncthreads();
    const uint64_t stride = (uint64_t)gridDim.x * 256;
    const uint64_t nround = (n + 255) / 256 * 256;  // keep whole waves in the loop
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < nround; i += stride) {
        const bool valid = i < n;
        const uint32_t k = valid ? keys[i] : 0u;
        const uint64_t act = ballot(valid);
        for (int p = 0; p < passes; ++p) {
            const uint32_t d = (k >> (begin_bit + 8 * p)) & 0xffu;
            const uint64_t peers = match_digit(d, act);
            if (valid && (peers & lanemask_lt()) == 0)
                atomicAdd(&s_h[p][d], (uint32_t)popc64(peers));
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < passes * kRadixBins; j += 256) {
        const uint32_t v = (&s_h[0][0])[j];
        if (v) atomicAdd(&hist[j], v);
    }
}

// The emission's staging index: one padding word per 16 slots, so a wave's
// blocked writes (16 slots per lane) and striped reads spread over the banks.
__device__ __forceinline__ int pad16(int slot) { return slot + (slot >> 4); }

// Expands the (tile, Gaussian) pairs of sort slots [base, base + nvalid) into
// s_keys / s_vals at pad16(slot) (kPacked: the one word (tile << gbits) | g in
// s_keys).  Pair slots are laid out by depth rank r at
// offsets[r] (ty outer, tx inner over the rank's tile rectangle), the order in
// which the reference emits keys per Gaussian (rasterize.cu:124-135).  Ranks
// r_lo..r_lo+nr-1 overlap the partition; the first kStageRanks of them have
// their offset, Gaussian id and tile rectangle staged in LDS by one parallel
// load (more only occur for partitions of very small Gaussians, or when ranks
// without pairs sit between ranks with pairs, and are read from global
// memory).  Each thread expands 16 consecutive slots: one binary search, one
// division, then a walk that steps the column and row.
constexpr int kStageRanks = 512;

struct RankStage {
    uint32_t off[kStageRanks];
    uint32_t g[kStageRanks];
    uint2 rect[kStageRanks];
};
constexpr int kRankStageWords = (int)(sizeof(RankStage) / 4);
static_assert(kRankStageWords >= 7 * kRadixBins, "the aux region also holds the digit counters");

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

// One LSD pass over 8-bit digit (key >> shift) & 0xff.  kEmit: the partition's
// (tile, Gaussian) pairs are generated from the depth order instead of being
// read (the first tile pass).  kPacked: each element is the one word
// (tile << gbits) | Gaussian id, sorted on its tile bits; kout receives the
// words and, when vout is not null (the last pass), vout the Gaussian ids.
// Otherwise keys and values are separate words, both written.
template <bool kEmit, bool kPacked, int kItems = kSortItems>
__global__ __launch_bounds__(kSortThreads) void onesweep_kernel(
    const uint32_t* __restrict__ kin, const uint32_t* __restrict__ vin,
    uint32_t* __restrict__ kout, uint32_t* __restrict__ vout, uint64_t n, int shift,
    int digit_bits, const uint32_t* __restrict__ hist, uint64_t* __restrict__ status,
    uint32_t* __restrict__ counter, int* __restrict__ err, EmitSource es, int gbits) {
    // s_aux holds the emission's staged offsets first, then the digit counters,
    // digit starts and global bases (7 KB).
    constexpr int kAuxWords = kEmit ? kRankStageWords : 7 * kRadixBins;
    constexpr int kPart = kSortThreads * kItems;  // elements per partition
    static_assert(!kEmit || kItems == kSortItems, "the emission expands kSortPartition slots");
    __shared__ uint32_t s_keys[kPart + kPart / 16];
    __shared__ uint32_t s_vals[kPacked ? 1 : kPart + kPart / 16];
    __shared__ __align__(16) uint32_t s_aux[kAuxWords];
    __shared__ uint32_t s_scan[4];
    __shared__ uint32_t s_hscan[4];
    __shared__ uint32_t s_part;
    uint32_t (*s_wcnt)[kRadixBins] = reinterpret_cast<uint32_t (*)[kRadixBins]>(s_aux);
    uint32_t* s_dstart = s_aux + 4 * kRadixBins;
    uint64_t* s_gbase = reinterpret_cast<uint64_t*>(s_aux + 5 * kRadixBins);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_part = atomicAdd(counter, 1u);
    __syncthreads();
    const uint64_t part = s_part;
    const uint64_t base = part * kPart;
    const int nvalid = (int)min((uint64_t)kPart, n - base);
    if constexpr (!kEmit) {
        // Every key has the same digit: the stable pass is the identity, so the
        // partition is copied through (no ranking, no look-back).
        if (__syncthreads_or(hist[tid] == (uint32_t)n)) {
            // 16-byte copies when every array is 16-byte aligned (partitions start
            // a multiple of 4 KB apart), the rest word by word
            const uint32_t mask = kPacked ? ((1u << gbits) - 1u) : 0u;
            const uintptr_t al = reinterpret_cast<uintptr_t>(kin) |
                                 reinterpret_cast<uintptr_t>(kout) |
                                 reinterpret_cast<uintptr_t>(vin) |
                                 reinterpret_cast<uintptr_t>(vout);
            const int n4 = (al & 15) ? 0 : nvalid / 4;
            const uint4* k4 = reinterpret_cast<const uint4*>(kin + base);
            uint4* ko4 = reinterpret_cast<uint4*>(kout + base);
#pragma unroll 4
            for (int e = tid; e < n4; e += kSortThreads) {
                const uint4 k = k4[e];
                ko4[e] = k;
                if constexpr (kPacked) {
                    if (vout)
                        reinterpret_cast<uint4*>(vout + base)[e] =
                            make_uint4(k.x & mask, k.y & mask, k.z & mask, k.w & mask);
                } else {
                    reinterpret_cast<uint4*>(vout + base)[e] =
                        reinterpret_cast<const uint4*>(vin + base)[e];
                }
            }
            for (int e = 4 * n4 + tid; e < nvalid; e += kSortThreads) {
                const uint32_t k = kin[base + e];
                kout[base + e] = k;
                if constexpr (kPacked) {
                    if (vout) vout[base + e] = k & mask;
                } else {
                    vout[base + e] = vin[base + e];
                }
            }
            return;
        }
    }

    uint32_t key[kItems], val[kItems], rank[kItems];
    (void)val;
    if constexpr (kEmit) {
        expand_pairs<kPacked>(es, base, nvalid, s_keys, s_vals,
                              reinterpret_cast<RankStage*>(s_aux), gbits);  // ends with a barrier
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            const bool v = e < nvalid;
            key[i] = v ? s_keys[pad16(e)] : 0u;
            if constexpr (!kPacked) val[i] = v ? s_vals[pad16(e)] : 0u;
        }
    } else {
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int e = wave * (kItems * 64) + i * 64 + lane;
            const bool v = e < nvalid;
            key[i] = v ? kin[base + e] : 0u;
            if constexpr (!kPacked) val[i] = v ? vin[base + e] : 0u;
        }
    }
    for (int j = tid; j < 4 * kRadixBins; j += kSortThreads) (&s_wcnt[0][0])[j] = 0;
    __syncthreads();
    // Stable ranks within the wave's slice, in element order.
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        const bool v = e < nvalid;
        const uint32_t d = (key[i] >> shift) & 0xffu;
        const uint64_t peers = match_digit(d, ballot(v), digit_bits);
        rank[i] = 0;
        if (v) {
            const uint32_t before = s_wcnt[wave][d];
            const uint64_t lower = peers & lanemask_lt();
            rank[i] = before + (uint32_t)popc64(lower);
            if (lower == 0) s_wcnt[wave][d] = before + (uint32_t)popc64(peers);
        }
    }
    __syncthreads();

    // One thread per digit: partition total, publish, prefixes.
    const int d = tid;
    const uint32_t c0 = s_wcnt[0][d], c1 = s_wcnt[1][d], c2 = s_wcnt[2][d], c3 = s_wcnt[3][d];
    const uint32_t total = c0 + c1 + c2 + c3;
    uint64_t* my_status = status + part * kRadixBins + d;
    store_agent(my_status, (part == 0 ? kFlagInclusive : kFlagAggregate) | (uint64_t)total);
    s_wcnt[0][d] = 0;
    s_wcnt[1][d] = c0;
    s_wcnt[2][d] = c0 + c1;
    s_wcnt[3][d] = c0 + c1 + c2;
    const uint32_t inc = wave_inclusive_scan(total);
    const uint32_t h = hist[d];
    const uint32_t hinc = wave_inclusive_scan(h);
    if (lane == 63) {
        s_scan[wave] = inc;
        s_hscan[wave] = hinc;
    }
    __syncthreads();
    uint32_t wpre = 0, hpre = 0;
    for (int w = 0; w < wave; ++w) {
        wpre += s_scan[w];
        hpre += s_hscan[w];
    }
    const uint32_t dstart = wpre + inc - total;
    const uint64_t hexcl = (uint64_t)(hpre + hinc - h);
    s_dstart[d] = dstart;
    __syncthreads();

    // Reorder the partition in LDS by digit (stable).
#pragma unroll
    for (int i = 0; i < kItems; ++i) {
        const int e = wave * (kItems * 64) + i * 64 + lane;
        if (e < nvalid) {
            const uint32_t dd = (key[i] >> shift) & 0xffu;
            const uint32_t pos = s_dstart[dd] + s_wcnt[wave][dd] + rank[i];
            s_keys[pos] = key[i];
            if constexpr (!kPacked) s_vals[pos] = val[i];
        }
    }

    // Decoupled look-back for digit d over earlier partitions, kLookback
    // status words per round trip (before partition 0 reads as inclusive 0).
    uint64_t excl = 0;
    if (part > 0) {
        int64_t p = (int64_t)part - 1;
        uint32_t spins = 0;
        while (true) {
            uint64_t sw[kLookback];
#pragma unroll
            for (int k = 0; k < kLookback; ++k)
                sw[k] = (p - k >= 0) ? load_agent(status + (uint64_t)(p - k) * kRadixBins + d)
                                     : kFlagInclusive;
            int k = 0;
            bool done = false;
            for (; k < kLookback; ++k) {
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
            if (k < kLookback) {
                if (++spins > kSpinLimit) {
                    atomicOr(err, 1);
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
        }
        store_agent(my_status, kFlagInclusive | (excl + total));
    }
    s_gbase[d] = hexcl + excl - (uint64_t)dstart;
    __syncthreads();

    for (int j = tid; j < nvalid; j += kSortThreads) {
        const uint32_t k = s_keys[j];
        const uint64_t o = s_gbase[(k >> shift) & 0xffu] + (uint64_t)j;
        if (o < n) {  // always true for consistent histograms; guards the stores
            if constexpr (kPacked) {
                kout[o] = k;
                if (vout) vout[o] = k & ((1u << gbits) - 1u);
            } else {
                kout[o] = k;
                vout[o] = s_vals[j];
            }
        }
    }
}

// ---- exclusive scan of counts[perm[r]] (decoupled look-back) -------------
constexpr int kScanThreads = 256;
constexpr int kScanItems = 16;
constexpr int kScanPartition = kScanThreads * kScanItems;

__global__ __launch_bounds__(kScanThreads) void scan_counts_kernel(
    int n, const uint32_t* __restrict__ perm, const uint32_t* __restrict__ counts,
    uint32_t* __restrict__ offsets, uint64_t* __restrict__ total, uint64_t* __restrict__ status,
    uint32_t* __restrict__ counter, int* __restrict__ err) {
    __shared__ uint32_t s_part;
    __shared__ uint32_t s_wsum[4];
    __shared__ uint64_t s_base;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid == 0) s_part = atomicAdd(counter, 1u);
    __syncthreads();
    const uint64_t part = s_part;
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
    // look-back by the first wave, 64 predecessors per step
    if (wave == 0) {
        const uint64_t excl = wave_lookback(status, part, (uint64_t)btot, err);
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

size_t sort_control_bytes(uint64_t n, int passes) {
    return align_up((size_t)passes * kRadixBins * 4, 256) + align_up((size_t)passes * 64, 256) +
           (size_t)passes * sort_parts(n) * kRadixBins * 8;
}

hipError_t launch_radix_sort(uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1, uint64_t n,
                             int begin_bit, int passes, void* control, int* err, hipStream_t st,
                             bool hist_ready) {
    if (n == 0 || passes <= 0) return hipSuccess;
    if (passes > kHistMaxPasses) return hipErrorInvalidValue;
    const uint64_t parts = sort_parts(n);
    const bool small = sort_items(n) == 4;
    SortCtl c = carve(control, n, passes);
    hipError_t e = hipSuccess;
    if (!hist_ready) {
        const unsigned hblocks = (unsigned)std::min<uint64_t>(parts, 512);
        hipLaunchKernelGGL(radix_hist_kernel, dim3(hblocks), dim3(256), 0, st, k0, n, begin_bit,
                           passes, c.hist);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    uint32_t *ki = k0, *vi = v0, *ko = k1, *vo = v1;
    for (int p = 0; p < passes; ++p) {
        if (small)
            hipLaunchKernelGGL((onesweep_kernel<false, false, 4>), dim3((unsigned)parts),
                               dim3(kSortThreads), 0, st, ki, vi, ko, vo, n, begin_bit + 8 * p, 8,
                               c.hist + p * kRadixBins,
                               c.status + (size_t)p * parts * kRadixBins, c.counters + p * 16,
                               err, EmitSource{}, 0);
        else
            hipLaunchKernelGGL((onesweep_kernel<false, false>), dim3((unsigned)parts),
                               dim3(kSortThreads), 0, st, ki, vi, ko, vo, n, begin_bit + 8 * p, 8,
                               c.hist + p * kRadixBins,
                               c.status + (size_t)p * parts * kRadixBins, c.counters + p * 16,
                               err, EmitSource{}, 0);
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
    if (passes < 1 || passes > 4 || !out_keys) return hipErrorInvalidValue;
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
            hipLaunchKernelGGL((onesweep_kernel<true, true>), grid, block, 0, st, ki, vi, ko, vo,
                               m, shift, bits, h, stat, ctr, err, es, gbits);
        else if (p == 0)
            hipLaunchKernelGGL((onesweep_kernel<true, false>), grid, block, 0, st, ki, vi, ko, vo,
                               m, shift, bits, h, stat, ctr, err, es, 0);
        else if (packed)
            hipLaunchKernelGGL((onesweep_kernel<false, true>), grid, block, 0, st, ki, vi, ko, vo,
                               m, shift, bits, h, stat, ctr, err, es, gbits);
        else
            hipLaunchKernelGGL((onesweep_kernel<false, false>), grid, block, 0, st, ki, vi, ko,
                               vo, m, shift, bits, h, stat, ctr, err, es, 0);
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
    hipLaunchKernelGGL(scan_counts_kernel, dim3(parts), dim3(kScanThreads), 0, st, n, perm, counts,
                       offsets, total, status, counter, err);
    return hipGetLastError();
}

}  // namespace gsr
