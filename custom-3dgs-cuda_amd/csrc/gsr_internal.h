// gsr_internal.h — launchers behind the C ABI (include/gsraster.h).  Each
// returns hipSuccess or the first HIP error; argument validation happens in
// gsr_capi.cpp before any launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace gsr {

// ---- per-device globals (gsr_device.hip) ----
// Bytes of the fixed scratch array of gsr_rasterize_backward_noalloc.
constexpr size_t kNoAllocScratchBytes = (size_t)256 << 20;
// Status-word bits set by kernels.
constexpr int kStatusSpin = 1;    // a look-back wait reached its spin bound
constexpr int kStatusCounts = 2;  // a scan found counts that disagree with the binning's
struct DeviceGlobals {
    int* status = nullptr;    // device address of the current device's status word
    void* scratch = nullptr;  // device address of its scratch array
};
// The current device's globals: their addresses are looked up once per
// device (hipGetSymbolAddress, with that device current) and kept.
hipError_t device_globals(DeviceGlobals* out);
// ORs bits into a status word from a one-thread kernel (a test hook).
hipError_t launch_raise_status(int* status, int bits, hipStream_t st);

// VALU issue-rate calibration kernels (gsr_calibrate.hip): kind 0 add, 1 fma,
// 2 exp, 3 permlane swaps, 4 DPP add; calibrate_valu_blocks() work-groups of
// 256 threads, one float of `out` per thread.
int calibrate_valu_blocks();
hipError_t launch_calibrate_valu(int kind, int iters, float* out, hipStream_t st);

hipError_t launch_project_fwd(int n, const float* mu, const float* q, const float* s,
                              const float* rot, const float* tr, float fx, float fy, float cx,
                              float cy, float* mean2d, float* cov2d, float* depth,
                              hipStream_t st);

hipError_t launch_screen_radii(int n, const float* cov2d, float* radii, hipStream_t st);
hipError_t launch_camera_position(const float* rot, const float* trans, float* cam,
                                  hipStream_t st);
hipError_t launch_project_bwd(int n, const float* dmean, const float* dcov, const float* mu,
                              const float* q, const float* s, const float* rot, const float* tr,
                              float fx, float fy, float* dmu, float* dq, float* ds, int ref_quat,
                              hipStream_t st);

hipError_t launch_sh_fwd(int n, const float* cam, const float* mu, const float* albedo,
                         const float* kj, float* colors, hipStream_t st);

hipError_t launch_sh_bwd(int n, const float* cgrad, const float* mu, const float* albedo,
                         const float* kj, const float* cam, float* dA, float* dkj, float* dmu,
                         hipStream_t st);

// Fused per-Gaussian passes: camera position + projection + screen radius +
// SH colour (cam: 3 floats out; with logits also the sigmoid opacity), and
// SH backward + projection backward with dL/dmu summed (with dop also the
// sigmoid's backward into dlogits).  Bit for bit the single-pass kernels'
// (and torch's sigmoid) results.
hipError_t launch_project_sh_fwd(int n, const float* mu, const float* q, const float* s,
                                 const float* rot, const float* tr, float fx, float fy, float cx,
                                 float cy, const float* albedo, const float* kj, float* mean2d,
                                 float* cov2d, float* depth, float* radii, float* colors,
                                 float* cam, const float* logits, float* opacity,
                                 hipStream_t st);
hipError_t launch_project_sh_bwd(int n, const float* dmean, const float* dcov,
                                 const float* cgrad, const float* mu, const float* q,
                                 const float* s, const float* rot, const float* tr, float fx,
                                 float fy, const float* albedo, const float* kj, const float* cam,
                                 float* dmu, float* dq, float* ds, float* dA, float* dkj,
                                 int ref_quat, const float* dop, const float* op,
                                 float* dlogits, hipStream_t st);

// ---- radix sort (u32 keys, u32 values), 8-bit digits ----------------------
// Partition of one onesweep work-group of the LSD tile sort.
constexpr int kSortThreads = 1024;
constexpr int kSortItems = 8;
constexpr int kSortPartition = kSortThreads * kSortItems;
constexpr int kRadixBins = 256;

// Device control block of one depth sort: the digit histograms of the key's
// four bytes ([4][256] u32 at its start), counters and per-partition words.
// All of it must be zero before the histogram kernel runs
// (sort_control_bytes / the fill kernel).
size_t sort_control_bytes(uint64_t n);
// Stable sort of keys[0..n) (n < 2^32) on all 32 bits, carrying vals: four
// LSD passes of 8-bit digits, ping-ponging through (k1, v1) and ending in
// (k0, v0).  Up to 2^20 keys each pass is one onesweep kernel over at most
// 256 partitions (a fan-in of their digit counts); beyond, each pass is an
// upsweep / scan / downsweep triple with no waits between work-groups.  A pass whose digit is the same for every key
// copies through.  `control` must be zeroed on the stream first (zero_fill).
// err (device int) is set when a look-back wait exceeds kSpinLimit.
// hist_ready: the histogram block at the start of `control` was accumulated
// already.
struct BinFinish;
hipError_t launch_radix_sort(uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1, uint64_t n,
                             void* control, int* err, hipStream_t st, bool hist_ready = false,
                             const BinFinish* finish = nullptr, hipEvent_t after_first = nullptr);
// Whether launch_radix_sort runs `finish` (in one extra work-group of its first
// pass, after which it records `after_first`) for n keys: up to 2^20.
bool radix_sort_takes_finish(uint64_t n);
// The depth order's input: keys = the bits of depth[i], vals = i, and the
// keys' histogram block at the start of `control` (zeroed first), so that
// launch_radix_sort runs with hist_ready.
hipError_t launch_depth_keys_hist(uint64_t n, const float* depth, uint32_t* keys, uint32_t* vals,
                                  void* control, hipStream_t st);

hipError_t zero_fill(void* p, size_t bytes, hipStream_t st);
// Several regions in one launch.
struct FillList {
    static constexpr int kMaxFills = 6;
    void* ptr[kMaxFills] = {};
    size_t bytes[kMaxFills] = {};
    int count = 0;
    void add(void* p, size_t b) {
        if (b > 0 && count < kMaxFills) {
            ptr[count] = p;
            bytes[count] = b;
            ++count;
        }
    }
};
hipError_t zero_fill(const FillList& f, hipStream_t st);

// Where the first tile-sort pass generates its (tile, Gaussian) pairs: depth
// order perm, per-Gaussian counts and packed tile rectangles, per-rank pair
// offsets, and part_rank[p] = the rank holding pair slot p * kSortPartition
// (nparts + 1 entries; the last is one past the last rank with pairs).
struct EmitSource {
    const uint32_t* perm = nullptr;
    const uint32_t* counts = nullptr;
    const uint2* rects = nullptr;
    const uint32_t* offsets = nullptr;
    const uint32_t* part_rank = nullptr;
    uint32_t nparts = 0;
    int tiles_x = 0;
};

// Status words and partition counters of `passes` onesweep passes over n
// elements (zero before use).
size_t onesweep_state_bytes(uint64_t n, int passes);
// Stable LSD sort of the m pairs described by es on tile-id digits 0..passes-1
// (tile ids below 2^key_bits).
// hist holds the passes' global digit histograms ([passes][256], from the
// tile rectangles).  Values (Gaussian ids) end in out_vals; keys (tile ids)
// in out_keys when it is not null.  k0/k1/vbuf are m-element scratch.
// gbits > 0: the packed form, one word (tile << gbits) | Gaussian id per pair
// (gbits + key_bits <= 32); out_keys then receives the sorted words.
hipError_t launch_tile_sort(const EmitSource& es, uint64_t m, int passes, int key_bits,
                            int gbits, const uint32_t* hist, void* state, uint32_t* k0,
                            uint32_t* k1, uint32_t* vbuf, uint32_t* out_vals, uint32_t* out_keys,
                            int* err, hipStream_t st);

// ---- two-level tile binning (8x8-tile blocks, then tiles) ----
// The tile grid in blocks of 8x8 tiles, row-major.
struct BlockGrid {
    int tiles_x = 0, tiles_y = 0;
    int bw = 0, bh = 0, nb = 0;
};
BlockGrid block_grid(int tiles_x, int tiles_y);

// The binning's hand-off after its count kernel (bin_finish_body): the pair
// count and the device status word to host_total[0, 1], the block and segment
// starts from the block histogram.
struct BinFinish {
    int nb;
    const uint32_t* block_hist;
    const uint64_t* pair_total;
    uint32_t* block_start;
    uint32_t* seg_start;
    uint64_t* host_total;
    int* status;
};
// Blocks the binning's per-work-group block histogram holds.
constexpr int kMaxBlocks = 8192;

// Row stride (u32) of the per-block chunk counts: n Gaussians in chunks of 64,
// rounded up to a multiple of 4.
size_t block_count_stride(int n);
// Upper bound on level-2 segments for m pairs.
uint64_t segment_bound(uint64_t m, const BlockGrid& bg);

struct TileBinning {
    int n = 0;
    uint64_t m = 0;
    BlockGrid grid;
    const uint32_t* perm = nullptr;         // depth order (n)
    const uint2* rects = nullptr;           // packed tile rectangles (n)
    uint2* drects = nullptr;                // optional: rects in depth order (n), gathered once
    const uint32_t* block_hist = nullptr;   // Gaussians per block (nb)
    const uint32_t* block_start = nullptr;  // nb + 1
    const uint32_t* seg_start = nullptr;    // nb + 1
    uint32_t* bcount = nullptr;             // nb * block_count_stride(n)
    uint32_t* lists = nullptr;              // block lists (m)
    uint16_t* lrects = nullptr;             // each list entry's rectangle in its block (m)
    uint32_t* seg_owner = nullptr;          // segment_bound(m)
    uint32_t* tcount = nullptr;             // 64 * segment_bound(m)
    uint32_t* ttotal = nullptr;             // tiles
    int32_t* ranges = nullptr;              // out: [tiles][2]
    uint32_t* ids = nullptr;                // out: sorted ids (m)
    int* err = nullptr;                     // bit 2: inconsistent counts
    // optional: tiles (nonzero) whose lists stay empty; the lists then hold
    // fewer than m entries
    const uint8_t* skip = nullptr;
    // optional: the blend records (n) from these, formed in extra work-groups
    // of the level-1 count kernel's launch (independent work, one launch fewer)
    const float* rec_mean2d = nullptr;
    const float* rec_cov2d = nullptr;
    const float* rec_colors = nullptr;
    const float* rec_alpha = nullptr;
    void* recs = nullptr;
};
// sorted ids and tile ranges from the depth order and tile rectangles.
hipError_t launch_tile_binning(const TileBinning& tb, hipStream_t st);
// Optional debug output from the ranges: (tile << 32) | float_bits(depth[id]).
hipError_t launch_range_keys(int T, const int32_t* ranges, const int32_t* ids, const float* depth,
                             int n, uint64_t m, uint64_t* keys, hipStream_t st);

// ---- binning ----
// Pairs per tile row of an H x W frame (rows[tiles_y], needs tiles_y + 1
// entries of room; tiles_y <= 4096).
hipError_t launch_row_pairs(int n, const float* mean2d, const float* cov2d, int H, int W,
                            uint64_t* rows, hipStream_t st);
// flags[i]: Gaussian i's tile rectangle, widened by one tile row each way,
// holds a tile marked in the summed-area table sat ((tiles_y+1) x (tiles_x+1)).
hipError_t launch_tiles_touch(int n, const float* mean2d, const float* cov2d, int H, int W,
                              const int32_t* sat, uint8_t* flags, hipStream_t st);
// counts[g], packed tile rect, depth key (float bits or 0xffffffff when the
// Gaussian touches no tile) and identity values, the digit histograms of the
// 4-pass depth sort (depth_hist), and either the digit histograms of the tile
// sort (tile_passes > 0: tile_hist) or the block histogram (block_hist), with
// the pair count added to *pair_total; in block histogram mode a one-group
// kernel behind it then writes the block and segment starts (block_start /
// seg_start, nb + 1 entries each) and, when host_total is not null, the final
// pair count to that host-mapped coherent word and the device status word
// (status, read and cleared) to host_total[1] (with finish false that kernel is
// not launched: the caller runs the hand-off itself, in the depth sort's
// first pass).  dkeys null: no depth keys, values or depth histograms (depth
// is then not read).
hipError_t launch_bin_count(int n, const float* mean2d, const float* cov2d, const float* depth,
                            int H, int W, uint32_t* counts, uint2* rects, uint32_t* dkeys,
                            uint32_t* dvals, int tile_passes, uint32_t* tile_hist,
                            uint32_t* depth_hist, uint32_t* block_hist, uint64_t* pair_total,
                            uint32_t* block_start, uint32_t* seg_start,
                            uint64_t* host_total, int* status, hipStream_t st,
                            bool finish = true);

// The backward's per-Gaussian pass: blend records, tile rectangles and counts,
// and the slot offsets goff (exclusive scan of the counts in Gaussian order,
// total to *total).  control: records_slots_control_bytes(n), zeroed.  With
// `work` (up to 2^18 Gaussians; returns true when taken) the same launch also
// computes the backward's per-tile work estimate from the tile ranges (num_pairs
// entries) and n_contrib into work (launch_bwd_schedule then runs with
// work_ready).
size_t records_slots_control_bytes(int n);
hipError_t launch_records_slots(int n, const float* mean2d, const float* cov2d,
                                const float* colors, const float* alpha, void* recs, int H, int W,
                                uint32_t* counts, uint2* rects, uint32_t* goff, uint64_t* total,
                                void* control, int* err, hipStream_t st,
                                const int32_t* ranges = nullptr, uint64_t num_pairs = 0,
                                const int32_t* ncontrib = nullptr, uint32_t* work = nullptr,
                                bool* work_done = nullptr);

// Exclusive scan of counts[perm[r]] over depth rank r -> offsets[r] (perm null:
// the identity); the total (u64) is written to *total.
size_t scan_control_bytes(int n);
hipError_t launch_scan_counts(int n, const uint32_t* perm, const uint32_t* counts,
                              uint32_t* offsets, uint64_t* total, void* control, int* err,
                              hipStream_t st);

// part_rank[p] for the fused emission of the first tile-sort pass (nparts + 1
// entries, nparts = ceil(m / kSortPartition)).
hipError_t launch_partition_starts(int n, const uint32_t* perm, const uint32_t* counts,
                                   const uint32_t* offsets, uint64_t m, uint32_t* part_rank,
                                   hipStream_t st);

// [start, end) per tile from sorted tile keys (tile = key >> shift); ranges
// must be zeroed.
hipError_t launch_tile_ranges(uint64_t m, uint32_t T, const uint32_t* sorted_tiles, int shift,
                              int32_t* ranges, hipStream_t st);

// Optional debug output: (tile << 32) | float_bits(depth[id]).
hipError_t launch_full_keys(uint64_t m, const uint32_t* sorted_tiles, int shift,
                            const int32_t* ids, const float* depth, int n, uint64_t* keys,
                            hipStream_t st);

// ---- blend ----
// With counts/rects (the backward) also the tile rectangle and count per
// Gaussian, as the binning forms them.
hipError_t launch_blend_records(int n, const float* mean2d, const float* cov2d,
                                const float* colors, const float* alpha, void* recs,
                                hipStream_t st, int H = 0, int W = 0, uint32_t* counts = nullptr,
                                uint2* rects = nullptr);

// Forward schedule: per-tile work estimates (work, T entries) and the launch
// order (order, T entries).
hipError_t launch_fwd_schedule(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                               uint64_t m, const void* recs, uint32_t* work, uint32_t* order,
                               hipStream_t st);
hipError_t launch_blend_fwd(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                            uint64_t m, const void* recs, float* img, float* finalT,
                            int32_t* ncontrib, const uint32_t* order, hipStream_t st);

// Backward schedule: entries up to each tile's largest n_contrib (unless
// work_ready: computed already), then the order.
hipError_t launch_bwd_schedule(int H, int W, const int32_t* ranges, uint64_t num_pairs,
                               const int32_t* ncontrib, uint32_t* work, uint32_t* order,
                               hipStream_t st, bool work_ready = false);

// Gradient slots: the (Gaussian, tile) pairs in Gaussian-major order, pair
// (g, t) at goff[g] + its index in g's tile rectangle (row-major); the backward
// claims each processed pair's slot (bit slot % 32 of flags[slot / 32], an
// atomic OR) and writes its nine sums to sums[9 slot ..], and
// pair_grad_reduce adds each Gaussian's claimed slots to the gradient
// outputs.  One bit per slot: at 4K with millions of Gaussians only about one
// slot in a thousand is claimed, and the flags are cleared and read in full.
// Pairs without a slot of their own (outside the rectangles, or an id repeated
// within one tile's list) fall back to atomics on the outputs.
struct GradSlots {
    const uint32_t* goff = nullptr;
    const uint32_t* counts = nullptr;
    const uint2* rects = nullptr;
    float* sums = nullptr;
    uint32_t* flags = nullptr;  // one bit per slot, padded to 64-bit words
    uint64_t slots = 0;
};

// Element strides of dL/dimage: pixel (y, x) channel c at grad[y h + x w + c c]
// ({3 W, 3, 1} for a contiguous [H, W, 3] image).
struct GradStrides {
    int64_t h = 0, w = 0, c = 0;
};

hipError_t launch_blend_bwd(int n, int H, int W, const float* grad, const GradStrides& gst,
                            const int32_t* ranges,
                            const int32_t* ids, uint64_t num_pairs, const void* recs,
                            const float* finalT, const int32_t* ncontrib, float* dmean,
                            float* dcov, float* dcol, float* dalpha, const GradSlots& gs,
                            const uint32_t* order, hipStream_t st);

// outputs += the per-Gaussian sums of the flagged slots (each slot holds its
// (tile, entry)'s covariance gradient, converted from the conic's in the blend).
hipError_t launch_pair_grad_reduce(int n, const GradSlots& gs, float* dmean, float* dcov,
                                   float* dcol, float* dalpha, hipStream_t st);

// ---- training loss (gsr_loss.hip) ----
// Work-group partial sums of the loss's forward kernel for an H x W image
// (float2 each).
size_t loss_partial_count(int H, int W);
// (1 - lambda) mean|gt - img| + lambda (1 - SSIM): out[0] = loss, out[1] =
// SSIM, out[2] = the L1 mean (device floats); gmaps (3 planes of H W 3 floats,
// or null) receives the SSIM index's derivatives for the backward.
hipError_t launch_l1_dssim_fwd(int H, int W, const float* img, const float* gt, float lambda,
                               float* gmaps, void* partial, float* out, hipStream_t st);
// dL/dimg, scaled by *grad_loss (a device float; null reads as 1).
hipError_t launch_l1_dssim_bwd(int H, int W, const float* img, const float* gt, float lambda,
                               const float* gmaps, const float* grad_loss, float* dimg,
                               hipStream_t st);

// ---- optimizer step (gsr_optim.hip) ----
constexpr int kAdamMaxTensors = 8;  // tensors per launch
struct AdamTensor {
    float* param;
    const float* grad;
    float* exp_avg;
    float* exp_avg_sq;
    uint64_t numel;
};
// A tensor's fp32 scalars, each rounded once from the host's double: 1 - b1,
// b2, 1 - b2, sqrt(1 - b2^t), -lr / (1 - b1^t), eps, and the clamp bounds.
struct AdamHostScalars {
    float w1, b2, w2, bc2s, neg_step, eps, lo, hi;
};
hipError_t launch_adam(int count, const AdamTensor* tensors, const AdamHostScalars* hs,
                       hipStream_t st);

// ---- PLY export (gsr_export.hip) ----
// Inria 3DGS vertex records [n, 17 + 3K] of n Gaussians with K rest SH
// coefficients per channel (q 16-byte aligned).
hipError_t launch_ply_pack(int n, int K, const float* mu, const float* q, const float* s,
                           const float* alpha, const float* A, const float* kj,
                           int from_probability, float* out, hipStream_t st);

// ---- adaptive density control (gsr_adc.hip) ----
// A cloud's six parameter arrays: mu [N,3], q [N,4], s [N,3], alpha [N],
// A [N,3], k_j [N,15,3]; its Adam moments: exp_avg of each, then exp_avg_sq
// of each (null entries: no state, read as zeros / not written).
struct AdcCloud {
    float* p[6];
};
struct AdcMoments {
    float* p[12];
};
// fp32 thresholds (the reference compares fp32 tensors with Python floats).
struct AdcConfig {
    float grad_threshold, dense_scale, max_scale, min_opacity, max_screen, split_scale,
        reset_logit;
    int densify, prune, has_screen, reset_opacity;
};
// Densification statistics: with mean2d_grad, its norm (the gradient scaled
// by (sx, sy) when `scale`) added to accum and 1 to denom where it is > 0;
// with radii, maxr = max(maxr, radii).
hipError_t launch_adc_stats(int n, const float* mean2d_grad, float sx, float sy, int scale,
                            const float* radii, float* accum, float* denom, float* maxr,
                            hipStream_t st);
size_t adc_workspace_bytes(int n);
// Flags and counts per source, then totals_dev[5] (device u64): kept
// originals, kept clones, kept split sources (two copies each), all split
// sources (noise rows: two per source), all clone sources.  The workspace's
// first 256 bytes are free for totals_dev.
hipError_t launch_adc_plan(int n, const AdcCloud& in, const float* accum, const float* denom,
                           const float* maxr, const AdcConfig& c, void* ws, uint64_t* totals_dev,
                           hipStream_t st);
hipError_t launch_adc_gather(int n, const AdcCloud& in, const AdcMoments& min_,
                             const float* noise, const AdcConfig& c, const void* ws,
                             const uint64_t* totals_dev, const AdcCloud& out,
                             const AdcMoments& mout, hipStream_t st);

}  // namespace gsr
