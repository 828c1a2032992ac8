// gsr_capi.cpp — the extern "C" entry points of libgsraster.so
// (declared in include/gsraster.h): argument checks, workspace carving and
// the launch sequence of each stage.  No allocation happens here; every
// buffer comes from the caller.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "gsr_internal.h"
#include "../../include/gsraster.h"

// "file=hash;..." over the sources this library was built from (build.py
// passes it); a build by other means reports that it recorded none.
#ifndef GSR_SOURCES
#define GSR_SOURCES ""
#endif

namespace {

thread_local std::string g_err;

int fail(int code, const std::string& msg) {
    g_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return fail(GSR_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

#define GSR_HIP(expr, what)                          \
    do {                                             \
        hipError_t gsr_e_ = (expr);                  \
        if (gsr_e_ != hipSuccess) return hip_fail(gsr_e_, what); \
    } while (0)

#define GSR_REQUIRE(cond, msg) \
    do {                       \
        if (!(cond)) return fail(GSR_ERR_INVALID_ARGUMENT, msg); \
    } while (0)

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// sorted_ids and tile ranges are int32, and the kernels add up to two list
// batches (well under 2^16) to int32 list positions: the pair count stays
// that far below 2^31.
constexpr int64_t kMaxPairs = 2147483647 - 65535;
constexpr size_t kRecBytes = 48;

int tiles_x_of(int W) { return (W + 15) / 16; }
int tiles_y_of(int H) { return (H + 15) / 16; }

// Digit passes of the tile sort for tile ids in [0, T): ceil(bits / 8), at
// least one (the pass that generates the pairs).
int tile_passes(int64_t T) {
    int bits = 0;
    uint64_t v = (uint64_t)(T > 1 ? T - 1 : 0);
    while (v) {
        ++bits;
        v >>= 1;
    }
    return bits > 8 ? (bits + 7) / 8 : 1;
}
constexpr int kMaxTilePasses = 4;

// Bits of a Gaussian id in the packed tile-sort word, or 0 for the two-word
// form (tile and id do not fit in 32 bits together).
int packed_id_bits(int n, int64_t T);

// Significant bits of tile ids in [0, T).
int tile_key_bits(int64_t T) {
    int bits = 0;
    for (uint64_t v = (uint64_t)(T > 1 ? T - 1 : 0); v; v >>= 1) ++bits;
    return bits;
}

// Misc block at the head of the bin workspace.  In the host's pinned copy,
// `status` receives the device status word.
struct Misc {
    uint64_t total;       // pair count
    int status;           // host copy only: the device status word
};

// The message for a non-zero device status word.
std::string status_message(int bits) {
    std::string m = "a kernel on this device";
    if (bits & gsr::kStatusSpin) m += " reached its look-back spin bound";
    if ((bits & gsr::kStatusSpin) && (bits & gsr::kStatusCounts)) m += " and one";
    if (bits & gsr::kStatusCounts) m += " found counts inconsistent with the binning";
    return m + " (status " + std::to_string(bits) +
           "; reported by the first forward or status call after it); its outputs are invalid";
}

// Which tile binning a frame uses: the two-level block binning, unless the
// grid has more 8x8-tile blocks than its histogram holds or GSR_TILE_BINNING
// is "sort" (the LSD tile sort).  Read on every call: it must not change
// between the bin and render calls of one frame.
bool block_binning(int H, int W) {
    const char* v = std::getenv("GSR_TILE_BINNING");
    if (v && std::strcmp(v, "sort") == 0) return false;
    return gsr::block_grid(tiles_x_of(W), tiles_y_of(H)).nb <= gsr::kMaxBlocks;
}

struct BinLayout {
    size_t misc, sortctl, scanctl, tilehist, blockhist, ctl_end;
    size_t counts, rects, dk0, dv0, dk1, dv1, offsets, block_start, seg_start, recs, end;
};

BinLayout bin_layout(int n, int H, int W) {
    BinLayout L;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t un = (size_t)(n > 0 ? n : 0);
    L.misc = take(sizeof(Misc));
    L.sortctl = take(gsr::sort_control_bytes(un));
    L.scanctl = take(gsr::scan_control_bytes(n));
    L.tilehist = take((size_t)kMaxTilePasses * 256 * 4);
    const gsr::BlockGrid bg = gsr::block_grid(tiles_x_of(W), tiles_y_of(H));
    const size_t nb = (size_t)bg.nb;
    L.blockhist = take(4 * nb);
    L.ctl_end = off;
    L.counts = take(4 * un);
    L.rects = take(8 * un);
    L.dk0 = take(4 * un);
    L.dv0 = take(4 * un);
    L.dk1 = take(4 * un);
    L.dv1 = take(4 * un);
    L.offsets = take(4 * un);
    L.block_start = take(4 * (nb + 1));
    L.seg_start = take(4 * (nb + 1));
    L.recs = take(kRecBytes * un);
    L.end = off;
    return L;
}

// Render workspace.  LSD tile sort: look-back state (cleared), then key,
// value and scratch words per pair.  Block binning: the per-block chunk
// counts, the block lists, segment owners and counts, and tile totals.  One
// size serves both; the schedule's work and order arrays follow.
struct SortLayout {
    size_t ctl, part_rank, ctl_end, tk0, tk1, vbuf;
    size_t bcount, lists, lrects, drects, seg_owner, tcount, ttotal;
    size_t work, order, end;
};

SortLayout sort_layout(int64_t m, int passes, int64_t T, int n, int H, int W) {
    SortLayout L;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t um = (size_t)(m > 0 ? m : 0);
    L.ctl = take(gsr::onesweep_state_bytes(um, passes));
    L.part_rank = take(4 * ((um + gsr::kSortPartition - 1) / gsr::kSortPartition + 1));
    L.ctl_end = off;
    const size_t pairs_end = off + 3 * align_up(4 * um, 256);
    L.tk0 = take(4 * um);
    L.tk1 = take(4 * um);
    L.vbuf = take(4 * um);
    // the block binning's arrays overlay the sort's
    off = L.ctl_end;
    const gsr::BlockGrid bg = gsr::block_grid(tiles_x_of(W), tiles_y_of(H));
    const uint64_t segs = gsr::segment_bound(um, bg);
    L.bcount = take(4 * (size_t)bg.nb * gsr::block_count_stride(n));
    L.lists = take(4 * um);
    L.lrects = take(2 * um);
    L.drects = take(8 * (size_t)(n > 0 ? n : 0));
    L.seg_owner = take(4 * (size_t)segs);
    L.tcount = take(4 * 64 * (size_t)segs);
    L.ttotal = take(4 * (size_t)(T > 0 ? T : 0));
    off = std::max(off, pairs_end);
    L.work = take(4 * (size_t)(T > 0 ? T : 0));
    L.order = take(4 * (size_t)(T > 0 ? T : 0));
    L.end = off;
    return L;
}

// Backward workspace: blend records, the tile schedule, the per-Gaussian tile
// rectangles, counts and gradient-slot offsets, then (cleared each call) the
// status block, the scan state and one flag byte per slot, then nine floats
// per slot.
struct BwdLayout {
    size_t recs, work, order, counts, rects, goff, ctl, misc, scanctl, flags, ctl_end, sums, end;
};

BwdLayout backward_layout(int n, int64_t m, int height, int width) {
    BwdLayout L;
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes, 256);
        return o;
    };
    const size_t un = (size_t)(n > 0 ? n : 0), um = (size_t)(m > 0 ? m : 0);
    const size_t T = (height > 0 && width > 0)
                         ? (size_t)tiles_x_of(width) * (size_t)tiles_y_of(height)
                         : 0;
    L.recs = take(kRecBytes * un);
    L.work = take(4 * T);
    L.order = take(4 * (T + 1));  // the tile order, then the backward's split count
    L.counts = take(4 * un);
    L.rects = take(8 * un);
    L.goff = take(4 * un);
    L.ctl = off;
    L.misc = take(sizeof(Misc));
    L.scanctl = take(gsr::records_slots_control_bytes(n));
    L.flags = take(align_up(um, 64) / 8);  // one bit per slot, read as 64-bit words
    L.ctl_end = off;
    L.sums = take(36 * um);
    L.end = off;
    return L;
}

template <typename T>
T* at(void* base, size_t off) {
    return reinterpret_cast<T*>(static_cast<char*>(base) + off);
}

// Pinned host slot for the one device-to-host read of the forward.
Misc* pinned_misc() {
    thread_local Misc* p = nullptr;
    if (!p) {
        void* h = nullptr;
        if (hipHostMalloc(&h, sizeof(Misc), hipHostMallocDefault) != hipSuccess) return nullptr;
        p = static_cast<Misc*>(h);
    }
    return p;
}

// The pair count as the kernel behind bin_count stores it: one host-mapped,
// coherent word per host thread, with its device address.
struct HostCount {
    volatile uint64_t* host = nullptr;
    uint64_t* dev = nullptr;
};
HostCount host_count() {
    thread_local HostCount c;
    if (!c.host) {
        void* h = nullptr;
        void* d = nullptr;
        if (hipHostMalloc(&h, 64, hipHostMallocMapped | hipHostMallocCoherent |
                                      hipHostMallocPortable) != hipSuccess)
            return HostCount{};
        if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess) {
            (void)hipHostFree(h);
            return HostCount{};
        }
        c.host = static_cast<volatile uint64_t*>(h);
        c.dev = static_cast<uint64_t*>(d);
    }
    return c;
}
// Stands in the host word until bin_count has stored the count.
constexpr uint64_t kNoCount = ~0ull;

// Marks bin_count's completion (one per host thread).  No system-scope fence:
// the count reaches the host through the kernel's own system-scope store to
// coherent host memory, so the event only has to say that the kernel is done.
hipEvent_t count_event() {
    thread_local hipEvent_t e = nullptr;
    if (!e && hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventDisableSystemFence) !=
                  hipSuccess)
        e = nullptr;
    return e;
}

// The quaternion gradient's mode, read on every call: 1 (GSR_REFERENCE_QUAT_GRAD
// set to 1) is the reference's literal formula, 0 the derivative of the forward.
int ref_quat_mode() {
    const char* v = std::getenv("GSR_REFERENCE_QUAT_GRAD");
    return (v && v[0] == '1' && v[1] == '\0') ? 1 : 0;
}

// ---- optional per-stage timing (gsr_profile_*): a pair of HIP events on the
// launch stream around each stage, collected after a synchronize ----
struct ProfState {
    std::mutex mu;
    bool on = false;
    std::vector<hipEvent_t> pool;
    struct Pending {
        const char* name;
        hipEvent_t a, b;
    };
    std::vector<Pending> pending;
    std::map<std::string, std::pair<int64_t, double>> acc;
};
ProfState& prof() {
    static ProfState* p = new ProfState();
    return *p;
}

class StageTimer {
  public:
    StageTimer(const char* name, hipStream_t st) : name_(name), st_(st) {
        ProfState& P = prof();
        std::lock_guard<std::mutex> lk(P.mu);
        if (!P.on) return;
        for (int i = 0; i < 2; ++i) {
            hipEvent_t e = nullptr;
            if (!P.pool.empty()) {
                e = P.pool.back();
                P.pool.pop_back();
            } else if (hipEventCreate(&e) != hipSuccess) {
                return;
            }
            (i == 0 ? a_ : b_) = e;
        }
        active_ = hipEventRecord(a_, st_) == hipSuccess;
    }
    ~StageTimer() {
        if (!active_) return;
        ProfState& P = prof();
        std::lock_guard<std::mutex> lk(P.mu);
        if (hipEventRecord(b_, st_) == hipSuccess) P.pending.push_back({name_, a_, b_});
    }

  private:
    const char* name_;
    hipStream_t st_;
    hipEvent_t a_ = nullptr, b_ = nullptr;
    bool active_ = false;
};

int packed_id_bits(int n, int64_t T) {
    int gb = 0;
    for (uint32_t v = (uint32_t)(n > 1 ? n - 1 : 1); v; v >>= 1) ++gb;
    return gb + tile_key_bits(T) <= 32 ? gb : 0;
}

int check_screen(int height, int width) {
    GSR_REQUIRE(height >= 0 && width >= 0, "height and width must be non-negative");
    GSR_REQUIRE(tiles_x_of(width) < 65536 && tiles_y_of(height) < 65536,
                "screen too large: at most 65535 tiles per axis");
    return GSR_OK;
}

}  // namespace

extern "C" {

const char* gsr_last_error(void) { return g_err.c_str(); }

const char* gsr_version(void) { return "gsraster 0.1 (gfx950)"; }

const char* gsr_build_sources(void) { return GSR_SOURCES; }

int gsr_project(int n, const float* mu, const float* q, const float* s, const float* rot,
                const float* trans, float fx, float fy, float cx, float cy, float* mean2d,
                float* cov2d, float* depth, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(mu && q && s && rot && trans && mean2d && cov2d && depth, "null pointer");
    GSR_REQUIRE(((uintptr_t)q & 15) == 0, "q must be 16-byte aligned");
    StageTimer timer("project", as_stream(stream));
    GSR_HIP(gsr::launch_project_fwd(n, mu, q, s, rot, trans, fx, fy, cx, cy, mean2d, cov2d, depth,
                                    as_stream(stream)),
            "project");
    return GSR_OK;
}

int gsr_screen_radii(int n, const float* cov2d, float* radii, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(cov2d && radii, "null pointer");
    GSR_HIP(gsr::launch_screen_radii(n, cov2d, radii, as_stream(stream)), "screen radii");
    return GSR_OK;
}

int gsr_camera_position(const float* rot, const float* trans, float* cam_pos, void* stream) {
    GSR_REQUIRE(rot && trans && cam_pos, "null pointer");
    GSR_HIP(gsr::launch_camera_position(rot, trans, cam_pos, as_stream(stream)),
            "camera position");
    return GSR_OK;
}

int gsr_sh(int n, const float* cam_pos, const float* mu, const float* albedo, const float* k_j,
           float* colors, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(cam_pos && mu && albedo && k_j && colors, "null pointer");
    GSR_REQUIRE(((uintptr_t)k_j & 15) == 0, "k_j must be 16-byte aligned");
    StageTimer timer("sh", as_stream(stream));
    GSR_HIP(gsr::launch_sh_fwd(n, cam_pos, mu, albedo, k_j, colors, as_stream(stream)), "SH");
    return GSR_OK;
}

int gsr_project_sh(int n, const float* mu, const float* q, const float* s, const float* rot,
                   const float* trans, float fx, float fy, float cx, float cy,
                   const float* albedo, const float* k_j, float* mean2d, float* cov2d,
                   float* depth, float* radii, float* colors, float* cam_pos,
                   const float* alpha_logits, float* opacity, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    GSR_REQUIRE(rot && trans && cam_pos, "null pointer");
    GSR_REQUIRE(!alpha_logits || opacity, "opacity must not be null when alpha_logits is given");
    if (n == 0) return gsr_camera_position(rot, trans, cam_pos, stream);
    GSR_REQUIRE(mu && q && s && albedo && k_j && mean2d && cov2d && depth && radii && colors,
                "null pointer");
    GSR_REQUIRE(((uintptr_t)q & 15) == 0, "q must be 16-byte aligned");
    GSR_REQUIRE(((uintptr_t)k_j & 15) == 0, "k_j must be 16-byte aligned");
    StageTimer timer("project_sh", as_stream(stream));
    GSR_HIP(gsr::launch_project_sh_fwd(n, mu, q, s, rot, trans, fx, fy, cx, cy, albedo, k_j,
                                       mean2d, cov2d, depth, radii, colors, cam_pos,
                                       alpha_logits, opacity, as_stream(stream)),
            "project_sh");
    return GSR_OK;
}

size_t gsr_bin_workspace_bytes(int n, int height, int width) {
    if (height < 0 || width < 0) return 0;
    return bin_layout(n, height, width).end;
}

}  // extern "C"

namespace {

// The bin step of gsr_rasterize_bin; with `order` (a depth order from
// gsr_depth_order) the depth keys and the depth sort are skipped and the
// order is copied in as the depth ranks' Gaussians.
int rasterize_bin(int n, const float* depth, const int32_t* order, const float* mean2d,
                  const float* cov2d, int height, int width, void* bin_ws, size_t bin_ws_bytes,
                  int64_t* num_pairs, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    GSR_REQUIRE(num_pairs, "num_pairs must not be null");
    if (int rc = check_screen(height, width)) return rc;
    *num_pairs = 0;
    const BinLayout L = bin_layout(n, height, width);
    GSR_REQUIRE(bin_ws, "bin workspace must not be null");
    if (bin_ws_bytes < L.end) return fail(GSR_ERR_WORKSPACE, "bin workspace too small");
    hipStream_t st = as_stream(stream);
    GSR_HIP(gsr::zero_fill(bin_ws, L.ctl_end, st), "rasterize: clear");
    if (n == 0 || height == 0 || width == 0) return GSR_OK;
    GSR_REQUIRE((depth || order) && mean2d && cov2d, "null pointer");
    gsr::DeviceGlobals dg;
    GSR_HIP(gsr::device_globals(&dg), "rasterize: device globals");
    Misc* misc = at<Misc>(bin_ws, L.misc);
    int* err = dg.status;
    uint32_t* counts = at<uint32_t>(bin_ws, L.counts);
    uint32_t* dk0 = at<uint32_t>(bin_ws, L.dk0);
    uint32_t* dv0 = at<uint32_t>(bin_ws, L.dv0);
    const bool blocks = block_binning(height, width);
    const HostCount hc = blocks ? host_count() : HostCount{};
    if (blocks && !hc.host) return fail(GSR_ERR_HIP, "rasterize: host-mapped count allocation failed");
    if (blocks) {
        hc.host[0] = kNoCount;
        hc.host[1] = 0;
    }
    // the binning's hand-off (the pair count to the host, the block starts)
    // runs in the depth sort's first pass when that pass can take it
    const bool finish_in_sort = blocks && !order && gsr::radix_sort_takes_finish((uint64_t)n);
    {
        StageTimer timer("bin_count", st);
        const int64_t T = (int64_t)tiles_x_of(width) * tiles_y_of(height);
        GSR_HIP(gsr::launch_bin_count(n, mean2d, cov2d, order ? nullptr : depth, height, width,
                                      counts, at<uint2>(bin_ws, L.rects),
                                      order ? nullptr : dk0, order ? nullptr : dv0,
                                      blocks ? 0 : tile_passes(T),
                                      at<uint32_t>(bin_ws, L.tilehist),
                                      at<uint32_t>(bin_ws, L.sortctl),
                                      blocks ? at<uint32_t>(bin_ws, L.blockhist) : nullptr,
                                      blocks ? &misc->total : nullptr,
                                      at<uint32_t>(bin_ws, L.block_start),
                                      at<uint32_t>(bin_ws, L.seg_start), hc.dev, dg.status,
                                      st, /*finish=*/!finish_in_sort),
                "rasterize: count");
    }
    Misc* host = pinned_misc();
    if (!host) return fail(GSR_ERR_HIP, "rasterize: pinned host buffer allocation failed");
    auto depth_sort = [&](const gsr::BinFinish* fin, hipEvent_t after_first) -> int {
        StageTimer timer("depth_sort", st);
        if (order) {
            GSR_HIP(hipMemcpyAsync(dv0, order, 4 * (size_t)n, hipMemcpyDeviceToDevice, st),
                    "rasterize: depth order");
            return GSR_OK;
        }
        GSR_HIP(gsr::launch_radix_sort(dk0, dv0, at<uint32_t>(bin_ws, L.dk1),
                                       at<uint32_t>(bin_ws, L.dv1), (uint64_t)n,
                                       at<void>(bin_ws, L.sortctl), err, st,
                                       /*hist_ready=*/true, fin, after_first),
                "rasterize: depth sort");
        return GSR_OK;
    };
    if (blocks) {
        // The pair count is final after bin_count; the hand-off (a work-group
        // of the depth sort's first pass, or a one-group kernel of its own)
        // stores it to host-mapped memory: queue the depth sort and wait only
        // for the hand-off, so the rest of the sort runs while the host
        // returns and queues the render.  The hand-off also passes on the
        // device status word: errors of every earlier kernel on the device
        // (an earlier frame's sorts, binning and backward) are reported here;
        // this frame's own, at the next forward or gsr_rasterize_status.
        hipEvent_t ev = count_event();
        if (!ev) return fail(GSR_ERR_HIP, "rasterize: event creation failed");
        if (finish_in_sort) {
            const gsr::BlockGrid bg = gsr::block_grid(tiles_x_of(width), tiles_y_of(height));
            const gsr::BinFinish fin{bg.nb, at<uint32_t>(bin_ws, L.blockhist), &misc->total,
                                     at<uint32_t>(bin_ws, L.block_start),
                                     at<uint32_t>(bin_ws, L.seg_start), hc.dev, dg.status};
            if (int rc = depth_sort(&fin, ev)) return rc;
        } else {
            GSR_HIP(hipEventRecord(ev, st), "rasterize: record");
            if (int rc = depth_sort(nullptr, nullptr)) return rc;
        }
        GSR_HIP(hipEventSynchronize(ev), "rasterize: synchronize");
        const uint64_t total = hc.host[0];
        if (total == kNoCount) return fail(GSR_ERR_DEVICE, "rasterize: pair count not stored");
        if (const int bits = (int)hc.host[1]) return fail(GSR_ERR_DEVICE, status_message(bits));
        if (total > (uint64_t)kMaxPairs)
            return fail(GSR_ERR_TOO_MANY_PAIRS,
                        "rasterize: " + std::to_string(total) +
                            " (Gaussian, tile) pairs exceed the int32 limit; render in screen "
                            "bands");
        *num_pairs = (int64_t)total;
        return GSR_OK;
    } else {
        if (int rc = depth_sort(nullptr, nullptr)) return rc;
        StageTimer timer("scan", st);
        GSR_HIP(gsr::launch_scan_counts(n, dv0, counts, at<uint32_t>(bin_ws, L.offsets),
                                        &misc->total, at<void>(bin_ws, L.scanctl), err, st),
                "rasterize: scan");
        GSR_HIP(hipMemcpyAsync(host, misc, sizeof(Misc), hipMemcpyDeviceToHost, st),
                "rasterize: read pair count");
        GSR_HIP(hipMemcpyAsync(&host->status, dg.status, sizeof(int), hipMemcpyDeviceToHost, st),
                "rasterize: read status");
        GSR_HIP(gsr::zero_fill(dg.status, sizeof(int), st), "rasterize: clear status");
        GSR_HIP(hipStreamSynchronize(st), "rasterize: synchronize");
    }
    if (host->status) return fail(GSR_ERR_DEVICE, status_message(host->status));
    if (host->total > (uint64_t)kMaxPairs)
        return fail(GSR_ERR_TOO_MANY_PAIRS,
                    "rasterize: " + std::to_string(host->total) +
                        " (Gaussian, tile) pairs exceed the int32 limit; render in screen bands");
    *num_pairs = (int64_t)host->total;
    return GSR_OK;
}

}  // namespace

extern "C" {

int gsr_rasterize_bin(int n, const float* depth, const float* mean2d, const float* cov2d,
                      int height, int width, void* bin_ws, size_t bin_ws_bytes,
                      int64_t* num_pairs, void* stream) {
    return rasterize_bin(n, depth, nullptr, mean2d, cov2d, height, width, bin_ws, bin_ws_bytes,
                         num_pairs, stream);
}

int gsr_rasterize_bin_ordered(int n, const int32_t* order, const float* mean2d,
                              const float* cov2d, int height, int width, void* bin_ws,
                              size_t bin_ws_bytes, int64_t* num_pairs, void* stream) {
    GSR_REQUIRE(n == 0 || order, "order must not be null");
    return rasterize_bin(n, nullptr, order, mean2d, cov2d, height, width, bin_ws, bin_ws_bytes,
                         num_pairs, stream);
}

size_t gsr_depth_order_workspace_bytes(int n) {
    if (n < 0) return 0;
    const size_t un = (size_t)n;
    return 3 * align_up(4 * un, 256) + gsr::sort_control_bytes(un);
}

int gsr_depth_order(int n, const float* depth, void* ws, size_t ws_bytes, int32_t* order,
                    void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(depth && order, "null pointer");
    GSR_REQUIRE(ws, "workspace must not be null");
    if (ws_bytes < gsr_depth_order_workspace_bytes(n))
        return fail(GSR_ERR_WORKSPACE, "depth order workspace too small");
    hipStream_t st = as_stream(stream);
    const size_t un = (size_t)n, w = align_up(4 * un, 256);
    uint32_t* k0 = at<uint32_t>(ws, 0);
    uint32_t* k1 = at<uint32_t>(ws, w);
    uint32_t* v1 = at<uint32_t>(ws, 2 * w);
    void* ctl = at<void>(ws, 3 * w);
    uint32_t* v0 = reinterpret_cast<uint32_t*>(order);  // the sort ends in (k0, v0)
    gsr::DeviceGlobals dg;
    GSR_HIP(gsr::device_globals(&dg), "depth order: device globals");
    GSR_HIP(gsr::zero_fill(ctl, gsr::sort_control_bytes(un), st), "depth order: clear");
    GSR_HIP(gsr::launch_depth_keys_hist((uint64_t)n, depth, k0, v0, ctl, st), "depth order: keys");
    GSR_HIP(gsr::launch_radix_sort(k0, v0, k1, v1, (uint64_t)n, ctl, dg.status, st,
                                   /*hist_ready=*/true),
            "depth order: sort");
    return GSR_OK;
}

size_t gsr_sort_workspace_bytes(int64_t num_pairs, int n, int height, int width) {
    if (height < 0 || width < 0 || n < 0) return 0;
    const int64_t T = (int64_t)tiles_x_of(width) * tiles_y_of(height);
    return sort_layout(num_pairs, tile_passes(T), T, n, height, width).end;
}

static int rasterize_render(int n, const float* depth, const float* mean2d, const float* cov2d,
                            const float* colors, const float* alpha, int height, int width,
                            void* bin_ws, size_t bin_ws_bytes, int64_t num_pairs, void* sort_ws,
                            size_t sort_ws_bytes, int32_t* sorted_ids, int32_t* tile_ranges,
                            float* img, float* final_T, int32_t* n_contrib,
                            uint64_t* sorted_keys, const uint8_t* tile_skip, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (int rc = check_screen(height, width)) return rc;
    GSR_REQUIRE(num_pairs >= 0 && num_pairs <= kMaxPairs, "num_pairs out of range");
    const int tiles_x = tiles_x_of(width);
    const int64_t T = (int64_t)tiles_x * tiles_y_of(height);
    if (T == 0) return GSR_OK;
    GSR_REQUIRE(tile_ranges && img && final_T && n_contrib, "null output pointer");
    const BinLayout BL = bin_layout(n, height, width);
    GSR_REQUIRE(bin_ws, "bin workspace must not be null");
    if (bin_ws_bytes < BL.end) return fail(GSR_ERR_WORKSPACE, "bin workspace too small");
    const int passes = tile_passes(T);
    const SortLayout SL = sort_layout(num_pairs, passes, T, n, height, width);
    hipStream_t st = as_stream(stream);
    const bool blocks = block_binning(height, width);
    // the block binning writes every tile range itself
    if (num_pairs == 0 || !blocks) {
        gsr::FillList clear;
        clear.add(tile_ranges, (size_t)T * 8);
        if (num_pairs > 0 && sort_ws && sort_ws_bytes >= SL.end) clear.add(sort_ws, SL.ctl_end);
        GSR_HIP(gsr::zero_fill(clear, st), "rasterize: clear");
    }
    const uint64_t m = (uint64_t)num_pairs;
    void* recs = at<void>(bin_ws, BL.recs);
    if (m > 0) {
        GSR_REQUIRE(sort_ws && sorted_ids, "null pointer");
        if (sort_ws_bytes < SL.end) return fail(GSR_ERR_WORKSPACE, "sort workspace too small");
        GSR_REQUIRE(mean2d && cov2d && colors && alpha && depth, "null pointer");
        // the block binning's first kernel forms the records in its own launch
        if (!blocks) {
            StageTimer timer("records", st);
            GSR_HIP(gsr::launch_blend_records(n, mean2d, cov2d, colors, alpha, recs, st),
                    "rasterize: records");
        }
        uint32_t* ids = reinterpret_cast<uint32_t*>(sorted_ids);
        gsr::DeviceGlobals dg;
        GSR_HIP(gsr::device_globals(&dg), "rasterize: device globals");
        if (blocks) {
            {
                StageTimer timer("tile_binning", st);
                gsr::TileBinning tb;
                tb.n = n;
                tb.m = m;
                tb.grid = gsr::block_grid(tiles_x, tiles_y_of(height));
                tb.perm = at<uint32_t>(bin_ws, BL.dv0);
                tb.rects = at<uint2>(bin_ws, BL.rects);
                tb.block_hist = at<uint32_t>(bin_ws, BL.blockhist);
                tb.block_start = at<uint32_t>(bin_ws, BL.block_start);
                tb.seg_start = at<uint32_t>(bin_ws, BL.seg_start);
                tb.bcount = at<uint32_t>(sort_ws, SL.bcount);
                tb.lists = at<uint32_t>(sort_ws, SL.lists);
                tb.lrects = at<uint16_t>(sort_ws, SL.lrects);
                // gathering the rectangles into depth order pays once the
                // level-1 passes' lookups by id are bandwidth-bound
                if (n >= (1 << 19)) tb.drects = at<uint2>(sort_ws, SL.drects);
                tb.seg_owner = at<uint32_t>(sort_ws, SL.seg_owner);
                tb.tcount = at<uint32_t>(sort_ws, SL.tcount);
                tb.ttotal = at<uint32_t>(sort_ws, SL.ttotal);
                tb.ranges = tile_ranges;
                tb.ids = ids;
                tb.err = dg.status;
                tb.skip = reinterpret_cast<const uint8_t*>(tile_skip);
                tb.rec_mean2d = mean2d;
                tb.rec_cov2d = cov2d;
                tb.rec_colors = colors;
                tb.rec_alpha = alpha;
                tb.recs = recs;
                GSR_HIP(gsr::launch_tile_binning(tb, st), "rasterize: tile binning");
            }
            if (sorted_keys)
                GSR_HIP(gsr::launch_range_keys((int)T, tile_ranges, sorted_ids, depth, n, m,
                                               sorted_keys, st),
                        "rasterize: keys");
        } else {
            uint32_t* tk0 = at<uint32_t>(sort_ws, SL.tk0);
            uint32_t* tk1 = at<uint32_t>(sort_ws, SL.tk1);
            uint32_t* ktiles = ((passes - 1) % 2 == 0) ? tk0 : tk1;  // the last pass's keys
            // one packed word per pair when tile and Gaussian id fit in 32 bits
            const int gbits = packed_id_bits(n, T);
            {
                StageTimer timer("tile_sort", st);
                uint32_t* part_rank = at<uint32_t>(sort_ws, SL.part_rank);
                gsr::EmitSource es;
                es.perm = at<uint32_t>(bin_ws, BL.dv0);
                es.counts = at<uint32_t>(bin_ws, BL.counts);
                es.rects = at<uint2>(bin_ws, BL.rects);
                es.offsets = at<uint32_t>(bin_ws, BL.offsets);
                es.part_rank = part_rank;
                es.nparts = (uint32_t)((m + gsr::kSortPartition - 1) / gsr::kSortPartition);
                es.tiles_x = tiles_x;
                GSR_HIP(gsr::launch_partition_starts(n, es.perm, es.counts, es.offsets, m,
                                                     part_rank, st),
                        "rasterize: partition starts");
                GSR_HIP(gsr::launch_tile_sort(es, m, passes, tile_key_bits(T), gbits,
                                              at<uint32_t>(bin_ws, BL.tilehist),
                                              at<void>(sort_ws, SL.ctl), tk0, tk1,
                                              at<uint32_t>(sort_ws, SL.vbuf), ids, ktiles,
                                              dg.status, st),
                        "rasterize: tile sort");
            }
            {
                StageTimer timer("ranges", st);
                GSR_HIP(gsr::launch_tile_ranges(m, (uint32_t)T, ktiles, gbits, tile_ranges, st),
                        "rasterize: ranges");
            }
            if (sorted_keys)
                GSR_HIP(gsr::launch_full_keys(m, ktiles, gbits, sorted_ids, depth, n,
                                              sorted_keys, st),
                        "rasterize: keys");
        }
    }
    uint32_t* order = m > 0 ? at<uint32_t>(sort_ws, SL.order) : nullptr;
    if (order) {
        StageTimer timer("fwd_schedule", st);
        GSR_HIP(gsr::launch_fwd_schedule(n, height, width, tile_ranges, sorted_ids, m, recs,
                                         at<uint32_t>(sort_ws, SL.work), order, st),
                "rasterize: schedule");
    }
    StageTimer timer("blend_fwd", st);
    GSR_HIP(gsr::launch_blend_fwd(n, height, width, tile_ranges, sorted_ids, m, recs, img, final_T,
                                  n_contrib, order, st),
            "rasterize: blend");
    return GSR_OK;
}

int gsr_rasterize_render(int n, const float* depth, const float* mean2d, const float* cov2d,
                         const float* colors, const float* alpha, int height, int width,
                         void* bin_ws, size_t bin_ws_bytes, int64_t num_pairs, void* sort_ws,
                         size_t sort_ws_bytes, int32_t* sorted_ids, int32_t* tile_ranges,
                         float* img, float* final_T, int32_t* n_contrib, uint64_t* sorted_keys,
                         void* stream) {
    return rasterize_render(n, depth, mean2d, cov2d, colors, alpha, height, width, bin_ws,
                            bin_ws_bytes, num_pairs, sort_ws, sort_ws_bytes, sorted_ids,
                            tile_ranges, img, final_T, n_contrib, sorted_keys, nullptr, stream);
}

int gsr_rasterize_render_skip(int n, const float* depth, const float* mean2d, const float* cov2d,
                              const float* colors, const float* alpha, int height, int width,
                              void* bin_ws, size_t bin_ws_bytes, int64_t num_pairs,
                              void* sort_ws, size_t sort_ws_bytes, const uint8_t* tile_skip,
                              int32_t* sorted_ids, int32_t* tile_ranges, float* img,
                              float* final_T, int32_t* n_contrib, void* stream) {
    GSR_REQUIRE(tile_skip, "tile_skip must not be null");
    return rasterize_render(n, depth, mean2d, cov2d, colors, alpha, height, width, bin_ws,
                            bin_ws_bytes, num_pairs, sort_ws, sort_ws_bytes, sorted_ids,
                            tile_ranges, img, final_T, n_contrib, nullptr, tile_skip, stream);
}

int gsr_tile_row_pairs(int n, const float* mean2d, const float* cov2d, int height, int width,
                       uint64_t* rows, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (int rc = check_screen(height, width)) return rc;
    GSR_REQUIRE(tiles_y_of(height) <= 4096, "height must be at most 65536");
    GSR_REQUIRE(rows != nullptr, "rows is null");
    GSR_REQUIRE(n == 0 || (mean2d && cov2d), "null pointer");
    GSR_HIP(gsr::launch_row_pairs(n, mean2d, cov2d, height, width, rows, as_stream(stream)),
            "tile row pairs");
    return GSR_OK;
}

int gsr_tiles_touch(int n, const float* mean2d, const float* cov2d, int height, int width,
                    const int32_t* sat, uint8_t* flags, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (int rc = check_screen(height, width)) return rc;
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(mean2d && cov2d && sat && flags, "null pointer");
    GSR_HIP(gsr::launch_tiles_touch(n, mean2d, cov2d, height, width, sat, flags,
                                    as_stream(stream)),
            "tiles touch");
    return GSR_OK;
}

int gsr_rasterize_status(void* bin_ws, size_t bin_ws_bytes, void* stream) {
    (void)bin_ws;
    (void)bin_ws_bytes;
    hipStream_t st = as_stream(stream);
    gsr::DeviceGlobals dg;
    GSR_HIP(gsr::device_globals(&dg), "status: device globals");
    Misc* host = pinned_misc();
    if (!host) return fail(GSR_ERR_HIP, "pinned host buffer allocation failed");
    GSR_HIP(hipMemcpyAsync(&host->status, dg.status, sizeof(int), hipMemcpyDeviceToHost, st),
            "status: read");
    GSR_HIP(gsr::zero_fill(dg.status, sizeof(int), st), "status: clear");
    GSR_HIP(hipStreamSynchronize(st), "status: synchronize");
    if (host->status) return fail(GSR_ERR_DEVICE, status_message(host->status));
    return GSR_OK;
}

int gsr_debug_raise_status(int bits, void* stream) {
    GSR_REQUIRE(bits > 0, "bits must be positive");
    gsr::DeviceGlobals dg;
    GSR_HIP(gsr::device_globals(&dg), "raise status: device globals");
    GSR_HIP(gsr::launch_raise_status(dg.status, bits, as_stream(stream)), "raise status");
    return GSR_OK;
}

size_t gsr_calibrate_valu_out_floats(void) {
    return (size_t)gsr::calibrate_valu_blocks() * 256;
}

int gsr_calibrate_valu(int kind, int iters, float* out, void* stream) {
    GSR_REQUIRE(kind >= 0 && kind <= 4, "kind must be 0..4");
    GSR_REQUIRE(iters >= 1 && iters <= 65536, "iters must be 1..65536");
    GSR_REQUIRE(out != nullptr, "out is null");
    GSR_HIP(gsr::launch_calibrate_valu(kind, iters, out, as_stream(stream)), "calibrate valu");
    return GSR_OK;
}

size_t gsr_backward_workspace_bytes(int n, int64_t num_pairs, int height, int width) {
    return backward_layout(n, num_pairs, height, width).end;
}

}  // extern "C"

namespace {

int rasterize_backward(int n, int height, int width, const float* grad_img,
                       const gsr::GradStrides& gst, const float* mean2d, const float* cov2d,
                       const float* colors, const float* alpha, const int32_t* sorted_ids,
                       int64_t num_pairs, const int32_t* tile_ranges, const float* final_T,
                       const int32_t* n_contrib, void* ws, size_t ws_bytes, float* d_mean2d,
                       float* d_cov2d, float* d_colors, float* d_alpha, void* stream,
                       bool accumulate = false) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (int rc = check_screen(height, width)) return rc;
    GSR_REQUIRE(num_pairs >= 0 && num_pairs <= kMaxPairs, "num_pairs out of range");
    hipStream_t st = as_stream(stream);
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(mean2d && cov2d && colors && alpha && d_mean2d && d_cov2d && d_colors && d_alpha,
                "null pointer");
    const BwdLayout L = backward_layout(n, num_pairs, height, width);
    if (ws_bytes < L.end || !ws) return fail(GSR_ERR_WORKSPACE, "backward workspace too small");
    const int64_t T = (int64_t)tiles_x_of(width) * tiles_y_of(height);
    const bool work = T > 0 && num_pairs > 0;
    if (work)
        GSR_REQUIRE(grad_img && sorted_ids && tile_ranges && final_T && n_contrib, "null pointer");
    gsr::FillList clear;
    if (!accumulate) {
        clear.add(d_mean2d, 8 * (size_t)n);
        clear.add(d_cov2d, 12 * (size_t)n);
        clear.add(d_colors, 12 * (size_t)n);
        clear.add(d_alpha, 4 * (size_t)n);
    }
    if (work) clear.add(at<void>(ws, L.ctl), L.ctl_end - L.ctl);
    GSR_HIP(gsr::zero_fill(clear, st), "backward: clear");
    if (!work) return GSR_OK;
    gsr::DeviceGlobals dg;
    GSR_HIP(gsr::device_globals(&dg), "backward: device globals");
    Misc* misc = at<Misc>(ws, L.misc);
    uint32_t* counts = at<uint32_t>(ws, L.counts);
    uint2* rects = at<uint2>(ws, L.rects);
    uint32_t* goff = at<uint32_t>(ws, L.goff);
    // the records kernel also computes the schedule's per-tile work when it can
    // (independent work in one launch)
    bool work_ready = false;
    {
        StageTimer timer("bwd_records", st);
        GSR_HIP(gsr::launch_records_slots(n, mean2d, cov2d, colors, alpha, at<void>(ws, L.recs),
                                          height, width, counts, rects, goff, &misc->total,
                                          at<void>(ws, L.scanctl), dg.status, st, tile_ranges,
                                          (uint64_t)num_pairs, n_contrib, at<uint32_t>(ws, L.work),
                                          &work_ready),
                "backward: records and slot layout");
    }
    gsr::GradSlots gs;
    gs.goff = goff;
    gs.counts = counts;
    gs.rects = rects;
    gs.sums = at<float>(ws, L.sums);
    gs.flags = at<uint32_t>(ws, L.flags);
    gs.slots = (uint64_t)num_pairs;
    uint32_t* order = at<uint32_t>(ws, L.order);
    {
        StageTimer timer("bwd_schedule", st);
        GSR_HIP(gsr::launch_bwd_schedule(height, width, tile_ranges, (uint64_t)num_pairs, n_contrib,
                                         at<uint32_t>(ws, L.work), order, st, work_ready),
                "backward: schedule");
    }
    {
        StageTimer timer("blend_bwd", st);
        GSR_HIP(gsr::launch_blend_bwd(n, height, width, grad_img, gst, tile_ranges, sorted_ids,
                                      (uint64_t)num_pairs, at<void>(ws, L.recs), final_T,
                                      n_contrib, d_mean2d, d_cov2d, d_colors, d_alpha, gs, order,
                                      st),
                "backward: blend");
    }
    StageTimer timer("grad_reduce", st);
    GSR_HIP(gsr::launch_pair_grad_reduce(n, gs, d_mean2d, d_cov2d, d_colors, d_alpha, st),
            "backward: gradient sums");
    return GSR_OK;
}

}  // namespace

extern "C" {

int gsr_rasterize_backward(int n, int height, int width, const float* grad_img,
                           const float* mean2d, const float* cov2d, const float* colors,
                           const float* alpha, const int32_t* sorted_ids, int64_t num_pairs,
                           const int32_t* tile_ranges, const float* final_T,
                           const int32_t* n_contrib, void* ws, size_t ws_bytes, float* d_mean2d,
                           float* d_cov2d, float* d_colors, float* d_alpha, void* stream) {
    gsr::GradStrides gst;
    gst.h = 3 * (int64_t)width;
    gst.w = 3;
    gst.c = 1;
    return rasterize_backward(n, height, width, grad_img, gst, mean2d, cov2d, colors, alpha,
                              sorted_ids, num_pairs, tile_ranges, final_T, n_contrib, ws,
                              ws_bytes, d_mean2d, d_cov2d, d_colors, d_alpha, stream);
}

int gsr_rasterize_backward_strided(int n, int height, int width, const float* grad_img,
                                   int64_t grad_stride_h, int64_t grad_stride_w,
                                   int64_t grad_stride_c, const float* mean2d,
                                   const float* cov2d, const float* colors, const float* alpha,
                                   const int32_t* sorted_ids, int64_t num_pairs,
                                   const int32_t* tile_ranges, const float* final_T,
                                   const int32_t* n_contrib, void* ws, size_t ws_bytes,
                                   float* d_mean2d, float* d_cov2d, float* d_colors,
                                   float* d_alpha, void* stream) {
    gsr::GradStrides gst;
    gst.h = grad_stride_h;
    gst.w = grad_stride_w;
    gst.c = grad_stride_c;
    return rasterize_backward(n, height, width, grad_img, gst, mean2d, cov2d, colors, alpha,
                              sorted_ids, num_pairs, tile_ranges, final_T, n_contrib, ws,
                              ws_bytes, d_mean2d, d_cov2d, d_colors, d_alpha, stream);
}

int gsr_rasterize_backward_accumulate(int n, int height, int width, const float* grad_img,
                                      int64_t grad_stride_h, int64_t grad_stride_w,
                                      int64_t grad_stride_c, const float* mean2d,
                                      const float* cov2d, const float* colors,
                                      const float* alpha, const int32_t* sorted_ids,
                                      int64_t num_pairs, const int32_t* tile_ranges,
                                      const float* final_T, const int32_t* n_contrib, void* ws,
                                      size_t ws_bytes, float* d_mean2d, float* d_cov2d,
                                      float* d_colors, float* d_alpha, void* stream) {
    gsr::GradStrides gst;
    gst.h = grad_stride_h;
    gst.w = grad_stride_w;
    gst.c = grad_stride_c;
    return rasterize_backward(n, height, width, grad_img, gst, mean2d, cov2d, colors, alpha,
                              sorted_ids, num_pairs, tile_ranges, final_T, n_contrib, ws,
                              ws_bytes, d_mean2d, d_cov2d, d_colors, d_alpha, stream,
                              /*accumulate=*/true);
}

int gsr_rasterize_backward_noalloc(int n, int height, int width, const float* grad_img,
                                   const float* mean2d, const float* cov2d, const float* colors,
                                   const float* alpha, const int32_t* sorted_ids,
                                   int64_t num_pairs, const int32_t* tile_ranges,
                                   const float* final_T, const int32_t* n_contrib,
                                   float* d_mean2d, float* d_cov2d, float* d_colors,
                                   float* d_alpha, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (int rc = check_screen(height, width)) return rc;
    GSR_REQUIRE(num_pairs >= 0 && num_pairs <= kMaxPairs, "num_pairs out of range");
    const size_t need = backward_layout(n, num_pairs, height, width).end;
    static_assert(gsr::kNoAllocScratchBytes == (size_t)GSR_NOALLOC_SCRATCH_BYTES,
                  "the header's scratch size is the array's");
    if (need > gsr::kNoAllocScratchBytes)
        return fail(GSR_ERR_WORKSPACE,
                    "backward (no allocation): the frame needs " + std::to_string(need) +
                        " bytes of workspace (about 36 per pair and 68 per Gaussian), more than "
                        "the fixed scratch's " +
                        std::to_string(gsr::kNoAllocScratchBytes) +
                        "; use gsr_rasterize_backward with a workspace");
    gsr::DeviceGlobals dg;
    GSR_HIP(gsr::device_globals(&dg), "backward (no allocation): device globals");
    gsr::GradStrides gst;
    gst.h = 3 * (int64_t)width;
    gst.w = 3;
    gst.c = 1;
    return rasterize_backward(n, height, width, grad_img, gst, mean2d, cov2d, colors, alpha,
                              sorted_ids, num_pairs, tile_ranges, final_T, n_contrib, dg.scratch,
                              gsr::kNoAllocScratchBytes, d_mean2d, d_cov2d, d_colors, d_alpha,
                              stream);
}

int gsr_sh_backward(int n, const float* colors_grad, const float* mu, const float* albedo,
                    const float* k_j, const float* cam_pos, float* d_albedo, float* d_k_j,
                    float* d_mu, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(colors_grad && mu && albedo && k_j && cam_pos && d_albedo && d_k_j && d_mu,
                "null pointer");
    GSR_REQUIRE(((uintptr_t)k_j & 15) == 0 && ((uintptr_t)d_k_j & 15) == 0,
                "k_j and d_k_j must be 16-byte aligned");
    StageTimer timer("sh_bwd", as_stream(stream));
    GSR_HIP(gsr::launch_sh_bwd(n, colors_grad, mu, albedo, k_j, cam_pos, d_albedo, d_k_j, d_mu,
                               as_stream(stream)),
            "backwards_SH");
    return GSR_OK;
}

int gsr_project_sh_backward(int n, const float* d_mean2d, const float* d_cov2d,
                            const float* d_colors, const float* mu, const float* q,
                            const float* s, const float* rot, const float* trans, float fx,
                            float fy, const float* albedo, const float* k_j,
                            const float* cam_pos, float* d_mu, float* d_q, float* d_s,
                            float* d_albedo, float* d_k_j, const float* d_opacity,
                            const float* opacity, float* d_alpha_logits, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    GSR_REQUIRE(!d_opacity || (opacity && d_alpha_logits),
                "opacity and d_alpha_logits must not be null when d_opacity is given");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(d_mean2d && d_cov2d && d_colors && mu && q && s && rot && trans && albedo && k_j &&
                    cam_pos && d_mu && d_q && d_s && d_albedo && d_k_j,
                "null pointer");
    GSR_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)d_q & 15) == 0,
                "q and d_q must be 16-byte aligned");
    GSR_REQUIRE(((uintptr_t)k_j & 15) == 0 && ((uintptr_t)d_k_j & 15) == 0,
                "k_j and d_k_j must be 16-byte aligned");
    StageTimer timer("project_sh_bwd", as_stream(stream));
    GSR_HIP(gsr::launch_project_sh_bwd(n, d_mean2d, d_cov2d, d_colors, mu, q, s, rot, trans, fx,
                                       fy, albedo, k_j, cam_pos, d_mu, d_q, d_s, d_albedo, d_k_j,
                                       ref_quat_mode(), d_opacity, opacity, d_alpha_logits,
                                       as_stream(stream)),
            "project_sh_backward");
    return GSR_OK;
}

int gsr_project_backward(int n, const float* d_mean2d, const float* d_cov2d, const float* mu,
                         const float* q, const float* s, const float* rot, const float* trans,
                         float fx, float fy, float cx, float cy, float* d_mu, float* d_q,
                         float* d_s, void* stream) {
    (void)cx;
    (void)cy;
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(d_mean2d && d_cov2d && mu && q && s && rot && trans && d_mu && d_q && d_s,
                "null pointer");
    GSR_REQUIRE(((uintptr_t)q & 15) == 0 && ((uintptr_t)d_q & 15) == 0,
                "q and d_q must be 16-byte aligned");
    StageTimer timer("project_bwd", as_stream(stream));
    GSR_HIP(gsr::launch_project_bwd(n, d_mean2d, d_cov2d, mu, q, s, rot, trans, fx, fy, d_mu, d_q,
                                    d_s, ref_quat_mode(), as_stream(stream)),
            "backwards_projection");
    return GSR_OK;
}

size_t gsr_loss_workspace_bytes(int height, int width) {
    if (height < 11 || width < 11) return 0;
    const size_t parts = align_up(8 * gsr::loss_partial_count(height, width), 256);
    return parts + 3 * 12 * (size_t)height * (size_t)width;
}

namespace {
int check_loss_args(int height, int width, const void* a, const void* b, const void* ws,
                    size_t ws_bytes) {
    GSR_REQUIRE(height >= 11 && width >= 11,
                "the SSIM needs images of at least 11 x 11 pixels (its window)");
    GSR_REQUIRE((int64_t)height * width <= ((int64_t)1 << 31) / 3, "image too large");
    GSR_REQUIRE(a && b, "null pointer");
    if (!ws || ws_bytes < gsr_loss_workspace_bytes(height, width))
        return fail(GSR_ERR_WORKSPACE, "loss workspace too small");
    return GSR_OK;
}
}  // namespace

int gsr_l1_dssim(int height, int width, const float* rendered, const float* gt,
                 float lambda_dssim, void* ws, size_t ws_bytes, float* out, void* stream) {
    if (int rc = check_loss_args(height, width, rendered, gt, ws, ws_bytes)) return rc;
    GSR_REQUIRE(out, "null pointer");
    const size_t parts = align_up(8 * gsr::loss_partial_count(height, width), 256);
    StageTimer timer("loss", as_stream(stream));
    GSR_HIP(gsr::launch_l1_dssim_fwd(height, width, rendered, gt, lambda_dssim,
                                     at<float>(ws, parts), ws, out, as_stream(stream)),
            "l1_dssim");
    return GSR_OK;
}

int gsr_l1_dssim_backward(int height, int width, const float* rendered, const float* gt,
                          float lambda_dssim, const void* ws, size_t ws_bytes,
                          const float* grad_loss, float* d_rendered, void* stream) {
    if (int rc = check_loss_args(height, width, rendered, gt, ws, ws_bytes)) return rc;
    GSR_REQUIRE(d_rendered, "null pointer");
    const size_t parts = align_up(8 * gsr::loss_partial_count(height, width), 256);
    StageTimer timer("loss_bwd", as_stream(stream));
    GSR_HIP(gsr::launch_l1_dssim_bwd(height, width, rendered, gt, lambda_dssim,
                                     at<float>(const_cast<void*>(ws), parts), grad_loss,
                                     d_rendered, as_stream(stream)),
            "l1_dssim_backward");
    return GSR_OK;
}

int gsr_ssim(int height, int width, const float* a, const float* b, void* ws, size_t ws_bytes,
             float* out, void* stream) {
    if (int rc = check_loss_args(height, width, a, b, ws, ws_bytes)) return rc;
    GSR_REQUIRE(out, "null pointer");
    GSR_HIP(gsr::launch_l1_dssim_fwd(height, width, a, b, 1.0f, nullptr, ws, out,
                                     as_stream(stream)),
            "ssim");
    return GSR_OK;
}

int gsr_adam_step(int count, const gsr_adam_tensor* tensors, double beta1, double beta2,
                  double eps, void* stream) {
    GSR_REQUIRE(count >= 0, "count must be non-negative");
    if (count == 0) return GSR_OK;
    GSR_REQUIRE(tensors, "null pointer");
    GSR_REQUIRE(beta1 >= 0.0 && beta1 < 1.0 && beta2 >= 0.0 && beta2 < 1.0,
                "betas must lie in [0, 1)");
    std::vector<gsr::AdamTensor> t((size_t)count);
    std::vector<gsr::AdamHostScalars> h((size_t)count);
    for (int i = 0; i < count; ++i) {
        const gsr_adam_tensor& a = tensors[i];
        GSR_REQUIRE(a.numel >= 0, "numel must be non-negative");
        GSR_REQUIRE(a.numel == 0 || (a.param && a.grad && a.exp_avg && a.exp_avg_sq),
                    "null pointer");
        GSR_REQUIRE(a.step >= 1, "step must be at least 1");
        t[(size_t)i] = gsr::AdamTensor{a.param, a.grad, a.exp_avg, a.exp_avg_sq,
                                       (uint64_t)a.numel};
        // torch forms these in Python floats (double) and rounds each to fp32
        const double bc1 = 1.0 - std::pow(beta1, (double)a.step);
        const double bc2 = 1.0 - std::pow(beta2, (double)a.step);
        h[(size_t)i] = gsr::AdamHostScalars{(float)(1.0 - beta1),     (float)beta2,
                                            (float)(1.0 - beta2),     (float)std::sqrt(bc2),
                                            (float)(-(a.lr / bc1)),   (float)eps,
                                            a.clamp_min,              a.clamp_max};
    }
    StageTimer timer("adam", as_stream(stream));
    GSR_HIP(gsr::launch_adam(count, t.data(), h.data(), as_stream(stream)), "adam_step");
    return GSR_OK;
}

int gsr_ply_pack(int n, int rest_coeffs, const float* mu, const float* q, const float* s,
                 const float* alpha, const float* albedo, const float* k_j,
                 int opacity_from_probability, float* records, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    GSR_REQUIRE(rest_coeffs >= 1 && rest_coeffs <= 63, "rest_coeffs must lie in [1, 63]");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(mu && q && s && alpha && albedo && k_j && records, "null pointer");
    GSR_REQUIRE(((uintptr_t)q & 15) == 0, "q must be 16-byte aligned");
    StageTimer timer("ply_pack", as_stream(stream));
    GSR_HIP(gsr::launch_ply_pack(n, rest_coeffs, mu, q, s, alpha, albedo, k_j,
                                 opacity_from_probability ? 1 : 0, records, as_stream(stream)),
            "ply_pack");
    return GSR_OK;
}

int gsr_adc_stats(int n, const float* mean2d_grad, int width, int height, const float* radii,
                  float* grad_accum, float* denom, float* max_radii2d, void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(!mean2d_grad || (grad_accum && denom), "null pointer");
    GSR_REQUIRE(!radii || max_radii2d, "null pointer");
    const bool scale = width > 0 && height > 0;
    StageTimer timer("adc_stats", as_stream(stream));
    // (width / 2.0, height / 2.0) as an fp32 tensor (adc.py:70-71)
    GSR_HIP(gsr::launch_adc_stats(n, mean2d_grad, (float)(width / 2.0), (float)(height / 2.0),
                                  scale ? 1 : 0, radii, grad_accum, denom, max_radii2d,
                                  as_stream(stream)),
            "adc_stats");
    return GSR_OK;
}

size_t gsr_adc_workspace_bytes(int n) { return gsr::adc_workspace_bytes(n > 0 ? n : 0); }

namespace {
gsr::AdcConfig adc_config(const gsr_adc_config& c) {
    gsr::AdcConfig a;
    a.grad_threshold = (float)c.grad_threshold;
    a.dense_scale = (float)(c.percent_dense * c.scene_extent);
    a.max_scale = (float)(0.1 * c.scene_extent);
    a.min_opacity = (float)c.min_opacity;
    a.max_screen = (float)c.max_screen_size;
    a.split_scale = (float)1.6;                          // adc.py:217 scale_factor
    a.reset_logit = (float)std::log(0.01 / (1.0 - 0.01));  // adc.py:297-298
    a.densify = c.densify ? 1 : 0;
    a.prune = c.prune ? 1 : 0;
    a.has_screen = c.has_max_screen_size ? 1 : 0;
    a.reset_opacity = c.reset_opacity ? 1 : 0;
    return a;
}
}  // namespace

int gsr_adc_plan(int n, float* const params[6], const float* grad_accum, const float* denom,
                 const float* max_radii2d, const gsr_adc_config* cfg, void* ws, size_t ws_bytes,
                 int64_t counts[5], void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    GSR_REQUIRE(cfg && counts, "null pointer");
    for (int k = 0; k < 5; ++k) counts[k] = 0;
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(params && grad_accum && denom, "null pointer");
    for (int a = 0; a < 6; ++a) GSR_REQUIRE(params[a], "null parameter array");
    if (!ws || ws_bytes < gsr::adc_workspace_bytes(n))
        return fail(GSR_ERR_WORKSPACE, "adc workspace too small");
    gsr::AdcCloud in;
    for (int a = 0; a < 6; ++a) in.p[a] = params[a];
    hipStream_t st = as_stream(stream);
    uint64_t* totals = static_cast<uint64_t*>(ws);
    {
        StageTimer timer("adc_plan", st);
        GSR_HIP(gsr::launch_adc_plan(n, in, grad_accum, denom, max_radii2d, adc_config(*cfg), ws,
                                     totals, st),
                "adc_plan");
    }
    uint64_t host[5];
    GSR_HIP(hipMemcpyAsync(host, totals, sizeof(host), hipMemcpyDeviceToHost, st), "adc_plan: read");
    GSR_HIP(hipStreamSynchronize(st), "adc_plan: synchronize");
    for (int k = 0; k < 5; ++k) counts[k] = (int64_t)host[k];
    return GSR_OK;
}

int gsr_adc_apply(int n, float* const params[6], float* const moments[12],
                  const float* split_noise, const gsr_adc_config* cfg, const void* ws,
                  size_t ws_bytes, float* const out_params[6], float* const out_moments[12],
                  void* stream) {
    GSR_REQUIRE(n >= 0, "n must be non-negative");
    if (n == 0) return GSR_OK;
    GSR_REQUIRE(params && out_params && cfg, "null pointer");
    GSR_REQUIRE(split_noise || !cfg->densify,
                "split_noise must not be null when densifying (2 counts[3] rows of 3 floats)");
    for (int a = 0; a < 6; ++a) GSR_REQUIRE(params[a] && out_params[a], "null parameter array");
    if (!ws || ws_bytes < gsr::adc_workspace_bytes(n))
        return fail(GSR_ERR_WORKSPACE, "adc workspace too small");
    gsr::AdcCloud in, out;
    gsr::AdcMoments min_{}, mout{};
    for (int a = 0; a < 6; ++a) {
        in.p[a] = params[a];
        out.p[a] = out_params[a];
    }
    for (int a = 0; a < 12; ++a) {
        min_.p[a] = moments ? moments[a] : nullptr;
        mout.p[a] = out_moments ? out_moments[a] : nullptr;
    }
    StageTimer timer("adc_apply", as_stream(stream));
    GSR_HIP(gsr::launch_adc_gather(n, in, min_, split_noise, adc_config(*cfg), ws,
                                   static_cast<const uint64_t*>(ws), out, mout,
                                   as_stream(stream)),
            "adc_apply");
    return GSR_OK;
}

void gsr_profile_enable(int on) {
    ProfState& P = prof();
    std::lock_guard<std::mutex> lk(P.mu);
    P.on = on != 0;
}

int gsr_profile_collect(void) {
    ProfState& P = prof();
    std::lock_guard<std::mutex> lk(P.mu);
    for (auto& e : P.pending) {
        GSR_HIP(hipEventSynchronize(e.b), "profile: synchronize");
        float ms = 0.0f;
        GSR_HIP(hipEventElapsedTime(&ms, e.a, e.b), "profile: elapsed");
        auto& slot = P.acc[e.name];
        slot.first += 1;
        slot.second += ms;
        P.pool.push_back(e.a);
        P.pool.push_back(e.b);
    }
    P.pending.clear();
    return GSR_OK;
}

int gsr_profile_get(const char* stage, int64_t* count, double* total_ms) {
    GSR_REQUIRE(stage && count && total_ms, "null pointer");
    ProfState& P = prof();
    std::lock_guard<std::mutex> lk(P.mu);
    auto it = P.acc.find(stage);
    *count = it == P.acc.end() ? 0 : it->second.first;
    *total_ms = it == P.acc.end() ? 0.0 : it->second.second;
    return GSR_OK;
}

const char* gsr_profile_stage(int index) {
    ProfState& P = prof();
    std::lock_guard<std::mutex> lk(P.mu);
    if (index < 0 || index >= (int)P.acc.size()) return nullptr;
    auto it = P.acc.begin();
    std::advance(it, index);
    return it->first.c_str();
}

void gsr_profile_reset(void) {
    ProfState& P = prof();
    std::lock_guard<std::mutex> lk(P.mu);
    P.acc.clear();
}

}  // extern "C"
