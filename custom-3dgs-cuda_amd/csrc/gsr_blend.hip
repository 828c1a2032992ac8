// gsr_blend.hip — front-to-back alpha blend and its backward.
//
// One work-group per 16x16 tile.  Layout template kPix (pixels per lane):
// 4 / kPix wave64s, each owning a 16 x (4 kPix) strip of the tile; lane l
// holds column l & 15 and rows (l >> 4) + 4p, p < kPix, of its strip.  More
// pixels per lane give each lane independent dependency chains and divide the
// per-pixel share of the batch loads and of the backward's wave reductions;
// more waves per tile shorten the longest tile's critical path.  A batch of
// one list entry per thread is staged in LDS as 48 B blend records (one
// coalesced record load per entry); lanes walk the batch with broadcast LDS
// reads.  The forward's per-pixel arithmetic is the reference's, operation
// for operation (rasterize.cu:241-270); the backward's decisions are too
// (rasterize_backward.cu:113-200).
//
// Exact strip culling: each record carries qthr, a bound on the quadratic
// form above which no pixel can reach alpha >= 1/255 (gsr_bin.hip).  When the
// batch is staged, each entry gets one bit per strip: clear when the least
// value of the quadratic form over the strip's rectangle exceeds qthr (with
// margins for the per-pixel fp32 rounding).  Every pixel of such a strip would
// skip the entry in the reference's own tests, so the wave skips it without
// changing any result.
//
// Forward early exit: a pixel is done once T < 1e-4; a wave leaves the batch
// when none of its pixels is live; the tile stops when all are done.
// Backward: the tile walks only entries [0, max n_contrib) of its list, back
// to front (the reference walks all K entries and skips the tail per pixel),
// and each wave skips entries beyond its own max n_contrib; each entry's nine
// gradient sums are formed in the lane, summed across the wave (one
// transposed permlane/DPP reduction) and across the waves through LDS, then
// stored with plain stores into the (Gaussian, tile) pair's own gradient slot
// (nine floats and a claim bit).  pair_grad_reduce_kernel adds each
// Gaussian's claimed slots.  Float atomics are used only for list entries
// that have no slot of their own: pairs outside the Gaussian's tile
// rectangle, and a repeated id within one tile's list (caller-supplied lists).
//
// Work-groups take their tile from a launch order, longest estimated work
// first (tile_order_kernel), so long tiles do not start last.
#include <algorithm>
#include <cstdlib>

#include <mutex>

#include "gsr_internal.h"
#include "gsr_common.h"
#include "gsr_schedule.h"

namespace gsr {

namespace {

template <int kPix>
struct Layout {
    static constexpr int kWaves = 4 / kPix;
    static constexpr int kThreads = kWaves * kWave;
    static constexpr int kBatch = kThreads;
    static constexpr int kRows = 4 * kPix;  // rows per wave strip
};

template <int kPix>
struct Pixels {
    int px;
    int py[kPix];
    bool in[kPix];
};

template <int kPix>
__device__ __forceinline__ Pixels<kPix> pixels_of(int tile, int tiles_x, int W, int H) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    Pixels<kPix> p;
    p.px = tx * kTileSize + (lane & 15);
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
        p.py[k] = ty * kTileSize + wave * Layout<kPix>::kRows + (lane >> 4) + 4 * k;
        p.in[k] = p.px < W && p.py[k] < H;
    }
    return p;
}

// Minimum over the pixel rectangle [x0, x1] x [y0, y1] of the quadratic form
// q = A u^2 + 2 B u v + C v^2, (u, v) = (x - mx, y - my), for a positive
// definite conic (A > 0, AC > B^2): 0 when the mean is inside, else the least
// of the four edges' minima (each a clamped 1D quadratic).  The computed
// minimiser is off by a few ulp, which raises q only at second order; the
// evaluation's own rounding is covered by the caller's margin.
__device__ __forceinline__ float qmin_rect(float mx, float my, float A, float B, float C,
                                          float rA, float rC, float x0, float x1, float y0,
                                          float y1) {
    if (mx >= x0 && mx <= x1 && my >= y0 && my <= y1) return 0.0f;
    const float ux0 = x0 - mx, ux1 = x1 - mx, vy0 = y0 - my, vy1 = y1 - my;
    auto q = [&](float u, float v) { return A * u * u + 2.0f * B * u * v + C * v * v; };
    float best = q(fminf(fmaxf(-B * vy0 * rA, ux0), ux1), vy0);
    best = fminf(best, q(fminf(fmaxf(-B * vy1 * rA, ux0), ux1), vy1));
    best = fminf(best, q(ux0, fminf(fmaxf(-B * ux0 * rC, vy0), vy1)));
    best = fminf(best, q(ux1, fminf(fmaxf(-B * ux1 * rC, vy0), vy1)));
    return best;
}

// Staged strip bits: bit w for wave w of the tile, and this flag for the
// backward (opacity in [0, 0.99)).
constexpr uint32_t kFastExpBit = 1u << 31;

// Bit w set: some pixel of strip w may reach alpha >= 1/255.  A strip is
// culled when the least q over its rectangle, lowered by 1e-5 of the largest
// sum of |terms| there (the fp32 rounding of the per-pixel q and of this
// bound are each within ~1e-6 of that sum), still exceeds qthr.  Conics that
// are not positive definite, and NaN anywhere, cull nothing.
template <int kPix>
__device__ __forceinline__ uint32_t strip_bits(const BlendRec& r, int tile, int tiles_x) {
    constexpr uint32_t kAll = (1u << Layout<kPix>::kWaves) - 1u;
    // the conic from the record's scaled coefficients (exact)
    const float A = -2.0f * r.a.z, B = -2.0f * r.c.y, C = -2.0f * r.b.x, thr = r.c.z;
    if (!(A > 0.0f) || !(C > 0.0f) || !((double)A * C - (double)B * B > 0.0)) return kAll;
    const float mx = r.a.x, my = r.a.y;
    const float rA = 1.0f / A, rC = 1.0f / C;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const float x0 = (float)(tx * kTileSize), x1 = x0 + (float)(kTileSize - 1);
    const float dxm = fmaxf(fabsf(x0 - mx), fabsf(x1 - mx));
    uint32_t bits = 0;
#pragma unroll 1
    for (int w = 0; w < Layout<kPix>::kWaves; ++w) {
        const float y0 = (float)(ty * kTileSize + w * Layout<kPix>::kRows);
        const float y1 = y0 + (float)(Layout<kPix>::kRows - 1);
        const float dym = fmaxf(fabsf(y0 - my), fabsf(y1 - my));
        const float absq = A * dxm * dxm + 2.0f * fabsf(B) * dxm * dym + C * dym * dym;
        const float q = qmin_rect(mx, my, A, B, C, rA, rC, x0, x1, y0, y1) - 1e-5f * absq;
        const bool skip = q > thr;  // false for NaN
        bits |= skip ? 0u : (1u << w);
    }
    return bits;
}

// The record of list entry g, zeros for an id outside [0, n) (such entries are
// skipped: rasterize_backward.cu:79-86).
__device__ __forceinline__ BlendRec load_record(const BlendRec* __restrict__ recs, int g, int n) {
    BlendRec r;
    if (g >= 0 && g < n) {
        r = recs[g];
    } else {
        r.a = r.b = r.c = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    return r;
}

template <int kPix>
__device__ __forceinline__ void stage_record(const BlendRec& r, bool ok, int g, int tile,
                                             int tiles_x, float4* s_a, float4* s_b, float4* s_c,
                                             uint32_t* s_bits, int* s_id, int slot) {
    s_a[slot] = r.a;
    s_b[slot] = r.b;
    if (s_bits) s_c[slot] = r.c;
    // bit 31: opacity in [0, 0.99), so alpha = opacity * G is never clamped
    const uint32_t fast = (__float_as_uint(r.b.y) < __float_as_uint(kAlphaMax)) ? kFastExpBit : 0u;
    const uint32_t bits = ok ? (strip_bits<kPix>(r, tile, tiles_x) | fast) : 0u;
    if (s_bits)
        s_bits[slot] = bits;
    else  // in the record's unused fourth word
        s_c[slot] = make_float4(r.c.x, r.c.y, r.c.z, __uint_as_float(bits));
    if (s_id) s_id[slot] = ok ? g : -1;
}

template <int kPix>
__device__ __forceinline__ void stage_entry(const BlendRec* __restrict__ recs, int g, int n,
                                            int tile, int tiles_x, float4* s_a, float4* s_b,
                                            float4* s_c, uint32_t* s_bits, int* s_id,
                                            int slot) {
    stage_record<kPix>(load_record(recs, g, n), g >= 0 && g < n, g, tile, tiles_x, s_a, s_b, s_c,
                       s_bits, s_id, slot);
}

// Forward pixel state.  A pixel is done once a blend takes T below 1e-4
// (rasterize.cu:264-267); T only changes on a blend, so "done" is T < 1e-4
// and needs no flag (pixels off the screen start with T = 0).
struct FwdPixel {
    float T, C0, C1, C2;
    int last;
};

__device__ __forceinline__ bool live(const FwdPixel& p) { return p.T >= kTransmittanceMin; }

// power = -0.5 (cx dx^2 + 2 cy dx dy + cz dy^2) (rasterize.cu:249-251) with
// its two additions fused, from the record's coefficients a = -cx/2 (A.z),
// b = -cy (A.w), c = -cz/2 (B.x): fma(c dy, dy, fma(b dx, dy, (a dx) dx)).
__device__ __forceinline__ float blend_power(float dx, float dy, const float4& A,
                                             const float4& B) {
    return __builtin_fmaf(B.x * dy, dy, __builtin_fmaf(A.w * dx, dy, (A.z * dx) * dx));
}

// One pixel's forward step for one list entry (rasterize.cu:243-268), with the
// reference's skips as selects: the same fp32 operations in the same order,
// the colour sums fused (pix_color += colour * weight).  `on` is live(p), the
// lane mask the caller's early-exit ballot already holds.
__device__ __forceinline__ void fwd_step(FwdPixel& p, bool on, float fx, float fy,
                                         const float4& A, const float4& B, float cb,
                                         int contributor) {
    const float dx = fx - A.x;
    const float dy = fy - A.y;
    const float power = blend_power(dx, dy, A, B);
    const float alpha = fminf(kAlphaMax, B.y * exp_blend_noclamp(power));
    const bool blend = on & !(power > 0.0f) & !(alpha < kAlphaMin);
    const float w = alpha * p.T;
    const float Tn = p.T * (1.0f - alpha);
    p.C0 = blend ? __builtin_fmaf(B.z, w, p.C0) : p.C0;
    p.C1 = blend ? __builtin_fmaf(B.w, w, p.C1) : p.C1;
    p.C2 = blend ? __builtin_fmaf(cb, w, p.C2) : p.C2;
    p.T = blend ? Tn : p.T;
    p.last = blend ? contributor : p.last;
}

template <int kPix>
__device__ __forceinline__ bool any_live(const FwdPixel (&p)[kPix]) {
    bool l = false;
#pragma unroll
    for (int k = 0; k < kPix; ++k) l |= live(p[k]);
    return l;
}

// A staged entry's strip bits as a wave-uniform (scalar) value: from the
// separate array, or from the record's unused fourth word.
__device__ __forceinline__ uint32_t uniform_bits(const uint32_t* s_bits, int j) {
    return __builtin_amdgcn_readfirstlane(s_bits[j]);
}
__device__ __forceinline__ uint32_t uniform_bits(const float4& c) {
    return __builtin_amdgcn_readfirstlane(__float_as_uint(c.w));
}

template <int kPix>
__global__ __launch_bounds__(Layout<kPix>::kThreads) void blend_fwd_kernel(
    int n, int H, int W, int tiles_x, uint64_t m, const int2* __restrict__ ranges,
    const int32_t* __restrict__ ids, const BlendRec* __restrict__ recs, float* __restrict__ img,
    float* __restrict__ finalT, int32_t* __restrict__ ncontrib,
    const uint32_t* __restrict__ order) {
    constexpr int kBatch = Layout<kPix>::kBatch;
    __shared__ float4 s_a[kBatch];
    __shared__ float4 s_b[kBatch];
    __shared__ float4 s_c[kBatch];
    __shared__ uint32_t s_bits[kBatch];
    const int tile = order ? (int)order[blockIdx.x] : (int)blockIdx.x;
    // a launch order is a permutation of the tiles; nothing else is touched
    if ((unsigned)tile >= (unsigned)(tiles_x * ((H + kTileSize - 1) / kTileSize))) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: uniform branches
    const uint32_t my_bit = 1u << wave;
    const Pixels<kPix> pp = pixels_of<kPix>(tile, tiles_x, W, H);
    const float fx = (float)pp.px;
    float fy[kPix];
    FwdPixel p[kPix];
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
        fy[k] = (float)pp.py[k];
        p[k] = FwdPixel{pp.in[k] ? 1.0f : 0.0f, 0.0f, 0.0f, 0.0f, 0};
    }
    int start, end;
    clamp_range(ranges[tile], m, start, end);
    // the range is the work-group's: scalar, so the loop counters are scalar
    start = __builtin_amdgcn_readfirstlane(start);
    end = __builtin_amdgcn_readfirstlane(end);

    // each batch's ids are loaded while the batch before it is blended
    int next_id = (start + tid < end) ? ids[start + tid] : -1;
    for (int b0 = start; b0 < end; b0 += kBatch) {
        // scalar, so the entry loop's counter is scalar
        const int cnt = __builtin_amdgcn_readfirstlane(min(kBatch, end - b0));
        const int g = next_id;
        __syncthreads();
        if (tid < cnt)
            stage_entry<kPix>(recs, g, n, tile, tiles_x, s_a, s_b, s_c, s_bits, nullptr, tid);
        if (b0 + kBatch + tid < end) next_id = ids[b0 + kBatch + tid];
        __syncthreads();
        if (ballot(any_live(p)) != 0) {
            const int cbase = b0 - start + 1;
            // 64 entries at a time: one ballot gives the entries this wave's
            // strip meets (lane e holds entry c0 + e), walked in order with a
            // scalar find-first; strip-culled entries cost nothing
            bool done = false;
            for (int c0 = 0; c0 < cnt && !done; c0 += kWave) {
                const int e = c0 + lane;
                uint64_t todo = ballot(e < cnt && (s_bits[min(e, kBatch - 1)] & my_bit) != 0u);
                while (todo) {
                    // the wave stops once no pixel is live, tested before each
                    // entry with the same compares the step's skip uses
                    if (ballot(any_live(p)) == 0) {
                        done = true;
                        break;
                    }
                    const int j = c0 + (int)__builtin_ctzll(todo);
                    todo &= todo - 1;
                    const float4 A = s_a[j];
                    const float4 B = s_b[j];
                    const float cb = s_c[j].x;
#pragma unroll
                    for (int k = 0; k < kPix; ++k)
                        fwd_step(p[k], live(p[k]), fx, fy[k], A, B, cb, cbase + j);
                }
            }
        }
        if (__syncthreads_and(!any_live(p))) break;
    }
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
        if (!pp.in[k]) continue;
        const size_t q = (size_t)pp.py[k] * W + pp.px;
        img[3 * q] = p[k].C0;
        img[3 * q + 1] = p[k].C1;
        img[3 * q + 2] = p[k].C2;
        finalT[q] = p[k].T;
        ncontrib[q] = p[k].last;
    }
}

// Backward pixel state: dL/dpixel, T (unwound back to front from final_T),
// accg = sum over channels of dL/dpixel * the reconstructed colour of what lies
// behind (the reference keeps the colour, accum_rec, and only ever uses its
// dot product with dL/dpixel), and n_contrib.
struct BwdPixel {
    float g0, g1, g2, T, accg;
    int last;
};

// Per pixel and list entry the walk forms dL/dpower = alpha dL/dalpha
// (rasterize_backward.cu:155-161: 0 for a clamped or skipped entry) and the
// colour weight alpha T; dL/dopacity = G dL/dalpha is dL/dpower / opacity,
// formed once per (tile, entry) at the flush.
struct BwdTerms {
    float aT;   // alpha * T_before: dL/dcolour = aT * dL/dpixel
    float dpw;  // dL/dpower
};

// One pixel's decision for one list entry (rasterize_backward.cu:117-140):
// G = exp(power), alpha = min(0.99, opacity G), and whether the entry blends
// (within n_contrib, power <= 0, alpha >= 1/255) and passes gradient through
// the clamp.  ae = alpha if it blends, else 0; ag = alpha if it also passes
// gradient (then alpha = opacity G unclamped), else 0.
struct BwdDecision {
    float dy, power, alpha, ae, ag;
    bool act;
};

// The forward's own evaluation: exp_blend and the same fp32 operations, so
// every skip agrees with the forward bit for bit.
__device__ __forceinline__ void decide_exact(BwdDecision& d, float o, int contributor, int last) {
    const float araw = o * exp_blend(d.power);
    d.alpha = fminf(kAlphaMax, araw);
    d.act = (contributor <= last) & !(d.power > 0.0f) & !(d.alpha < kAlphaMin);
    d.ae = d.act ? d.alpha : 0.0f;
    d.ag = (d.act & (araw < kAlphaMax)) ? d.alpha : 0.0f;
}

// For an entry with opacity in [0, 0.99): G from the hardware exp2, which is
// within 1e-6 relative of exp_blend wherever alpha can reach 1/255 (power in
// [-5.6, 0]), so the alpha >= 1/255 test agrees with the exact one unless
// alpha lies within kNearAlpha of 1/255; alpha <= opacity < 0.99 is never
// clamped.  Alpha at or above kAlphaMin + kNearAlpha passes the test, below
// kAlphaMin - kNearAlpha fails it; the returned mask holds the lanes in
// neither case (near the threshold, or a NaN alpha), which need the exact
// evaluation.  Two compares per pixel, each ballot a compare's own mask.
constexpr float kNearAlpha = kAlphaMin * 2e-5f;
constexpr float kAlphaLo = kAlphaMin - kNearAlpha, kAlphaHi = kAlphaMin + kNearAlpha;
__device__ __forceinline__ uint64_t decide_fast(BwdDecision& d, float o, int contributor,
                                                int last) {
    d.alpha = o * __builtin_amdgcn_exp2f(d.power * 1.44269504088896341f);
    const bool pass = d.alpha >= kAlphaHi;
    d.act = (contributor <= last) & !(d.power > 0.0f) & pass;
    d.ae = d.act ? d.alpha : 0.0f;
    d.ag = d.ae;
    return ballot(!(d.alpha < kAlphaLo)) & ~ballot(pass);
}

// The wave's decisions for one entry: the fast evaluation where the record
// allows it, the exact one for the whole wave when any lane is near the
// threshold.
template <int kPix>
__device__ __forceinline__ void decide_entry(BwdDecision (&d)[kPix], float o, bool fast,
                                             int contributor, const BwdPixel (&p)[kPix]) {
    bool exact = !fast;
    if (!exact) {
        uint64_t near = 0;
#pragma unroll
        for (int k = 0; k < kPix; ++k) near |= decide_fast(d[k], o, contributor, p[k].last);
        exact = near != 0;
    }
    if (exact) {
#pragma unroll
        for (int k = 0; k < kPix; ++k) decide_exact(d[k], o, contributor, p[k].last);
    }
}

// One pixel's gradient step for a decided entry (rasterize_backward.cu:
// 141-198).  A skipped entry enters with ae = ag = 0, which leaves T (x / 1)
// and accg unchanged and gives zero terms.  This arithmetic only has to meet
// the fp32 gradient tolerance and may use fused multiply-adds.
__device__ __forceinline__ BwdTerms bwd_update(BwdPixel& p, const BwdDecision& d,
                                               const float4& B, float cb) {
#pragma clang fp contract(fast)
    BwdTerms t;
    // T / (1 - alpha) with 1 - alpha in [0.01, 1]: the reference's 1e-4 floor
    // never applies.  The hardware reciprocal (1 ulp) times T: about 1.5 ulp
    // per entry where a division is 0.5, so over the two thousand entries of
    // the benchmark scene's longest lists T drifts by a few 1e-5, against the
    // 1e-5 that the reference's own fp32 division reaches there; both lie
    // within the 1e-4 gradient bar.  A correction step from the exact residual
    // T - q (1 - alpha) (two fused multiply-adds on the entry's dependency
    // chain) brought the quotient to a division's 0.5 ulp and cost 15 us of
    // the bench frame's 229 us backward blend; on c5's distributions (walks
    // of 1.5e4 entries) it left the gradients unchanged to 1e-3 of their
    // error against float64, as did the forward's own alpha in place of the
    // fast one.  A skipped entry (alpha 0) leaves T unchanged: the reciprocal
    // of 1 is exact.
    const float den = 1.0f - d.ae;
    const float Tb = p.T * __builtin_amdgcn_rcpf(den);
    const float cg = B.z * p.g0 + B.w * p.g1 + cb * p.g2;
    const float diff = cg - p.accg;
    t.aT = d.ae * Tb;
    t.dpw = d.ag * (diff * Tb);
    p.accg = __builtin_fmaf(d.ae, diff, p.accg);
    p.T = Tb;
    return t;
}

__device__ __forceinline__ BwdPixel load_bwd_pixel(bool in, int px, int py, int W,
                                                   const float* __restrict__ grad,
                                                   const GradStrides& gst,
                                                   const float* __restrict__ finalT,
                                                   const int32_t* __restrict__ ncontrib) {
    BwdPixel p{0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0};
    if (in) {
        const float* g = grad + (int64_t)py * gst.h + (int64_t)px * gst.w;
        p.g0 = g[0];
        p.g1 = g[gst.c];
        p.g2 = g[2 * gst.c];
        const size_t q = (size_t)py * W + px;
        p.T = finalT[q];
        p.last = max(ncontrib[q], 0);
    }
    return p;
}

// Per (tile, entry) the wave sums nine values.  A lane's pixels share dx
// (column lane & 15), so the reference's per-pixel mean and conic terms
// (rasterize_backward.cu:163-176) follow from per-lane sums of dpw = dL/dpower:
// S0 = sum dpw, P2 = sum dpw dy, P5 = sum dpw dy^2, with dx applied once the
// lanes of a column are summed (wave_reduce_columns): P1 = sum dx S0,
// Q1 = sum dx^2 S0, Q2 = sum dx P2.  Then dL/dmean = (cx P1 + cy P2,
// cy P1 + cz P2), dL/dconic = (-Q1 / 2, -Q2, -P5 / 2) (converted to dL/dcov2d
// per (tile, entry), before any sum over tiles), dL/dcolour the sums of
// alpha T dL/dpixel and dL/dopacity = S0 / opacity.  Value k sits in slot
// kCol* of the reduction's result.
constexpr int kTerms = 9;

// dL/dcov2d (a, b, c) from dL/dconic (x, y full off-diagonal, z) for conic =
// (cx, cy, cz) = cov^-1 (rasterize_backward.cu:211-221).
__device__ __forceinline__ void conic_to_cov_grad(float cx, float cy, float cz, float dx, float dy,
                                                  float dz, float out[3]) {
    const float gx = dx, gy = 0.5f * dy, gz = dz;
    out[0] = -(cx * cx * gx + 2.0f * cx * cy * gy + cy * cy * gz);
    out[1] = -2.0f * (cx * cy * gx + (cx * cz + cy * cy) * gy + cy * cz * gz);
    out[2] = -(cy * cy * gx + 2.0f * cy * cz * gy + cz * cz * gz);
}

// Long tiles' backward runs as two work items (tile_order_kernel picks them).
// The back part walks entries [mid, maxc) from the final transmittance, as a
// whole tile does.  The front part walks the same entries first with the
// pixel state only (state_walk) (the T and accumulated-colour steps of
// rasterize_backward.cu:141-198, no gradient sums), which hands it the exact
// state the sequential walk has at mid, then walks [0, mid) in full.  Both
// parts' gradients are bit for bit the whole tile's.  A state-only step costs
// about 0.4 of a full one, so mid = 0.37 maxc leaves each part ~0.63 of the
// tile's walk.
constexpr int kPartWhole = 0, kPartBack = 1, kPartFront = 2;
constexpr int kSplitNum = 37, kSplitDen = 100;
// Most tiles split per backward launch (the launch has this many extra groups).
constexpr int kSplitMax = 256;

// The entries of one 64-entry chunk of a staged batch [lo, lo + cnt) that a
// wave walks, one ballot each: bit e of `walk` for entry c0 + e when it is in
// the batch, within the wave's largest n_contrib and its strip bit is set;
// bit e of `fast` for its fast-exp flag.  Lane e reads entry c0 + e's bits.
struct ChunkMasks {
    uint64_t walk, fast;
};
template <int kBatch>
__device__ __forceinline__ ChunkMasks chunk_masks(const float4* s_c, int c0, int cnt, int lo,
                                                  int wave_last, uint32_t my_bit) {
    const int e = c0 + (int)(threadIdx.x & 63);
    const bool in = e < cnt;
    const uint32_t b = in ? __float_as_uint(s_c[min(e, kBatch - 1)].w) : 0u;
    return ChunkMasks{ballot(in && lo + e + 1 <= wave_last && (b & my_bit) != 0u),
                      ballot((b & kFastExpBit) != 0u)};
}

// The pixel state's walk over entries [lo0, hi0), back to front: the same
// decisions and T / accumulated-colour steps as the full walk, no sums.
template <int kPix, int kBatch>
__device__ __forceinline__ void state_walk(int lo0, int hi0, int n, int tile, int tiles_x,
                                           int start, int wave_last, uint32_t my_bit, float fx,
                                           const float (&fy)[kPix], BwdPixel (&p)[kPix],
                                           const int32_t* __restrict__ ids,
                                           const BlendRec* __restrict__ recs, float4* s_a,
                                           float4* s_b, float4* s_c) {
    const int tid = threadIdx.x;
    for (int hi = hi0; hi > lo0; hi -= kBatch) {
        const int lo = max(lo0, hi - kBatch);
        const int cnt = hi - lo;
        __syncthreads();
        if (tid < cnt)
            stage_entry<kPix>(recs, ids[start + lo + tid], n, tile, tiles_x, s_a, s_b, s_c,
                              nullptr, nullptr, tid);
        __syncthreads();
        for (int chunk = ((cnt - 1) / kWave) * kWave; chunk >= 0; chunk -= kWave) {
            const ChunkMasks cm = chunk_masks<kBatch>(s_c, chunk, cnt, lo, wave_last, my_bit);
            for (uint64_t todo = cm.walk; todo != 0;) {
                const int jj = 63 - (int)__builtin_clzll(todo);  // back to front
                todo ^= 1ull << jj;
                const int j = chunk + jj;
                const int contributor = lo + j + 1;
                const float4 A = s_a[j];
                const float4 B = s_b[j];
                const float cb = s_c[j].x;
                const float dx = fx - A.x;
                const float adxdx = (A.z * dx) * dx;
                const float bdx = A.w * dx;
                BwdDecision d[kPix];
#pragma unroll
                for (int k = 0; k < kPix; ++k) {
                    d[k].dy = fy[k] - A.y;
                    d[k].power = __builtin_fmaf(B.x * d[k].dy, d[k].dy,
                                                __builtin_fmaf(bdx, d[k].dy, adxdx));
                }
                decide_entry<kPix>(d, B.y, ((cm.fast >> jj) & 1u) != 0u, contributor, p);
#pragma unroll
                for (int k = 0; k < kPix; ++k) (void)bwd_update(p[k], d[k], B, cb);
            }
        }
    }
}

template <int kPix, int kBatch, bool kSplit>
__global__ __launch_bounds__(Layout<kPix>::kThreads) void blend_bwd_kernel(
    int n, int H, int W, int tiles_x, uint64_t m, const float* __restrict__ grad, GradStrides gst,
    const int2* __restrict__ ranges, const int32_t* __restrict__ ids,
    const BlendRec* __restrict__ recs, const float* __restrict__ finalT,
    const int32_t* __restrict__ ncontrib, float* __restrict__ dmean, float* __restrict__ dcov,
    float* __restrict__ dcol, float* __restrict__ dalpha, GradSlots gs,
    const uint32_t* __restrict__ order) {
    constexpr int kWaves = Layout<kPix>::kWaves;
    static_assert(kBatch <= Layout<kPix>::kThreads, "one staged entry per thread");
    __shared__ float4 s_a[kBatch];
    __shared__ float4 s_b[kBatch];
    __shared__ float4 s_c[kBatch];
    __shared__ int s_id[kBatch];
    __shared__ float s_part[kWaves][kTerms][kBatch + 1];  // +1: the 9 writers hit 9 banks
    __shared__ uint32_t s_max[kWaves];

    // Work item.  kSplit (a schedule is given): items 2i and 2i + 1 (i < K) are
    // the back and front parts of the schedule's i-th tile, and the later
    // items its tiles from K on, whole; order[T] holds K (at most kSplitMax).
    const int T = tiles_x * ((H + kTileSize - 1) / kTileSize);
    int part = kPartWhole, tile;
    if constexpr (kSplit) {
        const int K = (int)min((uint32_t)kSplitMax,
                               (uint32_t)__builtin_amdgcn_readfirstlane((int)order[T]));
        const int item = (int)blockIdx.x;
        if (item < 2 * K) {
            part = (item & 1) ? kPartFront : kPartBack;
            tile = (int)order[item >> 1];
        } else {
            const int idx = item - K;
            if (idx >= T) return;
            tile = (int)order[idx];
        }
    } else {
        tile = order ? (int)order[blockIdx.x] : (int)blockIdx.x;
    }
    tile = __builtin_amdgcn_readfirstlane(tile);
    // a launch order is a permutation of the tiles; nothing else is touched
    if ((unsigned)tile >= (unsigned)T) return;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // scalar: uniform branches
    const uint32_t my_bit = 1u << wave;
    const Pixels<kPix> pp = pixels_of<kPix>(tile, tiles_x, W, H);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const float fx = (float)pp.px;
    float fy[kPix];
    BwdPixel p[kPix];
    int my_last = 0;
#pragma unroll
    for (int k = 0; k < kPix; ++k) {
        fy[k] = (float)pp.py[k];
        p[k] = load_bwd_pixel(pp.in[k], pp.px, pp.py[k], W, grad, gst, finalT, ncontrib);
        my_last = max(my_last, p[k].last);
    }
    int start, end;
    clamp_range(ranges[tile], m, start, end);
    const int wave_last = __builtin_amdgcn_readfirstlane((int)wave_max_u32((uint32_t)my_last));
    if (lane == 0) s_max[wave] = (uint32_t)wave_last;
    __syncthreads();
    uint32_t tile_last = 0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) tile_last = max(tile_last, s_max[w]);
    const int maxc = __builtin_amdgcn_readfirstlane(min((int)tile_last, end - start));
    start = __builtin_amdgcn_readfirstlane(start);
    const int my_value = columns_value_of_lane(lane);
    // the entries [lo0, hi0) this item walks with gradients; the front part
    // first walks [mid, maxc) for the pixel state only
    int lo0 = 0, hi0 = maxc;
    if constexpr (kSplit) {
        const int mid = (int)(((int64_t)maxc * kSplitNum) / kSplitDen);
        if (part == kPartBack) lo0 = mid;
        if (part == kPartFront) {
            hi0 = mid;
            state_walk<kPix, kBatch>(mid, maxc, n, tile, tiles_x, start, wave_last, my_bit, fx,
                                     fy, p, ids, recs, s_a, s_b, s_c);
        }
    }

    // each batch's ids are loaded while the batch after it is walked
    int next_id =
        (tid < min(hi0 - lo0, kBatch)) ? ids[start + max(lo0, hi0 - kBatch) + tid] : -1;
    for (int hi = hi0; hi > lo0; hi -= kBatch) {
        const int lo = max(lo0, hi - kBatch);
        const int cnt = hi - lo;
        const int g = next_id;
        __syncthreads();
        if (tid < cnt)
            stage_entry<kPix>(recs, g, n, tile, tiles_x, s_a, s_b, s_c, nullptr, s_id, tid);
        if (lo > lo0) {
            const int nlo = max(lo0, lo - kBatch);
            if (tid < lo - nlo) next_id = ids[start + nlo + tid];
        }
        __syncthreads();
        // this wave's partial sums of the batch start at zero: entries it does
        // not walk (culled, or beyond its largest n_contrib) add nothing
        for (int e = lane; e < cnt; e += kWave)
#pragma unroll
            for (int k = 0; k < kTerms; ++k) s_part[wave][k][e] = 0.0f;
        // 64 entries at a time, back to front, the walked ones found with a
        // scalar find-last over one ballot
        for (int chunk = ((cnt - 1) / kWave) * kWave; chunk >= 0; chunk -= kWave) {
            const ChunkMasks cm = chunk_masks<kBatch>(s_c, chunk, cnt, lo, wave_last, my_bit);
            for (uint64_t todo = cm.walk; todo != 0;) {
                const int jj = 63 - (int)__builtin_clzll(todo);
                todo ^= 1ull << jj;
                const int j = chunk + jj;
                const int contributor = lo + j + 1;
                float w9;
                const float4 A = s_a[j];
                const float4 Cc = s_c[j];  // (b, -cy/2, qthr, strip bits)
                const float cb = Cc.x;
                const float4 B = s_b[j];
                const float dx = fx - A.x;
                // blend_power's shared column terms: (a dx) dx and b dx
                const float adxdx = (A.z * dx) * dx;
                const float bdx = A.w * dx;
                BwdDecision d[kPix];
#pragma unroll
                for (int k = 0; k < kPix; ++k) {
                    // the forward's power, bit for bit (blend_power)
                    d[k].dy = fy[k] - A.y;
                    d[k].power = __builtin_fmaf(B.x * d[k].dy, d[k].dy,
                                                __builtin_fmaf(bdx, d[k].dy, adxdx));
                }
                decide_entry<kPix>(d, B.y, ((cm.fast >> jj) & 1u) != 0u, contributor, p);
                // per-lane sums over its pixels, started from the first pixel's terms
                float S0, P2, P5, c0, c1, c2;
                {
                    const BwdTerms t = bwd_update(p[0], d[0], B, cb);
                    const float e = t.dpw * d[0].dy;
                    S0 = t.dpw;
                    P2 = e;
                    P5 = e * d[0].dy;
                    c0 = t.aT * p[0].g0;
                    c1 = t.aT * p[0].g1;
                    c2 = t.aT * p[0].g2;
                }
#pragma unroll
                for (int k = 1; k < kPix; ++k) {
                    const BwdTerms t = bwd_update(p[k], d[k], B, cb);
                    {
#pragma clang fp contract(fast)
                        const float e = t.dpw * d[k].dy;
                        S0 += t.dpw;
                        P2 += e;
                        P5 += e * d[k].dy;
                        c0 += t.aT * p[k].g0;
                        c1 += t.aT * p[k].g1;
                        c2 += t.aT * p[k].g2;
                    }
                }
                // a wave with no blending pixel (2% of the strip-passing
                // wave-entries on the bench scene) sums zeros
                w9 = wave_reduce_columns(S0, P2, P5, c0, c1, c2, dx);
                if (my_value >= 0) s_part[wave][my_value][j] = w9;
            }
        }
        __syncthreads();
        if (tid < cnt) {
            const int g = s_id[tid];
            float tot[kTerms];
            bool any = false;
#pragma unroll
            for (int k = 0; k < kTerms; ++k) {
                float acc = 0.0f;
#pragma unroll
                for (int w = 0; w < kWaves; ++w) acc += s_part[w][k][tid];
                tot[k] = acc;
                any |= acc != 0.0f;
            }
            if (g >= 0 && any) {
                float t[kTerms];
                // the record's -cx/2 (A.z), -cy/2 (C.y), -cz/2 (B.x), opacity (B.y)
                const float ha = s_a[tid].z, hb = s_c[tid].y, hc = s_b[tid].x, o = s_b[tid].y;
                const float S0 = tot[kColS0], P1 = tot[kColP1], P2 = tot[kColP2];
                t[0] = -2.0f * (ha * P1 + hb * P2);  // dL/dmean.x = cx P1 + cy P2
                t[1] = -2.0f * (hb * P1 + hc * P2);  // dL/dmean.y = cy P1 + cz P2
                // dL/dcov2d from this (tile, entry)'s dL/dconic (x, full
                // off-diagonal y, z), converted here as the reference converts
                // each flushed batch (rasterize_backward.cu:211-221): for a
                // near-singular covariance the conversion's terms cancel, and
                // they then cancel at one tile's magnitude instead of at the
                // Gaussian's total over all its tiles
                conic_to_cov_grad(-2.0f * ha, -2.0f * hb, -2.0f * hc, -0.5f * tot[kColQ1],
                                  -tot[kColQ2], -0.5f * tot[kColP5], t + 2);
                t[5] = tot[kColC0];                  // dL/dcolour
                t[6] = tot[kColC1];
                t[7] = tot[kColC2];
                // dL/dopacity: every dpw carries a factor opacity (no pixel
                // blends the entry when the opacity is 0)
                t[8] = (S0 == 0.0f) ? 0.0f : S0 / o;
                // the pair's slot: goff[g] + this tile's index in g's rectangle
                const uint2 rc = gs.rects[g];
                const int rx0 = (int)(rc.x & 0xffffu), rx1 = (int)(rc.x >> 16);
                const int ry0 = (int)(rc.y & 0xffffu), ry1 = (int)(rc.y >> 16);
                const uint64_t slot = (uint64_t)gs.goff[g] +
                                      (uint64_t)((ty - ry0) * (rx1 - rx0) + (tx - rx0));
                bool own = tx >= rx0 && tx < rx1 && ty >= ry0 && ty < ry1 && slot < gs.slots;
                if (own) {
                    // claim the slot: its flag bit.  Only an id repeated
                    // within this tile's list finds it claimed already.
                    const uint32_t bit = 1u << (uint32_t)(slot & 31u);
                    own = (atomicOr(gs.flags + (slot >> 5), bit) & bit) == 0u;
                }
                if (own) {
                    float* d = gs.sums + 9 * slot;
#pragma unroll
                    for (int k = 0; k < kTerms; ++k) d[k] = t[k];
                } else {
                    // no slot of its own (outside the rectangles, or a repeated
                    // id): straight to the outputs
                    unsafeAtomicAdd(&dmean[2 * (size_t)g], t[0]);
                    unsafeAtomicAdd(&dmean[2 * (size_t)g + 1], t[1]);
                    unsafeAtomicAdd(&dcov[3 * (size_t)g], t[2]);
                    unsafeAtomicAdd(&dcov[3 * (size_t)g + 1], t[3]);
                    unsafeAtomicAdd(&dcov[3 * (size_t)g + 2], t[4]);
                    unsafeAtomicAdd(&dcol[3 * (size_t)g], t[5]);
                    unsafeAtomicAdd(&dcol[3 * (size_t)g + 1], t[6]);
                    unsafeAtomicAdd(&dcol[3 * (size_t)g + 2], t[7]);
                    unsafeAtomicAdd(&dalpha[g], t[8]);
                }
            }
        }
    }
}

// One 16-lane row per Gaussian (four per wave): the nine sums of its flagged
// slots (d mean2d, d cov2d, d colour, d opacity), added to the outputs (which
// hold zeros and any fallback atomics from the blend).
// Sum over the kLanes (16 or 8) lanes of each row, result in every lane of
// the row.
template <int kLanes>
__device__ __forceinline__ float row_sum(float x) {
    if constexpr (kLanes == 16) x += dpp_move<kDppRowRor8>(x);
    x += lane_xor4(x);
    x += dpp_move<kDppQuadXor2>(x);
    x += dpp_move<kDppQuadXor1>(x);
    return x;
}

// kLanes per Gaussian: 16, or 8 when Gaussians have few slots (half the
// waves then wait on the dependent loads).  Each lane reads the flag bits of
// kGroup consecutive slots per step: 8 (one byte) when Gaussians average a
// few hundred slots or fewer, 64 (one word) beyond, where claimed slots are
// sparse and a row then covers 1024 slots per step.
template <int kReduceRowLanes, int kGroup>
__global__ __launch_bounds__(256) void pair_grad_reduce_kernel(
    int n, GradSlots gs, float* __restrict__ dmean, float* __restrict__ dcov,
    float* __restrict__ dcol, float* __restrict__ dalpha) {
    static_assert(kReduceRowLanes == 16 || kReduceRowLanes == 8, "rows of 16 or 8 lanes");
    static_assert(kGroup == 8 || kGroup == 64, "flag groups of 8 or 64 slots");
    constexpr int kReduceGaussiansPerBlock = 256 / kReduceRowLanes;
    const int sub = threadIdx.x & (kReduceRowLanes - 1);
    const int g = blockIdx.x * kReduceGaussiansPerBlock + (int)(threadIdx.x / kReduceRowLanes);
    // the flag bits of slots [grp, grp + kGroup), grp a multiple of kGroup
    // (the flag array is 256-byte aligned and padded to 64-bit words)
    auto group_bits = [&](uint64_t grp) -> uint64_t {
        if constexpr (kGroup == 8)
            return reinterpret_cast<const uint8_t*>(gs.flags)[grp >> 3];
        else
            return reinterpret_cast<const uint64_t*>(gs.flags)[grp >> 6];
    };
    float v[kTerms] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    bool claimed = false;
    if (g < n) {
        const uint64_t base = gs.goff[g];
        const uint64_t end = min(base + (uint64_t)gs.counts[g], gs.slots);
        // each group's flags are loaded while the group before is summed, and
        // the sums of two flagged slots are loaded together
        uint64_t grp = (base & ~(uint64_t)(kGroup - 1)) + (uint64_t)kGroup * sub;
        uint64_t bits = (grp < end) ? group_bits(grp) : 0ull;
        while (grp < end) {
            const uint64_t nxt = grp + (uint64_t)kGroup * kReduceRowLanes;
            const uint64_t nbits = (nxt < end) ? group_bits(nxt) : 0ull;
            // only the flags of [base, end)
            if (grp < base) bits &= ~0ull << (base - grp);
            if (end - grp < (uint64_t)kGroup) bits &= ~(~0ull << (end - grp));
            claimed |= bits != 0;
            while (bits) {
                const uint64_t s0 = grp + (uint64_t)__builtin_ctzll(bits);
                bits &= bits - 1;
                const bool two = bits != 0;
                const uint64_t s1 = two ? grp + (uint64_t)__builtin_ctzll(bits) : s0;
                if (two) bits &= bits - 1;
                const float* d0 = gs.sums + 9 * s0;
                const float* d1 = gs.sums + 9 * s1;
                float a[kTerms], b[kTerms];
#pragma unroll
                for (int k = 0; k < kTerms; ++k) {
                    a[k] = d0[k];
                    b[k] = d1[k];
                }
#pragma unroll
                for (int k = 0; k < kTerms; ++k) v[k] += two ? a[k] + b[k] : a[k];
            }
            grp = nxt;
            bits = nbits;
        }
    }
    // a Gaussian without claimed slots adds nothing (at 4K most Gaussians
    // have none in a given screen band): its outputs are not read or written,
    // and a wave without any skips the row sums
    const uint64_t wave_claims = ballot(claimed);
    if (wave_claims == 0ull) return;
    // every lane takes part in the row sums (rows past n add zeros)
    float t[kTerms];
#pragma unroll
    for (int k = 0; k < kTerms; ++k) t[k] = row_sum<kReduceRowLanes>(v[k]);
    const uint64_t row_claims =
        (wave_claims >> (lane_id() & (64 - kReduceRowLanes))) & ((1ull << kReduceRowLanes) - 1);
    if (g < n && sub == 0 && row_claims != 0) {
        const float m0 = dmean[2 * (size_t)g], m1 = dmean[2 * (size_t)g + 1];
        const float c0 = dcov[3 * (size_t)g], c1 = dcov[3 * (size_t)g + 1],
                    c2 = dcov[3 * (size_t)g + 2];
        const float k0 = dcol[3 * (size_t)g], k1 = dcol[3 * (size_t)g + 1],
                    k2 = dcol[3 * (size_t)g + 2];
        const float a0 = dalpha[g];
        dmean[2 * (size_t)g] = m0 + t[0];
        dmean[2 * (size_t)g + 1] = m1 + t[1];
        dcov[3 * (size_t)g] = c0 + t[2];
        dcov[3 * (size_t)g + 1] = c1 + t[3];
        dcov[3 * (size_t)g + 2] = c2 + t[4];
        dcol[3 * (size_t)g] = k0 + t[5];
        dcol[3 * (size_t)g + 1] = k1 + t[6];
        dcol[3 * (size_t)g + 2] = k2 + t[7];
        dalpha[g] = a0 + t[8];
    }
}

// ---- tile scheduling: work-groups start in descending order of estimated
// work, so the longest tiles do not start last and set the kernel's tail.
// The order changes no result: every tile's pixels are computed by one
// work-group on their own. ----

// Backward work of a tile: its list entries up to the largest n_contrib
// (tile_work_bwd_wave, one wave per tile).  Run here, or by the backward
// records kernel in work-groups of its own launch.
__global__ __launch_bounds__(kWorkTilesPerBlock * kWave) void tile_work_bwd_kernel(BwdWork b) {
    const int tile = blockIdx.x * kWorkTilesPerBlock + (int)(threadIdx.x >> 6);
    if (tile >= b.T) return;  // whole waves
    tile_work_bwd_wave(b, tile);
}

// Forward work of a tile: the list entries it takes until two sample pixels
// (on the diagonal, a quarter of the way in from opposite corners) are done
// (T < 1e-4), or the whole list when one never is (the forward walks a tile's
// list until every pixel is done).  An ordering heuristic only: it uses the
// hardware exp and log and no culling.  Measured against five points and a
// 1024-entry cap, it costs less than it loses in ordering (render -5 us at
// 1080p, -11 us at 720p on the bench scene, +3 us on c3).  Ordering by list
// length alone (no walk) made the bench scene's forward blend 32 us slower;
// one centre point cost c4's blend 5 us.
constexpr int kEstPoints = 2;

// One wave per tile, 64 entries per step, the next step's ids prefetched.  A
// sample pixel still live after kEstCap entries counts as never done.  256
// orders as well as 512 and 1024 on the bench scene, c3 and c4 and walks
// less (the estimate 22 to 19 us on the bench scene); 128 orders worse.
constexpr int kEstTilesPerBlock = 4;
constexpr int kEstCap = 256;

__global__ __launch_bounds__(kEstTilesPerBlock * kWave) void tile_work_fwd_kernel(
    int T, int tiles_x, int n, uint64_t m, const int2* __restrict__ ranges,
    const int32_t* __restrict__ ids, const BlendRec* __restrict__ recs,
    uint32_t* __restrict__ work) {
    constexpr float kLnTmin = -9.21034037f;  // ln(1e-4)
    const int lane = threadIdx.x & 63;
    const int tile = blockIdx.x * kEstTilesPerBlock + (int)(threadIdx.x >> 6);
    if (tile >= T) return;  // whole waves
    int start, end;
    clamp_range(ranges[tile], m, start, end);
    const int len = end - start;
    const float x0 = (float)((tile % tiles_x) * kTileSize);
    const float y0 = (float)((tile / tiles_x) * kTileSize);
    const float sx[kEstPoints] = {x0 + 3.0f, x0 + 12.0f};
    const float sy[kEstPoints] = {y0 + 3.0f, y0 + 12.0f};
    float carry[kEstPoints] = {0.0f, 0.0f};
    int sat[kEstPoints] = {-1, -1};
    int next = (lane < len) ? ids[start + lane] : -1;
    for (int c = 0; c < min(len, kEstCap); c += kWave) {
        const int g = next;
        const bool ok = g >= 0 && g < n;  // false past the list end as well
        BlendRec r;
        if (ok) r = recs[g];
        next = (c + kWave + lane < len) ? ids[start + c + kWave + lane] : -1;
        bool all = true;
#pragma unroll
        for (int q = 0; q < kEstPoints; ++q) {
            float l = 0.0f;
            if (ok) {
                const float dx = sx[q] - r.a.x, dy = sy[q] - r.a.y;
                const float power = blend_power(dx, dy, r.a, r.b);
                const float alpha = fminf(kAlphaMax, r.b.y * __expf(power));
                l = (power <= 0.0f && alpha >= kAlphaMin) ? __logf(1.0f - alpha) : 0.0f;
            }
            const float incl = wave_inclusive_scan_f(l);
            const uint64_t below = ballot(c + lane < len && carry[q] + incl < kLnTmin);
            if (sat[q] < 0 && below != 0) sat[q] = c + (int)__builtin_ctzll(below);
            carry[q] += __shfl(incl, 63, kWave);
            all &= sat[q] >= 0;
        }
        if (all) break;
    }
    if (lane == 0) {
        int w = 0;
        bool open = false;
#pragma unroll
        for (int q = 0; q < kEstPoints; ++q) {
            if (sat[q] < 0) open = true;
            else w = max(w, sat[q] + 1);
        }
        work[tile] = (uint32_t)(open ? len : w);
    }
}

// 256 buckets, ordered like the value: 5-bit exponent, 3-bit mantissa.
__device__ __forceinline__ uint32_t work_bucket(uint32_t w) {
    if (w == 0) return 0;
    const uint32_t e = 31u - (uint32_t)__builtin_clz(w);
    const uint32_t mant = (e >= 3) ? (w >> (e - 3)) & 7u : (w << (3 - e)) & 7u;
    return min(255u, e * 8u + mant + 1u);
}

constexpr int kOrderThreads = 1024;
constexpr int kOrderHeld = 8;  // 8192 tiles held in registers (1080p: 8160)
constexpr uint32_t kSplitBuckets = 5;
constexpr uint32_t kSplitMinWork = 256;
// A tile alone on a CU runs at roughly a quarter of the CU's rate.
constexpr uint64_t kSplitLoad = 4;

// order[i] = tiles by descending work bucket (one work-group); with split_max
// >= 0 also order[T], the backward's split count (below).  work == null:
// the forward's estimate, the tile's list length.
__global__ __launch_bounds__(kOrderThreads) void tile_order_kernel(
    int T, uint64_t m, const int2* __restrict__ ranges, const uint32_t* __restrict__ work,
    uint32_t* __restrict__ order, int split_max, int cus) {
    __shared__ uint32_t s_cnt[256];
    __shared__ uint32_t s_scan[4];
    __shared__ uint32_t s_top;
    __shared__ unsigned long long s_sum;
    __shared__ uint32_t s_wmax;
    const int tid = threadIdx.x;
    auto work_of = [&](int t) -> uint32_t {
        if (work) return work[t];
        int start, end;
        clamp_range(ranges[t], m, start, end);
        return (uint32_t)(end - start);
    };
    auto bucket = [](uint32_t w) -> uint32_t { return 255u - work_bucket(w); };  // descending
    auto bucket_of = [&](int t) -> uint32_t { return bucket(work_of(t)); };
    if (tid < 256) s_cnt[tid] = 0;
    if (tid == 0) {
        s_sum = 0ull;
        s_wmax = 0u;
    }
    // the first kOrderHeld tiles per thread are read once, all loads in
    // flight together, and their work kept for the scatter
    auto held_tile = [&](int i) { return tid + i * kOrderThreads; };
    uint32_t held[kOrderHeld];
#pragma unroll
    for (int i = 0; i < kOrderHeld; ++i) {
        const int t = held_tile(i);
        held[i] = (t < T) ? work_of(t) : 0u;
    }
    __syncthreads();
    uint64_t wsum = 0;
    uint32_t wmax = 0;
#pragma unroll
    for (int i = 0; i < kOrderHeld; ++i) {
        if (held_tile(i) < T) atomicAdd(&s_cnt[bucket(held[i])], 1u);
        wsum += held[i];
        wmax = max(wmax, held[i]);
    }
    for (int t = tid + kOrderHeld * kOrderThreads; t < T; t += kOrderThreads) {
        const uint32_t w = work_of(t);
        atomicAdd(&s_cnt[bucket(w)], 1u);
        wsum += w;
        wmax = max(wmax, w);
    }
    if (split_max > 0) {
        // one atomic per wave
        const uint64_t ws = wave_sum_u64(wsum);
        const uint32_t wm = wave_max_u32(wmax);
        if ((tid & 63) == 0) {
            atomicAdd(&s_sum, (unsigned long long)ws);
            atomicMax(&s_wmax, wm);
        }
    }
    __syncthreads();
    uint32_t c = 0, inc = 0;
    if (tid < 256) {
        c = s_cnt[tid];
        inc = wave_inclusive_scan(c);
        if ((tid & 63) == 63) s_scan[tid >> 6] = inc;
    }
    __syncthreads();
    if (tid < 256) {
        uint32_t pre = 0;
        for (int w = 0; w < (tid >> 6); ++w) pre += s_scan[w];
        s_cnt[tid] = pre + inc - c;  // first slot of the bucket
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kOrderHeld; ++i) {
        const int t = held_tile(i);
        if (t < T) {
            const uint32_t pos = atomicAdd(&s_cnt[bucket(held[i])], 1u);
            if (pos < (uint32_t)T) order[pos] = (uint32_t)t;
        }
    }
    for (int t = tid + kOrderHeld * kOrderThreads; t < T; t += kOrderThreads) {
        const uint32_t pos = atomicAdd(&s_cnt[bucket_of(t)], 1u);
        if (pos < (uint32_t)T) order[pos] = (uint32_t)t;
    }
    if (split_max == 0 && tid == 0) order[T] = 0u;
    if (split_max > 0) {
        // order[T] = how many of the first tiles the backward splits: those
        // within kSplitBuckets sub-buckets (a factor 2^(5/8) ~ 1.5) of the
        // longest, if it has kSplitMinWork entries or more and a long tail
        // (below).  s_cnt[b] now holds the end of bucket b, so the first
        // non-zero one is the top.
        if (tid == 0) s_top = 256u;
        __syncthreads();
        if (tid < 256 && s_cnt[tid] > 0u) atomicMin(&s_top, (uint32_t)tid);
        __syncthreads();
        if (tid == 0) {
            const uint32_t top = s_top;
            uint32_t k = 0;
            // only when the longest tile outlasts the balanced share of the
            // work: kSplitLoad x its work x the CUs against the total
            const bool tail = (uint64_t)s_wmax * (uint64_t)max(cus, 1) * kSplitLoad >= s_sum;
            if (tail && top < 256u && 255u - top >= work_bucket(kSplitMinWork))
                k = min(s_cnt[min(top + kSplitBuckets, 255u)], (uint32_t)split_max);
            order[T] = k;
        }
    }
}

// Splitting the backward's longest tiles in two (on unless GSR_BWD_SPLIT=0;
// read on every call, so a test can compare both).
bool bwd_split() {
    const char* v = std::getenv("GSR_BWD_SPLIT");
    return !(v && v[0] == '0');
}

// Per-device launch facts, looked up once per device and kept in a fixed
// table (no allocation after the first call): the compute units, and how many
// work-groups of the 64-entry-batch backward kernel fit on the device at once.
constexpr int kMaxDevices = 64;
struct DeviceFacts {
    int cus = 0;
    unsigned bwd_resident = 0;
};
DeviceFacts device_facts() {
    static std::mutex mu;
    static DeviceFacts table[kMaxDevices];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return DeviceFacts{1, 1};
    std::lock_guard<std::mutex> lock(mu);
    DeviceFacts& f = table[dev];
    if (f.cus == 0) {
        int per_cu = 0, cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess ||
            hipOccupancyMaxActiveBlocksPerMultiprocessor(
                &per_cu, reinterpret_cast<const void*>(&blend_bwd_kernel<2, 64, false>),
                Layout<2>::kThreads, 0) != hipSuccess)
            return DeviceFacts{1, 1};
        f.cus = std::max(1, cus);
        f.bwd_resident = (unsigned)std::max(1, per_cu * f.cus);
    }
    return f;
}

int cu_count() { return device_facts().cus; }

// Whether the backward's whole grid of tiles is resident on the device at once.
bool bwd_grid_fits(unsigned tiles) { return tiles <= device_facts().bwd_resident; }

// Lists that average this many entries per tile or more (the screen bands of
// config c5 average ~350k) are walked like a resident grid's: 128-entry
// batches with the longest tiles split.  Their longest tiles set the kernel's
// length there (c5: blend_bwd 8.0 ms per frame with 64-entry batches, 5.5 with
// 128, 4.5 with 128 and the split), while at 1080p (1.6k entries per tile) the
// 64-entry batch without the split stays ahead (251 us against 259).
constexpr uint64_t kLongListAvg = 32768;
bool bwd_long_lists(unsigned tiles, uint64_t pairs) {
    return pairs >= kLongListAvg * (uint64_t)tiles;
}

// Whether the backward walks 128-entry batches and may split long tiles.
bool bwd_wide(unsigned tiles, uint64_t pairs) {
    return bwd_grid_fits(tiles) || bwd_long_lists(tiles, pairs);
}

}  // namespace

hipError_t launch_fwd_schedule(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                               uint64_t m, const void* recs, uint32_t* work, uint32_t* order,
                               hipStream_t st) {
    const int tiles_x = (W + kTileSize - 1) / kTileSize;
    const unsigned tiles = (unsigned)(tiles_x * ((H + kTileSize - 1) / kTileSize));
    if (tiles == 0) return hipSuccess;
    const auto* r = reinterpret_cast<const int2*>(ranges);
    hipLaunchKernelGGL(tile_work_fwd_kernel,
                       dim3((tiles + kEstTilesPerBlock - 1) / kEstTilesPerBlock),
                       dim3(kEstTilesPerBlock * kWave), 0, st, (int)tiles, tiles_x, n, m, r, ids,
                       static_cast<const BlendRec*>(recs), work);
    hipLaunchKernelGGL(tile_order_kernel, dim3(1), dim3(kOrderThreads), 0, st, (int)tiles, m, r,
                       work, order, -1, 1);
    return hipGetLastError();
}

hipError_t launch_blend_fwd(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                            uint64_t m, const void* recs, float* img, float* finalT,
                            int32_t* ncontrib, const uint32_t* order, hipStream_t st) {
    const int tiles_x = (W + kTileSize - 1) / kTileSize;
    const int tiles_y = (H + kTileSize - 1) / kTileSize;
    const unsigned tiles = (unsigned)(tiles_x * tiles_y);
    if (tiles == 0) return hipSuccess;
    const auto* r = reinterpret_cast<const int2*>(ranges);
    const auto* rc = static_cast<const BlendRec*>(recs);
    // Two pixels per lane share each entry's record reads, column terms and
    // loop, which pays when the total work sets the kernel's length (1080p:
    // 135.4 -> 129.6 us).  Where the longest tiles set it (a grid resident at
    // once, or lists averaging 32k entries per tile), one pixel per lane in
    // four 16x4 strips culls finer and exits sooner per wave (720p bench frame
    // 0.4615 ms with two pixels per lane against 0.430; c5's blend_fwd 4.86
    // against 4.3 ms per frame).
    if (bwd_wide(tiles, m))
        hipLaunchKernelGGL(blend_fwd_kernel<1>, dim3(tiles), dim3(Layout<1>::kThreads), 0, st,
                           n, H, W, tiles_x, m, r, ids, rc, img, finalT, ncontrib, order);
    else
        hipLaunchKernelGGL(blend_fwd_kernel<2>, dim3(tiles), dim3(Layout<2>::kThreads), 0, st,
                           n, H, W, tiles_x, m, r, ids, rc, img, finalT, ncontrib, order);
    return hipGetLastError();
}

hipError_t launch_bwd_schedule(int H, int W, const int32_t* ranges, uint64_t num_pairs,
                               const int32_t* ncontrib, uint32_t* work, uint32_t* order,
                               hipStream_t st, bool work_ready) {
    const int tiles_x = (W + kTileSize - 1) / kTileSize;
    const unsigned tiles = (unsigned)(tiles_x * ((H + kTileSize - 1) / kTileSize));
    if (tiles == 0) return hipSuccess;
    const auto* r = reinterpret_cast<const int2*>(ranges);
    if (!work_ready)
        hipLaunchKernelGGL(tile_work_bwd_kernel,
                           dim3((tiles + kWorkTilesPerBlock - 1) / kWorkTilesPerBlock),
                           dim3(kWorkTilesPerBlock * kWave), 0, st,
                           make_bwd_work(H, W, ranges, num_pairs, ncontrib, work));
    hipLaunchKernelGGL(tile_order_kernel, dim3(1), dim3(kOrderThreads), 0, st, (int)tiles,
                       num_pairs, r, work, order,
                       (bwd_split() && bwd_wide(tiles, num_pairs)) ? kSplitMax : 0,
                       cu_count());
    return hipGetLastError();
}

hipError_t launch_blend_bwd(int n, int H, int W, const float* grad, const GradStrides& gst,
                            const int32_t* ranges,
                            const int32_t* ids, uint64_t num_pairs, const void* recs,
                            const float* finalT, const int32_t* ncontrib, float* dmean,
                            float* dcov, float* dcol, float* dalpha, const GradSlots& gs,
                            const uint32_t* order, hipStream_t st) {
    const int tiles_x = (W + kTileSize - 1) / kTileSize;
    const int tiles_y = (H + kTileSize - 1) / kTileSize;
    const unsigned tiles = (unsigned)(tiles_x * tiles_y);
    if (tiles == 0) return hipSuccess;
    const auto* r = reinterpret_cast<const int2*>(ranges);
    const auto* rc = static_cast<const BlendRec*>(recs);
    // With a schedule and the whole grid resident at once, or lists long
    // enough that the longest tiles set the kernel's length, up to kSplitMax
    // of the longest run as two items each.  Otherwise the total work does,
    // and the split's extra state-only walk costs more than it saves.
    const bool wide = bwd_wide(tiles, num_pairs);
    const bool split = order && bwd_split() && wide;
    // The 64-entry batch halves the work-group's LDS (8 KB), so registers, not
    // LDS, bound the resident waves; it pays when the grid does not fit on the
    // device at once.  When it would, the 128-entry batch leaves part of the
    // grid to be placed as CUs free up, which balances the long tiles better.
    if (!wide)
        hipLaunchKernelGGL((blend_bwd_kernel<2, 64, false>), dim3(tiles),
                           dim3(Layout<2>::kThreads), 0, st, n, H, W, tiles_x, num_pairs, grad, gst,
                           r, ids, rc, finalT, ncontrib, dmean, dcov, dcol, dalpha, gs, order);
    else if (split)
        hipLaunchKernelGGL((blend_bwd_kernel<2, 128, true>), dim3(tiles + kSplitMax),
                           dim3(Layout<2>::kThreads), 0, st, n, H, W, tiles_x, num_pairs, grad, gst,
                           r, ids, rc, finalT, ncontrib, dmean, dcov, dcol, dalpha, gs, order);
    else
        hipLaunchKernelGGL((blend_bwd_kernel<2, 128, false>), dim3(tiles),
                           dim3(Layout<2>::kThreads), 0, st, n, H, W, tiles_x, num_pairs, grad, gst,
                           r, ids, rc, finalT, ncontrib, dmean, dcov, dcol, dalpha, gs, order);
    return hipGetLastError();
}

hipError_t launch_pair_grad_reduce(int n, const GradSlots& gs, float* dmean, float* dcov,
                                   float* dcol, float* dalpha, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    // 8-lane rows when a Gaussian averages at most 64 slots (one flag load per
    // lane); word-sized flag groups beyond 256 slots per Gaussian
    if (gs.slots <= 64ull * (uint64_t)n)
        hipLaunchKernelGGL((pair_grad_reduce_kernel<8, 8>), dim3((unsigned)((n + 31) / 32)),
                           dim3(256), 0, st, n, gs, dmean, dcov, dcol, dalpha);
    else if (gs.slots <= 256ull * (uint64_t)n)
        hipLaunchKernelGGL((pair_grad_reduce_kernel<16, 8>), dim3((unsigned)((n + 15) / 16)),
                           dim3(256), 0, st, n, gs, dmean, dcov, dcol, dalpha);
    else
        hipLaunchKernelGGL((pair_grad_reduce_kernel<16, 64>), dim3((unsigned)((n + 15) / 16)),
                           dim3(256), 0, st, n, gs, dmean, dcov, dcol, dalpha);
    return hipGetLastError();
}

}  // namespace gsr
