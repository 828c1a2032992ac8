// gsr_adc.hip — adaptive density control (gaussian_splatting/utils/adc.py of
// kmurungi/custom-3dgs-cuda): the per-step densification statistics
// (:58-87) and the densify / prune pass (:209-294, :316-393) with the
// optimizer state carried along (:122-165).
//
// The reference runs the pass as a chain of torch ops: clone (concatenate the
// selected), split (concatenate two perturbed copies, then drop the
// originals), prune (boolean masks), each rebuilding every parameter and both
// Adam moments.  Here every output slot of the final cloud is known from each
// source Gaussian's own data, so the pass is one plan kernel, one scan and one
// gather:
//   plan:    per Gaussian, the densify decision (clone / split from the mean
//            gradient norm and the largest scale) and, for each copy it would
//            put in the cloud (itself unless split, its clone, its two split
//            copies), the prune decision as the reference takes it on the
//            densified cloud: opacity below the floor, the largest scale above
//            a tenth of the scene, the screen radius above the cap (new
//            Gaussians start at radius 0); flags and per-block counts;
//   scan:    one work-group: block offsets of the five counts (kept
//            originals, kept clones, kept split copies, all split sources,
//            for the noise rows) and their totals;
//   gather:  each source writes its kept copies at their final positions:
//            [kept originals] [kept clones] [kept first split copies]
//            [kept second split copies], the reference's order.  Split copies
//            get mu + R(q) (z * exp(s)) with z the caller's N(0, 1) rows (the
//            reference's torch.normal draws) and log(exp(s) / 1.6); new
//            Gaussians' moments are zero; the opacity reset clamps the logits
//            and zeroes their moments.
// Decisions compare fp32 values against fp32 thresholds, as torch compares an
// fp32 tensor with a Python float.
#include <hip/hip_runtime.h>

#include <cfloat>

#include "gsr_common.h"
#include "gsr_internal.h"

namespace gsr {

namespace {

constexpr int kAdcThreads = 256;
// Elements per thread whose loads copy_rows issues together.
constexpr int kAdcUnroll = 4;

// flag bits of a source Gaussian
constexpr uint8_t kKeepOrig = 1, kKeepClone = 2, kKeepSplit = 4, kSplitSrc = 8, kCloneSrc = 16;
constexpr int kKinds = 5;

__device__ __forceinline__ bool isnan_f(float x) { return x != x; }

// torch.maximum (NaN propagates)
__device__ __forceinline__ float max_nan(float a, float b) {
    return (isnan_f(a) || isnan_f(b)) ? __builtin_nanf("") : fmaxf(a, b);
}

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + exp_gs(-x)); }

__global__ __launch_bounds__(kAdcThreads) void adc_stats_kernel(
    int n, const float* __restrict__ mg, float sx, float sy, int scale,
    const float* __restrict__ radii, float* __restrict__ accum, float* __restrict__ denom,
    float* __restrict__ maxr) {
    const int i = blockIdx.x * kAdcThreads + threadIdx.x;
    if (i >= n) return;
    if (mg) {
        float gx = mg[2 * (size_t)i], gy = mg[2 * (size_t)i + 1];
        if (scale) {
            gx = gx * sx;
            gy = gy * sy;
        }
        // torch's norm over the last dimension: squares summed in order
        const float nrm = sqrt_rn(gx * gx + gy * gy);
        if (nrm > 0.0f) {
            accum[i] = accum[i] + nrm;
            denom[i] = denom[i] + 1.0f;
        }
    }
    if (radii) maxr[i] = max_nan(maxr[i], radii[i]);
}

__device__ __forceinline__ float max3_nan(float a, float b, float c) {
    return max_nan(max_nan(a, b), c);
}

__device__ uint8_t adc_flags(int i, const AdcCloud& in, const float* __restrict__ accum,
                             const float* __restrict__ denom, const float* __restrict__ maxr,
                             const AdcConfig& c) {
    // grads = nan_to_num(accum / denom.clamp_min(1), nan=0) (adc.py:345-346)
    const float d = denom[i];
    float g = accum[i] / (isnan_f(d) ? d : fmaxf(d, 1.0f));
    g = isnan_f(g) ? 0.0f : fminf(fmaxf(g, -FLT_MAX), FLT_MAX);
    const float* s = in.p[2] + 3 * (size_t)i;
    const float e0 = exp_gs(s[0]), e1 = exp_gs(s[1]), e2 = exp_gs(s[2]);
    const float smax = max3_nan(e0, e1, e2);
    const bool big = g >= c.grad_threshold;
    const bool clone = c.densify && big && smax <= c.dense_scale;
    const bool split = c.densify && big && smax > c.dense_scale;
    // the prune test of a copy with largest scale sm and screen radius r
    const float op = sigmoid_f(in.p[3][i]);
    auto pruned = [&](float sm, float r) {
        return c.prune && (op < c.min_opacity || sm > c.max_scale ||
                           (c.has_screen && r > c.max_screen));
    };
    uint8_t f = 0;
    if (!split && !pruned(smax, maxr ? maxr[i] : 0.0f)) f |= kKeepOrig;
    if (clone) f |= kCloneSrc;
    if (clone && !pruned(smax, 0.0f)) f |= kKeepClone;
    if (split) {
        f |= kSplitSrc;
        // the copies' log-scales log(exp(s) / 1.6), and the scales the
        // reference's prune then takes as exp of those
        const float t0 = exp_gs(logf(e0 / c.split_scale)), t1 = exp_gs(logf(e1 / c.split_scale)),
                    t2 = exp_gs(logf(e2 / c.split_scale));
        if (!pruned(max3_nan(t0, t1, t2), 0.0f)) f |= kKeepSplit;
    }
    return f;
}

// Per-block counts of kept originals, kept clones, kept split sources, all
// split sources and all clone sources (counts[block][kKinds]).
__global__ __launch_bounds__(kAdcThreads) void adc_plan_kernel(
    int n, AdcCloud in, const float* __restrict__ accum, const float* __restrict__ denom,
    const float* __restrict__ maxr, AdcConfig c, uint8_t* __restrict__ flags,
    uint32_t* __restrict__ counts) {
    __shared__ uint32_t s_c[kKinds][kAdcThreads / kWave];
    const int i = blockIdx.x * kAdcThreads + threadIdx.x;
    uint8_t f = 0;
    if (i < n) {
        f = adc_flags(i, in, accum, denom, maxr, c);
        flags[i] = f;
    }
    const int w = threadIdx.x / kWave;
#pragma unroll
    for (int k = 0; k < kKinds; ++k) {
        const uint32_t cnt = (uint32_t)popc64(ballot((f >> k) & 1));
        if ((threadIdx.x & (kWave - 1)) == 0) s_c[k][w] = cnt;
    }
    __syncthreads();
    if (threadIdx.x < kKinds) {
        uint32_t t = 0;
        for (int j = 0; j < kAdcThreads / kWave; ++j) t += s_c[threadIdx.x][j];
        counts[kKinds * (size_t)blockIdx.x + threadIdx.x] = t;
    }
}

// Exclusive scan of the blocks' counts, per kind, in place; totals[kKinds].
__global__ __launch_bounds__(1024) void adc_scan_kernel(int blocks, uint32_t* __restrict__ counts,
                                                       uint64_t* __restrict__ totals) {
    __shared__ uint32_t s_part[kKinds][1024];
    const int tid = threadIdx.x;
    // each thread a contiguous run of blocks
    const int per = (blocks + 1023) / 1024;
    const int b0 = min(blocks, tid * per), b1 = min(blocks, b0 + per);
    uint32_t sum[kKinds] = {0, 0, 0, 0, 0};
    for (int b = b0; b < b1; ++b)
        for (int k = 0; k < kKinds; ++k) sum[k] += counts[kKinds * (size_t)b + k];
    for (int k = 0; k < kKinds; ++k) s_part[k][tid] = sum[k];
    __syncthreads();
    if (tid < kKinds) {
        uint32_t run = 0;
        for (int j = 0; j < 1024; ++j) {
            const uint32_t v = s_part[tid][j];
            s_part[tid][j] = run;
            run += v;
        }
        totals[tid] = run;
    }
    __syncthreads();
    uint32_t run[kKinds];
    for (int k = 0; k < kKinds; ++k) run[k] = s_part[k][tid];
    for (int b = b0; b < b1; ++b)
        for (int k = 0; k < kKinds; ++k) {
            const uint32_t v = counts[kKinds * (size_t)b + k];
            counts[kKinds * (size_t)b + k] = run[k];
            run[k] += v;
        }
}

// Destinations of a block's Gaussians in the new cloud (row indices, or
// kNoRow): itself, its clone, its two split copies.
constexpr uint32_t kNoRow = 0xffffffffu;

// Copies one [N, W] array of the block's Gaussians to their destinations,
// element-parallel: the block's source rows are contiguous, so the loads are
// coalesced, and each destination kind's rows are contiguous too (the order
// is kept), so are the stores up to the dropped rows.  mode 0: a parameter
// (every destination gets the value; with `skip_split` the split copies are
// left to the caller; with `clamp` the value is min(v, clamp_hi), NaN kept);
// mode 1: a moment (the Gaussian's own row gets the value, new rows zero;
// `zero_all` zeroes every row).
template <int W>
__device__ __forceinline__ void copy_rows(const float* __restrict__ src, float* __restrict__ dst,
                                          int g0, int cnt, const uint32_t (*s_dst)[kAdcThreads],
                                          int mode, bool skip_split, bool clamp, float clamp_hi,
                                          bool zero_all) {
    const float* sp = src ? src + (size_t)g0 * W : nullptr;
    const int total = cnt * W;
    // kAdcUnroll elements per thread and step, their loads issued together
    for (int e0 = threadIdx.x; e0 < total; e0 += kAdcUnroll * kAdcThreads) {
        float v[kAdcUnroll];
#pragma unroll
        for (int u = 0; u < kAdcUnroll; ++u) {
            const int e = e0 + u * kAdcThreads;
            v[u] = (sp && e < total) ? sp[e] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < kAdcUnroll; ++u) {
            const int e = e0 + u * kAdcThreads;
            if (e >= total) break;
            const int g = e / W, k = e - g * W;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint32_t row = s_dst[d][g];
                if (row == kNoRow) continue;
                if (mode == 0) {
                    if (skip_split && d >= 2) continue;
                    float x = v[u];
                    if (clamp) x = isnan_f(x) ? x : fminf(x, clamp_hi);
                    dst[(size_t)row * W + k] = x;
                } else {
                    dst[(size_t)row * W + k] = (d == 0 && !zero_all) ? v[u] : 0.0f;
                }
            }
        }
    }
}

__global__ __launch_bounds__(kAdcThreads) void adc_gather_kernel(
    int n, AdcCloud in, AdcMoments min_, const uint8_t* __restrict__ flags,
    const uint32_t* __restrict__ offs, const uint64_t* __restrict__ totals,
    const float* __restrict__ noise, AdcConfig c, AdcCloud out, AdcMoments mout) {
    __shared__ uint32_t s_w[4][kAdcThreads / kWave];
    __shared__ uint32_t s_dst[4][kAdcThreads];
    const int g0 = blockIdx.x * kAdcThreads;
    const int cnt = min(kAdcThreads, n - g0);
    const int i = g0 + threadIdx.x;
    const uint8_t f = (i < n) ? flags[i] : 0;
    const int w = threadIdx.x / kWave;
    uint32_t rank[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint64_t b = ballot((f >> k) & 1);
        rank[k] = (uint32_t)popc64(b & lanemask_lt());
        if ((threadIdx.x & (kWave - 1)) == 0) s_w[k][w] = (uint32_t)popc64(b);
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t pre = offs[kKinds * (size_t)blockIdx.x + k];
        for (int j = 0; j < w; ++j) pre += s_w[k][j];
        rank[k] += pre;
    }
    const uint64_t n_orig = totals[0], n_clone = totals[1], n_split = totals[2];
    const uint64_t n_src = totals[3];
    s_dst[0][threadIdx.x] = (f & kKeepOrig) ? (uint32_t)rank[0] : kNoRow;
    s_dst[1][threadIdx.x] = (f & kKeepClone) ? (uint32_t)(n_orig + rank[1]) : kNoRow;
    s_dst[2][threadIdx.x] = (f & kKeepSplit) ? (uint32_t)(n_orig + n_clone + rank[2]) : kNoRow;
    s_dst[3][threadIdx.x] =
        (f & kKeepSplit) ? (uint32_t)(n_orig + n_clone + n_split + rank[2]) : kNoRow;
    __syncthreads();
    if (cnt <= 0) return;
    const bool reset = c.reset_opacity != 0;
    // the parameters (the split copies' mu and s below), then the moments
    copy_rows<3>(in.p[0], out.p[0], g0, cnt, s_dst, 0, true, false, 0.0f, false);
    copy_rows<4>(in.p[1], out.p[1], g0, cnt, s_dst, 0, false, false, 0.0f, false);
    copy_rows<3>(in.p[2], out.p[2], g0, cnt, s_dst, 0, true, false, 0.0f, false);
    copy_rows<1>(in.p[3], out.p[3], g0, cnt, s_dst, 0, false, reset, c.reset_logit, false);
    copy_rows<3>(in.p[4], out.p[4], g0, cnt, s_dst, 0, false, false, 0.0f, false);
    copy_rows<45>(in.p[5], out.p[5], g0, cnt, s_dst, 0, false, false, 0.0f, false);
    for (int m = 0; m < 2; ++m) {
        const int o = 6 * m;
        if (mout.p[o + 0]) copy_rows<3>(min_.p[o + 0], mout.p[o + 0], g0, cnt, s_dst, 1, false, false, 0.0f, false);
        if (mout.p[o + 1]) copy_rows<4>(min_.p[o + 1], mout.p[o + 1], g0, cnt, s_dst, 1, false, false, 0.0f, false);
        if (mout.p[o + 2]) copy_rows<3>(min_.p[o + 2], mout.p[o + 2], g0, cnt, s_dst, 1, false, false, 0.0f, false);
        if (mout.p[o + 3]) copy_rows<1>(min_.p[o + 3], mout.p[o + 3], g0, cnt, s_dst, 1, false, false, 0.0f, reset);
        if (mout.p[o + 4]) copy_rows<3>(min_.p[o + 4], mout.p[o + 4], g0, cnt, s_dst, 1, false, false, 0.0f, false);
        if (mout.p[o + 5]) copy_rows<45>(min_.p[o + 5], mout.p[o + 5], g0, cnt, s_dst, 1, false, false, 0.0f, false);
    }
    if (i >= n) return;
    // the kept original's and clone's mu and s were copied above; the split
    // copies' are the perturbed ones
    if (f & kKeepSplit) {
        const float* q = in.p[1] + 4 * (size_t)i;
        const float* sv = in.p[2] + 3 * (size_t)i;
        const float* mu = in.p[0] + 3 * (size_t)i;
        // R of the normalized quaternion (adc.py:103-119: F.normalize, eps
        // 1e-12, then the rotation matrix)
        const float len = fmaxf(
            sqrt_rn(((q[0] * q[0] + q[1] * q[1]) + q[2] * q[2]) + q[3] * q[3]), 1e-12f);
        const float qw = q[0] / len, qx = q[1] / len, qy = q[2] / len, qz = q[3] / len;
        const float r[3][3] = {
            {1.0f - 2.0f * (qy * qy + qz * qz), 2.0f * (qx * qy - qw * qz),
             2.0f * (qx * qz + qw * qy)},
            {2.0f * (qx * qy + qw * qz), 1.0f - 2.0f * (qx * qx + qz * qz),
             2.0f * (qy * qz - qw * qx)},
            {2.0f * (qx * qz - qw * qy), 2.0f * (qy * qz + qw * qx),
             1.0f - 2.0f * (qx * qx + qy * qy)}};
        const float sc[3] = {exp_gs(sv[0]), exp_gs(sv[1]), exp_gs(sv[2])};
        for (int copy = 0; copy < 2; ++copy) {
            const size_t d = (size_t)s_dst[2 + copy][threadIdx.x];
            // the split source's noise row: copy k of source j is row k n_src + j
            const float* z = noise + 3 * ((size_t)copy * n_src + rank[3]);
            float smp[3];
            for (int a = 0; a < 3; ++a) smp[a] = z[a] * sc[a];
            float* om = out.p[0] + 3 * d;
            float* os = out.p[2] + 3 * d;
            for (int a = 0; a < 3; ++a) {
                om[a] = ((r[a][0] * smp[0] + r[a][1] * smp[1]) + r[a][2] * smp[2]) + mu[a];
                os[a] = logf(sc[a] / c.split_scale);
            }
        }
    }
}

}  // namespace

hipError_t launch_adc_stats(int n, const float* mean2d_grad, float sx, float sy, int scale,
                            const float* radii, float* accum, float* denom, float* maxr,
                            hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(adc_stats_kernel, dim3((unsigned)((n + kAdcThreads - 1) / kAdcThreads)),
                       dim3(kAdcThreads), 0, st, n, mean2d_grad, sx, sy, scale, radii, accum,
                       denom, maxr);
    return hipGetLastError();
}

size_t adc_workspace_bytes(int n) {
    const size_t blocks = (size_t)(n + kAdcThreads - 1) / kAdcThreads;
    return 256 + ((size_t)n + 255) / 256 * 256 + blocks * 4 * kKinds;
}

hipError_t launch_adc_plan(int n, const AdcCloud& in, const float* accum, const float* denom,
                           const float* maxr, const AdcConfig& c, void* ws, uint64_t* totals_dev,
                           hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n + kAdcThreads - 1) / kAdcThreads);
    char* base = static_cast<char*>(ws);
    uint8_t* flags = reinterpret_cast<uint8_t*>(base + 256);
    uint32_t* counts = reinterpret_cast<uint32_t*>(base + 256 + ((size_t)n + 255) / 256 * 256);
    hipLaunchKernelGGL(adc_plan_kernel, dim3(blocks), dim3(kAdcThreads), 0, st, n, in, accum,
                       denom, maxr, c, flags, counts);
    hipLaunchKernelGGL(adc_scan_kernel, dim3(1), dim3(1024), 0, st, (int)blocks, counts,
                       totals_dev);
    return hipGetLastError();
}

hipError_t launch_adc_gather(int n, const AdcCloud& in, const AdcMoments& min_,
                             const float* noise, const AdcConfig& c, const void* ws,
                             const uint64_t* totals_dev, const AdcCloud& out,
                             const AdcMoments& mout, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const unsigned blocks = (unsigned)((n + kAdcThreads - 1) / kAdcThreads);
    const char* base = static_cast<const char*>(ws);
    const uint8_t* flags = reinterpret_cast<const uint8_t*>(base + 256);
    const uint32_t* offs =
        reinterpret_cast<const uint32_t*>(base + 256 + ((size_t)n + 255) / 256 * 256);
    hipLaunchKernelGGL(adc_gather_kernel, dim3(blocks), dim3(kAdcThreads), 0, st, n, in, min_,
                       flags, offs, totals_dev, noise, c, out, mout);
    return hipGetLastError();
}

}  // namespace gsr
