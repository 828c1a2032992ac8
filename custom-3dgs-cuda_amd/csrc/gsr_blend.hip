// gsr_blend.hip — front-to-back alpha blend (a8) and its backward (a10).
//
// One work-group per 16x16 tile, four wave64s, each wave owning an 8x8 pixel
// quadrant (compact quadrants let a whole wave finish together).  A batch of
// 256 list entries is staged in LDS as 48 B blend records (one coalesced
// record load per entry); every lane then walks the batch with broadcast LDS
// reads.  Per-pixel arithmetic is the reference's, operation for operation
// (rasterize.cu:241-270, rasterize_backward.cu:113-200).
//
// Forward early exit: a lane is done once T < 1e-4; a wave leaves the batch
// when its ballot of live lanes is empty; the tile stops when all 256 are done.
// Backward: the tile walks only entries [0, max n_contrib) of its list, back
// to front (the reference walks all K entries and skips the tail per pixel);
// each entry's 9 per-pixel gradient terms are summed across the wave (64 -> 1,
// one transposed permlane/DPP reduction), across the four waves through LDS,
// and then added to HBM with one set of 9 float atomics per (tile, entry).
#include "gsr_internal.h"
#include "gsr_common.h"

namespace gsr {

namespace {

constexpr int kThreads = 256;
constexpr int kBatch = 256;

struct PixelMap {
    int px, py;
    bool inside;
};

__device__ __forceinline__ PixelMap pixel_of(int tile, int tiles_x, int W, int H) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    PixelMap p;
    p.px = tx * kTileSize + (wave & 1) * 8 + (lane & 7);
    p.py = ty * kTileSize + (wave >> 1) * 8 + (lane >> 3);
    p.inside = p.px < W && p.py < H;
    return p;
}

__device__ __forceinline__ void clamp_range(int2 rg, uint64_t m, int& start, int& end) {
    const int64_t s = min<int64_t>(max<int64_t>(rg.x, 0), (int64_t)m);
    const int64_t e = min<int64_t>(max<int64_t>(rg.y, s), (int64_t)m);
    start = (int)s;
    end = (int)e;
}

__global__ __launch_bounds__(kThreads) void blend_fwd_kernel(
    int n, int H, int W, int tiles_x, uint64_t m, const int2* __restrict__ ranges,
    const int32_t* __restrict__ ids, const BlendRec* __restrict__ recs, float* __restrict__ img,
    float* __restrict__ finalT, int32_t* __restrict__ ncontrib) {
    __shared__ float4 s_a[kBatch];
    __shared__ float4 s_b[kBatch];
    __shared__ float4 s_c[kBatch];
    const int tile = blockIdx.x;
    const PixelMap pm = pixel_of(tile, tiles_x, W, H);
    const float fpx = (float)pm.px, fpy = (float)pm.py;
    int start, end;
    clamp_range(ranges[tile], m, start, end);

    float T = 1.0f, C0 = 0.0f, C1 = 0.0f, C2 = 0.0f;
    int last = 0;
    bool done = !pm.inside;
    const int tid = threadIdx.x;
    for (int b0 = start; b0 < end; b0 += kBatch) {
        const int cnt = min(kBatch, end - b0);
        __syncthreads();
        if (tid < cnt) {
            const int g = ids[b0 + tid];
            BlendRec r;
            if (g >= 0 && g < n) {
                r = recs[g];
            } else {  // ids come from the sort; a zero record is never blended
                r.a = r.b = r.c = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            s_a[tid] = r.a;
            s_b[tid] = r.b;
            s_c[tid] = r.c;
        }
        __syncthreads();
        if (ballot(!done) != 0) {
            const int cbase = b0 - start;
            for (int j = 0; j < cnt; ++j) {
                if (!done) {
                    const float4 A = s_a[j];
                    const float4 B = s_b[j];
                    const float dx = fpx - A.x;
                    const float dy = fpy - A.y;
                    const float power = -0.5f * (A.z * dx * dx + A.w * dx * dy + B.x * dy * dy);
                    if (!(power > 0.0f)) {
                        const float alpha = fminf(kAlphaMax, B.y * exp_gs(power));
                        if (!(alpha < kAlphaMin)) {
                            const float w = alpha * T;
                            C0 = C0 + B.z * w;
                            C1 = C1 + B.w * w;
                            C2 = C2 + s_c[j].x * w;
                            T = T * (1.0f - alpha);
                            last = cbase + j + 1;
                            if (T < kTransmittanceMin) done = true;
                        }
                    }
                }
                if (ballot(!done) == 0) break;
            }
        }
        if (__syncthreads_and(done)) break;
    }
    if (pm.inside) {
        const size_t p = (size_t)pm.py * W + pm.px;
        img[3 * p] = C0;
        img[3 * p + 1] = C1;
        img[3 * p + 2] = C2;
        finalT[p] = T;
        ncontrib[p] = last;
    }
}

__global__ __launch_bounds__(kThreads) void blend_bwd_kernel(
    int n, int H, int W, int tiles_x, uint64_t m, const float* __restrict__ grad,
    const int2* __restrict__ ranges, const int32_t* __restrict__ ids,
    const BlendRec* __restrict__ recs, const float* __restrict__ finalT,
    const int32_t* __restrict__ ncontrib, float* __restrict__ dmean, float* __restrict__ dcov,
    float* __restrict__ dcol, float* __restrict__ dalpha) {
    __shared__ float4 s_a[kBatch];
    __shared__ float4 s_b[kBatch];
    __shared__ float4 s_c[kBatch];
    __shared__ int s_id[kBatch];
    __shared__ float s_part[4][9][kBatch];
    __shared__ uint32_t s_max[4];

    const int tile = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const PixelMap pm = pixel_of(tile, tiles_x, W, H);
    const float fpx = (float)pm.px, fpy = (float)pm.py;
    int start, end;
    clamp_range(ranges[tile], m, start, end);

    float g0 = 0.0f, g1 = 0.0f, g2 = 0.0f, T = 0.0f;
    int last = 0;
    if (pm.inside) {
        const size_t p = (size_t)pm.py * W + pm.px;
        g0 = grad[3 * p];
        g1 = grad[3 * p + 1];
        g2 = grad[3 * p + 2];
        T = finalT[p];
        last = ncontrib[p];
    }
    const uint32_t wmax = wave_max_u32((uint32_t)max(last, 0));
    if (lane == 0) s_max[wave] = wmax;
    __syncthreads();
    const int maxc = min((int)max(max(s_max[0], s_max[1]), max(s_max[2], s_max[3])), end - start);

    float acc0 = 0.0f, acc1 = 0.0f, acc2 = 0.0f;
    const int my_value = reduce9_value_of_lane(lane);
    for (int hi = maxc; hi > 0; hi -= kBatch) {
        const int lo = max(0, hi - kBatch);
        const int cnt = hi - lo;
        __syncthreads();
        if (tid < cnt) {
            const int g = ids[start + lo + tid];
            const bool ok = g >= 0 && g < n;  // corrupt ids are skipped (rasterize_backward.cu:79-86)
            s_id[tid] = ok ? g : -1;
            BlendRec r;
            if (ok) {
                r = recs[g];
            } else {
                r.a = r.b = r.c = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
            s_a[tid] = r.a;
            s_b[tid] = r.b;
            s_c[tid] = r.c;
        }
        __syncthreads();
        for (int j = cnt - 1; j >= 0; --j) {
            const int contributor = lo + j + 1;
            // Branch-free form of the reference's per-pixel skips: an entry the
            // pixel did not blend (beyond n_contrib, power > 0, alpha < 1/255,
            // corrupt id) contributes zero terms and leaves T and the
            // background colour unchanged.
            const float4 A = s_a[j];
            const float4 B = s_b[j];
            const float4 Cc = s_c[j];
            const float dx = fpx - A.x;
            const float dy = fpy - A.y;
            const float power = -0.5f * (A.z * dx * dx + A.w * dx * dy + B.x * dy * dy);
            const float G = exp_gs(power);
            const float araw = B.y * G;
            const float alpha = fminf(kAlphaMax, araw);
            const bool id_ok = s_id[j] >= 0;
            const bool act = (contributor <= last) & id_ok & !(power > 0.0f) &
                             !(alpha < kAlphaMin);
            const float om = 1.0f - alpha;
            const float Tb = T / fmaxf(om, 1e-4f);
            const float aT = act ? alpha * Tb : 0.0f;
            const float dal =
                act ? ((B.z - acc0) * g0 + (B.w - acc1) * g1 + (Cc.x - acc2) * g2) * Tb : 0.0f;
            // alpha = min(0.99, o G): a clamped alpha passes no gradient to o or G
            const bool unclamped = araw < kAlphaMax;
            const float dop = unclamped ? G * dal : 0.0f;
            const float dpw = unclamped ? alpha * dal : 0.0f;
            const float cy = Cc.y;
            float v[9];
            v[0] = dpw * (A.z * dx + cy * dy);
            v[1] = dpw * (cy * dx + B.x * dy);
            v[2] = -0.5f * dpw * dx * dx;
            v[3] = -dpw * dx * dy;
            v[4] = -0.5f * dpw * dy * dy;
            v[5] = aT * g0;
            v[6] = aT * g1;
            v[7] = aT * g2;
            v[8] = dop;
            acc0 = act ? alpha * B.z + om * acc0 : acc0;
            acc1 = act ? alpha * B.w + om * acc1 : acc1;
            acc2 = act ? alpha * Cc.x + om * acc2 : acc2;
            T = act ? Tb : T;
            // Wave totals of the nine terms: one transposed reduction, then the
            // nine lanes that hold a total write it (zeros when no lane blended).
            const float w9 = (ballot(act) != 0) ? wave_reduce9(v) : 0.0f;
            if (my_value >= 0) s_part[wave][my_value][j] = w9;
        }
        __syncthreads();
        if (tid < cnt) {
            const int g = s_id[tid];
            if (g >= 0) {
                float t[9];
#pragma unroll
                for (int k = 0; k < 9; ++k)
                    t[k] = s_part[0][k][tid] + s_part[1][k][tid] + s_part[2][k][tid] +
                           s_part[3][k][tid];
                // conic gradient -> covariance gradient (rasterize_backward.cu:211-221)
                const float vx = s_a[tid].z, vy = s_c[tid].y, vz = s_b[tid].x;
                const float gx = t[2], gy = 0.5f * t[3], gz = t[4];
                const float dA = -(vx * vx * gx + 2.0f * vx * vy * gy + vy * vy * gz);
                const float dB = -2.0f * (vx * vy * gx + (vx * vz + vy * vy) * gy + vy * vz * gz);
                const float dC = -(vy * vy * gx + 2.0f * vy * vz * gy + vz * vz * gz);
                unsafeAtomicAdd(&dmean[2 * (size_t)g], t[0]);
                unsafeAtomicAdd(&dmean[2 * (size_t)g + 1], t[1]);
                unsafeAtomicAdd(&dcov[3 * (size_t)g], dA);
                unsafeAtomicAdd(&dcov[3 * (size_t)g + 1], dB);
                unsafeAtomicAdd(&dcov[3 * (size_t)g + 2], dC);
                unsafeAtomicAdd(&dcol[3 * (size_t)g], t[5]);
                unsafeAtomicAdd(&dcol[3 * (size_t)g + 1], t[6]);
                unsafeAtomicAdd(&dcol[3 * (size_t)g + 2], t[7]);
                unsafeAtomicAdd(&dalpha[g], t[8]);
            }
        }
    }
}

}  // namespace

hipError_t launch_blend_fwd(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                            uint64_t m, const void* recs, float* img, float* finalT,
                            int32_t* ncontrib, hipStream_t st) {
    const int tiles_x = (W + kTileSize - 1) / kTileSize;
    const int tiles_y = (H + kTileSize - 1) / kTileSize;
    const unsigned tiles = (unsigned)(tiles_x * tiles_y);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(blend_fwd_kernel, dim3(tiles), dim3(kThreads), 0, st, n, H, W, tiles_x, m,
                       reinterpret_cast<const int2*>(ranges), ids,
                       static_cast<const BlendRec*>(recs), img, finalT, ncontrib);
    return hipGetLastError();
}

hipError_t launch_blend_bwd(int n, int H, int W, const float* grad, const int32_t* ranges,
                            const int32_t* ids, uint64_t num_pairs, const void* recs,
                            const float* finalT, const int32_t* ncontrib, float* dmean,
                            float* dcov, float* dcol, float* dalpha, hipStream_t st) {
    const int tiles_x = (W + kTileSize - 1) / kTileSize;
    const int tiles_y = (H + kTileSize - 1) / kTileSize;
    const unsigned tiles = (unsigned)(tiles_x * tiles_y);
    if (tiles == 0) return hipSuccess;
    hipLaunchKernelGGL(blend_bwd_kernel, dim3(tiles), dim3(kThreads), 0, st, n, H, W, tiles_x,
                       num_pairs, grad, reinterpret_cast<const int2*>(ranges), ids,
                       static_cast<const BlendRec*>(recs), finalT, ncontrib, dmean, dcov, dcol,
                       dalpha);
    return hipGetLastError();
}

}  // namespace gsr
