// gsr_loss.hip — the trainer's reconstruction loss
// (gaussian_splatting/utils/loss.py:12-33 of kmurungi/custom-3dgs-cuda):
//   loss = (1 - lambda) mean|gt - img| + lambda (1 - SSIM(clamp(img), clamp(gt)))
// with the SSIM of torchmetrics (>= 1.0, the reference's requirement; not
// vendored): an 11x11 Gaussian window of sigma 1.5 normalised to sum 1,
// C1 = (0.01)^2, C2 = (0.03)^2 for data range 1, per-window statistics
// sigma_x^2 = max(E[x^2] - mu_x^2, 0) (torchmetrics clamps both variances at 0
// since its releases after 1.0) and sigma_xy = E[xy] - mu_x mu_y, averaged over
// the windows whose 11x11 support lies inside the image (torchmetrics pads by
// reflection and crops the 5-pixel margin of the index map, which leaves
// exactly those windows) and over the 3 channels.  Images are [H, W, 3] fp32.
//
// Two kernels, each one pass over HBM with LDS-staged 2D tiles:
//   ssim_fwd_kernel   per 32x16 tile: the tile and its 5-pixel halo of both
//                     images into LDS (one coalesced sweep of the interleaved
//                     channels), a horizontal then a vertical 11-tap pass for
//                     the five window moments, the SSIM index, and per window
//                     the three partial derivatives of the index with respect
//                     to mu_x, E[x^2] and E[xy] (stored for the backward);
//                     per-work-group sums of the index and of |gt - img|;
//   ssim_bwd_kernel   per tile: the derivative maps and their halo into LDS,
//                     their 11x11 window sums (the window is symmetric, so the
//                     adjoint of the moments' blur is the same blur), and
//                     dL/dimg = g ((1 - lambda)/(3HW) sgn(img - gt)
//                               - lambda/(3 n_win) [clamp mask] (B1 + 2 x B2 + y B3)).
// Only the loss's own arithmetic is fp32-tolerance work: the convolutions use
// fused multiply-adds.
#include <hip/hip_runtime.h>

#include <cmath>

#include "gsr_common.h"
#include "gsr_internal.h"

namespace gsr {

namespace {

constexpr int kLossTW = 32, kLossTH = 16;  // output tile (columns x rows)
constexpr int kWinR = 5;                   // window radius: 11 taps
constexpr int kWinTaps = 2 * kWinR + 1;
constexpr int kInW = kLossTW + 2 * kWinR, kInH = kLossTH + 2 * kWinR;  // 42 x 26
constexpr int kLossThreads = 256;
constexpr int kRowElems = kInW * 3;                // floats of one halo row
constexpr int kHaloElems = kInH * kRowElems;       // floats of a tile + halo
constexpr int kHaloIters = (kHaloElems + kLossThreads - 1) / kLossThreads;
constexpr float kC1 = 0.01f * 0.01f, kC2 = 0.03f * 0.03f;

struct Window {
    float w[kWinTaps];
};

// torch.clamp(v, 0, 1): NaN stays NaN.
__device__ __forceinline__ float clamp01(float v) { return v < 0.0f ? 0.0f : (v > 1.0f ? 1.0f : v); }

// Windows whose support lies inside the image: centres in [5, H - 5) x [5, W - 5).
__device__ __forceinline__ bool interior(int y, int x, int H, int W) {
    return y >= kWinR && y < H - kWinR && x >= kWinR && x < W - kWinR;
}

__global__ __launch_bounds__(kLossThreads) void ssim_fwd_kernel(
    int H, int W, const float* __restrict__ img, const float* __restrict__ gt, Window win,
    float* __restrict__ gmaps, float2* __restrict__ partial) {
#pragma clang fp contract(fast)
    __shared__ float s_x[3][kInH][kInW];
    __shared__ float s_y[3][kInH][kInW];
    __shared__ float s_h[5][kInH][kLossTW];
    __shared__ float s_red[2][kLossThreads / kWave];
    const int tid = threadIdx.x;
    const int x0 = blockIdx.x * kLossTW, y0 = blockIdx.y * kLossTH;
    const size_t plane = (size_t)H * W * 3;

    // the tile and its halo, channels interleaved as in HBM, every thread's
    // loads issued together; |gt - img| of the tile's own pixels on the way
    float l1 = 0.0f;
    {
        float xv[kHaloIters], yv[kHaloIters];
#pragma unroll
        for (int it = 0; it < kHaloIters; ++it) {
            const int e = tid + it * kLossThreads;
            const int r = e / kRowElems, q = e - r * kRowElems;
            const int gy = y0 - kWinR + r, gx = x0 - kWinR + q / 3;
            const bool in = e < kHaloElems && gy >= 0 && gy < H && gx >= 0 && gx < W;
            const size_t idx = (size_t)gy * W * 3 + (size_t)(x0 - kWinR) * 3 + q;
            xv[it] = in ? img[idx] : 0.0f;
            yv[it] = in ? gt[idx] : 0.0f;
        }
#pragma unroll
        for (int it = 0; it < kHaloIters; ++it) {
            const int e = tid + it * kLossThreads;
            if (e >= kHaloElems) continue;
            const int r = e / kRowElems, q = e - r * kRowElems;
            const int cx = q / 3, ch = q - cx * 3;
            if (r >= kWinR && r < kWinR + kLossTH && cx >= kWinR && cx < kWinR + kLossTW)
                l1 += fabsf(yv[it] - xv[it]);
            s_x[ch][r][cx] = clamp01(xv[it]);
            s_y[ch][r][cx] = clamp01(yv[it]);
        }
    }
    __syncthreads();

    float ssum = 0.0f;
    const int vc = tid & (kLossTW - 1), vr = 2 * (tid / kLossTW);  // 2 window rows per thread
    for (int ch = 0; ch < 3; ++ch) {
        // horizontal pass: the five moments of 11 columns, for every halo row
        for (int t = tid; t < kInH * kLossTW; t += kLossThreads) {
            const int r = t / kLossTW, c = t - r * kLossTW;
            float mx = 0.0f, my = 0.0f, xx = 0.0f, yy = 0.0f, xy = 0.0f;
#pragma unroll
            for (int k = 0; k < kWinTaps; ++k) {
                const float xv = s_x[ch][r][c + k], yv = s_y[ch][r][c + k], w = win.w[k];
                const float wx = w * xv, wy = w * yv;
                mx += wx;
                my += wy;
                xx += wx * xv;
                yy += wy * yv;
                xy += wx * yv;
            }
            s_h[0][r][c] = mx;
            s_h[1][r][c] = my;
            s_h[2][r][c] = xx;
            s_h[3][r][c] = yy;
            s_h[4][r][c] = xy;
        }
        __syncthreads();
        // vertical pass: two windows per thread, from 12 rows
        float m[2][5] = {};
#pragma unroll
        for (int k = 0; k < kWinTaps + 1; ++k) {
            float v[5];
#pragma unroll
            for (int i = 0; i < 5; ++i) v[i] = s_h[i][vr + k][vc];
            if (k < kWinTaps) {
#pragma unroll
                for (int i = 0; i < 5; ++i) m[0][i] += win.w[k] * v[i];
            }
            if (k >= 1) {
#pragma unroll
                for (int i = 0; i < 5; ++i) m[1][i] += win.w[k - 1] * v[i];
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int gy = y0 + vr + j, gx = x0 + vc;
            if (!interior(gy, gx, H, W)) continue;
            const float mux = m[j][0], muy = m[j][1];
            // the variances clamped at 0 (torch.clamp: NaN stays NaN)
            const float vxx = m[j][2] - mux * mux, vyy = m[j][3] - muy * muy;
            const float sxx = vxx < 0.0f ? 0.0f : vxx, syy = vyy < 0.0f ? 0.0f : vyy;
            const float sxy = m[j][4] - mux * muy;
            const float a1 = 2.0f * mux * muy + kC1, a2 = 2.0f * sxy + kC2;
            const float b1 = mux * mux + muy * muy + kC1, b2 = sxx + syy + kC2;
            const float rb1 = 1.0f / b1, rb2 = 1.0f / b2;
            const float inv = rb1 * rb2;
            const float s = a1 * a2 * inv;
            ssum += s;
            if (gmaps) {
                // dS/dA1 = a2 inv, dS/dA2 = a1 inv, dS/dB1 = -S / b1, dS/dB2 = -S / b2;
                // A1 = 2 mux muy + C1, A2 = 2 (E[xy] - mux muy) + C2,
                // B1 = mux^2 + muy^2 + C1, B2 = E[x^2] - mux^2 + E[y^2] - muy^2 + C2
                const float dA1 = a2 * inv, dA2 = a1 * inv, dB1 = -s * rb1, dB2 = -s * rb2;
                // the clamp of sigma_x^2 passes its gradient where sigma_x^2 >= 0
                const float dBx = (vxx >= 0.0f) ? dB2 : 0.0f;
                const float g1 = 2.0f * muy * (dA1 - dA2) + 2.0f * mux * (dB1 - dBx);
                const size_t idx = ((size_t)gy * W + gx) * 3 + ch;
                gmaps[idx] = g1;              // dS/dmu_x
                gmaps[plane + idx] = dBx;     // dS/dE[x^2]
                gmaps[2 * plane + idx] = 2.0f * dA2;  // dS/dE[xy]
            }
        }
        __syncthreads();  // s_h is rewritten for the next channel
    }
    const float ws = wave_sum(ssum), wl = wave_sum(l1);
    if ((tid & (kWave - 1)) == 0) {
        s_red[0][tid / kWave] = ws;
        s_red[1][tid / kWave] = wl;
    }
    __syncthreads();
    if (tid == 0) {
        float a = 0.0f, b = 0.0f;
        for (int w = 0; w < kLossThreads / kWave; ++w) {
            a += s_red[0][w];
            b += s_red[1][w];
        }
        partial[blockIdx.y * gridDim.x + blockIdx.x] = make_float2(a, b);
    }
}

// out[0] = loss, out[1] = SSIM, out[2] = mean |gt - img|, from the work-groups'
// partial sums (added in double, in work-group order: deterministic).
__global__ __launch_bounds__(kLossThreads) void loss_finalize_kernel(
    int parts, const float2* __restrict__ partial, double n_win, double n_px, float lambda,
    float* __restrict__ out) {
    __shared__ double s_a[kLossThreads], s_b[kLossThreads];
    const int tid = threadIdx.x;
    double a = 0.0, b = 0.0;
    for (int i = tid; i < parts; i += kLossThreads) {
        const float2 p = partial[i];
        a += (double)p.x;
        b += (double)p.y;
    }
    s_a[tid] = a;
    s_b[tid] = b;
    __syncthreads();
    for (int s = kLossThreads / 2; s > 0; s >>= 1) {
        if (tid < s) {
            s_a[tid] += s_a[tid + s];
            s_b[tid] += s_b[tid + s];
        }
        __syncthreads();
    }
    if (tid == 0) {
        const double ssim = s_a[0] / n_win, l1 = s_b[0] / n_px;
        out[0] = (float)((1.0 - (double)lambda) * l1 + (double)lambda * (1.0 - ssim));
        out[1] = (float)ssim;
        out[2] = (float)l1;
    }
}

__global__ __launch_bounds__(kLossThreads) void ssim_bwd_kernel(
    int H, int W, const float* __restrict__ img, const float* __restrict__ gt, Window win,
    const float* __restrict__ gmaps, float c_l1, float c_ssim, const float* __restrict__ grad_loss,
    float* __restrict__ dimg) {
#pragma clang fp contract(fast)
    __shared__ float s_g[3][3][kInH][kInW];  // [map][channel][row][column]
    __shared__ float s_h[3][kInH][kLossTW];
    const int tid = threadIdx.x;
    const int x0 = blockIdx.x * kLossTW, y0 = blockIdx.y * kLossTH;
    const size_t plane = (size_t)H * W * 3;
    // the derivative maps of the windows centred in the tile and its halo;
    // zero for windows that are not inside the image.  One map at a time,
    // every thread's loads of it issued together.
#pragma unroll 1
    for (int mp = 0; mp < 3; ++mp) {
        float v[kHaloIters];
#pragma unroll
        for (int it = 0; it < kHaloIters; ++it) {
            const int e = tid + it * kLossThreads;
            const int r = e / kRowElems, q = e - r * kRowElems;
            const int gy = y0 - kWinR + r, gx = x0 - kWinR + q / 3;
            const bool in = e < kHaloElems && gy >= 0 && gy < H && gx >= 0 && gx < W &&
                            interior(gy, gx, H, W);
            v[it] = in ? gmaps[mp * plane + (size_t)gy * W * 3 + (size_t)(x0 - kWinR) * 3 + q]
                       : 0.0f;
        }
#pragma unroll
        for (int it = 0; it < kHaloIters; ++it) {
            const int e = tid + it * kLossThreads;
            if (e >= kHaloElems) continue;
            const int r = e / kRowElems, q = e - r * kRowElems;
            const int cx = q / 3, ch = q - cx * 3;
            s_g[mp][ch][r][cx] = v[it];
        }
    }
    const float g = grad_loss ? *grad_loss : 1.0f;
    __syncthreads();
    const int vc = tid & (kLossTW - 1), vr = 2 * (tid / kLossTW);
    for (int ch = 0; ch < 3; ++ch) {
        for (int t = tid; t < kInH * kLossTW; t += kLossThreads) {
            const int r = t / kLossTW, c = t - r * kLossTW;
            float b0 = 0.0f, b1 = 0.0f, b2 = 0.0f;
#pragma unroll
            for (int k = 0; k < kWinTaps; ++k) {
                const float w = win.w[k];
                b0 += w * s_g[0][ch][r][c + k];
                b1 += w * s_g[1][ch][r][c + k];
                b2 += w * s_g[2][ch][r][c + k];
            }
            s_h[0][r][c] = b0;
            s_h[1][r][c] = b1;
            s_h[2][r][c] = b2;
        }
        __syncthreads();
        float m[2][3] = {};
#pragma unroll
        for (int k = 0; k < kWinTaps + 1; ++k) {
            float v[3];
#pragma unroll
            for (int i = 0; i < 3; ++i) v[i] = s_h[i][vr + k][vc];
            if (k < kWinTaps) {
#pragma unroll
                for (int i = 0; i < 3; ++i) m[0][i] += win.w[k] * v[i];
            }
            if (k >= 1) {
#pragma unroll
                for (int i = 0; i < 3; ++i) m[1][i] += win.w[k - 1] * v[i];
            }
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int gy = y0 + vr + j, gx = x0 + vc;
            if (gy >= H || gx >= W) continue;
            const size_t idx = ((size_t)gy * W + gx) * 3 + ch;
            const float xv = img[idx], yv = gt[idx];
            const float xc = clamp01(xv), yc = clamp01(yv);
            // torch's clamp passes the gradient where 0 <= x <= 1
            const float ds = (xv >= 0.0f && xv <= 1.0f)
                                 ? m[j][0] + 2.0f * xc * m[j][1] + yc * m[j][2]
                                 : 0.0f;
            // d|gt - x|/dx = -sgn(gt - x) (0 at 0, as torch's abs backward)
            const float u = yv - xv;
            const float sg = (u > 0.0f) ? -1.0f : ((u < 0.0f) ? 1.0f : (u != u ? u : 0.0f));
            dimg[idx] = g * (c_l1 * sg - c_ssim * ds);
        }
        __syncthreads();
    }
}

Window gaussian_window() {
    Window w;
    double g[kWinTaps], sum = 0.0;
    for (int k = 0; k < kWinTaps; ++k) {
        const double d = (double)(k - kWinR) / 1.5;
        g[k] = std::exp(-0.5 * d * d);
        sum += g[k];
    }
    for (int k = 0; k < kWinTaps; ++k) w.w[k] = (float)(g[k] / sum);
    return w;
}

dim3 loss_grid(int H, int W) {
    return dim3((unsigned)((W + kLossTW - 1) / kLossTW), (unsigned)((H + kLossTH - 1) / kLossTH));
}

}  // namespace

size_t loss_partial_count(int H, int W) {
    const dim3 g = loss_grid(H, W);
    return (size_t)g.x * g.y;
}

hipError_t launch_l1_dssim_fwd(int H, int W, const float* img, const float* gt, float lambda,
                               float* gmaps, void* partial, float* out, hipStream_t st) {
    const dim3 grid = loss_grid(H, W);
    hipLaunchKernelGGL(ssim_fwd_kernel, grid, dim3(kLossThreads), 0, st, H, W, img, gt,
                       gaussian_window(), gmaps, static_cast<float2*>(partial));
    const double n_win = 3.0 * (double)(H - 2 * kWinR) * (double)(W - 2 * kWinR);
    const double n_px = 3.0 * (double)H * (double)W;
    hipLaunchKernelGGL(loss_finalize_kernel, dim3(1), dim3(kLossThreads), 0, st,
                       (int)(grid.x * grid.y), static_cast<const float2*>(partial), n_win, n_px,
                       lambda, out);
    return hipGetLastError();
}

hipError_t launch_l1_dssim_bwd(int H, int W, const float* img, const float* gt, float lambda,
                               const float* gmaps, const float* grad_loss, float* dimg,
                               hipStream_t st) {
    const double n_win = 3.0 * (double)(H - 2 * kWinR) * (double)(W - 2 * kWinR);
    const double n_px = 3.0 * (double)H * (double)W;
    const float c_l1 = (float)((1.0 - (double)lambda) / n_px);
    const float c_ssim = (float)((double)lambda / n_win);
    hipLaunchKernelGGL(ssim_bwd_kernel, loss_grid(H, W), dim3(kLossThreads), 0, st, H, W, img,
                       gt, gaussian_window(), gmaps, c_l1, c_ssim, grad_loss, dimg);
    return hipGetLastError();
}

}  // namespace gsr
