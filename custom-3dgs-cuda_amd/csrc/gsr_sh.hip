// gsr_sh.hip — degree-3 SH colour forward and backward, one thread per
// Gaussian, one wave per work-group.  The 45 coefficients of a Gaussian are
// 180 contiguous bytes; a work-group's 64 x 45 floats (11.25 KB, 16-byte
// aligned) are staged through LDS with coalesced 16-byte loads (and dk_j
// leaves the same way), so every HBM access of the dominant stream is a full,
// contiguous transaction and many work-groups per CU keep loads in flight.
// HBM bytes per Gaussian: 216 forward, 420 backward.
#include "gsr_internal.h"
#include "gsr_math.h"

namespace gsr {

namespace {

constexpr int kThreads = 64;
constexpr int kCoef = 45;  // 15 x 3 band-1..3 coefficients per Gaussian

// Copy floats [base*45, base*45 + cnt*45) of src into LDS: 16-byte chunks
// (base is a multiple of 64, so the block's span starts 16-byte aligned),
// then the remainder singly.
__device__ __forceinline__ void stage_coeffs(float* __restrict__ lds,
                                             const float* __restrict__ src, size_t base,
                                             int cnt) {
    const int total = cnt * kCoef, total4 = total / 4;
    const float4* g4 = reinterpret_cast<const float4*>(src + base * kCoef);
    float4* l4 = reinterpret_cast<float4*>(lds);
#pragma unroll 4
    for (int j = threadIdx.x; j < total4; j += kThreads) l4[j] = g4[j];
    for (int j = total4 * 4 + threadIdx.x; j < total; j += kThreads) lds[j] = src[base * kCoef + j];
}

// The reverse: LDS floats [0, cnt*45) to dst[base*45 ..].
__device__ __forceinline__ void unstage_coeffs(float* __restrict__ dst,
                                               const float* __restrict__ lds, size_t base,
                                               int cnt) {
    const int total = cnt * kCoef, total4 = total / 4;
    float4* g4 = reinterpret_cast<float4*>(dst + base * kCoef);
    const float4* l4 = reinterpret_cast<const float4*>(lds);
#pragma unroll 4
    for (int j = threadIdx.x; j < total4; j += kThreads) g4[j] = l4[j];
    for (int j = total4 * 4 + threadIdx.x; j < total; j += kThreads) dst[base * kCoef + j] = lds[j];
}

// SH.cu:57-93.  dir = glm::normalize(mu - cam) = v * (1 / sqrt(dot(v, v))).
__global__ __launch_bounds__(kThreads) void sh_fwd_kernel(int n, const float* __restrict__ cam,
                                                          const float* __restrict__ mu,
                                                          const float* __restrict__ albedo,
                                                          const float* __restrict__ kj,
                                                          float* __restrict__ colors) {
    __shared__ __align__(16) float s_k[kThreads * kCoef];
    const size_t base = (size_t)blockIdx.x * kThreads;
    const int cnt = (int)min((size_t)kThreads, (size_t)n - base);
    stage_coeffs(s_k, kj, base, cnt);
    __syncthreads();
    if ((int)threadIdx.x >= cnt) return;
    const size_t i = base + threadIdx.x;
    const float v0 = mu[3 * i] - cam[0], v1 = mu[3 * i + 1] - cam[1], v2 = mu[3 * i + 2] - cam[2];
    const float inv = 1.0f / __builtin_sqrtf(v0 * v0 + v1 * v1 + v2 * v2);
    float Y[15];
    sh_basis15(v0 * inv, v1 * inv, v2 * inv, Y);
    const float* k = s_k + threadIdx.x * kCoef;
    float r = 0.5f + SH_C0 * albedo[3 * i];
    float g = 0.5f + SH_C0 * albedo[3 * i + 1];
    float b = 0.5f + SH_C0 * albedo[3 * i + 2];
#pragma unroll
    for (int j = 0; j < 15; ++j) {
        r = r + Y[j] * k[3 * j];
        g = g + Y[j] * k[3 * j + 1];
        b = b + Y[j] * k[3 * j + 2];
    }
    colors[3 * i] = fminf(fmaxf(r, 0.0f), 1.0f);
    colors[3 * i + 1] = fminf(fmaxf(g, 0.0f), 1.0f);
    colors[3 * i + 2] = fminf(fmaxf(b, 0.0f), 1.0f);
}

// delight_backward.cu:107-174.  The backward direction uses
// 1/sqrt(|v|^2 + 1e-8) (the reference's rsqrtf, here correctly rounded).
__global__ __launch_bounds__(kThreads) void sh_bwd_kernel(
    int n, const float* __restrict__ cgrad, const float* __restrict__ mu,
    const float* __restrict__ albedo, const float* __restrict__ kj, const float* __restrict__ cam,
    float* __restrict__ dA, float* __restrict__ dkj, float* __restrict__ dmu) {
    __shared__ __align__(16) float s_k[kThreads * kCoef];
    const size_t base = (size_t)blockIdx.x * kThreads;
    const int cnt = (int)min((size_t)kThreads, (size_t)n - base);
    stage_coeffs(s_k, kj, base, cnt);
    __syncthreads();
    const bool live = (int)threadIdx.x < cnt;
    float* k = s_k + threadIdx.x * kCoef;
    if (live) {
        const size_t i = base + threadIdx.x;
        const float v0 = mu[3 * i] - cam[0], v1 = mu[3 * i + 1] - cam[1], v2 = mu[3 * i + 2] - cam[2];
        const float inv = 1.0f / __builtin_sqrtf(v0 * v0 + v1 * v1 + v2 * v2 + 1e-8f);
        const float x = v0 * inv, y = v1 * inv, z = v2 * inv;
        float Y[15];
        sh_basis15(x, y, z, Y);
        float rgb[3];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) rgb[ch] = 0.5f + SH_C0 * albedo[3 * i + ch];
#pragma unroll
        for (int j = 0; j < 15; ++j)
#pragma unroll
            for (int ch = 0; ch < 3; ++ch) rgb[ch] = rgb[ch] + Y[j] * k[3 * j + ch];
        float g[3];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch)
            g[ch] = (rgb[ch] < 0.0f || rgb[ch] > 1.0f) ? 0.0f : cgrad[3 * i + ch];
#pragma unroll
        for (int ch = 0; ch < 3; ++ch) dA[3 * i + ch] = g[ch] * SH_C0;
        float dY[15];
#pragma unroll
        for (int j = 0; j < 15; ++j) {
            dY[j] = g[0] * k[3 * j] + g[1] * k[3 * j + 1] + g[2] * k[3 * j + 2];
            // coefficients are consumed: reuse the LDS slots for dk_j
            k[3 * j] = g[0] * Y[j];
            k[3 * j + 1] = g[1] * Y[j];
            k[3 * j + 2] = g[2] * Y[j];
        }
        const float xx = x * x, yy = y * y, zz = z * z;
        float gx = 0.0f, gy = 0.0f, gz = 0.0f;
        // accumulate_dY_ddir (delight_backward.cu:50-105), same term order
        gy += dY[0] * (-SH_C1);
        gz += dY[1] * (SH_C1);
        gx += dY[2] * (-SH_C1);
        gx += dY[3] * (SH_C2_0 * y);
        gy += dY[3] * (SH_C2_0 * x);
        gy += dY[4] * (SH_C2_1 * z);
        gz += dY[4] * (SH_C2_1 * y);
        gx += dY[5] * (-2.0f * SH_C2_2 * x);
        gy += dY[5] * (-2.0f * SH_C2_2 * y);
        gz += dY[5] * (4.0f * SH_C2_2 * z);
        gx += dY[6] * (SH_C2_3 * z);
        gz += dY[6] * (SH_C2_3 * x);
        gx += dY[7] * (2.0f * SH_C2_4 * x);
        gy += dY[7] * (-2.0f * SH_C2_4 * y);
        gx += dY[8] * (SH_C3_0 * y * 6.0f * x);
        gy += dY[8] * (SH_C3_0 * (3.0f * xx - 3.0f * yy));
        gx += dY[9] * (SH_C3_1 * y * z);
        gy += dY[9] * (SH_C3_1 * x * z);
        gz += dY[9] * (SH_C3_1 * x * y);
        gx += dY[10] * (SH_C3_2 * y * (-2.0f * x));
        gy += dY[10] * (SH_C3_2 * (4.0f * zz - xx - 3.0f * yy));
        gz += dY[10] * (SH_C3_2 * y * 8.0f * z);
        gx += dY[11] * (SH_C3_3 * z * (-6.0f * x));
        gy += dY[11] * (SH_C3_3 * z * (-6.0f * y));
        gz += dY[11] * (SH_C3_3 * (6.0f * zz - 3.0f * xx - 3.0f * yy));
        gx += dY[12] * (SH_C3_4 * (4.0f * zz - 3.0f * xx - yy));
        gy += dY[12] * (SH_C3_4 * x * (-2.0f * y));
        gz += dY[12] * (SH_C3_4 * x * 8.0f * z);
        gx += dY[13] * (SH_C3_5 * z * 2.0f * x);
        gy += dY[13] * (SH_C3_5 * z * (-2.0f * y));
        gz += dY[13] * (SH_C3_5 * (xx - yy));
        gx += dY[14] * (SH_C3_6 * (3.0f * xx - 3.0f * yy));
        gy += dY[14] * (SH_C3_6 * x * (-6.0f * y));
        const float ddot = x * gx + y * gy + z * gz;
        dmu[3 * i] = inv * (gx - x * ddot);
        dmu[3 * i + 1] = inv * (gy - y * ddot);
        dmu[3 * i + 2] = inv * (gz - z * ddot);
    }
    __syncthreads();
    unstage_coeffs(dkj, s_k, base, cnt);
}

inline int blocks_for(int n) { return (n + kThreads - 1) / kThreads; }

}  // namespace

hipError_t launch_sh_fwd(int n, const float* cam, const float* mu, const float* albedo,
                         const float* kj, float* colors, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sh_fwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, cam, mu,
                       albedo, kj, colors);
    return hipGetLastError();
}

hipError_t launch_sh_bwd(int n, const float* cgrad, const float* mu, const float* albedo,
                         const float* kj, const float* cam, float* dA, float* dkj, float* dmu,
                         hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(sh_bwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, cgrad, mu,
                       albedo, kj, cam, dA, dkj, dmu);
    return hipGetLastError();
}

}  // namespace gsr
