// gsr_sh.hip — degree-3 SH colour forward and backward, one thread per
// Gaussian, one wave per work-group.  The 45 coefficients of a Gaussian are
// 180 contiguous bytes; a work-group's 64 x 45 floats (11.25 KB, 16-byte
// aligned) are staged through LDS with coalesced 16-byte loads (and dk_j
// leaves the same way), so every HBM access of the dominant stream is a full,
// contiguous transaction and many work-groups per CU keep loads in flight.
// HBM bytes per Gaussian: 216 forward, 420 backward.
#include "gsr_internal.h"
#include "gsr_gaussian.h"

namespace gsr {

namespace {

constexpr int kThreads = kShThreads;

// SH.cu:57-93 (sh_colour).
__global__ __launch_bounds__(kThreads) void sh_fwd_kernel(int n, const float* __restrict__ cam,
                                                          const float* __restrict__ mu,
                                                          const float* __restrict__ albedo,
                                                          const float* __restrict__ kj,
                                                          float* __restrict__ colors) {
    __shared__ __align__(16) float s_k[kThreads * kShCoef];
    const size_t base = (size_t)blockIdx.x * kThreads;
    const int cnt = (int)min((size_t)kThreads, (size_t)n - base);
    stage_coeffs(s_k, kj, base, cnt);
    __syncthreads();
    if ((int)threadIdx.x >= cnt) return;
    const size_t i = base + threadIdx.x;
    float rgb[3];
    sh_colour(cam, mu, albedo, s_k + threadIdx.x * kShCoef, i, rgb);
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) colors[3 * i + ch] = rgb[ch];
}

// delight_backward.cu:107-174 (sh_backward_one).
__global__ __launch_bounds__(kThreads) void sh_bwd_kernel(
    int n, const float* __restrict__ cgrad, const float* __restrict__ mu,
    const float* __restrict__ albedo, const float* __restrict__ kj, const float* __restrict__ cam,
    float* __restrict__ dA, float* __restrict__ dkj, float* __restrict__ dmu) {
    __shared__ __align__(16) float s_k[kThreads * kShCoef];
    const size_t base = (size_t)blockIdx.x * kThreads;
    const int cnt = (int)min((size_t)kThreads, (size_t)n - base);
    stage_coeffs(s_k, kj, base, cnt);
    __syncthreads();
    if ((int)threadIdx.x < cnt) {
        const size_t i = base + threadIdx.x;
        float g[3];
        sh_backward_one(cgrad, mu, albedo, s_k + threadIdx.x * kShCoef, cam, dA, i, g);
#pragma unroll
        for (int k = 0; k < 3; ++k) dmu[3 * i + k] = g[k];
    }
    __syncthreads();
    unstage_coeffs(dkj, s_k, base, cnt);
}

// The autograd glue's forward head in one pass (rasterize.py:43-56): camera
// position, projection, screen radius and SH colour of each Gaussian, with
// the operations of camera_position_kernel, project_fwd_kernel,
// screen_radii_kernel and sh_fwd_kernel, so every output is bit for bit
// theirs.  Thread 0 of work-group 0 also stores cam.  With logits, also the
// opacity 1 / (1 + exp(-logit)): torch's fp32 sigmoid, operation for
// operation (the device expf and a correctly rounded division).
__global__ __launch_bounds__(kThreads) void project_sh_fwd_kernel(
    int n, const float* __restrict__ mu, const float* __restrict__ q,
    const float* __restrict__ s, const float* __restrict__ rot, const float* __restrict__ tr,
    float fx, float fy, float cx, float cy, const float* __restrict__ albedo,
    const float* __restrict__ kj, float* __restrict__ mean2d, float* __restrict__ cov2d,
    float* __restrict__ depth, float* __restrict__ radii, float* __restrict__ colors,
    float* __restrict__ cam_out, const float* __restrict__ logits, float* __restrict__ opacity) {
    __shared__ __align__(16) float s_k[kThreads * kShCoef];
    const size_t base = (size_t)blockIdx.x * kThreads;
    const int cnt = (int)min((size_t)kThreads, (size_t)n - base);
    stage_coeffs(s_k, kj, base, cnt);
    float cam[3];
    camera_position_of(rot, tr, cam);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
#pragma unroll
        for (int k = 0; k < 3; ++k) cam_out[k] = cam[k];
    }
    const bool live = (int)threadIdx.x < cnt;
    const size_t i = base + threadIdx.x;
    if (live) {
        const Pose pose = load_pose(rot, tr);
        const Projected p = project_one(pose, mu, q, s, fx, fy, cx, cy, i);
        mean2d[2 * i] = p.m0;
        mean2d[2 * i + 1] = p.m1;
        cov2d[3 * i] = p.a;
        cov2d[3 * i + 1] = p.b;
        cov2d[3 * i + 2] = p.c;
        depth[i] = p.d;
        radii[i] = screen_radius(p.a, p.b, p.c);
        if (logits) opacity[i] = 1.0f / (1.0f + expf(-logits[i]));
    }
    __syncthreads();
    if (!live) return;
    float rgb[3];
    sh_colour(cam, mu, albedo, s_k + threadIdx.x * kShCoef, i, rgb);
#pragma unroll
    for (int ch = 0; ch < 3; ++ch) colors[3 * i + ch] = rgb[ch];
}

// The glue's backward tail in one pass (rasterize.py:100-125): the SH
// backward and the projection backward of each Gaussian, with dL/dmu the sum
// of the two (projection's + SH's, the glue's one fp32 addition), with the
// operations of sh_bwd_kernel and project_bwd_kernel.  With d_opacity, also
// dL/dlogit = (d_opacity (1 - s)) s for s = the opacity: torch's fp32 sigmoid
// backward, operation for operation.
__global__ __launch_bounds__(kThreads) void project_sh_bwd_kernel(
    int n, const float* __restrict__ dmean, const float* __restrict__ dcov,
    const float* __restrict__ cgrad, const float* __restrict__ mu, const float* __restrict__ q,
    const float* __restrict__ s, const float* __restrict__ rot, const float* __restrict__ tr,
    float fx, float fy, const float* __restrict__ albedo, const float* __restrict__ kj,
    const float* __restrict__ cam, float* __restrict__ dmu, float* __restrict__ dq,
    float* __restrict__ ds, float* __restrict__ dA, float* __restrict__ dkj, int ref_quat,
    const float* __restrict__ dop, const float* __restrict__ op, float* __restrict__ dlogits) {
    __shared__ __align__(16) float s_k[kThreads * kShCoef];
    const size_t base = (size_t)blockIdx.x * kThreads;
    const int cnt = (int)min((size_t)kThreads, (size_t)n - base);
    stage_coeffs(s_k, kj, base, cnt);
    __syncthreads();
    if ((int)threadIdx.x < cnt) {
        const size_t i = base + threadIdx.x;
        float gsh[3];
        sh_backward_one(cgrad, mu, albedo, s_k + threadIdx.x * kShCoef, cam, dA, i, gsh);
        const Pose pose = load_pose(rot, tr);
        float omu[3], oq[4], os[3];
        project_backward_one(pose, dmean, dcov, mu, q, s, fx, fy, ref_quat, i, omu, oq, os);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            dmu[3 * i + k] = omu[k] + gsh[k];
            ds[3 * i + k] = os[k];
        }
        *reinterpret_cast<float4*>(dq + 4 * i) = make_float4(oq[0], oq[1], oq[2], oq[3]);
        if (dop) {
            const float sg = op[i];
            dlogits[i] = (dop[i] * (1.0f - sg)) * sg;
        }
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

hipError_t launch_project_sh_fwd(int n, const float* mu, const float* q, const float* s,
                                 const float* rot, const float* tr, float fx, float fy, float cx,
                                 float cy, const float* albedo, const float* kj, float* mean2d,
                                 float* cov2d, float* depth, float* radii, float* colors,
                                 float* cam, const float* logits, float* opacity,
                                 hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(project_sh_fwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, mu,
                       q, s, rot, tr, fx, fy, cx, cy, albedo, kj, mean2d, cov2d, depth, radii,
                       colors, cam, logits, opacity);
    return hipGetLastError();
}

hipError_t launch_project_sh_bwd(int n, const float* dmean, const float* dcov,
                                 const float* cgrad, const float* mu, const float* q,
                                 const float* s, const float* rot, const float* tr, float fx,
                                 float fy, const float* albedo, const float* kj, const float* cam,
                                 float* dmu, float* dq, float* ds, float* dA, float* dkj,
                                 int ref_quat, const float* dop, const float* op,
                                 float* dlogits, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(project_sh_bwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n,
                       dmean, dcov, cgrad, mu, q, s, rot, tr, fx, fy, albedo, kj, cam, dmu, dq,
                       ds, dA, dkj, ref_quat, dop, op, dlogits);
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
