// gsr_project.hip — projection forward and backward, one thread per
// Gaussian.  Both are HBM-stream kernels: 64 B per Gaussian forward
// (mu 12, q 16, s 12 in; mean 8, cov 12, depth 4 out), 100 B backward.
#include "gsr_internal.h"
#include "gsr_gaussian.h"

namespace gsr {

namespace {

constexpr int kThreads = 256;

// projection.cu:12-107 (project_one).
__global__ __launch_bounds__(kThreads) void project_fwd_kernel(
    int n, const float* __restrict__ mu, const float* __restrict__ q,
    const float* __restrict__ s, const float* __restrict__ rot, const float* __restrict__ tr,
    float fx, float fy, float cx, float cy, float* __restrict__ mean2d,
    float* __restrict__ cov2d, float* __restrict__ depth) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const Pose pose = load_pose(rot, tr);
    const Projected p = project_one(pose, mu, q, s, fx, fy, cx, cy, (size_t)i);
    mean2d[2 * (size_t)i] = p.m0;
    mean2d[2 * (size_t)i + 1] = p.m1;
    cov2d[3 * (size_t)i] = p.a;
    cov2d[3 * (size_t)i + 1] = p.b;
    cov2d[3 * (size_t)i + 2] = p.c;
    depth[i] = p.d;
}

// projection_backward.cu:11-140 (project_backward_one).
__global__ __launch_bounds__(kThreads) void project_bwd_kernel(
    int n, const float* __restrict__ dmean, const float* __restrict__ dcov,
    const float* __restrict__ mu, const float* __restrict__ q, const float* __restrict__ s,
    const float* __restrict__ rot, const float* __restrict__ tr, float fx, float fy,
    float* __restrict__ dmu, float* __restrict__ dq, float* __restrict__ ds, int ref_quat) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const Pose pose = load_pose(rot, tr);
    float omu[3], oq[4], os[3];
    project_backward_one(pose, dmean, dcov, mu, q, s, fx, fy, ref_quat, (size_t)i, omu, oq, os);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        dmu[3 * (size_t)i + k] = omu[k];
        ds[3 * (size_t)i + k] = os[k];
    }
    *reinterpret_cast<float4*>(dq + 4 * (size_t)i) = make_float4(oq[0], oq[1], oq[2], oq[3]);
}

inline int blocks_for(int n) { return (n + kThreads - 1) / kThreads; }

// The autograd glue's screen radius for densification (screen_radius).
__global__ __launch_bounds__(256) void screen_radii_kernel(int n, const float* __restrict__ cov,
                                                           float* __restrict__ radii) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    radii[i] = screen_radius(cov[3 * (size_t)i], cov[3 * (size_t)i + 1], cov[3 * (size_t)i + 2]);
}

// cam = -R^T t (the glue's -matmul(R.T, t)), one thread.
__global__ void camera_position_kernel(const float* __restrict__ R, const float* __restrict__ t,
                                       float* __restrict__ cam) {
    if (threadIdx.x != 0) return;
    float c[3];
    camera_position_of(R, t, c);
#pragma unroll
    for (int i = 0; i < 3; ++i) cam[i] = c[i];
}

}  // namespace

hipError_t launch_screen_radii(int n, const float* cov2d, float* radii, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(screen_radii_kernel, dim3((n + 255) / 256), dim3(256), 0, st, n, cov2d,
                       radii);
    return hipGetLastError();
}

hipError_t launch_camera_position(const float* rot, const float* trans, float* cam,
                                  hipStream_t st) {
    hipLaunchKernelGGL(camera_position_kernel, dim3(1), dim3(64), 0, st, rot, trans, cam);
    return hipGetLastError();
}

hipError_t launch_project_fwd(int n, const float* mu, const float* q, const float* s,
                              const float* rot, const float* tr, float fx, float fy, float cx,
                              float cy, float* mean2d, float* cov2d, float* depth,
                              hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(project_fwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, mu, q,
                       s, rot, tr, fx, fy, cx, cy, mean2d, cov2d, depth);
    return hipGetLastError();
}

hipError_t launch_project_bwd(int n, const float* dmean, const float* dcov, const float* mu,
                              const float* q, const float* s, const float* rot, const float* tr,
                              float fx, float fy, float* dmu, float* dq, float* ds, int ref_quat,
                              hipStream_t st) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(project_bwd_kernel, dim3(blocks_for(n)), dim3(kThreads), 0, st, n, dmean,
                       dcov, mu, q, s, rot, tr, fx, fy, dmu, dq, ds, ref_quat);
    return hipGetLastError();
}

}  // namespace gsr
