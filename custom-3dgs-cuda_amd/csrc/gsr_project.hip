// gsr_project.hip — projection forward (a1) and backward (a12), one thread
// per Gaussian.  Both are HBM-stream kernels: 64 B per Gaussian forward
// (mu 12, q 16, s 12 in; mean 8, cov 12, depth 4 out), 100 B backward.
#include "gsr_internal.h"
#include "gsr_math.h"

namespace gsr {

namespace {

constexpr int kThreads = 256;

// projection.cu:12-107.  Culled Gaussians (z <= 0.2, or NaN-free z at or
// below the plane) keep zero mean, covariance and depth.
__global__ __launch_bounds__(kThreads) void project_fwd_kernel(
    int n, const float* __restrict__ mu, const float* __restrict__ q,
    const float* __restrict__ s, const float* __restrict__ rot, const float* __restrict__ tr,
    float fx, float fy, float cx, float cy, float* __restrict__ mean2d,
    float* __restrict__ cov2d, float* __restrict__ depth) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const Pose pose = load_pose(rot, tr);
    float mc[3];
    to_camera(pose, mu[3 * (size_t)i], mu[3 * (size_t)i + 1], mu[3 * (size_t)i + 2], mc);
    float m0 = 0.0f, m1 = 0.0f, a = 0.0f, b = 0.0f, c = 0.0f, d = 0.0f;
    if (!(mc[2] <= kNearZ)) {
        d = mc[2];
        m0 = (fx * mc[0]) / mc[2] + cx;
        m1 = (fy * mc[1]) / mc[2] + cy;
        const float4 qq = *reinterpret_cast<const float4*>(q + 4 * (size_t)i);
        const Cov3 cv = covariance3d(pose, qq.x, qq.y, qq.z, qq.w, s[3 * (size_t)i],
                                     s[3 * (size_t)i + 1], s[3 * (size_t)i + 2]);
        const float z2 = mc[2] * mc[2];
        const float J00 = fx / mc[2];
        const float J02 = -(fx * mc[0]) / z2;
        const float J11 = fy / mc[2];
        const float J12 = -(fy * mc[1]) / z2;
        const Mat3& Sc = cv.Sc;
        a = J00 * (J00 * Sc.m[0][0] + J02 * Sc.m[0][2]) + J02 * (J00 * Sc.m[2][0] + J02 * Sc.m[2][2]);
        b = J00 * (J11 * Sc.m[1][0] + J12 * Sc.m[2][0]) + J02 * (J11 * Sc.m[1][2] + J12 * Sc.m[2][2]);
        c = J11 * (J11 * Sc.m[1][1] + J12 * Sc.m[2][1]) + J12 * (J11 * Sc.m[1][2] + J12 * Sc.m[2][2]);
        a = a + 0.3f;  // 0.3 px anti-aliasing on the diagonal (projection.cu:101-102)
        c = c + 0.3f;
    }
    mean2d[2 * (size_t)i] = m0;
    mean2d[2 * (size_t)i + 1] = m1;
    cov2d[3 * (size_t)i] = a;
    cov2d[3 * (size_t)i + 1] = b;
    cov2d[3 * (size_t)i + 2] = c;
    depth[i] = d;
}

// projection_backward.cu:11-140: dL/dmu through the mean and through J,
// dL/dlog-scale through exp, dL/dq through toMat3 and normalize.
// ref_quat selects the reference's literal quaternion formula, which reads
// transpose(dL/dR) with indices meant for dL/dR (it fails finite
// differences); 0 gives the derivative of glm::toMat3.
__global__ __launch_bounds__(kThreads) void project_bwd_kernel(
    int n, const float* __restrict__ dmean, const float* __restrict__ dcov,
    const float* __restrict__ mu, const float* __restrict__ q, const float* __restrict__ s,
    const float* __restrict__ rot, const float* __restrict__ tr, float fx, float fy,
    float* __restrict__ dmu, float* __restrict__ dq, float* __restrict__ ds, int ref_quat) {
    const int i = blockIdx.x * kThreads + threadIdx.x;
    if (i >= n) return;
    const Pose pose = load_pose(rot, tr);
    float mc[3];
    to_camera(pose, mu[3 * (size_t)i], mu[3 * (size_t)i + 1], mu[3 * (size_t)i + 2], mc);
    float omu[3] = {0.0f, 0.0f, 0.0f}, oq[4] = {0.0f, 0.0f, 0.0f, 0.0f},
          os[3] = {0.0f, 0.0f, 0.0f};
    if (!(mc[2] <= kNearZ)) {
        const float z = mc[2], z2 = z * z, z3 = z2 * z;
        const float gdx = dmean[2 * (size_t)i], gdy = dmean[2 * (size_t)i + 1];
        float dmc[3] = {(fx / z) * gdx, (fy / z) * gdy,
                        (-fx * mc[0] / z2) * gdx + (-fy * mc[1] / z2) * gdy};
        const float ga = dcov[3 * (size_t)i], gb = dcov[3 * (size_t)i + 1],
                    gc = dcov[3 * (size_t)i + 2];
        const float G00 = ga, G01 = 0.5f * gb, G10 = 0.5f * gb, G11 = gc;
        const float J[2][3] = {{fx / z, 0.0f, -(fx * mc[0]) / z2}, {0.0f, fy / z, -(fy * mc[1]) / z2}};
        const float4 qq = *reinterpret_cast<const float4*>(q + 4 * (size_t)i);
        const Cov3 cv = covariance3d(pose, qq.x, qq.y, qq.z, qq.w, s[3 * (size_t)i],
                                     s[3 * (size_t)i + 1], s[3 * (size_t)i + 2]);
        // dl_dcam = (J^T G) J
        float JtG[3][2];
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            JtG[r][0] = J[0][r] * G00 + J[1][r] * G10;
            JtG[r][1] = J[0][r] * G01 + J[1][r] * G11;
        }
        Mat3 dcam;
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int k = 0; k < 3; ++k) dcam.m[r][k] = JtG[r][0] * J[0][k] + JtG[r][1] * J[1][k];
        // dl_dworld = (R_cam^T dl_dcam) R_cam ; dl_dM = (2 dl_dworld) M
        const Mat3 Rct = transpose(pose.R);
        Mat3 dw = mul(mul(Rct, dcam), pose.R);
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int k = 0; k < 3; ++k) dw.m[r][k] = 2.0f * dw.m[r][k];
        const Mat3 dM = mul(dw, cv.M);
        const Mat3 dR = mul(dM, cv.S);
        const Mat3 dS = mul(transpose(cv.R), dM);
        os[0] = dS.m[0][0] * cv.S.m[0][0];
        os[1] = dS.m[1][1] * cv.S.m[1][1];
        os[2] = dS.m[2][2] * cv.S.m[2][2];
        // dL/dJ = ((2 G) J) Sigma_cam, entries (0,0), (1,1), (0,2), (1,2)
        const float G2[2][2] = {{2.0f * G00, 2.0f * G01}, {2.0f * G10, 2.0f * G11}};
        float GJ[2][3];
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int k = 0; k < 3; ++k) GJ[r][k] = G2[r][0] * J[0][k] + G2[r][1] * J[1][k];
        const Mat3& Sc = cv.Sc;
        auto dJ = [&](int r, int k) {
            return GJ[r][0] * Sc.m[0][k] + GJ[r][1] * Sc.m[1][k] + GJ[r][2] * Sc.m[2][k];
        };
        const float dJ00 = dJ(0, 0), dJ11 = dJ(1, 1), dJ02 = dJ(0, 2), dJ12 = dJ(1, 2);
        dmc[0] = dmc[0] + dJ02 * (-fx / z2);
        dmc[1] = dmc[1] + dJ12 * (-fy / z2);
        dmc[2] = dmc[2] + (dJ00 * (-fx / z2) + dJ11 * (-fy / z2) + dJ02 * (2.0f * fx * mc[0] / z3) +
                           dJ12 * (2.0f * fy * mc[1] / z3));
#pragma unroll
        for (int r = 0; r < 3; ++r)
            omu[r] = Rct.m[r][0] * dmc[0] + Rct.m[r][1] * dmc[1] + Rct.m[r][2] * dmc[2];
        // quaternion (projection_backward.cu:334-344); L[i][j] is the value
        // the reference reads as dL_dRt[i][j].
        float L[3][3];
#pragma unroll
        for (int r = 0; r < 3; ++r)
#pragma unroll
            for (int k = 0; k < 3; ++k) L[r][k] = ref_quat ? dR.m[r][k] : dR.m[k][r];
        const float qw = cv.qn[0], qx = cv.qn[1], qy = cv.qn[2], qz = cv.qn[3];
        const float gw = 2.0f * qz * (L[0][1] - L[1][0]) + 2.0f * qy * (L[2][0] - L[0][2]) +
                         2.0f * qx * (L[1][2] - L[2][1]);
        const float gx = 2.0f * qy * (L[1][0] + L[0][1]) + 2.0f * qz * (L[2][0] + L[0][2]) +
                         2.0f * qw * (L[1][2] - L[2][1]) - 4.0f * qx * (L[2][2] + L[1][1]);
        const float gy = 2.0f * qx * (L[1][0] + L[0][1]) + 2.0f * qw * (L[2][0] - L[0][2]) +
                         2.0f * qz * (L[1][2] + L[2][1]) - 4.0f * qy * (L[2][2] + L[0][0]);
        const float gz = 2.0f * qw * (L[0][1] - L[1][0]) + 2.0f * qx * (L[2][0] + L[0][2]) +
                         2.0f * qy * (L[1][2] + L[2][1]) - 4.0f * qz * (L[1][1] + L[0][0]);
        // through normalize (projection_backward.cu:346-356)
        const float inv_norm =
            1.0f / __builtin_sqrtf(qq.x * qq.x + qq.y * qq.y + qq.z * qq.z + qq.w * qq.w + 1e-8f);
        const float qdot = qw * gw + qx * gx + qy * gy + qz * gz;
        oq[0] = inv_norm * (gw - qw * qdot);
        oq[1] = inv_norm * (gx - qx * qdot);
        oq[2] = inv_norm * (gy - qy * qdot);
        oq[3] = inv_norm * (gz - qz * qdot);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        dmu[3 * (size_t)i + k] = omu[k];
        ds[3 * (size_t)i + k] = os[k];
    }
    *reinterpret_cast<float4*>(dq + 4 * (size_t)i) = make_float4(oq[0], oq[1], oq[2], oq[3]);
}

inline int blocks_for(int n) { return (n + kThreads - 1) / kThreads; }

// The autograd glue's screen radius for densification
// (gaussian_splatting/rasterizer/rasterize.py:49-53), one op per rounding in
// torch's order: mid = 0.5 (a + c); radius = mid + sqrt(clamp((0.5 (a - c))^2
// + b b, min 0.1)); radii = 3 sqrt(clamp(radius, min 0)).  A clamp keeps NaN,
// as torch's does.
__global__ __launch_bounds__(256) void screen_radii_kernel(int n, const float* __restrict__ cov,
                                                           float* __restrict__ radii) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float a = cov[3 * (size_t)i], b = cov[3 * (size_t)i + 1], c = cov[3 * (size_t)i + 2];
    const float mid = 0.5f * (a + c);
    const float h = 0.5f * (a - c);
    const float q = h * h + b * b;
    const float qc = (q < 0.1f) ? 0.1f : q;
    const float radius = mid + __builtin_sqrtf(qc);
    const float rc = (radius < 0.0f) ? 0.0f : radius;
    radii[i] = 3.0f * __builtin_sqrtf(rc);
}

// cam = -R^T t (the glue's -matmul(R.T, t)), one thread.
__global__ void camera_position_kernel(const float* __restrict__ R, const float* __restrict__ t,
                                       float* __restrict__ cam) {
    if (threadIdx.x != 0) return;
#pragma unroll
    for (int i = 0; i < 3; ++i)
        cam[i] = -(R[i] * t[0] + R[3 + i] * t[1] + R[6 + i] * t[2]);
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
