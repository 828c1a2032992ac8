// gsr_gaussian.h — per-Gaussian bodies of the projection, screen-radius and SH
// colour passes and of their backwards, shared by the single-pass kernels
// (gsr_project.hip, gsr_sh.hip) and the fused ones (gsr_sh.hip), so both run
// the same fp32 operations in the same order.
#pragma once

#include <hip/hip_runtime.h>

#include "gsr_common.h"
#include "gsr_math.h"

namespace gsr {

// The 45 band-1..3 SH coefficients of a Gaussian (15 x 3 floats).
constexpr int kShCoef = 45;
// Threads (one Gaussian each) of the SH work-groups; their coefficients are
// staged through LDS together.
constexpr int kShThreads = 64;

// Rows [base, base + cnt) of a row-major [N, kW] float array to LDS (row r
// of the span at lds[r * kW]), by the kT threads of the work-group: 16-byte
// loads when the span starts 16-byte aligned (base is a multiple of kT, so
// that holds when the array does), single floats otherwise.  Per-Gaussian
// rows of 2, 3 or 45 floats read one per thread are strided accesses; staged,
// every global access of the work-group is a coalesced 16-byte one.
template <int kW, int kT>
__device__ __forceinline__ void stage_rows(float* __restrict__ lds, const float* __restrict__ src,
                                           size_t base, int cnt) {
    const int total = cnt * kW;
    const float* g = src + base * kW;
    int done = 0;
    if ((reinterpret_cast<uintptr_t>(g) & 15u) == 0) {
        const int total4 = total / 4;
        // rows are read once: non-temporal (streaming) loads
        const f32x4* g4 = reinterpret_cast<const f32x4*>(g);
        f32x4* l4 = reinterpret_cast<f32x4*>(lds);
#pragma unroll 4
        for (int j = threadIdx.x; j < total4; j += kT) l4[j] = __builtin_nontemporal_load(g4 + j);
        done = total4 * 4;
    }
    for (int j = done + (int)threadIdx.x; j < total; j += kT) lds[j] = g[j];
}

// The reverse: LDS floats [0, cnt * kW) to rows [base, base + cnt) of dst.
template <int kW, int kT>
__device__ __forceinline__ void unstage_rows(float* __restrict__ dst, const float* __restrict__ lds,
                                             size_t base, int cnt) {
    const int total = cnt * kW;
    float* g = dst + base * kW;
    int done = 0;
    if ((reinterpret_cast<uintptr_t>(g) & 15u) == 0) {
        const int total4 = total / 4;
        f32x4* g4 = reinterpret_cast<f32x4*>(g);
        const f32x4* l4 = reinterpret_cast<const f32x4*>(lds);
#pragma unroll 4
        for (int j = threadIdx.x; j < total4; j += kT) __builtin_nontemporal_store(l4[j], g4 + j);
        done = total4 * 4;
    }
    for (int j = done + (int)threadIdx.x; j < total; j += kT) g[j] = lds[j];
}

// The SH work-groups' coefficients: 45 floats per Gaussian.
__device__ __forceinline__ void stage_coeffs(float* __restrict__ lds,
                                             const float* __restrict__ src, size_t base,
                                             int cnt) {
    stage_rows<kShCoef, kShThreads>(lds, src, base, cnt);
}
__device__ __forceinline__ void unstage_coeffs(float* __restrict__ dst,
                                               const float* __restrict__ lds, size_t base,
                                               int cnt) {
    unstage_rows<kShCoef, kShThreads>(dst, lds, base, cnt);
}

// cam = -R^T t (the glue's -matmul(R.T, t), rasterize.py:43-44).
__device__ __forceinline__ void camera_position_of(const float* __restrict__ R,
                                                   const float* __restrict__ t, float cam[3]) {
#pragma unroll
    for (int i = 0; i < 3; ++i) cam[i] = -(R[i] * t[0] + R[3 + i] * t[1] + R[6 + i] * t[2]);
}

// Screen-space mean, upper-triangular covariance (a, b, c) and depth.
struct Projected {
    float m0, m1, a, b, c, d;
};

// projection.cu:12-107.  Culled Gaussians (z <= 0.2, or NaN-free z at or
// below the plane) keep zero mean, covariance and depth.
__device__ __forceinline__ Projected project_one(const Pose& pose, const float* __restrict__ mu,
                                                 const float* __restrict__ q,
                                                 const float* __restrict__ s, float fx, float fy,
                                                 float cx, float cy, size_t i) {
    float mc[3];
    to_camera(pose, mu[3 * i], mu[3 * i + 1], mu[3 * i + 2], mc);
    Projected p{0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
    if (!(mc[2] <= kNearZ)) {
        p.d = mc[2];
        p.m0 = (fx * mc[0]) / mc[2] + cx;
        p.m1 = (fy * mc[1]) / mc[2] + cy;
        const float4 qq = *reinterpret_cast<const float4*>(q + 4 * i);
        const Cov3 cv = covariance3d(pose, qq.x, qq.y, qq.z, qq.w, s[3 * i], s[3 * i + 1],
                                     s[3 * i + 2]);
        const float z2 = mc[2] * mc[2];
        const float J00 = fx / mc[2];
        const float J02 = -(fx * mc[0]) / z2;
        const float J11 = fy / mc[2];
        const float J12 = -(fy * mc[1]) / z2;
        const Mat3& Sc = cv.Sc;
        float a = J00 * (J00 * Sc.m[0][0] + J02 * Sc.m[0][2]) +
                  J02 * (J00 * Sc.m[2][0] + J02 * Sc.m[2][2]);
        const float b = J00 * (J11 * Sc.m[1][0] + J12 * Sc.m[2][0]) +
                        J02 * (J11 * Sc.m[1][2] + J12 * Sc.m[2][2]);
        float c = J11 * (J11 * Sc.m[1][1] + J12 * Sc.m[2][1]) +
                  J12 * (J11 * Sc.m[1][2] + J12 * Sc.m[2][2]);
        a = a + 0.3f;  // 0.3 px anti-aliasing on the diagonal (projection.cu:101-102)
        c = c + 0.3f;
        p.a = a;
        p.b = b;
        p.c = c;
    }
    return p;
}

// The autograd glue's screen radius for densification
// (gaussian_splatting/rasterizer/rasterize.py:49-53), one op per rounding in
// torch's order: mid = 0.5 (a + c); radius = mid + sqrt(clamp((0.5 (a - c))^2
// + b b, min 0.1)); radii = 3 sqrt(clamp(radius, min 0)).  A clamp keeps NaN,
// as torch's does.
__device__ __forceinline__ float screen_radius(float a, float b, float c) {
    const float mid = 0.5f * (a + c);
    const float h = 0.5f * (a - c);
    const float q = h * h + b * b;
    const float qc = (q < 0.1f) ? 0.1f : q;
    const float radius = mid + __builtin_sqrtf(qc);
    const float rc = (radius < 0.0f) ? 0.0f : radius;
    return 3.0f * __builtin_sqrtf(rc);
}

// SH.cu:57-93, from the Gaussian's 45 coefficients k.  dir =
// glm::normalize(mu - cam) = v * (1 / sqrt(dot(v, v))).
__device__ __forceinline__ void sh_colour(const float* __restrict__ cam,
                                          const float* __restrict__ mu,
                                          const float* __restrict__ albedo, const float* k,
                                          size_t i, float rgb[3]) {
    const float v0 = mu[3 * i] - cam[0], v1 = mu[3 * i + 1] - cam[1], v2 = mu[3 * i + 2] - cam[2];
    const float inv = 1.0f / __builtin_sqrtf(v0 * v0 + v1 * v1 + v2 * v2);
    float Y[15];
    sh_basis15(v0 * inv, v1 * inv, v2 * inv, Y);
    float r = 0.5f + SH_C0 * albedo[3 * i];
    float g = 0.5f + SH_C0 * albedo[3 * i + 1];
    float b = 0.5f + SH_C0 * albedo[3 * i + 2];
#pragma unroll
    for (int j = 0; j < 15; ++j) {
        r = r + Y[j] * k[3 * j];
        g = g + Y[j] * k[3 * j + 1];
        b = b + Y[j] * k[3 * j + 2];
    }
    rgb[0] = fminf(fmaxf(r, 0.0f), 1.0f);
    rgb[1] = fminf(fmaxf(g, 0.0f), 1.0f);
    rgb[2] = fminf(fmaxf(b, 0.0f), 1.0f);
}

// delight_backward.cu:107-174 for one Gaussian: dA[3i..] written, the 45
// coefficients k replaced in place by dL/dk_j, dL/dmu (through the view
// direction) returned in dmu.  The direction uses 1/sqrt(|v|^2 + 1e-8) (the
// reference's rsqrtf, here correctly rounded).
__device__ __forceinline__ void sh_backward_one(const float* __restrict__ cgrad,
                                                const float* __restrict__ mu,
                                                const float* __restrict__ albedo, float* k,
                                                const float* __restrict__ cam,
                                                float* __restrict__ dA, size_t i, float dmu[3]) {
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
        // coefficients are consumed: reuse their slots for dk_j
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
    dmu[0] = inv * (gx - x * ddot);
    dmu[1] = inv * (gy - y * ddot);
    dmu[2] = inv * (gz - z * ddot);
}

// projection_backward.cu:11-140 for one Gaussian: dL/dmu through the mean and
// through J, dL/dlog-scale through exp, dL/dq through toMat3 and normalize;
// zeros for a culled Gaussian.  ref_quat selects the reference's literal
// quaternion formula, which reads transpose(dL/dR) with indices meant for
// dL/dR (it fails finite differences); 0 gives the derivative of glm::toMat3.
__device__ __forceinline__ void project_backward_one(
    const Pose& pose, const float* __restrict__ dmean, const float* __restrict__ dcov,
    const float* __restrict__ mu, const float* __restrict__ q, const float* __restrict__ s,
    float fx, float fy, int ref_quat, size_t i, float omu[3], float oq[4], float os[3]) {
    float mc[3];
    to_camera(pose, mu[3 * i], mu[3 * i + 1], mu[3 * i + 2], mc);
#pragma unroll
    for (int k = 0; k < 3; ++k) omu[k] = os[k] = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; ++k) oq[k] = 0.0f;
    if (mc[2] <= kNearZ) return;
    const float z = mc[2], z2 = z * z, z3 = z2 * z;
    const float gdx = dmean[2 * i], gdy = dmean[2 * i + 1];
    float dmc[3] = {(fx / z) * gdx, (fy / z) * gdy,
                    (-fx * mc[0] / z2) * gdx + (-fy * mc[1] / z2) * gdy};
    const float ga = dcov[3 * i], gb = dcov[3 * i + 1], gc = dcov[3 * i + 2];
    const float G00 = ga, G01 = 0.5f * gb, G10 = 0.5f * gb, G11 = gc;
    const float J[2][3] = {{fx / z, 0.0f, -(fx * mc[0]) / z2}, {0.0f, fy / z, -(fy * mc[1]) / z2}};
    const float4 qq = *reinterpret_cast<const float4*>(q + 4 * i);
    const Cov3 cv = covariance3d(pose, qq.x, qq.y, qq.z, qq.w, s[3 * i], s[3 * i + 1], s[3 * i + 2]);
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
    // quaternion (projection_backward.cu:116-127); L[i][j] is the value the
    // reference reads as dL_dRt[i][j].
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
    // through normalize (projection_backward.cu:129-138)
    const float inv_norm =
        1.0f / __builtin_sqrtf(qq.x * qq.x + qq.y * qq.y + qq.z * qq.z + qq.w * qq.w + 1e-8f);
    const float qdot = qw * gw + qx * gx + qy * gy + qz * gz;
    oq[0] = inv_norm * (gw - qw * qdot);
    oq[1] = inv_norm * (gx - qx * qdot);
    oq[2] = inv_norm * (gy - qy * qdot);
    oq[3] = inv_norm * (gz - qz * qdot);
}

}  // namespace gsr
