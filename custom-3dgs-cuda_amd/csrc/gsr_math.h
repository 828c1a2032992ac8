// gsr_math.h — per-Gaussian fp32 math shared by the forward and backward
// kernels: camera transform, quaternion rotation, 3D/2D covariance and the
// degree-3 SH basis.  Matrices are plain row-major float[3][3] in math
// (row, col) order; every dot product sums its terms left to right, the order
// glm's operator* uses in the reference (projection.cu:33-105, SH.cu:31-55).
#pragma once

#include "gsr_common.h"

namespace gsr {

struct Mat3 {
    float m[3][3];
};

__device__ __forceinline__ Mat3 mul(const Mat3& a, const Mat3& b) {
    Mat3 c;
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k)
            c.m[r][k] = a.m[r][0] * b.m[0][k] + a.m[r][1] * b.m[1][k] + a.m[r][2] * b.m[2][k];
    return c;
}

__device__ __forceinline__ Mat3 transpose(const Mat3& a) {
    Mat3 c;
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) c.m[r][k] = a.m[k][r];
    return c;
}

// World-to-camera pose: rows of R (row-major [3,3]) and t [3].
struct Pose {
    Mat3 R;
    float t[3];
};

__device__ __forceinline__ Pose load_pose(const float* __restrict__ rot,
                                          const float* __restrict__ tr) {
    Pose p;
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) p.R.m[r][k] = rot[r * 3 + k];
#pragma unroll
    for (int i = 0; i < 3; ++i) p.t[i] = tr[i];
    return p;
}

__device__ __forceinline__ void to_camera(const Pose& p, float x, float y, float z,
                                          float out[3]) {
#pragma unroll
    for (int r = 0; r < 3; ++r)
        out[r] = (p.R.m[r][0] * x + p.R.m[r][1] * y + p.R.m[r][2] * z) + p.t[r];
}

// glm::normalize(quat (w,x,y,z)) then glm::toMat3 (projection.cu:64-65).
// The quaternion dot is (w*w + x*x) + (y*y + z*z); length <= 0 gives identity.
__device__ __forceinline__ Mat3 quat_rotation(float w, float x, float y, float z,
                                              float qn[4]) {
    const float len = __builtin_sqrtf((w * w + x * x) + (y * y + z * z));
    if (len <= 0.0f) {
        w = 1.0f; x = 0.0f; y = 0.0f; z = 0.0f;
    } else {
        const float inv = 1.0f / len;
        w = w * inv; x = x * inv; y = y * inv; z = z * inv;
    }
    qn[0] = w; qn[1] = x; qn[2] = y; qn[3] = z;
    const float qxx = x * x, qyy = y * y, qzz = z * z;
    const float qxz = x * z, qxy = x * y, qyz = y * z;
    const float qwx = w * x, qwy = w * y, qwz = w * z;
    Mat3 R;
    R.m[0][0] = 1.0f - 2.0f * (qyy + qzz);
    R.m[1][0] = 2.0f * (qxy + qwz);
    R.m[2][0] = 2.0f * (qxz - qwy);
    R.m[0][1] = 2.0f * (qxy - qwz);
    R.m[1][1] = 1.0f - 2.0f * (qxx + qzz);
    R.m[2][1] = 2.0f * (qyz + qwx);
    R.m[0][2] = 2.0f * (qxz + qwy);
    R.m[1][2] = 2.0f * (qyz - qwx);
    R.m[2][2] = 1.0f - 2.0f * (qxx + qyy);
    return R;
}

// R, S = diag(exp s) as a full matrix, M = R S, and
// Sigma_cam = (R_cam (M M^T)) R_cam^T (projection.cu:63-81).
struct Cov3 {
    Mat3 R, S, M, Sc;
    float qn[4];
};

__device__ __forceinline__ Cov3 covariance3d(const Pose& pose, float qw, float qx, float qy,
                                             float qz, float s0, float s1, float s2) {
    Cov3 c;
    c.R = quat_rotation(qw, qx, qy, qz, c.qn);
#pragma unroll
    for (int r = 0; r < 3; ++r)
#pragma unroll
        for (int k = 0; k < 3; ++k) c.S.m[r][k] = 0.0f;
    c.S.m[0][0] = exp_gs(s0);
    c.S.m[1][1] = exp_gs(s1);
    c.S.m[2][2] = exp_gs(s2);
    c.M = mul(c.R, c.S);
    const Mat3 Sw = mul(c.M, transpose(c.M));
    c.Sc = mul(mul(pose.R, Sw), transpose(pose.R));
    return c;
}

// SH band constants (SH.cu:12-28), rounded to fp32 like the reference's literals.
constexpr float SH_C0 = 0.28209479177387814f;
constexpr float SH_C1 = 0.4886025119029199f;
constexpr float SH_C2_0 = 1.0925484305920792f;
constexpr float SH_C2_1 = -1.0925484305920792f;
constexpr float SH_C2_2 = 0.31539156525252005f;
constexpr float SH_C2_3 = -1.0925484305920792f;
constexpr float SH_C2_4 = 0.5462742152960396f;
constexpr float SH_C3_0 = -0.5900435899266435f;
constexpr float SH_C3_1 = 2.890611442640554f;
constexpr float SH_C3_2 = -0.4570457994644658f;
constexpr float SH_C3_3 = 0.3731763325901154f;
constexpr float SH_C3_4 = -0.4570457994644658f;
constexpr float SH_C3_5 = 1.445305721320277f;
constexpr float SH_C3_6 = -0.5900435899266435f;

// The 15 basis values of bands 1..3 at unit direction (x, y, z) (SH.cu:31-55).
__device__ __forceinline__ void sh_basis15(float x, float y, float z, float Y[15]) {
    Y[0] = -SH_C1 * y;
    Y[1] = SH_C1 * z;
    Y[2] = -SH_C1 * x;
    const float xx = x * x, yy = y * y, zz = z * z;
    const float xy = x * y, yz = y * z, xz = x * z;
    Y[3] = SH_C2_0 * xy;
    Y[4] = SH_C2_1 * yz;
    Y[5] = SH_C2_2 * (2.0f * zz - xx - yy);
    Y[6] = SH_C2_3 * xz;
    Y[7] = SH_C2_4 * (xx - yy);
    Y[8] = SH_C3_0 * y * (3.0f * xx - yy);
    Y[9] = SH_C3_1 * xy * z;
    Y[10] = SH_C3_2 * y * (4.0f * zz - xx - yy);
    Y[11] = SH_C3_3 * z * (2.0f * zz - 3.0f * xx - 3.0f * yy);
    Y[12] = SH_C3_4 * x * (4.0f * zz - xx - yy);
    Y[13] = SH_C3_5 * z * (xx - yy);
    Y[14] = SH_C3_6 * x * (xx - 3.0f * yy);
}

}  // namespace gsr
