// gs_oracle.cpp — TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline).
//
// CPU restatement of the hot path of the reference rasterizer
// (kmurungi/custom-3dgs-cuda): projection, degree-3 SH colour, tile binning,
// stable 64-bit key sort, tile ranges, front-to-back alpha blend and the three
// backward passes.  Only tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg load this library; the HIP product never links it.
//
// Every function is templated on the real type:
//   * float  — the reference's fp32 semantics, operation by operation, in the
//              order the reference source writes them.  Built with
//              -ffp-contract=off so no multiply-add is fused except the
//              explicit fma calls: inside orc_expf, and in the blend's
//              power and colour sums, where they stand for the
//              multiply-adds nvcc forms from the reference's a * b + c
//              expressions by default (--fmad=true).  The HIP kernels
//              evaluate the same operations, so fp32 forward outputs agree
//              bit for bit.
//   * double — the same mathematics in float64 (std::exp), used for tight
//              finite-difference pins of the backward formulas.
//
// GLM (header-only, unpinned, not vendored by the reference) is restated with
// explicit scalar code: glm matrices are column-major (m[col][row]); every
// product below is written in math (row, col) form with the inner index
// summed left to right, which is what glm's operator* does.
//
// Pins (tests/test_oracle_*.py): closed forms (identity-rotation EWA
// covariance, SH band constants, isotropic blend), brute-force tile
// enumeration, std::stable_sort, finite differences in float64 against every
// backward formula, and the reference's own four gradcheck scenes.

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>
#include <parallel/algorithm>
#include <omp.h>

#define ORC_EXPORT extern "C" __attribute__((visibility("default")))

// ---------------------------------------------------------------------------
// exp: Cody–Waite two-constant range reduction (fdlibm's ln2 split,
// 0x3f317200 / 0x35bfbe8e) + degree-6 polynomial for e^r on [-ln2/2, ln2/2]
// (coefficients from a weighted least-squares fit on Chebyshev nodes,
// iterated towards minimax; custom-3dgs-cuda_amd/csrc/gen_exp_poly.py).
// Max error 0.955 ulp over every float in [-87.34, 88.72] (exhaustive sweep
// against float64 exp).  Results below FLT_MIN are flushed to +0.  The
// reference uses CUDA's __expf (rasterize.cu:255, rasterize_backward.cu:131)
// and expf (projection.cu:70-72); neither is reproducible on a CPU, so the
// build fixes this one function on host and device.
// ---------------------------------------------------------------------------
ORC_EXPORT float orc_expf(float x) {
    if (x > 88.72283935546875f) return std::numeric_limits<float>::infinity();
    if (!(x >= -87.33654022216796875f)) return (x != x) ? x : 0.0f;
    const float k = std::rint(x * 1.44269502162933349609375f);
    float r = std::fma(-k, 0.693145751953125f, x);
    r = std::fma(-k, 1.428606765330187045e-06f, r);
    float p = 0.0013766406336799264f;
    p = std::fma(p, r, 0.00837041437625885f);
    p = std::fma(p, r, 0.041669245809316635f);
    p = std::fma(p, r, 0.16666485369205475f);
    p = std::fma(p, r, 0.49999988079071045f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    return std::ldexp(p, (int)k);
}

ORC_EXPORT void orc_expf_array(int64_t n, const float* x, float* y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

namespace {

template <typename T> struct M;
template <> struct M<float> {
    static float exp(float x) { return orc_expf(x); }
    static float sqrt(float x) { return std::sqrt(x); }
};
template <> struct M<double> {
    static double exp(double x) { return std::exp(x); }
    static double sqrt(double x) { return std::sqrt(x); }
};

// 3x3 / 2x3 / 3x2 helpers in math (row, col) order; sums run left to right.
template <typename T>
void mm33(const T a[3][3], const T b[3][3], T c[3][3]) {
    for (int r = 0; r < 3; ++r)
        for (int k = 0; k < 3; ++k)
            c[r][k] = a[r][0] * b[0][k] + a[r][1] * b[1][k] + a[r][2] * b[2][k];
}
template <typename T>
void tr33(const T a[3][3], T c[3][3]) {
    for (int r = 0; r < 3; ++r)
        for (int k = 0; k < 3; ++k) c[r][k] = a[k][r];
}

// Saturating float -> int32 conversion with NaN -> 0: what a GPU's
// v_cvt_i32_f32 / PTX cvt.rzi.s32.f32 return for the casts at
// rasterize.cu:38-41 (x86 cvttss2si would return INT_MIN instead).
inline int f2i_sat(float x) {
    if (x != x) return 0;
    if (x >= 2147483648.0f) return 2147483647;
    if (x <= -2147483648.0f) return (-2147483647 - 1);
    return (int)x;
}

// Quaternion (w,x,y,z) -> rotation matrix after glm::normalize
// (projection.cu:64-65).  glm::dot(quat) sums (w*w + x*x) + (y*y + z*z);
// a non-positive length yields the identity quaternion.
template <typename T>
void quat_to_rot(const T* q4, T R[3][3], T qn[4]) {
    T w = q4[0], x = q4[1], y = q4[2], z = q4[3];
    T len = M<T>::sqrt((w * w + x * x) + (y * y + z * z));
    if (len <= T(0)) {
        w = T(1); x = T(0); y = T(0); z = T(0);
    } else {
        T inv = T(1) / len;
        w = w * inv; x = x * inv; y = y * inv; z = z * inv;
    }
    qn[0] = w; qn[1] = x; qn[2] = y; qn[3] = z;
    T qxx = x * x, qyy = y * y, qzz = z * z;
    T qxz = x * z, qxy = x * y, qyz = y * z;
    T qwx = w * x, qwy = w * y, qwz = w * z;
    // glm mat3_cast: Result[col][row]; written here as R[row][col].
    R[0][0] = T(1) - T(2) * (qyy + qzz);
    R[1][0] = T(2) * (qxy + qwz);
    R[2][0] = T(2) * (qxz - qwy);
    R[0][1] = T(2) * (qxy - qwz);
    R[1][1] = T(1) - T(2) * (qxx + qzz);
    R[2][1] = T(2) * (qyz + qwx);
    R[0][2] = T(2) * (qxz + qwy);
    R[1][2] = T(2) * (qyz - qwx);
    R[2][2] = T(1) - T(2) * (qxx + qyy);
}

template <typename T>
struct Cam {
    T R[3][3];
    T t[3];
};
template <typename T>
Cam<T> load_cam(const T* rot, const T* tr) {
    Cam<T> c;
    for (int r = 0; r < 3; ++r)
        for (int k = 0; k < 3; ++k) c.R[r][k] = rot[r * 3 + k];
    for (int i = 0; i < 3; ++i) c.t[i] = tr[i];
    return c;
}
template <typename T>
void world_to_cam(const Cam<T>& c, const T* mu, T out[3]) {
    for (int r = 0; r < 3; ++r)
        out[r] = (c.R[r][0] * mu[0] + c.R[r][1] * mu[1] + c.R[r][2] * mu[2]) + c.t[r];
}

// Sigma_world = (R S)(R S)^T and Sigma_cam = (R_cam Sigma_world) R_cam^T
// (projection.cu:69-81).  S = diag(exp(s)) is multiplied as a full matrix
// the way glm does; the zero products are kept so signed zeros agree.
template <typename T>
void covariances(const Cam<T>& c, const T* q4, const T* s3, T R[3][3], T S[3][3],
                 T Mm[3][3], T Sc[3][3], T qn[4]) {
    quat_to_rot(q4, R, qn);
    for (int r = 0; r < 3; ++r)
        for (int k = 0; k < 3; ++k) S[r][k] = T(0);
    S[0][0] = M<T>::exp(s3[0]);
    S[1][1] = M<T>::exp(s3[1]);
    S[2][2] = M<T>::exp(s3[2]);
    mm33(R, S, Mm);
    T Mt[3][3], Sw[3][3], A[3][3], Rt[3][3];
    tr33(Mm, Mt);
    mm33(Mm, Mt, Sw);
    mm33(c.R, Sw, A);
    tr33(c.R, Rt);
    mm33(A, Rt, Sc);
}

// ----- a1: projection (projection.cu:33-105) -------------------------------
template <typename T>
void project_one(const Cam<T>& c, const T* mu, const T* q4, const T* s3, T fx, T fy, T cx,
                 T cy, T* mean2d, T* cov2d, T* depth) {
    T mc[3];
    world_to_cam(c, mu, mc);
    mean2d[0] = mean2d[1] = T(0);
    cov2d[0] = cov2d[1] = cov2d[2] = T(0);
    *depth = T(0);
    if (mc[2] <= T(0.2f)) return;  // frustum cull, outputs stay zero
    *depth = mc[2];
    mean2d[0] = (fx * mc[0]) / mc[2] + cx;
    mean2d[1] = (fy * mc[1]) / mc[2] + cy;
    T R[3][3], S[3][3], Mm[3][3], Sc[3][3], qn[4];
    covariances(c, q4, s3, R, S, Mm, Sc, qn);
    T z2 = mc[2] * mc[2];
    T J00 = fx / mc[2];
    T J02 = -(fx * mc[0]) / z2;
    T J11 = fy / mc[2];
    T J12 = -(fy * mc[1]) / z2;
    // glm Sigma_cam[i][j] is (row j, col i).
    T a = J00 * (J00 * Sc[0][0] + J02 * Sc[0][2]) + J02 * (J00 * Sc[2][0] + J02 * Sc[2][2]);
    T b = J00 * (J11 * Sc[1][0] + J12 * Sc[2][0]) + J02 * (J11 * Sc[1][2] + J12 * Sc[2][2]);
    T cc = J11 * (J11 * Sc[1][1] + J12 * Sc[2][1]) + J12 * (J11 * Sc[1][2] + J12 * Sc[2][2]);
    a = a + T(0.3f);
    cc = cc + T(0.3f);
    cov2d[0] = a;
    cov2d[1] = b;
    cov2d[2] = cc;
}

template <typename T>
void project_all(int n, const T* mu, const T* q, const T* s, const T* rot, const T* tr, T fx,
                 T fy, T cx, T cy, T* mean2d, T* cov2d, T* depth) {
    Cam<T> c = load_cam(rot, tr);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i)
        project_one(c, mu + 3 * (size_t)i, q + 4 * (size_t)i, s + 3 * (size_t)i, fx, fy, cx, cy,
                    mean2d + 2 * (size_t)i, cov2d + 3 * (size_t)i, depth + i);
}

// ----- a2: SH colour (SH.cu:12-91) -----------------------------------------
constexpr double SH_C0 = 0.28209479177387814;
constexpr double SH_C1 = 0.4886025119029199;
constexpr double SH_C2_0 = 1.0925484305920792;
constexpr double SH_C2_1 = -1.0925484305920792;
constexpr double SH_C2_2 = 0.31539156525252005;
constexpr double SH_C2_3 = -1.0925484305920792;
constexpr double SH_C2_4 = 0.5462742152960396;
constexpr double SH_C3_0 = -0.5900435899266435;
constexpr double SH_C3_1 = 2.890611442640554;
constexpr double SH_C3_2 = -0.4570457994644658;
constexpr double SH_C3_3 = 0.3731763325901154;
constexpr double SH_C3_4 = -0.4570457994644658;
constexpr double SH_C3_5 = 1.445305721320277;
constexpr double SH_C3_6 = -0.5900435899266435;
// The reference's constants are float literals: round each once to T.
template <typename T> constexpr T K(double v) { return (T)(float)v; }

template <typename T>
void sh_basis(T x, T y, T z, T* Y) {
    Y[0] = -K<T>(SH_C1) * y;
    Y[1] = K<T>(SH_C1) * z;
    Y[2] = -K<T>(SH_C1) * x;
    T xx = x * x, yy = y * y, zz = z * z;
    T xy = x * y, yz = y * z, xz = x * z;
    Y[3] = K<T>(SH_C2_0) * xy;
    Y[4] = K<T>(SH_C2_1) * yz;
    Y[5] = K<T>(SH_C2_2) * (T(2) * zz - xx - yy);
    Y[6] = K<T>(SH_C2_3) * xz;
    Y[7] = K<T>(SH_C2_4) * (xx - yy);
    Y[8] = K<T>(SH_C3_0) * y * (T(3) * xx - yy);
    Y[9] = K<T>(SH_C3_1) * xy * z;
    Y[10] = K<T>(SH_C3_2) * y * (T(4) * zz - xx - yy);
    Y[11] = K<T>(SH_C3_3) * z * (T(2) * zz - T(3) * xx - T(3) * yy);
    Y[12] = K<T>(SH_C3_4) * x * (T(4) * zz - xx - yy);
    Y[13] = K<T>(SH_C3_5) * z * (xx - yy);
    Y[14] = K<T>(SH_C3_6) * x * (xx - T(3) * yy);
}

// rgb before the clamp: 0.5 + C0*A + sum_k Y_k k_j[k] (SH.cu:80-85).
template <typename T>
void sh_rgb(const T* Y, const T* A, const T* kj, T rgb[3]) {
    for (int ch = 0; ch < 3; ++ch) rgb[ch] = T(0.5f) + K<T>(SH_C0) * A[ch];
    for (int k = 0; k < 15; ++k)
        for (int ch = 0; ch < 3; ++ch) rgb[ch] = rgb[ch] + Y[k] * kj[k * 3 + ch];
}

template <typename T>
void sh_all(int n, const T* cam, const T* mu, const T* A, const T* kj, T* colors) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        const T* m = mu + 3 * (size_t)i;
        T v0 = m[0] - cam[0], v1 = m[1] - cam[1], v2 = m[2] - cam[2];
        // glm::normalize: v * (1 / sqrt(dot(v, v)))
        T inv = T(1) / M<T>::sqrt(v0 * v0 + v1 * v1 + v2 * v2);
        T Y[15], rgb[3];
        sh_basis(v0 * inv, v1 * inv, v2 * inv, Y);
        sh_rgb(Y, A + 3 * (size_t)i, kj + 45 * (size_t)i, rgb);
        for (int ch = 0; ch < 3; ++ch)
            colors[3 * (size_t)i + ch] = std::fmin(std::fmax(rgb[ch], T(0)), T(1));
    }
}

// ----- a3/a5: tile rectangle of one Gaussian (rasterize.cu:19-59) ----------
struct Rect {
    int x0, x1, y0, y1;
};
inline Rect tile_rect(const float* mean, const float* cov, int W, int H, bool* ok) {
    Rect r{0, 0, 0, 0};
    float a = cov[0], b = cov[1], c = cov[2];
    float det = a * c - b * b;
    *ok = false;
    if (det <= 0.0f) return r;
    float mid = 0.5f * (a + c);
    float lambda_max = mid + std::sqrt(std::fmax(0.1f, mid * mid - det));
    float radius = std::ceil(3.0f * std::sqrt(lambda_max));
    int min_x = std::max(0, f2i_sat(std::floor(mean[0] - radius)));
    int max_x = std::min(W, f2i_sat(std::ceil(mean[0] + radius)));
    int min_y = std::max(0, f2i_sat(std::floor(mean[1] - radius)));
    int max_y = std::min(H, f2i_sat(std::ceil(mean[1] + radius)));
    int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
    int mtx = min_x / 16, Mtx = (max_x + 15) / 16;
    int mty = min_y / 16, Mty = (max_y + 15) / 16;
    r.x0 = std::max(0, std::min(tiles_x, mtx));
    r.x1 = std::max(0, std::min(tiles_x, Mtx));
    r.y0 = std::max(0, std::min(tiles_y, mty));
    r.y1 = std::max(0, std::min(tiles_y, Mty));
    *ok = true;
    return r;
}
inline int rect_count(const Rect& r) {
    return std::max(0, r.x1 - r.x0) * std::max(0, r.y1 - r.y0);
}

// Conic = cov^-1 with 1/det computed first (rasterize.cu:224-232).
inline void conic_of(const float* cov, float* cn) {
    float det = cov[0] * cov[2] - cov[1] * cov[1];
    float det_inv = (det > 0.0f) ? (1.0f / det) : 0.0f;
    cn[0] = cov[2] * det_inv;
    cn[1] = -cov[1] * det_inv;
    cn[2] = cov[0] * det_inv;
}
template <typename T>
void conic_of_t(const T* cov, T* cn) {
    T det = cov[0] * cov[2] - cov[1] * cov[1];
    T det_inv = (det > T(0)) ? (T(1) / det) : T(0);
    cn[0] = cov[2] * det_inv;
    cn[1] = -cov[1] * det_inv;
    cn[2] = cov[0] * det_inv;
}

// power = -0.5 (cx dx^2 + 2 cy dx dy + cz dy^2) (rasterize.cu:249-251), the
// two additions fused: -0.5 fma(cz dy, dy, fma(2 cy dx, dy, (cx dx) dx)).
// The -0.5 is applied to the coefficients first (exact scalings by powers of
// two), which gives the same value: fma(c dy, dy, fma(b dx, dy, (a dx) dx))
// with a = -cx/2, b = -cy, c = -cz/2.
template <typename T>
inline T power_of(const T* cn, T dx, T dy) {
    const T a = T(-0.5f) * cn[0], b = -cn[1], c = T(-0.5f) * cn[2];
    return std::fma(c * dy, dy, std::fma(b * dx, dy, (a * dx) * dx));
}

// ----- a8: per-pixel front-to-back blend (rasterize.cu:184-280) ------------
template <typename T>
void blend_fwd_all(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                   const T* mean2d, const T* cov2d, const T* colors, const T* alpha, T* img,
                   T* finalT, int32_t* ncontrib) {
    const int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
#pragma omp parallel for schedule(dynamic, 4)
    for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
        const int tx = tile % tiles_x, ty = tile / tiles_x;
        const int start = ranges[2 * tile], end = ranges[2 * tile + 1];
        for (int ly = 0; ly < 16; ++ly)
            for (int lx = 0; lx < 16; ++lx) {
                const int px = tx * 16 + lx, py = ty * 16 + ly;
                if (px >= W || py >= H) continue;
                T C[3] = {T(0), T(0), T(0)};
                T Tr = T(1);
                int contributor = 0, last = 0;
                for (int i = start; i < end; ++i) {
                    ++contributor;
                    const int g = ids[i];
                    T cn[3];
                    conic_of_t(cov2d + 3 * (size_t)g, cn);
                    T dx = (T)px - mean2d[2 * (size_t)g];
                    T dy = (T)py - mean2d[2 * (size_t)g + 1];
                    T power = power_of(cn, dx, dy);
                    if (power > T(0)) continue;
                    T a = std::fmin(T(0.99f), alpha[g] * M<T>::exp(power));
                    if (a < T(1.0f / 255.0f)) continue;
                    T wgt = a * Tr;
                    // pix_color += colour * weight, fused (rasterize.cu:259-261)
                    for (int ch = 0; ch < 3; ++ch)
                        C[ch] = std::fma(colors[3 * (size_t)g + ch], wgt, C[ch]);
                    Tr = Tr * (T(1) - a);
                    last = contributor;
                    if (Tr < T(1e-4f)) break;
                }
                const size_t p = (size_t)py * W + px;
                for (int ch = 0; ch < 3; ++ch) img[3 * p + ch] = C[ch];
                finalT[p] = Tr;
                ncontrib[p] = last;
            }
    }
}

// ----- a10: per-pixel back-to-front gradient (rasterize_backward.cu:60-234) -
// Per-pixel arithmetic in T exactly as the reference; the per-Gaussian sums
// over pixels and tiles are accumulated in double (9 values per Gaussian:
// dmean 2, dconic 3, dcolor 3, dopacity 1), plus the matching sums of
// absolute values so tests can bound fp32 summation error.  The conic->cov
// conversion (rasterize_backward.cu:211-221) is linear in the summed conic
// gradient, so it is applied once per Gaussian to the total.
template <typename T>
void blend_bwd_all(int n, int H, int W, const T* grad, const T* mean2d, const T* cov2d,
                   const T* colors, const T* alpha, const int32_t* ids, const int32_t* ranges,
                   const T* finalT, const int32_t* ncontrib, double* acc9, double* abs9) {
    const int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
    const int nthreads = omp_get_max_threads();
    std::vector<std::vector<double>> part(nthreads), pabs(nthreads);
#pragma omp parallel
    {
        const int tid = omp_get_thread_num();
        std::vector<double>& acc = part[tid];
        std::vector<double>& ab = pabs[tid];
        acc.assign((size_t)n * 9, 0.0);
        if (abs9) ab.assign((size_t)n * 9, 0.0);
#pragma omp for schedule(dynamic, 4)
        for (int tile = 0; tile < tiles_x * tiles_y; ++tile) {
            const int tx = tile % tiles_x, ty = tile / tiles_x;
            const int start = ranges[2 * tile], end = ranges[2 * tile + 1];
            const int K = end - start;
            for (int ly = 0; ly < 16; ++ly)
                for (int lx = 0; lx < 16; ++lx) {
                    const int px = tx * 16 + lx, py = ty * 16 + ly;
                    if (px >= W || py >= H) continue;
                    const size_t p = (size_t)py * W + px;
                    const int last = ncontrib[p];
                    if (last == 0) continue;
                    T dLdC[3] = {grad[3 * p], grad[3 * p + 1], grad[3 * p + 2]};
                    T Tr = finalT[p];
                    T accr[3] = {T(0), T(0), T(0)};
                    for (int c = std::min(last, K); c >= 1; --c) {
                        const int g = ids[start + c - 1];
                        if (g < 0 || g >= n) continue;
                        T cn[3];
                        conic_of_t(cov2d + 3 * (size_t)g, cn);
                        T dx = (T)px - mean2d[2 * (size_t)g];
                        T dy = (T)py - mean2d[2 * (size_t)g + 1];
                        T power = power_of(cn, dx, dy);
                        if (power > T(0)) continue;
                        T G = M<T>::exp(power);
                        T araw = alpha[g] * G;
                        T a = std::fmin(T(0.99f), araw);
                        if (a < T(1.0f / 255.0f)) continue;
                        T om = T(1) - a;
                        T Tb = Tr / std::fmax(om, T(1e-4f));
                        const T* col = colors + 3 * (size_t)g;
                        T dcol[3] = {a * Tb * dLdC[0], a * Tb * dLdC[1], a * Tb * dLdC[2]};
                        T dal = ((col[0] - accr[0]) * dLdC[0] + (col[1] - accr[1]) * dLdC[1] +
                                 (col[2] - accr[2]) * dLdC[2]) *
                                Tb;
                        T dop = T(0), dpw = T(0);
                        if (araw < T(0.99f)) {
                            dop = G * dal;
                            dpw = a * dal;
                        }
                        T v[9];
                        v[0] = dpw * (cn[0] * dx + cn[1] * dy);
                        v[1] = dpw * (cn[1] * dx + cn[2] * dy);
                        v[2] = T(-0.5f) * dpw * dx * dx;
                        v[3] = -dpw * dx * dy;
                        v[4] = T(-0.5f) * dpw * dy * dy;
                        v[5] = dcol[0];
                        v[6] = dcol[1];
                        v[7] = dcol[2];
                        v[8] = dop;
                        double* dst = &acc[(size_t)g * 9];
                        for (int k = 0; k < 9; ++k) dst[k] += (double)v[k];
                        if (abs9) {
                            double* da = &ab[(size_t)g * 9];
                            for (int k = 0; k < 9; ++k) da[k] += std::fabs((double)v[k]);
                        }
                        for (int ch = 0; ch < 3; ++ch) accr[ch] = a * col[ch] + om * accr[ch];
                        Tr = Tb;
                        if (c == 1) break;
                    }
                }
        }
    }
    for (size_t i = 0; i < (size_t)n * 9; ++i) {
        double s = 0.0, sa = 0.0;
        for (int t = 0; t < nthreads; ++t) {
            s += part[t][i];
            if (abs9) sa += pabs[t][i];
        }
        acc9[i] = s;
        if (abs9) abs9[i] = sa;
    }
    // conic gradient -> covariance gradient (packed a, b, c; b carries both
    // off-diagonals): dSigma = -V Gs V with Gs = [[gx, gy/2], [gy/2, gz]].
    for (int g = 0; g < n; ++g) {
        double cn[3];
        T cnt[3];
        conic_of_t(cov2d + 3 * (size_t)g, cnt);
        for (int k = 0; k < 3; ++k) cn[k] = (double)cnt[k];
        double* d = acc9 + (size_t)g * 9;
        double gx = d[2], gy = 0.5 * d[3], gz = d[4];
        double vx = cn[0], vy = cn[1], vz = cn[2];
        d[2] = -(vx * vx * gx + 2.0 * vx * vy * gy + vy * vy * gz);
        d[3] = -2.0 * (vx * vy * gx + (vx * vz + vy * vy) * gy + vy * vz * gz);
        d[4] = -(vy * vy * gx + 2.0 * vy * vz * gy + vz * vz * gz);
        if (abs9) {
            double* a = abs9 + (size_t)g * 9;
            double ax = a[2], ay = 0.5 * a[3], az = a[4];
            double ux = std::fabs(vx), uy = std::fabs(vy), uz = std::fabs(vz);
            a[2] = ux * ux * ax + 2.0 * ux * uy * ay + uy * uy * az;
            a[3] = 2.0 * (ux * uy * ax + (ux * uz + uy * uy) * ay + uy * uz * az);
            a[4] = uy * uy * ax + 2.0 * uy * uz * ay + uz * uz * az;
        }
    }
}

// ----- a11: SH backward (delight_backward.cu:107-173) ----------------------
template <typename T>
void sh_bwd_all(int n, const T* cgrad, const T* mu, const T* A, const T* kj, const T* cam,
                T* dA, T* dkj, T* dmu) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        const T* m = mu + 3 * (size_t)i;
        const T* kk = kj + 45 * (size_t)i;
        T v[3] = {m[0] - cam[0], m[1] - cam[1], m[2] - cam[2]};
        T inv = T(1) / M<T>::sqrt(v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + T(1e-8f));
        T d[3] = {v[0] * inv, v[1] * inv, v[2] * inv};
        T Y[15], rgb[3];
        sh_basis(d[0], d[1], d[2], Y);
        sh_rgb(Y, A + 3 * (size_t)i, kk, rgb);
        T g[3];
        for (int ch = 0; ch < 3; ++ch)
            g[ch] = (rgb[ch] < T(0) || rgb[ch] > T(1)) ? T(0) : cgrad[3 * (size_t)i + ch];
        for (int ch = 0; ch < 3; ++ch) dA[3 * (size_t)i + ch] = g[ch] * K<T>(SH_C0);
        T dY[15];
        for (int k = 0; k < 15; ++k) {
            for (int ch = 0; ch < 3; ++ch) dkj[45 * (size_t)i + k * 3 + ch] = g[ch] * Y[k];
            dY[k] = g[0] * kk[k * 3 + 0] + g[1] * kk[k * 3 + 1] + g[2] * kk[k * 3 + 2];
        }
        const T x = d[0], y = d[1], z = d[2];
        const T xx = x * x, yy = y * y, zz = z * z;
        T gx = T(0), gy = T(0), gz = T(0);
        // accumulate_dY_ddir (delight_backward.cu:50-105), same term order.
        gy += dY[0] * (-K<T>(SH_C1));
        gz += dY[1] * (K<T>(SH_C1));
        gx += dY[2] * (-K<T>(SH_C1));
        gx += dY[3] * (K<T>(SH_C2_0) * y);
        gy += dY[3] * (K<T>(SH_C2_0) * x);
        gy += dY[4] * (K<T>(SH_C2_1) * z);
        gz += dY[4] * (K<T>(SH_C2_1) * y);
        gx += dY[5] * (T(-2) * K<T>(SH_C2_2) * x);
        gy += dY[5] * (T(-2) * K<T>(SH_C2_2) * y);
        gz += dY[5] * (T(4) * K<T>(SH_C2_2) * z);
        gx += dY[6] * (K<T>(SH_C2_3) * z);
        gz += dY[6] * (K<T>(SH_C2_3) * x);
        gx += dY[7] * (T(2) * K<T>(SH_C2_4) * x);
        gy += dY[7] * (T(-2) * K<T>(SH_C2_4) * y);
        gx += dY[8] * (K<T>(SH_C3_0) * y * T(6) * x);
        gy += dY[8] * (K<T>(SH_C3_0) * (T(3) * xx - T(3) * yy));
        gx += dY[9] * (K<T>(SH_C3_1) * y * z);
        gy += dY[9] * (K<T>(SH_C3_1) * x * z);
        gz += dY[9] * (K<T>(SH_C3_1) * x * y);
        gx += dY[10] * (K<T>(SH_C3_2) * y * (T(-2) * x));
        gy += dY[10] * (K<T>(SH_C3_2) * (T(4) * zz - xx - T(3) * yy));
        gz += dY[10] * (K<T>(SH_C3_2) * y * T(8) * z);
        gx += dY[11] * (K<T>(SH_C3_3) * z * (T(-6) * x));
        gy += dY[11] * (K<T>(SH_C3_3) * z * (T(-6) * y));
        gz += dY[11] * (K<T>(SH_C3_3) * (T(6) * zz - T(3) * xx - T(3) * yy));
        gx += dY[12] * (K<T>(SH_C3_4) * (T(4) * zz - T(3) * xx - yy));
        gy += dY[12] * (K<T>(SH_C3_4) * x * (T(-2) * y));
        gz += dY[12] * (K<T>(SH_C3_4) * x * T(8) * z);
        gx += dY[13] * (K<T>(SH_C3_5) * z * T(2) * x);
        gy += dY[13] * (K<T>(SH_C3_5) * z * (T(-2) * y));
        gz += dY[13] * (K<T>(SH_C3_5) * (xx - yy));
        gx += dY[14] * (K<T>(SH_C3_6) * (T(3) * xx - T(3) * yy));
        gy += dY[14] * (K<T>(SH_C3_6) * x * (T(-6) * y));
        // d(normalize)/dv = (I - d d^T) / |v|
        T ddot = x * gx + y * gy + z * gz;
        dmu[3 * (size_t)i + 0] = inv * (gx - x * ddot);
        dmu[3 * (size_t)i + 1] = inv * (gy - y * ddot);
        dmu[3 * (size_t)i + 2] = inv * (gz - z * ddot);
    }
}

// ----- a12: projection backward (projection_backward.cu:33-138) ------------
// ref_quat = 1 evaluates the reference's quaternion formula literally
// (projection_backward.cu:116-127): it indexes transpose(dL/dR) with the
// index pattern of a formula derived for dL/dR itself, so every term that
// multiplies w changes sign and the result fails finite differences (the
// reference's own test_projection_backward_matches_finite_differences).
// ref_quat = 0 (the default everywhere) feeds dL/dR so the same
// formula gives the derivative of glm::toMat3.
template <typename T>
void proj_bwd_all(int n, const T* dmean, const T* dcov, const T* mu, const T* q, const T* s,
                  const T* rot, const T* tr, T fx, T fy, T cx, T cy, T* dmu, T* dq, T* ds,
                  int ref_quat) {
    (void)cx;
    (void)cy;
    Cam<T> c = load_cam(rot, tr);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        T* omu = dmu + 3 * (size_t)i;
        T* oq = dq + 4 * (size_t)i;
        T* os = ds + 3 * (size_t)i;
        for (int k = 0; k < 3; ++k) omu[k] = os[k] = T(0);
        for (int k = 0; k < 4; ++k) oq[k] = T(0);
        T mc[3];
        world_to_cam(c, mu + 3 * (size_t)i, mc);
        if (mc[2] <= T(0.2f)) continue;
        const T z = mc[2], z2 = z * z, z3 = z2 * z;
        const T gdx = dmean[2 * (size_t)i], gdy = dmean[2 * (size_t)i + 1];
        T dmc[3] = {(fx / z) * gdx, (fy / z) * gdy,
                    (-fx * mc[0] / z2) * gdx + (-fy * mc[1] / z2) * gdy};
        const T ga = dcov[3 * (size_t)i], gb = dcov[3 * (size_t)i + 1], gc = dcov[3 * (size_t)i + 2];
        const T G[2][2] = {{ga, T(0.5f) * gb}, {T(0.5f) * gb, gc}};
        // J as the 2x3 math matrix of glm::mat3x2 J(fx/z, 0, 0, fy/z, J02, J12)
        const T J[2][3] = {{fx / z, T(0), -(fx * mc[0]) / z2}, {T(0), fy / z, -(fy * mc[1]) / z2}};
        T R[3][3], S[3][3], Mm[3][3], Sc[3][3], qn[4];
        covariances(c, q + 4 * (size_t)i, s + 3 * (size_t)i, R, S, Mm, Sc, qn);
        // dl_dcam = (J^T G) J
        T JtG[3][2], dcam[3][3];
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 2; ++k) JtG[r][k] = J[0][r] * G[0][k] + J[1][r] * G[1][k];
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 3; ++k) dcam[r][k] = JtG[r][0] * J[0][k] + JtG[r][1] * J[1][k];
        // dl_dworld = (R_cam^T dl_dcam) R_cam
        T Rct[3][3], tmp[3][3], dw[3][3];
        tr33(c.R, Rct);
        mm33(Rct, dcam, tmp);
        mm33(tmp, c.R, dw);
        // dl_dM = (2 dl_dworld) M ; dl_dR = dl_dM S ; dl_dS = R^T dl_dM
        T dw2[3][3], dM[3][3], dR[3][3], Rt[3][3], dS[3][3];
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 3; ++k) dw2[r][k] = T(2) * dw[r][k];
        mm33(dw2, Mm, dM);
        mm33(dM, S, dR);
        tr33(R, Rt);
        mm33(Rt, dM, dS);
        os[0] = dS[0][0] * S[0][0];
        os[1] = dS[1][1] * S[1][1];
        os[2] = dS[2][2] * S[2][2];
        // dL/dJ = ((2 G) J) Sigma_cam  (2x3)
        T G2[2][2] = {{T(2) * G[0][0], T(2) * G[0][1]}, {T(2) * G[1][0], T(2) * G[1][1]}};
        T GJ[2][3], dJ[2][3];
        for (int r = 0; r < 2; ++r)
            for (int k = 0; k < 3; ++k) GJ[r][k] = G2[r][0] * J[0][k] + G2[r][1] * J[1][k];
        for (int r = 0; r < 2; ++r)
            for (int k = 0; k < 3; ++k)
                dJ[r][k] = GJ[r][0] * Sc[0][k] + GJ[r][1] * Sc[1][k] + GJ[r][2] * Sc[2][k];
        const T dJ00 = dJ[0][0], dJ11 = dJ[1][1], dJ02 = dJ[0][2], dJ12 = dJ[1][2];
        dmc[0] = dmc[0] + dJ02 * (-fx / z2);
        dmc[1] = dmc[1] + dJ12 * (-fy / z2);
        dmc[2] = dmc[2] + (dJ00 * (-fx / z2) + dJ11 * (-fy / z2) + dJ02 * (T(2) * fx * mc[0] / z3) +
                           dJ12 * (T(2) * fy * mc[1] / z3));
        // dmu_world = R_cam^T dmu_cam
        for (int r = 0; r < 3; ++r)
            omu[r] = Rct[r][0] * dmc[0] + Rct[r][1] * dmc[1] + Rct[r][2] * dmc[2];
        // quaternion: L[i][j] is what the reference reads as dL_dRt[i][j]
        T L[3][3];
        for (int r = 0; r < 3; ++r)
            for (int k = 0; k < 3; ++k) L[r][k] = ref_quat ? dR[r][k] : dR[k][r];
        const T qw = qn[0], qx = qn[1], qy = qn[2], qz = qn[3];
        T gw = T(2) * qz * (L[0][1] - L[1][0]) + T(2) * qy * (L[2][0] - L[0][2]) +
               T(2) * qx * (L[1][2] - L[2][1]);
        T gxq = T(2) * qy * (L[1][0] + L[0][1]) + T(2) * qz * (L[2][0] + L[0][2]) +
                T(2) * qw * (L[1][2] - L[2][1]) - T(4) * qx * (L[2][2] + L[1][1]);
        T gyq = T(2) * qx * (L[1][0] + L[0][1]) + T(2) * qw * (L[2][0] - L[0][2]) +
                T(2) * qz * (L[1][2] + L[2][1]) - T(4) * qy * (L[2][2] + L[0][0]);
        T gzq = T(2) * qw * (L[0][1] - L[1][0]) + T(2) * qx * (L[2][0] + L[0][2]) +
                T(2) * qy * (L[1][2] + L[2][1]) - T(4) * qz * (L[1][1] + L[0][0]);
        // through normalize (projection_backward.cu:129-138)
        const T* qr = q + 4 * (size_t)i;
        T inv_norm = T(1) / M<T>::sqrt(qr[0] * qr[0] + qr[1] * qr[1] + qr[2] * qr[2] +
                                       qr[3] * qr[3] + T(1e-8f));
        T qdot = qw * gw + qx * gxq + qy * gyq + qz * gzq;
        oq[0] = inv_norm * (gw - qw * qdot);
        oq[1] = inv_norm * (gxq - qx * qdot);
        oq[2] = inv_norm * (gyq - qy * qdot);
        oq[3] = inv_norm * (gzq - qz * qdot);
    }
}

}  // namespace

// =========================== exported entry points ==========================

ORC_EXPORT int orc_num_threads(void) { return omp_get_max_threads(); }
ORC_EXPORT void orc_set_num_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

ORC_EXPORT void orc_project_f32(int n, const float* mu, const float* q, const float* s,
                                const float* rot, const float* tr, float fx, float fy, float cx,
                                float cy, float* mean2d, float* cov2d, float* depth) {
    project_all<float>(n, mu, q, s, rot, tr, fx, fy, cx, cy, mean2d, cov2d, depth);
}
ORC_EXPORT void orc_project_f64(int n, const double* mu, const double* q, const double* s,
                                const double* rot, const double* tr, double fx, double fy,
                                double cx, double cy, double* mean2d, double* cov2d,
                                double* depth) {
    project_all<double>(n, mu, q, s, rot, tr, fx, fy, cx, cy, mean2d, cov2d, depth);
}
ORC_EXPORT void orc_sh_f32(int n, const float* cam, const float* mu, const float* A,
                           const float* kj, float* colors) {
    sh_all<float>(n, cam, mu, A, kj, colors);
}
ORC_EXPORT void orc_sh_f64(int n, const double* cam, const double* mu, const double* A,
                           const double* kj, double* colors) {
    sh_all<double>(n, cam, mu, A, kj, colors);
}

// a3: overlap counts (rasterize.cu:19-60); rect4 (optional) gets the
// clamped tile rectangle [x0, x1) x [y0, y1) per Gaussian.
ORC_EXPORT void orc_bin_count(int n, const float* mean2d, const float* cov2d, int H, int W,
                              int32_t* counts, int32_t* rect4) {
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        bool ok;
        Rect r = tile_rect(mean2d + 2 * (size_t)i, cov2d + 3 * (size_t)i, W, H, &ok);
        counts[i] = ok ? rect_count(r) : 0;
        if (rect4) {
            rect4[4 * (size_t)i + 0] = r.x0;
            rect4[4 * (size_t)i + 1] = r.x1;
            rect4[4 * (size_t)i + 2] = r.y0;
            rect4[4 * (size_t)i + 3] = r.y1;
        }
    }
}

// a4+a5: exclusive scan of counts, then Gaussian-major key emission,
// ty outer / tx inner (rasterize.cu:124-135).  Returns M.  keys/ids may be
// null to only compute M.
ORC_EXPORT int64_t orc_emit_keys(int n, const float* mean2d, const float* cov2d,
                                 const float* depth, int H, int W, uint64_t* keys, int32_t* ids) {
    std::vector<int32_t> counts(n);
    orc_bin_count(n, mean2d, cov2d, H, W, counts.data(), nullptr);
    std::vector<int64_t> off((size_t)n + 1, 0);
    for (int i = 0; i < n; ++i) off[i + 1] = off[i] + counts[i];
    const int64_t m = off[n];
    if (!keys || !ids) return m;
    const int tiles_x = (W + 15) / 16;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        if (counts[i] == 0) continue;
        bool ok;
        Rect r = tile_rect(mean2d + 2 * (size_t)i, cov2d + 3 * (size_t)i, W, H, &ok);
        uint32_t dbits;
        std::memcpy(&dbits, depth + i, 4);
        int64_t slot = off[i];
        for (int ty = r.y0; ty < r.y1; ++ty)
            for (int tx = r.x0; tx < r.x1; ++tx) {
                uint64_t tile = (uint64_t)(ty * tiles_x + tx);
                keys[slot] = (tile << 32) | (uint64_t)dbits;
                ids[slot] = i;
                ++slot;
            }
    }
    return m;
}

// a6: stable ascending sort of (key, id) pairs by all 64 key bits
// (cub::DeviceRadixSort::SortPairs, rasterize.cu:423-435).
ORC_EXPORT void orc_sort_pairs(int64_t m, uint64_t* keys, int32_t* ids) {
    struct P {
        uint64_t k;
        int32_t v;
    };
    std::vector<P> buf((size_t)m);
    for (int64_t i = 0; i < m; ++i) buf[i] = P{keys[i], ids[i]};
    __gnu_parallel::stable_sort(buf.begin(), buf.end(),
                                [](const P& a, const P& b) { return a.k < b.k; });
    for (int64_t i = 0; i < m; ++i) {
        keys[i] = buf[i].k;
        ids[i] = buf[i].v;
    }
}

// a7: per-tile [start, end) from sorted keys; unseen tiles stay (0, 0)
// (identify_tile_ranges_kernel, rasterize.cu:140-166).
ORC_EXPORT void orc_tile_ranges(int64_t m, const uint64_t* skeys, int T, int32_t* ranges) {
    std::memset(ranges, 0, sizeof(int32_t) * 2 * (size_t)T);
    for (int64_t i = 0; i < m; ++i) {
        uint32_t cur = (uint32_t)(skeys[i] >> 32);
        if (i == 0) {
            ranges[2 * (size_t)cur] = 0;
        } else {
            uint32_t prev = (uint32_t)(skeys[i - 1] >> 32);
            if (cur != prev) {
                ranges[2 * (size_t)prev + 1] = (int32_t)i;
                ranges[2 * (size_t)cur] = (int32_t)i;
            }
        }
        if (i == m - 1) ranges[2 * (size_t)cur + 1] = (int32_t)m;
    }
}

ORC_EXPORT void orc_blend_fwd_f32(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                                  const float* mean2d, const float* cov2d, const float* colors,
                                  const float* alpha, float* img, float* finalT,
                                  int32_t* ncontrib) {
    blend_fwd_all<float>(n, H, W, ranges, ids, mean2d, cov2d, colors, alpha, img, finalT,
                         ncontrib);
}
ORC_EXPORT void orc_blend_fwd_f64(int n, int H, int W, const int32_t* ranges, const int32_t* ids,
                                  const double* mean2d, const double* cov2d, const double* colors,
                                  const double* alpha, double* img, double* finalT,
                                  int32_t* ncontrib) {
    blend_fwd_all<double>(n, H, W, ranges, ids, mean2d, cov2d, colors, alpha, img, finalT,
                          ncontrib);
}

// acc9/abs9: [n, 9] = (dmean2d x, y | dcov2d a, b, c | dcolor r, g, b | dalpha)
ORC_EXPORT void orc_blend_bwd_f32(int n, int H, int W, const float* grad, const float* mean2d,
                                  const float* cov2d, const float* colors, const float* alpha,
                                  const int32_t* ids, const int32_t* ranges, const float* finalT,
                                  const int32_t* ncontrib, double* acc9, double* abs9) {
    blend_bwd_all<float>(n, H, W, grad, mean2d, cov2d, colors, alpha, ids, ranges, finalT,
                         ncontrib, acc9, abs9);
}
ORC_EXPORT void orc_blend_bwd_f64(int n, int H, int W, const double* grad, const double* mean2d,
                                  const double* cov2d, const double* colors, const double* alpha,
                                  const int32_t* ids, const int32_t* ranges, const double* finalT,
                                  const int32_t* ncontrib, double* acc9, double* abs9) {
    blend_bwd_all<double>(n, H, W, grad, mean2d, cov2d, colors, alpha, ids, ranges, finalT,
                          ncontrib, acc9, abs9);
}

ORC_EXPORT void orc_sh_bwd_f32(int n, const float* cgrad, const float* mu, const float* A,
                               const float* kj, const float* cam, float* dA, float* dkj,
                               float* dmu) {
    sh_bwd_all<float>(n, cgrad, mu, A, kj, cam, dA, dkj, dmu);
}
ORC_EXPORT void orc_sh_bwd_f64(int n, const double* cgrad, const double* mu, const double* A,
                               const double* kj, const double* cam, double* dA, double* dkj,
                               double* dmu) {
    sh_bwd_all<double>(n, cgrad, mu, A, kj, cam, dA, dkj, dmu);
}

ORC_EXPORT void orc_project_bwd_f32(int n, const float* dmean, const float* dcov, const float* mu,
                                    const float* q, const float* s, const float* rot,
                                    const float* tr, float fx, float fy, float cx, float cy,
                                    float* dmu, float* dq, float* ds, int ref_quat) {
    proj_bwd_all<float>(n, dmean, dcov, mu, q, s, rot, tr, fx, fy, cx, cy, dmu, dq, ds, ref_quat);
}
ORC_EXPORT void orc_project_bwd_f64(int n, const double* dmean, const double* dcov,
                                    const double* mu, const double* q, const double* s,
                                    const double* rot, const double* tr, double fx, double fy,
                                    double cx, double cy, double* dmu, double* dq, double* ds,
                                    int ref_quat) {
    proj_bwd_all<double>(n, dmean, dcov, mu, q, s, rot, tr, fx, fy, cx, cy, dmu, dq, ds,
                         ref_quat);
}

// ---- the trainer's optimizer step: torch.optim.Adam (the reference's
// utils/optim.py:12-31, eps 1e-15, default betas) on an fp32 tensor, followed
// by the trainer's clamps of the updated parameter (scripts/train.py:171-176,
// utils/adc.py:90-93).  Two paths of torch/optim/adam.py, which differ only in
// rounding:
//   device (_multi_tensor_adam, the default on the GPU, where the trainer runs;
//   device_path != 0):
//     m = fma(1 - b1, g - m, m)               _foreach_lerp_
//     v = fma(1 - b2, g g, v b2)              _foreach_mul_, _foreach_addcmul_
//     p = fma(-(lr / (1 - b1^t)), m / d, p)   _foreach_addcdiv_
//   CPU (_single_tensor_adam):
//     m = fma(1 - b1, g - m, m)               exp_avg.lerp_(grad, 1 - b1)
//     v = fma((1 - b2) g, g, v b2)            exp_avg_sq.mul_(b2).addcmul_(grad, grad, 1 - b2)
//     p = p + (-(lr / (1 - b1^t)) m) / d      param.addcdiv_(exp_avg, denom, -step_size)
// with d = sqrt(v) / sqrt(1 - b2^t) + eps and then p = min(max(p, lo), hi),
// NaN kept (param.clamp_(lo, hi)).  The scalars are formed in double (Python
// floats) and rounded to fp32 once, as torch does when it applies a Python
// scalar to an fp32 tensor; the fused multiply-adds are the ones torch's
// kernels form (the CPU path pinned against torch on the CPU in
// tests/test_oracle_adam.py, the device path against torch on the GPU in
// tests/test_gpu_optim.py).
ORC_EXPORT void orc_adam_step_f32(int64_t n, float* p, const float* g, float* m, float* v,
                                  double lr, double beta1, double beta2, double eps, int64_t step,
                                  float lo, float hi, int device_path) {
    const float w1 = (float)(1.0 - beta1), b2 = (float)beta2, w2 = (float)(1.0 - beta2);
    const double bc1 = 1.0 - std::pow(beta1, (double)step);
    const double bc2 = 1.0 - std::pow(beta2, (double)step);
    const float neg_step = (float)(-(lr / bc1));
    const float bc2s = (float)std::sqrt(bc2);
    const float e = (float)eps;
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        const float gi = g[i];
        const float mi = std::fma(w1, gi - m[i], m[i]);
        const float vi = device_path ? std::fma(w2, gi * gi, v[i] * b2)
                                     : std::fma(w2 * gi, gi, v[i] * b2);
        const float d = std::sqrt(vi) / bc2s + e;
        float pi = device_path ? std::fma(neg_step, mi / d, p[i]) : p[i] + (neg_step * mi) / d;
        pi = (pi < lo) ? lo : pi;
        pi = (pi > hi) ? hi : pi;
        m[i] = mi;
        v[i] = vi;
        p[i] = pi;
    }
}
