// gsr_export.hip — the Inria 3DGS vertex records of a PLY export
// (scripts/run.py:66-165 of kmurungi/custom-3dgs-cuda, save_ply), packed on the
// device so the host writes the file body with one copy.
//
// Record of Gaussian n, 17 + 3K fp32 (K rest SH coefficients per channel):
//   x y z | nx ny nz (0) | f_dc_0..2 = A | f_rest_0..3K-1, channel-major:
//   f_rest[c K + k] = k_j[n][k][c] (run.py:98-108: transpose(1, 2) then
//   flatten) | opacity | scale_0..2 = s | rot_0..3 = q / max(|q|, 1e-8)
// opacity is the stored logit, or (a legacy checkpoint of probabilities,
// run.py:110-118) log(a / (1 - a)) of a clamped to [1e-6, 1 - 1e-6].
//
// One work-group of 256 threads per 64 Gaussians: the inputs of its 64
// Gaussians are contiguous in HBM and are read with coalesced loads straight
// into their places in the 64 records staged in LDS; the 64 records are then
// stored as one contiguous run.  |q| sums the squares in order in fp32 as
// torch's norm over the last dimension does, with a square root rounded to
// nearest; the divisions are correctly rounded.
#include <hip/hip_runtime.h>

#include "gsr_common.h"
#include "gsr_internal.h"

namespace gsr {

namespace {

constexpr int kPackThreads = 256;
constexpr int kPackGaussians = 64;

__global__ __launch_bounds__(kPackThreads) void ply_pack_kernel(
    int n, int K, const float* __restrict__ mu, const float* __restrict__ q,
    const float* __restrict__ s, const float* __restrict__ alpha, const float* __restrict__ A,
    const float* __restrict__ kj, int from_probability, float* __restrict__ out) {
    extern __shared__ float s_rec[];  // kPackGaussians records
    const int R = 17 + 3 * K;
    const int tid = threadIdx.x;
    const int g0 = blockIdx.x * kPackGaussians;
    const int cnt = min(kPackGaussians, n - g0);
    // contiguous inputs of the block's Gaussians, each to its record columns
    for (int e = tid; e < cnt * 3; e += kPackThreads) {
        const int g = e / 3, j = e - 3 * g;
        const size_t src = (size_t)g0 * 3 + e;
        s_rec[g * R + j] = mu[src];
        s_rec[g * R + 3 + j] = 0.0f;
        s_rec[g * R + 6 + j] = A[src];
        s_rec[g * R + 10 + 3 * K + j] = s[src];
    }
    const int kr = 3 * K;
    for (int e = tid; e < cnt * kr; e += kPackThreads) {
        const int g = e / kr, r = e - kr * g;
        const int k = r / 3, c = r - 3 * k;
        s_rec[g * R + 9 + c * K + k] = kj[(size_t)g0 * kr + e];
    }
    if (tid < cnt) {
        const int g = tid;
        const float a = alpha[(size_t)g0 + g];
        float op = a;
        if (from_probability) {
            const float ac = fminf(fmaxf(a, 1e-6f), 1.0f - 1e-6f);
            op = (float)log((double)(ac / (1.0f - ac)));
        }
        s_rec[g * R + 9 + kr] = op;
        const float4 qq = reinterpret_cast<const float4*>(q)[(size_t)g0 + g];
        // torch's fp32 vector norm of four elements: the squares summed in order
        const float n2 = ((qq.x * qq.x + qq.y * qq.y) + qq.z * qq.z) + qq.w * qq.w;
        const float nrm = fmaxf(sqrt_rn(n2), 1e-8f);
        float* rot = s_rec + g * R + 13 + kr;
        rot[0] = qq.x / nrm;
        rot[1] = qq.y / nrm;
        rot[2] = qq.z / nrm;
        rot[3] = qq.w / nrm;
    }
    __syncthreads();
    float* dst = out + (size_t)g0 * R;
    for (int e = tid; e < cnt * R; e += kPackThreads) dst[e] = s_rec[e];
}

}  // namespace

hipError_t launch_ply_pack(int n, int K, const float* mu, const float* q, const float* s,
                           const float* alpha, const float* A, const float* kj,
                           int from_probability, float* out, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    const size_t lds = sizeof(float) * kPackGaussians * (size_t)(17 + 3 * K);
    hipLaunchKernelGGL(ply_pack_kernel, dim3((unsigned)((n + kPackGaussians - 1) / kPackGaussians)),
                       dim3(kPackThreads), lds, st, n, K, mu, q, s, alpha, A, kj, from_probability,
                       out);
    return hipGetLastError();
}

}  // namespace gsr
